// BSCK decode: the GPU-native chunked entropy-coded format of the BigSmall
// decode engine, decoded on CDNA4 (gfx950), with either of two coders.
//
// Format (little-endian; produced by bsck_encode.cpp):
//   [0]  "BSCK"  [4] u8 version (3; 2 = the earlier chunk-contiguous layout,
//        read too)  [5] u8 elem_bytes (1|2)  [6] u8 plane_mode
//   [7]  u8 prec_log2 = 12  [8] u64 n  [16] u32 steps  [20] u16 lanes = 64*K
//   [22] u16 n_syms  [24] u32 n_chunks  [28] u8 coder (0 rANS; tANS: 1 with a
//        state array, 2 with the states at the stream head), 3 zero bytes
//   [32] n_syms x u32 symbol entries: bits 0..15 output value (bf16 word with
//        zero sign/mantissa for exponent symbols, the exact word/byte, or an
//        exponent pair e0 | e1 << 4), bits 16..28 quantised frequency (sum
//        4096), bit 31 = reads one plane byte
//   pad to 16; tANS only: 4096 x u32 decode table {newX:12, nb:4, symbol:8, 0:8}
//   n_chunks x {u64 offset, u32 n_words (rANS: renorm words; tANS: stream
//        bits), u32 n_plane}
//   pad to 256; plane_mode 1 and 3 only: the dense plane region, nf*per bytes
//   chunk (16-aligned): 64*K x u32 initial states (state v = g*64 + l; not
//        in coder 2) | the stream (rANS: n_words x u16 renorm words; tANS:
//        whole u32 words of an LSB-first bit stream, in coder 2 starting with
//        the 12-bit initial states, lane l's state g at bit 12*(l*K + g)),
//        pad 16 | n_plane plane bytes (pad 16), the plane bytes omitted for a
//        full chunk in plane_mode 1 and 3
//   pad to 256 (the blob length is a multiple of 256; coder 2: and at least
//        the last chunk's offset + 256, so 256 bytes from any chunk's start
//        are inside the blob)
// Version 2 has no plane region (every plane inline), coder 0, no plane mode
// 3, chunks holding contiguous elements (c*per + j) and 16-byte padding.
//
// Chunks and elements: per = 64*K*steps coded elements per chunk (at most
// 2^24), nf = ne / per full chunks (ne = n, or n / 2 in plane mode 3, whose
// coded elements are byte pairs), and a partial chunk (c = nf) when per does
// not divide ne. A full chunk's elements are 512-element units of the tensor
// interleaved across the full chunks: chunk element j is tensor element
// ((j/512)*nf + c)*512 + j%512. The partial chunk holds the tail: chunk
// element j is element nf*per + j. The chunks that run side by side therefore
// read and write neighbouring addresses, which the memory system serves faster
// than one separate stream per chunk. The dense planes of the full chunks are
// interleaved the same way, per plane block (B*64*K bytes, below): block b of
// full chunk c is block b*nf + c of the plane region.
//
// A chunk is decoded by one wavefront. Lane l owns K interleaved states
// (g = 0..K-1); at step t state (g, l) decodes element t*64K + l*K + g of the
// chunk, so a lane's K outputs of a step are adjacent and one step of the
// wavefront produces 64*K consecutive elements.
// Plane bytes complete the symbols that have one:
//   plane_mode 1 (dense): every element has one (sign<<7 | mantissa of a bf16
//                         word), stored per block of B steps (B = 8 for
//                         K <= 2, 4 for K = 4) with lane l's B*K bytes
//                         contiguous, step-major (byte q*K+g); the blocks of a
//                         full chunk in the plane region, of the partial chunk
//                         inline;
//   plane_mode 3 (pairs): as mode 1, the plane byte of a pair of fp8 e4m3
//                         bytes being m0 | s1 << 3 | m1 << 4 | s0 << 7;
//   plane_mode 2 (compact): only elements whose symbol has bit 31 set have one,
//                         in decode order (rANS: a byte area after the words,
//                         ballot + mbcnt placed; tANS: 8 bits in the stream
//                         after the element's state bits);
//   plane_mode 0: no plane (every symbol is an exact value).
//
// rANS (coder 0; the reference's state machine, bigsmall/codecs/rans.py:165-207:
// 32-bit state, L = 2^16, 16-bit renormalisation, M = 2^12):
//   slot = x & 4095; s = sym(slot); x = f[s]*(x>>12) + slot - cf[s];
//   if x < L: x = (x << 16) | next_word
// The 64*K states share one 16-bit renorm word stream, consumed per step
// group by group (g ascending), lanes ascending among the lanes whose state
// fell below L = 2^16; the words are placed with a wavefront ballot + mbcnt
// prefix. A valid chunk ends with every state back at x == L and every word
// and plane byte consumed.
// tANS (coders 1 and 2): X in [0, 4096); e = table[X]; s = e's symbol;
//   X = newX | next nb bits  (newX has nb zero low bits)
// Each step every lane reads its K states' bits in order (and a compact
// symbol's 8 plane bits after its state bits) from one stream position:
// the wavefront's inclusive prefix sum of the lanes' bit counts (DPP). A
// valid chunk ends with every X == 0 and every bit read.
// Anything else is reported as BS_DEV_ERR_STREAM.
//
// Decode-table layouts in LDS (4096 slots):
//   rANS dense bf16 (plane_mode 1): {f | exponent << 24, slot - cf}; the update is
//     one shift and one v_mad_u32_u24 (which ignores bits 24..31 of f's word),
//     and the exponent byte is placed with v_perm;
//   rANS bytes and pairs (elem_bytes 1): {f | value << 24, slot - cf}, the same
//     update, the output byte taken from bits 24..31 with v_perm;
//   rANS generic (bf16 plane modes 0/2): {f, value | (slot - cf) << 16 | consume << 31};
//     the update is one shift, one bit-field extract and one v_mad_u32_u24;
//   tANS dense: one word {newX:12, nb:4, exponent word (e << 7):16};
//   tANS pairs: one word {newX:12, nb:4, e0 << 3 | e1 << 11:16};
//   tANS bytes: one word {newX:12, nb:4, -:8, byte:8};
//   tANS generic: {newX | nb << 12 | mask << 16, nt | value << 16}: nt = nb + raw bits, and
//     mask = 0x807F for a compact-mode symbol that takes a plane byte (raw = 8), else 0.
#include <stdint.h>

#include "simt.h"

#include "../../include/bigsmall_hip.h"
#include "lds_limit.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr uint32_t kVersion = 3;
constexpr uint32_t kUnit = 512;           // elements per interleave unit of the output
constexpr int kWave = 64;                 // lanes of a wavefront
#ifndef BSCK_WAVES
#define BSCK_WAVES 8
#endif
constexpr int kWaves = BSCK_WAVES;        // chunks (wavefronts) per workgroup
constexpr int kThreads = kWaves * kWave;
static_assert(kThreads >= 256, "the table build reads one symbol entry per thread (up to 256)");
// Steps per block (dense-plane block, refill check): 8 for K <= 2 states per
// lane, 4 for K = 4, so a block is at most 1024 elements (1024 renorm words of
// worst-case demand) and a lane's plane bytes of a block are 16 bytes.
template <int K>
constexpr int block_steps() { return K == 4 ? 4 : 8; }
constexpr int kBlockMax = 8;
constexpr uint32_t kMirror = 64;          // word-ring entries [0, 64) are mirrored after the ring end
constexpr uint32_t kPMirror = 64;         // compact plane-ring bytes [0, 64) likewise
// per-wave ring area: a 2048-word ring and its mirror, or (compact chunks) a
// 1024-word ring and its mirror, a 2048-byte plane ring and its mirror, and a
// 16-byte zero slot that non-consuming lanes read as their plane byte
constexpr uint32_t kRingBytes = (1024 + kMirror) * 2 + 2048 + kPMirror + 16;
static_assert(kRingBytes >= (2048 + kMirror) * 2, "ring area");
constexpr uint32_t kL = 1u << 16;
// elements per chunk at most (lanes * steps): byte offsets inside a chunk fit 32 bits
constexpr uint64_t kMaxChunk = 1ull << 24;
// s_waitcnt immediate for gfx9: vmcnt(n), expcnt and lgkmcnt not waited on
// (vmcnt bits 3:0 and 15:14, expcnt bits 6:4, lgkmcnt bits 11:8)
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// dynamic LDS layout (bytes): per-wave ring areas | decode table | per-wave
// output staging. The rings come first, so a wave's ring starts at one
// wave-uniform offset (wave * kRingBytes) and a ring read's address is that
// plus the word offset, one instruction; the table's fixed offset fits the
// immediate offset field of its reads.
constexpr uint32_t kTblBytes = 4096 * 8;
constexpr uint32_t kTblOff = kWaves * kRingBytes;
constexpr uint32_t kStageMax = 1024;      // per wave: half a block of bf16 outputs (512 elements)
static_assert(kTblOff % 16 == 0 && kTblOff <= 65535, "table offset in a ds_read immediate");
// each wave's progress in block pairs (u16 per wave), read by the others
constexpr uint32_t kProgOff = kTblOff + kTblBytes + kWaves * kStageMax;
// a workgroup-wide flag set by any thread whose run of a tANS table fails its check
constexpr uint32_t kFlagOff = kProgOff + ((2 * kWaves + 15) & ~15u);
constexpr uint32_t kLds = kFlagOff + 16;           // 75424: two workgroups per CU
constexpr uint32_t kTansSlots = 4096;              // tANS table positions (12-bit states)

template <bool HALF> struct SegVec { typedef u32x4 T; };
template <> struct SegVec<true> { typedef u32x2 T; };

// Ring geometry of a chunk. Plane modes 0 and 1 use the whole ring area as a
// 2048-word renorm ring, refilled in 512-word segments (64 lanes x 16 bytes),
// with blocks of block_steps<K>() steps (up to 1024 elements). Compact-plane
// chunks (mode 2) run at half scale: blocks of 512 elements, a 1024-word renorm
// ring and a 2048-byte plane ring sharing the same area, segments of 64 lanes x
// 8 bytes. Every ring then holds the same multiple of a block's worst-case
// demand, and a compact launch needs no more LDS than any other (two
// workgroups per CU).
template <int K, int MODE>
struct Geo {
  static constexpr bool kHalf = MODE == 2;
  static constexpr int kBlock = kHalf ? 8 / K : block_steps<K>();
  static constexpr uint32_t kBlkElems = (uint32_t)kBlock * kWave * K;   // worst-case words/plane bytes per block
  static constexpr uint32_t kRing = kHalf ? 1024 : 2048;                 // renorm-word ring entries
  static constexpr uint32_t kLaneSeg = kHalf ? 8 : 16;                   // bytes per lane per segment
  static constexpr uint32_t kWSeg = kLaneSeg * kWave / 2;                // words per segment
  static constexpr uint32_t kPRing = 2048;                               // plane ring bytes (mode 2)
  static constexpr uint32_t kPSeg = kLaneSeg * kWave;                    // plane bytes per segment
  static constexpr uint32_t kPRingOff = (kRing + kMirror) * 2;           // plane ring offset in the ring area
  static constexpr uint32_t kPZero = kPRing + kPMirror;                  // zero slot, from the plane ring
  typedef typename SegVec<kHalf>::T Seg;
  static_assert(!kHalf || kPRingOff + kPZero + 16 <= kRingBytes, "compact rings exceed the ring area");
  static_assert(kHalf || (kRing + kMirror) * 2 <= kRingBytes, "word ring exceeds the ring area");
};

// rank of this lane among the set lanes of m
__device__ __forceinline__ uint32_t lane_rank(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Workgroup barrier that publishes LDS only: its fences cover the LDS address
// space, so loads from global memory issued before it stay in flight across
// it (__syncthreads() also waits for every outstanding vector-memory load).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Makes the values available at this point: every load producing them is
// issued before it, and nothing can sink them under a later branch.
template <int K>
__device__ __forceinline__ void consume(const uint32_t (&v)[K]) {
  if (K == 1) BS_KEEP1(v[0]);
  if (K == 2) BS_KEEP2(v[0], v[K - 1]);
  if (K == 4) BS_KEEP4(v[0], v[1 % K], v[2 % K], v[3 % K]);
}

__device__ __forceinline__ uint32_t pad16(uint32_t v) { return (v + 15u) & ~15u; }

// readfirstlane of a 32-bit value, as unsigned (the builtin returns int, and
// widening an int to 64 bits would copy its bit 31 into the high half)
__device__ __forceinline__ uint32_t rfl(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

// The builtin returns int: each half goes through uint32_t so that the low
// half is zero-extended (a plain cast would copy its bit 31 into the high half).
__device__ __forceinline__ uint64_t readlane64(uint64_t v, uint32_t l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, (int)l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), (int)l);
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

__device__ __forceinline__ void report(int32_t* status, int32_t bits) {
  if (__lane_id() == 0) atomicOr(status, bits);
}

__device__ __forceinline__ uint32_t byte_merge(uint32_t v, uint32_t b) { return ((b * 0x101u) & 0x807Fu) | v; }

// Inclusive prefix sum over the wavefront's 64 lanes: DPP adds of the value
// 1, 2, 4 and 8 lanes below within each 16-lane row, then of lane 15's row
// total into rows 1 and 3 and of lane 31's (rows 0-1) into rows 2 and 3.
// Six VALU instructions; lanes without a source add 0.
__device__ __forceinline__ uint32_t wave_prefix_sum(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);   // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);   // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);   // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);   // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);   // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);   // row_bcast:31
  return v;
}

// 32 bits of a tANS chunk's stream from bit `pos` (LSB first), out of the
// wave's word ring seen as 1,024 u32 words: two ring words, the second
// covered by the ring's mirrored head when the first is the last.
__device__ __forceinline__ uint32_t stream_bits(const LDS uint32_t* ring, uint32_t pos) {
  uint32_t w;
  BS_BFE_U32(w, pos, 5, 10);                            // (pos >> 5) & 1023: the address is then one lshl_add
  return __builtin_amdgcn_alignbit(ring[w + 1], ring[w], pos);   // shifts by pos mod 32
}

// ---- ring refills. A segment is 64 lanes x Geo::kLaneSeg bytes; segment
// positions are multiples of the segment size.

// Load this lane's part of the segment at `pos` (in units of V); out-of-range
// lanes read `safe` (the chunk's state words, 256 bytes or more, always in
// bounds), so every call issues exactly one load per lane. The source lies
// after `safe` inside the chunk, so the lane's address is one 32-bit offset
// from the wave-uniform `safe` (a select of two offsets, not of two 64-bit
// addresses).
template <typename V>
__device__ __forceinline__ V load_seg(const GLB uint8_t* src, uint32_t pos, uint32_t valid, uint32_t lane,
                                      const GLB uint8_t* safe) {
  const uint32_t slot = pos + lane;
  const uint32_t src_off = (uint32_t)(src - safe) + pos * (uint32_t)sizeof(V);   // wave-uniform
  const uint32_t off = slot < valid ? src_off + lane * (uint32_t)sizeof(V)
                                    : (lane & (256u / sizeof(V) - 1u)) * (uint32_t)sizeof(V);
  return *(const GLB V*)(safe + off);
}
// Word ring: words [0, kMirror) also live at [kRing, kRing + kMirror), so a
// read at (ring position mod kRing) + rank, rank < 64, never wraps.
template <class G>
__device__ __forceinline__ void store_wseg(LDS uint16_t* ring, uint32_t pos, typename G::Seg v, uint32_t lane) {
  const uint32_t r = (pos + lane * (G::kLaneSeg / 2u)) & (G::kRing - 1u);
  *(LDS typename G::Seg*)(ring + r) = v;
  if (r < kMirror) *(LDS typename G::Seg*)(ring + G::kRing + r) = v;
}
// Plane ring (compact chunks): bytes [0, kPMirror) also live after the ring
// end, so a read at (ring position mod kPRing) + rank, rank < 64, never wraps.
template <class G>
__device__ __forceinline__ void store_pseg(LDS uint8_t* ring, uint32_t pos, typename G::Seg v, uint32_t lane) {
  const uint32_t r = (pos + lane * G::kLaneSeg) & (G::kPRing - 1u);
  *(LDS typename G::Seg*)(ring + r) = v;
  if (r < kPMirror) *(LDS typename G::Seg*)(ring + G::kPRing + r) = v;
}

template <int K>
struct PlaneRegs {   // dense plane bytes of one block: 8 (K = 1) or 16 (K = 2, 4) per lane
  static constexpr int kWords = K == 1 ? 1 : 2;
  uint64_t b[kWords];
};
template <int K>
__device__ __forceinline__ PlaneRegs<K> load_plane(const GLB uint8_t* dplane, uint64_t stride, uint32_t blk,
                                                   uint32_t lane) {
  PlaneRegs<K> r;
  constexpr uint32_t kLaneBytes = block_steps<K>() * K;   // 8 (K=1) or 16 (K=2, 4)
  const GLB uint8_t* p = dplane + (uint64_t)blk * stride + lane * kLaneBytes;
  if (kLaneBytes == 16) {
    // Streaming load: a dense plane block is read once, in whole 256-byte
    // aligned lines, so it need not stay in the caches (8B-shaped layer:
    // 141.7 -> 140.7 us per launch). The renorm-word segments keep normal
    // loads (152.9 us with streaming loads; likely because a segment that a
    // wave does not need is issued as a load of its chunk's state words,
    // which then stop being cache hits).
    const u32x4 v = __builtin_nontemporal_load((const GLB u32x4*)p);
    r.b[0] = (uint64_t)v.x | ((uint64_t)v.y << 32);
    r.b[PlaneRegs<K>::kWords - 1] = (uint64_t)v.z | ((uint64_t)v.w << 32);
  } else {
    r.b[0] = *(const GLB uint64_t*)p;
  }
  return r;
}

template <int K>
__device__ __forceinline__ void consume_plane(const PlaneRegs<K>& p) {
  if (PlaneRegs<K>::kWords == 1) BS_KEEP1(p.b[0]);
  else BS_KEEP2(p.b[0], p.b[PlaneRegs<K>::kWords - 1]);
}

// Per-wavefront decode state of one chunk.
template <int K>
struct ChunkState {
  uint32_t x[K];         // rANS states, or tANS states X in [0, 4096)
  uint32_t wptr, wld;    // word ring holds words [wptr, wld)
  uint32_t pptr, pld;    // plane ring (compact mode) holds bytes [pptr, pld)
  uint32_t bpos;         // tANS: bits of the chunk's stream read so far
};

// Loads issued at a pair start (two blocks) and landed at the next one: up to
// two word-ring segments, up to two compact-plane segments, and the dense
// plane of the next pair's two blocks. Every load is issued unconditionally
// (unneeded ones read an always-valid dummy address) so the wait counts are
// the same on every path.
template <int K, int MODE>
struct Inflight {
  typename Geo<K, MODE>::Seg w[2], p[2];
  bool wn[2], pn[2];
  PlaneRegs<K> pl[2];
};

// Chunk-constant parameters.
struct ChunkParams {
  const GLB uint8_t* wsrc;      // renorm words
  const GLB uint8_t* psrc;      // compact plane
  const GLB uint8_t* dplane;    // dense plane block 0: B*K bytes per lane per block of B steps
  uint64_t pstride;             // bytes from one dense plane block of the chunk to its next
  const GLB uint8_t* safe;      // the chunk's state words: an always-valid dummy address
  GLB uint8_t* out8;
  uint64_t ubase, ustride;      // chunk element j is element (j/512)*ustride + ubase + j%512
  uint32_t n_words, n_plane;
  uint32_t wvalid, pvalid;      // readable words / plane bytes, in segment-lane units
  uint32_t nc, nsteps, nblk, lane;
};

// Store the staged outputs of half-block `hb` (HS steps) to the output.
template <int K, int EB, bool PARTIAL, int HS>
__device__ __forceinline__ void flush_half(uint32_t hb, const ChunkParams& C, LDS uint8_t* stage) {
  constexpr uint32_t kBlkElems = (uint32_t)HS * kWave * K;
  constexpr uint32_t kBlkBytes = kBlkElems * EB;
  const uint32_t e0 = hb * kBlkElems;                  // a half block lies inside one 512-element unit
  const uint64_t blk_byte0 = ((uint64_t)(e0 / kUnit) * C.ustride + C.ubase + e0 % kUnit) * EB;
  // Streaming stores: the decoded tensor is far larger than the L2 (the hint
  // measured 3-4% faster than plain stores on an 8B layer). A full chunk's
  // half block is 256, 512 or 1024 bytes: every lane stores its 4, 8 or 16
  // bytes with one unconditional instruction, which keeps the wait counts of
  // the pipeline exact.
  if (!PARTIAL) {
    static_assert(kBlkBytes == 256 || kBlkBytes == 512 || kBlkBytes == 1024, "half block size");
    constexpr uint32_t kLB = kBlkBytes / kWave;
    const uint32_t o = C.lane * kLB;
    if (kLB == 16) {
      const u32x4 d = *(const LDS u32x4*)(stage + o);
      __builtin_nontemporal_store(d, (GLB u32x4*)(C.out8 + blk_byte0 + o));
    } else if (kLB == 8) {
      const uint64_t d = *(const LDS uint64_t*)(stage + o);
      __builtin_nontemporal_store(d, (GLB uint64_t*)(C.out8 + blk_byte0 + o));
    } else {
      const uint32_t d = *(const LDS uint32_t*)(stage + o);
      __builtin_nontemporal_store(d, (GLB uint32_t*)(C.out8 + blk_byte0 + o));
    }
    return;
  }
  const uint32_t valid_bytes = min(kBlkBytes, (C.nc - min(C.nc, hb * kBlkElems)) * EB);
#pragma unroll
  for (uint32_t i = 0; i < (kBlkBytes + 1023) / 1024; ++i) {
    const uint32_t o = i * 1024u + C.lane * 16u;
    if (o + 16u <= valid_bytes) {
      const u32x4 d = *(const LDS u32x4*)(stage + o);
      *(GLB u32x4*)(C.out8 + blk_byte0 + o) = d;
    } else if (o < valid_bytes) {
      for (uint32_t k = o; k < min(o + 16u, valid_bytes); ++k) C.out8[blk_byte0 + k] = stage[k];
    }
  }
}

// Full chunks with K >= 2 store each step's outputs straight from registers:
// a step's 64*K elements are contiguous in the output (a quarter or half of a
// 512-element unit), so every lane writes its K adjacent elements (4 or 8
// bytes of bf16, 2 or 4 bytes of fp8) and the wavefront writes 128 to 512
// contiguous bytes, whole cache lines, with no LDS staging. K = 1 and the
// partial chunk stage their outputs in LDS and store whole half blocks.
template <int K, int EB, bool PARTIAL>
constexpr bool direct_stores() { return !PARTIAL && K >= 2; }

// Output stores a chunk issues per pair of blocks (the pipeline's wait counts).
template <int K, int MODE, int EB, bool PARTIAL>
constexpr int stores_per_pair() { return direct_stores<K, EB, PARTIAL>() ? 2 * Geo<K, MODE>::kBlock : 4; }

// Store step q of block blk (KB steps per block): lane l's K words go to
// chunk elements t*64K + l*K .. +K-1, t = blk*KB + q, which lie in 512-element
// unit t*K/8 at offset (t*K % 8)*64.
template <int K, int KB, int EB>
__device__ __forceinline__ void store_step(const ChunkParams& C, uint32_t blk, int q, uint32_t v0, uint32_t v1) {
  static_assert((KB * K) % 8 == 0, "a block is whole units");
  const uint32_t unit = blk * (uint32_t)(KB * K / 8) + (uint32_t)(q * K / 8);   // wave-uniform
  GLB uint8_t* p = C.out8 + ((uint64_t)unit * C.ustride + C.ubase) * EB + (uint32_t)((q * K) % 8) * (64u * EB) +
                   C.lane * (EB * K);
  if (EB * K == 2) __builtin_nontemporal_store((uint16_t)v0, (GLB uint16_t*)p);
  else if (EB * K == 4) __builtin_nontemporal_store(v0, (GLB uint32_t*)p);
  else __builtin_nontemporal_store((uint64_t)v0 | ((uint64_t)v1 << 32), (GLB uint64_t*)p);
}

// One step of the K states of every lane. Phased so the K dependency chains of
// a lane overlap: K table reads, then the K state updates with their ballots,
// then the K ring reads (one wait for all), then the renormalisations.
// FAST = dense bf16 or byte table layout (d = the table word holding the
// exponent or byte in bits 24..31); otherwise d = value | consume << 31, and
// for MODE 2 the compact-plane byte
// of each consuming element is read beside the renorm words (same wait) and
// merged into d.
template <int K, int MODE, bool FAST, bool PARTIAL>
__device__ __forceinline__ void rans_step(uint32_t t, ChunkState<K>& S, const ChunkParams& C,
                                          const LDS uint64_t* __restrict__ tbl, const LDS uint16_t* wring,
                                          const LDS uint8_t* pring, uint32_t (&d)[K]) {
  typedef Geo<K, MODE> G;
  uint64_t e[K];
#pragma unroll
  for (int g = 0; g < K; ++g) e[g] = tbl[S.x[g] & 4095u];
  uint32_t xn[K], w[K], pb[K];
  bool need[K], cons[K];
  uint32_t pos = S.wptr, ppos = S.pptr;
#pragma unroll
  for (int g = 0; g < K; ++g) {
    const uint32_t lo = (uint32_t)e[g], hi = (uint32_t)(e[g] >> 32);
    if (FAST) {
      xn[g] = __umul24(lo, S.x[g] >> 12) + hi;             // v_mad_u32_u24: f = bits 0..23 of lo
      d[g] = lo;                                           // exponent or byte value in byte 3
    } else {
      xn[g] = __umul24(lo, S.x[g] >> 12) + ((hi >> 16) & 0xFFFu);
      d[g] = hi;                                           // value | (slot - cf) << 16 | consume << 31
    }
    bool act = true;
    if (PARTIAL) {
      act = t * (kWave * K) + C.lane * K + g < C.nc;
      if (!act) xn[g] = S.x[g];
    }
    need[g] = xn[g] < kL;
    const uint64_t m = __ballot(need[g]);
    w[g] = wring[(pos & (G::kRing - 1u)) + lane_rank(m)];   // < kRing + 64: the mirror covers it
    pos += (uint32_t)__popcll(m);
    if (MODE == 2) {
      // plane bytes follow decode order: groups ascending, then lanes ascending;
      // a non-consuming lane reads the zero slot, so the merge below needs no select
      cons[g] = act && (int32_t)hi < 0;
      const uint64_t cm = __ballot(cons[g]);
      // ring position + rank (< kPRing + 64: the mirror covers it), the position
      // added by mbcnt's accumulator
      const uint32_t at = __builtin_amdgcn_mbcnt_hi((uint32_t)(cm >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)cm, ppos & (G::kPRing - 1u)));
      pb[g] = pring[cons[g] ? at : G::kPZero];
      ppos += (uint32_t)__popcll(cm);
    }
  }
  consume<K>(w);
  if (MODE == 2) consume<K>(pb);
  S.wptr = pos;
  if (MODE == 2) S.pptr = ppos;
#pragma unroll
  for (int g = 0; g < K; ++g) {
    S.x[g] = need[g] ? ((xn[g] << 16) | w[g]) : xn[g];
    if (MODE == 2) d[g] = byte_merge(d[g], pb[g]);       // pb = 0 for a non-consuming element
  }
}

// One tANS step of the K states of every lane. Table entries: FAST (dense
// bf16, bytes, exponent pairs) {newX:12, nb:4, -:8, output byte:8}, 4 bytes;
// otherwise {lo: newX:12, nb:4, mask:16; hi: nt:5, -:11, value:16}, 8 bytes,
// nt = nb + raw with raw = 8 for a compact-mode symbol that takes a plane
// byte, whose mask is then 0x807F (else 0). Each lane reads its states' bits
// in order (state bits, then raw plane bits) from one stream position per
// lane: the wavefront prefix sum of the lanes' bit counts. newX has nb low
// zero bits, so X = newX | bits. d as for rans_step for FAST; for the generic
// layout the output word is d's high half: (8 bits after the state bits,
// duplicated into bytes 2 and 3) & lo | hi, which leaves the value alone when
// the mask is 0 and merges the plane byte's sign and mantissa when it is
// 0x807F, with no step spent on the raw count (hi's nt, in bits 0..4, is the
// alignbit shift as it stands).
//
// In compact chunks (MODE 2) the step calls `ensure` with the ring words it
// reads once their count is known: the block-level refill checks only
// 6 bits per element there (a compact symbol takes up to 20), and ensure
// lands the rest in the step that needs it.
template <int K, int MODE, bool FAST, bool PARTIAL, class Ensure>
__device__ __forceinline__ void tans_step(uint32_t t, ChunkState<K>& S, const ChunkParams& C, const LDS void* tbl,
                                          const LDS uint32_t* ring, uint32_t (&d)[K], Ensure&& ensure) {
  uint32_t e[K], hv[K], nb[K], nt[K];
  bool act[K];
  uint32_t tot = 0;
#pragma unroll
  for (int g = 0; g < K; ++g) {
    if (FAST) {
      e[g] = ((const LDS uint32_t*)tbl)[S.x[g]];
      hv[g] = 0;
    } else {
      const uint64_t v = ((const LDS uint64_t*)tbl)[S.x[g]];
      e[g] = (uint32_t)v;
      hv[g] = (uint32_t)(v >> 32);
    }
    nb[g] = __builtin_amdgcn_ubfe(e[g], 12, 4);
    // generic layout: hv itself, whose low half is nt (bits 0..4) and whose
    // high half the value: a lane's sum of at most 4 x 20 bits, and the
    // wavefront's of at most 5,120, never carry into bit 16, so the sums' low
    // halves are the bit counts and their high halves are ignored
    nt[g] = FAST ? nb[g] : hv[g];
    act[g] = true;
    if (PARTIAL) {
      act[g] = t * (kWave * K) + C.lane * K + g < C.nc;
      if (!act[g]) nb[g] = nt[g] = 0;
    }
    tot += nt[g];
  }
  const uint32_t incl = wave_prefix_sum(tot);
  // this lane's first bit; generic layout: exact in bits 0..15, of which the
  // step reads bits 0..14 (the ring word, 1024 words, and the shift), the
  // high half carrying the values' sums
  uint32_t pos = S.bpos + incl - tot;
  S.bpos += (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1) & (FAST ? 0xFFFFFFFFu : 0xFFFFu);
  S.wptr = (S.bpos >> 5) << 1;                          // ring words no longer needed: [.., wptr)
  if constexpr (MODE == 2) ensure(((S.bpos + 31u) >> 5) << 1);   // the ring words up to the step's last bit
  // The lane's states are read in pairs: a one-word-layout pair takes at most
  // 2 x 12 bits (one 32-bit window), a generic pair at most 2 x 20 (a 64-bit
  // window from three ring words, the second state's bits funnel-shifted out
  // of it).
#pragma unroll
  for (int g = 0; g < K; g += 2) {
    const bool two = g + 1 < K;
    if (FAST) {
      const uint32_t win = stream_bits(ring, pos);
      const uint32_t x0 = (e[g] & 0xFFFu) | __builtin_amdgcn_ubfe(win, 0, nb[g]);
      S.x[g] = PARTIAL && !act[g] ? S.x[g] : x0;
      d[g] = e[g];
      if (two) {
        const uint32_t x1 = (e[g + 1] & 0xFFFu) | __builtin_amdgcn_ubfe(win, nb[g], nb[g + 1]);
        S.x[g + 1] = PARTIAL && !act[g + 1] ? S.x[g + 1] : x1;
        d[g + 1] = e[g + 1];
        if (g + 2 < K) pos += nb[g] + nb[g + 1];
      }
    } else {
      uint32_t w;
      BS_BFE_U32(w, pos, 5, 10);
      const uint32_t r0 = ring[w], r1 = ring[w + 1];
      const uint32_t lo = __builtin_amdgcn_alignbit(r1, r0, pos);
      uint32_t win[2] = {lo, lo};
      if (two) {
        // bits 32..63 from `pos` come from the third word (w + 2 <= 1025:
        // inside the ring's mirrored head)
        const uint32_t hi = __builtin_amdgcn_alignbit(ring[w + 2], r1, pos);
        // from bit nt[g] on (nt <= 20): alignbit shifts by its operand's low 5 bits, hv's nt
        win[1] = __builtin_amdgcn_alignbit(hi, lo, hv[g]);
      }
#pragma unroll
      for (int h = 0; h < (two ? 2 : 1); ++h) {
        const int gg = g + h;
        const uint32_t x = (e[gg] & 0xFFFu) | __builtin_amdgcn_ubfe(win[h], 0, nb[gg]);
        S.x[gg] = PARTIAL && !act[gg] ? S.x[gg] : x;
        // the plane byte follows the state bits; the mask drops it for a symbol without one
        if (MODE == 2) {
          const uint32_t b = __builtin_amdgcn_ubfe(win[h], nb[gg], 8);
          d[gg] = (__builtin_amdgcn_perm(0u, b, 0x00000C0Cu) & e[gg]) | hv[gg];
        } else {
          d[gg] = hv[gg];
        }
      }
      if (g + 2 < K) pos += nt[g] + (two ? nt[g + 1] : 0u);
    }
  }
}

// Ring upkeep and prefetch, at block granularity.
//
// Word-ring and compact-plane segments are requested at a pair start (every
// other block) when the ring has room, and landed at the next pair start: the
// two blocks in between cover their latency. So does the dense plane, loaded
// one pair ahead. The output stores of a block (mid-block and at its end)
// come after the pair's loads; on gfx9 one vector-memory counter covers loads
// and stores and retires in issue order, so waiting for the loads at the next
// pair start leaves the four stores of the pair in flight.

// Land the in-flight ring segments, in request order.
template <int K, int MODE>
__device__ __forceinline__ void land_segments(ChunkState<K>& S, Inflight<K, MODE>& F, LDS uint16_t* wring,
                                              LDS uint8_t* pring, uint32_t lane) {
  typedef Geo<K, MODE> G;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    if (F.wn[i]) { store_wseg<G>(wring, S.wld, F.w[i], lane); S.wld += G::kWSeg; F.wn[i] = false; }
  if (MODE == 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (F.pn[i]) { store_pseg<G>(pring, S.pld, F.p[i], lane); S.pld += G::kPSeg; F.pn[i] = false; }
  }
}

// Request up to two segments per ring (as many as fit behind the unconsumed
// and landed data).
template <int K, int MODE>
__device__ __forceinline__ void request_segments(const ChunkState<K>& S, Inflight<K, MODE>& F, const ChunkParams& C) {
  typedef Geo<K, MODE> G;
  typedef typename G::Seg V;
  const uint32_t lane = C.lane;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t at = S.wld + i * G::kWSeg;
    F.wn[i] = at < C.n_words && at + G::kWSeg - S.wptr <= G::kRing;
    F.w[i] = load_seg<V>(C.wsrc, F.wn[i] ? at / (G::kLaneSeg / 2u) : 0u, C.wvalid, lane, C.safe);
  }
  if (MODE == 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t at = S.pld + i * G::kPSeg;
      F.pn[i] = at < C.n_plane && at + G::kPSeg - S.pptr <= G::kPRing;
      F.p[i] = load_seg<V>(C.psrc, F.pn[i] ? at / G::kLaneSeg : 0u, C.pvalid, lane, C.safe);
    }
  }
}

// Make sure the rings hold a block's worst-case demand. Rare: it lands the
// in-flight segments early (waiting for them) and loads synchronously. A
// block needs at most one renorm word per element (rANS), or MAXB bits per
// element (tANS: 12, a state's worst case) plus the second word of the last
// 32-bit window, in ring words; compact tANS blocks ask for 6 bits per
// element, and a step that takes more (plane bits: up to 20 per element)
// lands the rest itself.
template <int K, int MODE, int MAXB = 0>
__device__ __forceinline__ void refill(ChunkState<K>& S, Inflight<K, MODE>& F, const ChunkParams& C,
                                       LDS uint16_t* wring, LDS uint8_t* pring) {
  typedef Geo<K, MODE> G;
  typedef typename G::Seg V;
  constexpr uint32_t kBlkElems = G::kBlkElems;
  constexpr uint32_t kNeed = MAXB ? kBlkElems * MAXB / 16u + 8u : kBlkElems;
  static_assert(kNeed + G::kWSeg <= G::kRing, "a block's worst case and a segment fit the ring");
  const uint32_t lane = C.lane;
  const uint32_t need_w = min(kNeed, C.n_words - min(S.wptr, C.n_words));
  const uint32_t need_p = MODE == 2 ? min(kBlkElems, C.n_plane - S.pptr) : 0u;
  // wld < wptr + need, not wld - wptr < need: a coder-2 chunk starts with
  // wptr past the ring words of its states, before any word has landed
  if (S.wld < S.wptr + need_w || (MODE == 2 && S.pld - S.pptr < need_p)) {
    land_segments<K, MODE>(S, F, wring, pring, lane);
    while (S.wld < S.wptr + need_w) {
      store_wseg<G>(wring, S.wld, load_seg<V>(C.wsrc, S.wld / (G::kLaneSeg / 2u), C.wvalid, lane, C.safe), lane);
      S.wld += G::kWSeg;
    }
    if (MODE == 2) {
      while (S.pld - S.pptr < need_p) {
        store_pseg<G>(pring, S.pld, load_seg<V>(C.psrc, S.pld / G::kLaneSeg, C.pvalid, lane, C.safe), lane);
        S.pld += G::kPSeg;
      }
    }
  }
}

// Ring geometry of a plane mode under a coder: pair mode (3) loads its dense
// plane as mode 1 does, and tANS compact chunks keep their plane bytes in the
// stream, so they need no plane ring (full-scale geometry, as mode 0).
template <int MODE, int CODER>
constexpr int ring_mode() { return MODE == 3 ? 1 : (CODER == 1 && MODE == 2 ? 0 : MODE); }

// Two exponent-pair symbols into four fp8 bytes. `dup` holds their plane
// bytes as [pA, pA, pB, pB] (p = m0 | s1 << 3 | m1 << 4 | s0 << 7), dA and dB
// the symbols (e0 | e1 << 4) in byte 3. Bytes out: pA's s0|m0 and e0, then
// pA's nibbles swapped (s1|m1) and e1, then the same for B. Per byte, bits 7
// and 0-2 come from the plane and bits 3-6 from the exponent field.
template <int CODER>
__device__ __forceinline__ uint32_t pair_merge(uint32_t dup, uint32_t dA, uint32_t dB) {
  const uint32_t plane = ((dup << 4) & 0xFF00FF00u) | (dup & 0x00FF00FFu);   // bytes 1, 3: nibbles swapped
  uint32_t ex;                                                              // e0, e1, e0, e1 at bits 3-6
  if (CODER == 1) {
    ex = __builtin_amdgcn_perm(dB, dA, 0x07060302u);     // tANS entries hold e0 << 3 | e1 << 11 in bits 16..31
  } else {
    const uint32_t y = __builtin_amdgcn_perm(dB, dA, 0x07070303u);          // [bA, bA, bB, bB]
    ex = ((y >> 1) & 0xFF00FF00u) | ((y << 3) & 0x00FF00FFu);
  }
  return (plane & 0x87878787u) | (ex & 0x78787878u);
}

// The steps of one block, staging outputs in LDS and storing each half block
// once it is complete (a partial chunk stores its second half at the next
// block start, or after the last block). Pair mode (MODE 3) runs with EB = 2:
// a coded element is a pair of bytes.
template <int K, int MODE, int EB, bool PARTIAL, int CODER>
__device__ __forceinline__ void decode_block(uint32_t blk, const PlaneRegs<K>& pl, ChunkState<K>& S,
                                             Inflight<K, ring_mode<MODE, CODER>()>& F, const ChunkParams& C,
                                             const LDS uint64_t* __restrict__ tbl, LDS uint16_t* wring,
                                             LDS uint8_t* pring, LDS uint8_t* stage) {
  constexpr int RM = ring_mode<MODE, CODER>();
  constexpr uint32_t kStates = kWave * K;
  constexpr int kBlock = Geo<K, RM>::kBlock;
  constexpr int kHalf = kBlock / 2;
  constexpr bool DENSE = MODE == 1 && EB == 2;
  constexpr bool PAIR = MODE == 3;
  constexpr bool FAST = DENSE || PAIR || EB == 1;       // one-word table layouts (the output bits in the word)
  constexpr bool DIRECT = direct_stores<K, EB, PARTIAL>();
  const uint32_t lane = C.lane;
#pragma unroll
  for (int q = 0; q < kBlock; ++q) {
    const uint32_t t = blk * kBlock + q;
    if (PARTIAL && t >= C.nsteps) break;                 // wave-uniform
    if (!DIRECT && q == kHalf) {                         // first half of the block is staged: store it
      wave_sync();
      flush_half<K, EB, PARTIAL, kHalf>(2 * blk, C, stage);
    }
    const uint32_t qs = q % kHalf;                       // step within the staged half
    uint32_t d[K];
    if (CODER == 0) {
      rans_step<K, RM, FAST, PARTIAL>(t, S, C, tbl, wring, pring, d);
    } else {
      // compact tANS: lands ring words up to `need` (16-bit words, at most the stream's) when a
      // step takes more than the block-level refill provided (a wave-uniform branch)
      tans_step<K, MODE, FAST, PARTIAL>(t, S, C, tbl, (const LDS uint32_t*)wring, d, [&](uint32_t need) {
        typedef Geo<K, RM> G;
        need = min(need, C.n_words);
        if (S.wld < need) {
          land_segments<K, RM>(S, F, wring, pring, lane);
          while (S.wld < need) {
            store_wseg<G>(wring, S.wld, load_seg<typename G::Seg>(C.wsrc, S.wld / (G::kLaneSeg / 2u), C.wvalid,
                                                                  lane, C.safe), lane);
            S.wld += G::kWSeg;
          }
          wave_sync();
        }
      });
    }
    if (PAIR) {
      // plane bytes of this step: bytes q*K .. q*K+K-1 of the lane's 8K bytes
      const uint64_t pw = pl.b[(q * K) / 8];
      const uint32_t o = (q * K) % 8;
      const uint32_t phi = (uint32_t)(pw >> 32), plo = (uint32_t)pw;
      if (K >= 2) {
        constexpr int kPairs = K >= 2 ? K / 2 : 1;
        uint32_t v[kPairs];
#pragma unroll
        for (int h = 0; h < kPairs; ++h) {
          const uint32_t ob = o + 2 * h;
          const uint32_t dup = __builtin_amdgcn_perm(phi, plo, (ob + 1) * 0x01010000u | ob * 0x0101u);
          v[h] = pair_merge<CODER>(dup, d[(2 * h) % K], d[(2 * h + 1) % K]);
        }
        if (DIRECT) {
          store_step<K, kBlock, EB>(C, blk, q, v[0], v[kPairs - 1]);
        } else {
          LDS uint8_t* dst = stage + qs * (kStates * 2) + lane * (2u * K);
          if (K == 2) *(LDS uint32_t*)dst = v[0];
          else *(LDS uint64_t*)dst = (uint64_t)v[0] | ((uint64_t)v[kPairs - 1] << 32);
        }
      } else {
        const uint32_t dup = __builtin_amdgcn_perm(phi, plo, 0x0C0C0000u | o * 0x0101u);
        *(LDS uint16_t*)(stage + qs * (kStates * 2) + lane * 2u) = (uint16_t)pair_merge<CODER>(dup, d[0], d[0]);
      }
    } else if (DENSE) {
      // plane bytes of this step: bytes q*K .. q*K+K-1 of the lane's 8K bytes
      const uint64_t pw = pl.b[(q * K) / 8];
      const uint32_t o = (q * K) % 8;                    // byte offset in pw
      const uint32_t phi = (uint32_t)(pw >> 32), plo = (uint32_t)pw;
      if (K >= 2) {
        // word pairs: (p | p<<8) & 0x807F per half, exponents from byte 3 of d
        constexpr int kPairs = K >= 2 ? K / 2 : 1;
        uint32_t v[kPairs];
#pragma unroll
        for (int h = 0; h < kPairs; ++h) {
          const uint32_t ob = o + 2 * h;
          const uint32_t dup = __builtin_amdgcn_perm(phi, plo, (ob + 1) * 0x01010000u | ob * 0x0101u);
          // the two exponent words: rANS entries hold the exponent byte in bits
          // 24..31, tANS entries the word itself in bits 16..31
          const uint32_t ex = CODER == 1 ? __builtin_amdgcn_perm(d[(2 * h + 1) % K], d[(2 * h) % K], 0x07060302u)
                                         : __builtin_amdgcn_perm(d[(2 * h + 1) % K], d[(2 * h) % K], 0x070C030Cu) >> 1;
          v[h] = (dup & 0x807F807Fu) | ex;
        }
        if (DIRECT) {
          store_step<K, kBlock, EB>(C, blk, q, v[0], v[kPairs - 1]);
        } else {
          LDS uint8_t* dst = stage + qs * (kStates * 2) + lane * (2u * K);
          if (K == 2) *(LDS uint32_t*)dst = v[0];
          else *(LDS uint64_t*)dst = (uint64_t)v[0] | ((uint64_t)v[kPairs - 1] << 32);
        }
      } else {
        const uint32_t dup = __builtin_amdgcn_perm(phi, plo, 0x0C0C0000u | o * 0x0101u);
        const uint32_t v = (dup & 0x807Fu) | (CODER == 1 ? d[0] >> 16 : d[0] >> 17);
        *(LDS uint16_t*)(stage + qs * (kStates * 2) + lane * 2u) = (uint16_t)v;
      }
    } else {
      // the lane's K outputs of this step are adjacent: one LDS store. The
      // generic tANS layout leaves each output word in d's high half
      constexpr uint32_t kW = CODER == 1 ? 0x07060302u : 0x05040100u;
      constexpr uint32_t kW1 = CODER == 1 ? 16u : 0u;
      LDS uint8_t* dst = stage + (qs * kStates + lane * K) * EB;
      if (DIRECT && EB == 2) {
        store_step<K, kBlock, EB>(C, blk, q, __builtin_amdgcn_perm(d[1 % K], d[0], kW),
                                  __builtin_amdgcn_perm(d[3 % K], d[2 % K], kW));
      } else if (DIRECT) {                               // bytes: K = 2 in one half word, K = 4 in one word
        store_step<K, kBlock, EB>(C, blk, q,
                                  __builtin_amdgcn_perm(d[1 % K], d[0], 0x0C0C0703u) |
                                      (K == 4 ? __builtin_amdgcn_perm(d[3 % K], d[2 % K], 0x0C0C0703u) << 16 : 0u),
                                  0u);
      } else if (EB == 2) {
        if (K == 1) *(LDS uint16_t*)dst = (uint16_t)(d[0] >> kW1);
        else if (K == 2) *(LDS uint32_t*)dst = __builtin_amdgcn_perm(d[K - 1], d[0], kW);
        else *(LDS uint64_t*)dst = (uint64_t)__builtin_amdgcn_perm(d[1 % K], d[0], kW) |
                                   ((uint64_t)__builtin_amdgcn_perm(d[3 % K], d[2 % K], kW) << 32);
      } else {                                           // byte values in bits 24..31 of d
        if (K == 1) *dst = (uint8_t)(d[0] >> 24);
        else if (K == 2) *(LDS uint16_t*)dst = (uint16_t)__builtin_amdgcn_perm(d[K - 1], d[0], 0x0C0C0703u);
        else *(LDS uint32_t*)dst = __builtin_amdgcn_perm(d[1 % K], d[0], 0x0C0C0703u) |
                                   (__builtin_amdgcn_perm(d[3 % K], d[2 % K], 0x0C0C0703u) << 16);
      }
    }
  }
  if (!PARTIAL && !DIRECT) {
    wave_sync();
    flush_half<K, EB, PARTIAL, kHalf>(2 * blk + 1, C, stage);
  }
}

// A wavefront's issue priority falls as its chunk progresses, from 3 to 0 in
// four bands. The SIMD arbiter otherwise favours the oldest waves, so the
// first of a CU's two workgroups ran ahead and the CU's last 20-30 us ran the
// second one alone, at lower throughput; with the priority the waves that
// are behind issue first and the chunks of a CU end closer together. The
// dispatcher places workgroups in index order, one per CU before any CU gets
// a second, so workgroups from index `first_round` (the device's CU count) on
// are the younger of their CU's two: their bands end at 40/60/80 % of the
// chunk's blocks, the others' at 20/40/60 %. Partial chunks, which have fewer
// blocks, lower their priority sooner. A wrong guess (another kernel sharing
// the CUs) changes only the order of issue. Within a band the oldest wave
// still issues first, so the first waves of a workgroup ran ahead of the
// others on their SIMD and ended some microseconds before them; a wave that
// is two or more block pairs ahead of the slowest wave of its workgroup
// (`lead`) therefore takes the next band's priority. Llama-3-8B-shaped
// layer: 157.4 us per launch without the priority, 154.9 with quarter bands
// for every wave, 148.5 with the shifted bands (and the later prologue
// changes), 145.6 with the lead rule (147.8 without it on the same boxes).
__device__ __forceinline__ void progress_priority(uint32_t blk, uint32_t nblk, bool younger, uint32_t lead) {
  const uint32_t fifth = (blk * 5u) / nblk + (younger ? 0u : 1u) + (lead >= 2u ? 1u : 0u);   // wave-uniform, 0..6
  if (fifth <= 1) __builtin_amdgcn_s_setprio(3);
  else if (fifth == 2) __builtin_amdgcn_s_setprio(2);
  else if (fifth == 3) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// Decode one chunk with one wavefront: K interleaved states per lane, MODE =
// plane mode, EB = element bytes (2 for pair mode, whose elements are byte
// pairs), PARTIAL = chunk may be shorter than 64*K*steps (the tensor's last
// chunk), CODER = 0 rANS, 1 tANS. n_words is the chunk table's count: renorm
// words (rANS) or stream bits (tANS, whose stream is whole u32 words). fl:
// bit 0 = the later of its CU's two workgroups, bit 1 = tANS states at the
// stream head (coder 2; the stream then holds at least their 12 * 64K bits).
template <int K, int MODE, int EB, bool PARTIAL, int CODER>
__device__ __forceinline__ void decode_chunk(const LDS uint64_t* __restrict__ tbl, LDS uint16_t* wring,
                                             LDS uint8_t* pring, LDS uint8_t* stage,
                                             const GLB uint8_t* __restrict__ cbase, uint32_t n_words,
                                             uint32_t n_plane, const GLB uint8_t* dplane, uint64_t pstride,
                                             GLB uint8_t* __restrict__ out8, uint64_t ubase, uint64_t ustride,
                                             uint32_t nc, uint32_t nsteps, int32_t* status, uint32_t fl) {
  constexpr int RM = ring_mode<MODE, CODER>();
  // tANS: bits per element the block-level refill provides. The one-word
  // layouts take at most 12 (a state's worst case). Compact steps land what
  // they need beyond it themselves (tans_step's ensure), so their blocks ask
  // for 6, about what a compact element takes on average: a larger reserve
  // made blocks wait for segments more often (12 bits: 0.3-1 % slower on the
  // half-zeros tensor and the pruned layer).
  constexpr int MAXB = CODER == 0 ? 0 : (MODE == 2 ? 6 : 12);
  typedef Geo<K, RM> G;
  constexpr uint32_t kStates = kWave * K;
  ChunkParams C;
  C.lane = __lane_id();
  const uint32_t n_bits = n_words;                               // tANS: the stream's length in bits
  if (CODER == 1) n_words = 2u * ((n_bits + 31u) / 32u);          // in 16-bit ring words
  const uint32_t wbytes = pad16(n_words * 2u);
  const bool younger = fl & 1u;
  const bool head = CODER == 1 && (fl & 2u);
  const uint32_t sarr = head ? 0u : 4u * kStates;                // bytes of the u32 state array
  C.wsrc = cbase + sarr;
  C.psrc = cbase + sarr + wbytes;
  C.dplane = dplane ? dplane : C.psrc;
  C.pstride = pstride;
  C.safe = cbase;
  C.out8 = out8;
  C.ubase = ubase;
  C.ustride = ustride;
  C.n_words = n_words;
  C.n_plane = n_plane;
  C.wvalid = wbytes / G::kLaneSeg;
  C.pvalid = pad16(n_plane) / G::kLaneSeg;
  C.nc = nc;
  C.nsteps = nsteps;
  C.nblk = (nsteps + G::kBlock - 1) / G::kBlock;

  ChunkState<K> S;
  bool bad_init = false;
  S.wptr = S.wld = S.pptr = S.pld = S.bpos = 0;
  if (head) {
    // the lane's K 12-bit states at bit 12K * lane of the stream: at most 48
    // bits from a shift below 32, so inside three words; words past the
    // stream's last are not read (the last is read again in their place, and
    // its bits beyond the states are not used)
    const uint32_t b0 = 12u * K * C.lane, w0 = b0 >> 5, last = (n_bits + 31u) / 32u - 1u;
    const GLB uint32_t* s32 = (const GLB uint32_t*)cbase;
    const uint32_t r0 = s32[w0], r1 = s32[min(w0 + 1u, last)];
    const uint32_t lo = __builtin_amdgcn_alignbit(r1, r0, b0);
    const uint32_t hi = K == 4 ? __builtin_amdgcn_alignbit(s32[min(w0 + 2u, last)], r1, b0) : 0u;
    const uint64_t win = (uint64_t)lo | ((uint64_t)hi << 32);
#pragma unroll
    for (int g = 0; g < K; ++g) S.x[g] = (uint32_t)(win >> (12 * g)) & 4095u;
    S.bpos = 12u * kStates;
    S.wptr = (S.bpos >> 5) << 1;                        // ring words before the first element's bits
  } else {
#pragma unroll
    for (int g = 0; g < K; ++g) {
      S.x[g] = ((const GLB uint32_t*)cbase)[g * kWave + C.lane];
      if (CODER == 1) {                                 // a table index: kept inside the table
        bad_init |= S.x[g] > 4095u;
        S.x[g] &= 4095u;
      }
    }
  }

  if (RM == 2 && C.lane == 0) *(LDS u32x4*)(pring + G::kPZero) = u32x4{0u, 0u, 0u, 0u};

  // First loads; land all of them before the loop so that the loop header's
  // wait-count state holds no load issued here.
  Inflight<K, RM> F;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    F.pl[i] = RM == 1 ? load_plane<K>(C.dplane, C.pstride, min((uint32_t)i, C.nblk - 1), C.lane) : PlaneRegs<K>{};
  request_segments<K, RM>(S, F, C);
  consume<K>(S.x);
  if (RM == 1) { consume_plane(F.pl[0]); consume_plane(F.pl[1]); }
  BS_KEEP2(F.w[0].x, F.w[1].x);
  if (RM == 2) BS_KEEP2(F.p[0].x, F.p[1].x);

  LDS uint16_t* prog = (LDS uint16_t*)((LDS uint8_t*)tbl + (kProgOff - kTblOff));   // kWaves entries
  const uint32_t pwave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  for (uint32_t blk = 0;;) {
    {
      // publish this wave's pair count and take the workgroup's lowest (0xFFFF:
      // no chunk, or done); a stale entry is lower than the true one, so the
      // lead read here is never less than the true lead
      const uint32_t pair = min(blk >> 1, 0xFFFEu);
      if (C.lane == 0) *(volatile LDS uint16_t*)(prog + pwave) = (uint16_t)pair;
      uint32_t m = 0xFFFFu;
      if constexpr (kWaves == 8) {             // one 16-byte read
        const u32x4 pv = *(volatile LDS u32x4*)prog;
#pragma unroll
        for (int i = 0; i < 4; ++i) m = min(m, min(pv[i] & 0xFFFFu, pv[i] >> 16));
      } else {
#pragma unroll
        for (int i = 0; i < kWaves; ++i) m = min(m, (uint32_t)((volatile LDS uint16_t*)prog)[i]);
      }
      progress_priority(blk, C.nblk, younger, rfl(pair - min(m, pair)));
    }
    // ---- pair start: land the previous pair's loads, issue the next pair's
    const PlaneRegs<K> cur0 = F.pl[0], cur1 = F.pl[1];
    land_segments<K, RM>(S, F, wring, pring, C.lane);
    refill<K, RM, MAXB>(S, F, C, wring, pring);
    wave_sync();
    if (PARTIAL && blk > 0) flush_half<K, EB, PARTIAL, G::kBlock / 2>(2 * blk - 1, C, stage);
    request_segments<K, RM>(S, F, C);
    if (RM == 1) {
      F.pl[0] = load_plane<K>(C.dplane, C.pstride, min(blk + 2, C.nblk - 1), C.lane);
      F.pl[1] = load_plane<K>(C.dplane, C.pstride, min(blk + 3, C.nblk - 1), C.lane);
    }
    wave_sync();
    decode_block<K, MODE, EB, PARTIAL, CODER>(blk, cur0, S, F, C, tbl, wring, pring, stage);
    if (PARTIAL && blk + 1 >= C.nblk) break;
    // ---- second block of the pair
    refill<K, RM, MAXB>(S, F, C, wring, pring);
    wave_sync();
    if (PARTIAL) flush_half<K, EB, PARTIAL, G::kBlock / 2>(2 * blk + 1, C, stage);
    decode_block<K, MODE, EB, PARTIAL, CODER>(blk + 1, cur1, S, F, C, tbl, wring, pring, stage);
    blk += 2;
    if (blk >= C.nblk) break;
    if (!PARTIAL) {
      // The pair's loads were followed by its output stores: vmcnt(stores)
      // lands the loads and leaves the stores in flight. Stating it gives the
      // compiler's wait-count tracking an exact state here; the uses below
      // keep its own waits for these registers at this point.
      __builtin_amdgcn_s_waitcnt(wait_vm(stores_per_pair<K, RM, EB, PARTIAL>()));
      if (RM == 1) { consume_plane(F.pl[0]); consume_plane(F.pl[1]); }
      BS_KEEP2(F.w[0].x, F.w[1].x);
      if (RM == 2) BS_KEEP2(F.p[0].x, F.p[1].x);
    }
  }
  // a partial chunk's last staged half: the second half of its last block, or
  // the first if that block has at most half a block of steps
  if (PARTIAL) {
    wave_sync();
    flush_half<K, EB, PARTIAL, G::kBlock / 2>((C.nsteps - 1) / (G::kBlock / 2), C, stage);
  }
  // segments requested but never landed need no wait: nothing reads them
  if (C.lane == 0) *(volatile LDS uint16_t*)(prog + pwave) = 0xFFFFu;   // out of the workgroup's lowest

  // a valid chunk ends in the encoder's start states (rANS x = L, tANS X = 0)
  // with every word, bit and plane byte read
  bool bad_state = bad_init;
#pragma unroll
  for (int g = 0; g < K; ++g) bad_state |= S.x[g] != (CODER == 0 ? kL : 0u);
  const bool bad = __ballot(bad_state) != 0 || (CODER == 0 ? S.wptr != n_words : S.bpos != n_bits) ||
                   (RM == 2 && S.pptr != n_plane);
  if (bad) report(status, BS_DEV_ERR_STREAM);
}

template <int K, int EB, bool PARTIAL, bool COMPACT, int CODER>
__device__ __forceinline__ void decode_chunk_mode(uint32_t mode, const LDS uint64_t* tbl, LDS uint16_t* wring,
                                                  LDS uint8_t* pring, LDS uint8_t* stage, const GLB uint8_t* cbase,
                                                  uint32_t nw, uint32_t np, const GLB uint8_t* dplane,
                                                  uint64_t pstride, GLB uint8_t* out, uint64_t ubase, uint64_t ustride,
                                                  uint32_t nc, uint32_t nsteps, int32_t* status, uint32_t fl) {
  if constexpr (EB == 1) {   // byte symbols (no plane); exponent pairs run as 2-byte elements
    if (mode == 3)
      decode_chunk<K, 3, 2, PARTIAL, CODER>(tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
    else
      decode_chunk<K, 0, EB, PARTIAL, CODER>(tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
  } else {
    if (mode == 0) {
      decode_chunk<K, 0, EB, PARTIAL, CODER>(tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
    } else if (mode == 1) {
      decode_chunk<K, 1, EB, PARTIAL, CODER>(tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
    } else {
      if constexpr (COMPACT)
        decode_chunk<K, 2, EB, PARTIAL, CODER>(tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
    }
  }
}

template <int K, bool COMPACT, int CODER>
__device__ __forceinline__ void decode_chunk_c(uint32_t eb, bool partial, uint32_t mode, const LDS uint64_t* tbl,
                                               LDS uint16_t* wring, LDS uint8_t* pring, LDS uint8_t* stage,
                                               const GLB uint8_t* cbase, uint32_t nw, uint32_t np,
                                               const GLB uint8_t* dplane, uint64_t pstride, GLB uint8_t* out,
                                               uint64_t ubase, uint64_t ustride, uint32_t nc, uint32_t nsteps,
                                               int32_t* status, uint32_t fl) {
  if (eb == 2) {
    if (partial) decode_chunk_mode<K, 2, true, COMPACT, CODER>(mode, tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
    else decode_chunk_mode<K, 2, false, COMPACT, CODER>(mode, tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
  } else {
    if (partial) decode_chunk_mode<K, 1, true, COMPACT, CODER>(mode, tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
    else decode_chunk_mode<K, 1, false, COMPACT, CODER>(mode, tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
  }
}

template <int K, bool COMPACT>
__device__ __forceinline__ void decode_chunk_k(uint32_t eb, bool partial, uint32_t mode, uint32_t coder,
                                               const LDS uint64_t* tbl, LDS uint16_t* wring, LDS uint8_t* pring,
                                               LDS uint8_t* stage, const GLB uint8_t* cbase, uint32_t nw, uint32_t np,
                                               const GLB uint8_t* dplane, uint64_t pstride, GLB uint8_t* out,
                                               uint64_t ubase, uint64_t ustride, uint32_t nc, uint32_t nsteps,
                                               int32_t* status, uint32_t fl) {
  if (coder == 0)
    decode_chunk_c<K, COMPACT, 0>(eb, partial, mode, tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
  else
    decode_chunk_c<K, COMPACT, 1>(eb, partial, mode, tbl, wring, pring, stage, cbase, nw, np, dplane, pstride, out, ubase, ustride, nc, nsteps, status, fl);
}

template <bool COMPACT>
__global__ __launch_bounds__(kThreads) void bsck_decode_kernel(const bs_chunk_task* __restrict__ tasks,
                                                               uint32_t n_tasks, bs_chunk_task single,
                                                               int32_t* __restrict__ status, uint32_t first_round) {
  BS_DYNAMIC_LDS(smem);
  LDS uint64_t* s_tbl = (LDS uint64_t*)(smem + kTblOff);
  LDS uint8_t* s_wring = (LDS uint8_t*)smem;
  LDS uint8_t* s_stage = (LDS uint8_t*)(smem + kTblOff + kTblBytes);
  // table-build scratch overlaps the staging area (unused until decoding starts)
  LDS uint32_t* s_cum = (LDS uint32_t*)s_stage + 3;    // 257 entries; s_cum + 1 is 16-byte aligned
  LDS uint32_t* s_val = s_cum + 257;                    // 256 entries, 16-byte aligned
  LDS uint32_t* s_flag = s_val + 256;                   // table-check flag

  // ---- which tensor does this workgroup serve. The prologue is a chain of
  // dependent global loads (task, header and symbols, chunk entry, states),
  // each a full memory latency at launch, so it is kept short: tasks are read
  // by the lanes together and found by ballots (wg_begin ascends, so the tasks
  // starting at or before this workgroup are a prefix).
  bs_chunk_task T = single;
  if (tasks != nullptr) {
    // The workgroup's task is the last one whose wg_begin is at or before it
    // (wg_begin ascends). Each round the 64 lanes read evenly spaced wg_begin
    // values of the range that holds it and a vote narrows the range 64-fold,
    // so up to 4,096 tasks take two dependent loads and any count fits 64 in
    // a few; the last round reads whole tasks, one per lane.
    const uint32_t l = __lane_id();
    uint32_t lo = 0, span = n_tasks;                   // the task lies in [lo, lo + span)
    while (span > (uint32_t)kWave) {                   // wave-uniform
      const uint32_t stride = (span + kWave - 1) / kWave;
      const bool in = l * stride < span;
      const uint32_t wb = in ? tasks[lo + l * stride].wg_begin : 0xFFFFFFFFu;
      const uint64_t before = __ballot(in && wb <= blockIdx.x);
      const uint32_t k = before ? (uint32_t)__popcll(before) - 1u : 0u;
      lo += k * stride;
      span = min(stride, span - k * stride);
    }
    const bs_chunk_task mine = l < span ? tasks[lo + l] : bs_chunk_task{};
    const uint64_t before = __ballot(l < span && mine.wg_begin <= blockIdx.x);
    const uint32_t k = before ? (uint32_t)__popcll(before) - 1u : 0u;
    T.blob = (const uint8_t*)readlane64((uint64_t)mine.blob, k);
    T.blob_bytes = readlane64(mine.blob_bytes, k);
    T.out = (void*)readlane64((uint64_t)mine.out, k);
    T.n = readlane64(mine.n, k);
    T.wg_begin = (uint32_t)__builtin_amdgcn_readlane((int)mine.wg_begin, (int)k);
    T.n_chunks = (uint32_t)__builtin_amdgcn_readlane((int)mine.n_chunks, (int)k);
  }
  const uint32_t group = blockIdx.x - T.wg_begin;
  const GLB uint8_t* __restrict__ b = (const GLB uint8_t*)T.blob;
  const uint32_t tid = threadIdx.x;
  // The loads of the prologue are issued without branches around them, at
  // clamped or known-valid addresses, so that the compiler's in-order count
  // of outstanding loads stays exact and a use of one load waits for it alone,
  // not for the loads issued after it. A valid blob has at least 64 bytes
  // (header, one symbol entry padded to 16, one chunk-table entry).
  if (T.blob_bytes < 64) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  const uint32_t lane = __lane_id();
  // The 32-byte header (two 16-byte loads at one address for the whole
  // wavefront) and the symbol entries are requested together: both need only
  // the blob address, and the header fields are then taken from registers,
  // not read one dependent byte load at a time.
  const u32x4 h0 = ((const GLB u32x4*)b)[0], h1 = ((const GLB u32x4*)b)[1];
  // symbol entries: lane l entries 4l..4l+3 in one 16-byte load (every wave
  // loads them, wavefront 0 uses them); lanes past the blob's end read its
  // last 16 bytes, which belong to no live symbol when the header is valid
  const u32x4 ent4 =
      *(const GLB u32x4*)(b + (32u + 16u * lane + 16u <= T.blob_bytes ? (uint64_t)(32u + 16u * lane)
                                                                         : (T.blob_bytes - 16u) & ~(uint64_t)15));

  // ---- header checks (uniform across the workgroup)
  const uint32_t magic = rfl(h0.x), w1 = rfl(h0.y);
  const uint32_t ver = w1 & 0xFFu, eb = (w1 >> 8) & 0xFFu, mode = (w1 >> 16) & 0xFFu;
  const uint32_t w7 = rfl(h1.w), coder = w7;             // byte 28: coder; bytes 29..31 zero
  if (magic != 0x4B435342u ||                                             // "BSCK"
      (ver != 2 && ver != kVersion) || (eb != 1 && eb != 2) || mode > 3 || (w1 >> 24) != 12 || coder > 2 ||
      (ver == 2 && (coder != 0 || mode == 3)) || (!COMPACT && mode == 2) ||
      (eb == 1 ? (mode != 0 && mode != 3) : mode == 3)) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  const uint64_t n = (uint64_t)rfl(h0.z) | ((uint64_t)rfl(h0.w) << 32);
  const uint64_t ne = mode == 3 ? n / 2 : n;                 // coded elements (pair mode: byte pairs)
  const uint32_t steps = rfl(h1.x);
  const uint32_t w5 = rfl(h1.y);
  const uint32_t lanes = w5 & 0xFFFFu, nsym = w5 >> 16;
  const uint32_t nch = rfl(h1.z);
  const uint64_t per = (uint64_t)lanes * steps;
  // an empty tensor (n = 0, no chunks) has no blob to decode: only a task
  // table out of order can send a workgroup to one, and it stops here
  if ((lanes != 64 && lanes != 128 && lanes != 256) || steps == 0 || (steps % (2 * kBlockMax)) != 0 || nsym == 0 ||
      nsym > 256 || (mode == 3 && (n & 1)) || nch == 0 || nch != T.n_chunks || per > kMaxChunk ||
      nch != (ne + per - 1) / per) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  if (n != T.n) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_COUNT);
    return;
  }
  const uint32_t stab = pad16(32u + 4u * nsym);               // tANS decode table (coders 1 and 2)
  const uint32_t ctab = stab + (coder ? 4u * kTansSlots : 0u);
  const uint64_t nf = ne / per;                               // full chunks
  // layout version 3 keeps the full chunks' dense planes in one region;
  // version 2 keeps every plane inline and lays chunks out contiguously
  const bool region = ver == kVersion && (mode == 1 || mode == 3);
  const uint64_t preg = ((uint64_t)ctab + 16ull * nch + 255u) & ~255ull;   // dense plane region
  if ((uint64_t)ctab + 16ull * nch > T.blob_bytes ||
      (region && (preg > T.blob_bytes || nf * per > T.blob_bytes - preg))) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_BOUNDS);
    return;
  }
  const bool dense = eb == 2 && mode == 1;                    // exponent symbols of bf16 words
  const bool fast = dense || eb == 1;                         // one-word table layouts (bytes, pairs too)
  // tANS: this thread's run of the stored decode table (kRun entries), in
  // flight during the symbol checks below (inside the blob: checked above)
  constexpr uint32_t kRun = 4096u / kThreads;
  static_assert(4096u % kThreads == 0 && kRun % 4 == 0, "slot runs");
  u32x4 trun[kRun / 4];
#pragma unroll
  for (uint32_t i = 0; i < kRun / 4; ++i) trun[i] = u32x4{0u, 0u, 0u, 0u};
  if (coder) {
#pragma unroll
    for (uint32_t i = 0; i < kRun / 4; ++i) trun[i] = *(const GLB u32x4*)(b + stab + 4u * (tid * kRun + 4u * i));
  }

  // this wave's chunk-table entry, requested before the table build so that
  // its latency passes under it (the build's barriers wait for LDS only)
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);   // wave-uniform: keeps chunk state scalar
  const uint32_t chunk = group * kWaves + wave;
  // (nch >= 1 here: checked above; a wave past the last chunk reads the last entry and does not use it)
  // a scalar load (the address is wave-uniform): its wait is on the scalar
  // counter, apart from the vector loads issued around it
  const u32x4 centry = *(const CST u32x4*)((const CST uint8_t*)b + ctab + 16ull * min(chunk, nch - 1u));


  // ---- decode table in LDS (layouts in the file comment). Wavefront 0
  // checks the symbol entries and writes their values and the inclusive
  // prefix of their frequencies (each lane sums its four, a shuffle scan over
  // the lanes adds the sums before it); one barrier publishes them. Then every
  // thread fills a run of consecutive slots: a binary search for the run's
  // first symbol, a walk that reloads only where the symbol changes, and the
  // entries written two at a time.
  if (tid < (uint32_t)kWave) {
    const uint32_t l = tid;
    uint32_t f[4], c = 0;
    bool bad = false;
    u32x4 vals;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t e = ent4[i];
      const bool live = 4u * l + i < nsym;
      f[i] = live ? (e >> 16) & 0x1FFFu : 0u;
      // dense-mode symbols are exponent classes: value e<<7 with zero sign/mantissa, one plane byte each;
      // byte symbols are bytes, exponent-pair symbols bytes with one plane byte each
      bad |= live && (f[i] == 0 || (dense && ((e & 0x807Fu) != 0 || (e >> 31) == 0)) ||
                      (eb == 1 && ((e & 0xFF00u) != 0 || (e >> 31) != (mode == 3 ? 1u : 0u))));
      vals[i] = (e & 0xFFFFu) | (e & 0x80000000u);
      c += f[i];
    }
    uint32_t incl = c;
#pragma unroll
    for (uint32_t d = 1; d < (uint32_t)kWave; d <<= 1) {
      const uint32_t u = (uint32_t)__builtin_amdgcn_ds_bpermute((int)(((l - d) & 63u) << 2), (int)incl);
      if (l >= d) incl += u;
    }
    const uint32_t c1 = incl - c + f[0], c2 = c1 + f[1], c3 = c2 + f[2];
    *(LDS u32x4*)(s_cum + 1 + 4 * l) = u32x4{c1, c2, c3, incl};
    *(LDS u32x4*)(s_val + 4 * l) = vals;
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
    const bool any_bad = __ballot(bad) != 0;
    if (l == 0) {
      s_cum[0] = 0;
      *s_flag = any_bad || total != 4096u;
      *(volatile LDS uint32_t*)(smem + kFlagOff) = 0u;   // the tANS table check's flag
    }
  }
  lds_barrier();
  const uint64_t off = (uint64_t)rfl(centry.x) | ((uint64_t)rfl(centry.y) << 32);
  const uint32_t nw = rfl(centry.z), np = rfl(centry.w);
  // Warm the chunk's first 2 KB (its initial states and first ring words) while
  // the table is built: decode_chunk's own loads of them come after the next
  // barrier and then hit L2 instead of waiting on HBM, which every workgroup of
  // a launch's first round reaches at once. Only inside the blob (a uniform
  // test); the values are dropped.
  u32x4 warm0 = {0u, 0u, 0u, 0u}, warm1 = {0u, 0u, 0u, 0u};
  if (chunk < nch && (off & 15u) == 0 && off + 2048u <= T.blob_bytes) {
    warm0 = *(const GLB u32x4*)(b + off + 16u * lane);
    warm1 = *(const GLB u32x4*)(b + off + 1024u + 16u * lane);
  }
  if (*s_flag) {                                  // the same value for every thread
    if (tid == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  if (coder) {
    // tANS: the blob's table {newX:12, nb:4, symbol:8, 0:8}, checked (a
    // symbol of the tensor, nb <= 12, newX + 2^nb <= 4096 with nb zero low
    // bits, so every next state stays in the table) and laid out for the
    // step: one word {newX, nb, output bits} for dense bf16, bytes and
    // pairs (layouts in the file comment); else two, {newX, nb, plane-byte
    // mask} and {nb + raw, value} (raw = 8 plane bits, mask 0x807F, for a
    // compact symbol that has one)
    const uint32_t slot0 = tid * kRun;
    bool bad = false;
    uint32_t lo[kRun], hi[kRun];
#pragma unroll
    for (uint32_t k = 0; k < kRun; ++k) {
      const uint32_t e = trun[k / 4][k % 4], sym = (e >> 16) & 0xFFu, nb = (e >> 12) & 15u, nx = e & 0xFFFu;
      bad |= (e >> 24) != 0 || sym >= nsym || nb > 12u || nx + (1u << nb) > 4096u || (nx & ((1u << nb) - 1u)) != 0;
      const uint32_t v = s_val[sym];
      const uint32_t rw = mode == 2 && (v >> 31) ? 8u : 0u;
      // dense: the symbol's word (exponent in place) in bits 16..31; pairs:
      // e0 << 3 | e1 << 11 (both exponent fields in place); bytes: the byte
      // in bits 24..31; generic: the plane-byte mask in bits 16..31, and a
      // second word of the bit count and the value
      lo[k] = dense       ? (e & 0xFFFFu) | ((v & 0x7F80u) << 16)
              : mode == 3 ? (e & 0xFFFFu) | (((v & 0xFu) << 19) | ((v & 0xF0u) << 23))
              : fast      ? (e & 0xFFFFu) | ((v & 0xFFu) << 24)
                          : (e & 0xFFFFu) | (rw ? 0x807F0000u : 0u);
      hi[k] = (nb + rw) | (v << 16);
    }
    if (fast) {
      LDS uint32_t* t32 = (LDS uint32_t*)s_tbl + slot0;
#pragma unroll
      for (uint32_t k = 0; k < kRun; k += 4) *(LDS u32x4*)(t32 + k) = u32x4{lo[k], lo[k + 1], lo[k + 2], lo[k + 3]};
    } else {
#pragma unroll
      for (uint32_t k = 0; k < kRun; k += 2)
        *(LDS u32x4*)(s_tbl + slot0 + k) = u32x4{lo[k], hi[k], lo[k + 1], hi[k + 1]};
    }
    if (bad) *(volatile LDS uint32_t*)(smem + kFlagOff) = 1u;
  } else {
    const uint32_t slot0 = tid * kRun;
    uint32_t lo = 0, hi = nsym;                      // cum[lo] <= slot0 < cum[hi]
    while (hi - lo > 1) {
      const uint32_t mid = (lo + hi) >> 1;
      if (s_cum[mid] <= slot0) lo = mid; else hi = mid;
    }
    uint32_t c0 = s_cum[lo], c1 = s_cum[lo + 1], val = s_val[lo];
#pragma unroll
    for (uint32_t k = 0; k < kRun; k += 2) {
      uint64_t e2[2];
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t slot = slot0 + k + h;
        while (c1 <= slot) {                         // cum[nsym] = 4096 > slot ends it
          ++lo;
          c0 = c1;
          c1 = s_cum[lo + 1];
          val = s_val[lo];
        }
        const uint32_t f = c1 - c0;
        e2[h] = dense  ? ((uint64_t)(f | ((val & 0x7F80u) << 17)) | ((uint64_t)(slot - c0) << 32))
                : fast ? ((uint64_t)(f | ((val & 0xFFu) << 24)) | ((uint64_t)(slot - c0) << 32))
                       : ((uint64_t)f | ((uint64_t)(val | ((slot - c0) << 16)) << 32));
      }
      *(LDS u32x4*)(s_tbl + slot0 + k) =
          u32x4{(uint32_t)e2[0], (uint32_t)(e2[0] >> 32), (uint32_t)e2[1], (uint32_t)(e2[1] >> 32)};
    }
  }
  // progress entries (decode_chunk): 0 for a wave with a chunk, 0xFFFF for one without
  // (and for one that leaves on an error below)
  if ((tid & (kWave - 1)) == 0) *(volatile LDS uint16_t*)((LDS uint8_t*)smem + kProgOff + 2 * wave) = chunk < nch ? 0u : 0xFFFFu;
  BS_KEEP2(warm0.x, warm1.x);                           // landed long ago: the table build took longer
  lds_barrier();
  if (coder && *(volatile LDS uint32_t*)(smem + kFlagOff)) {   // the same value for every thread
    if (tid == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }

  // ---- one chunk per wavefront
  if (chunk >= nch) return;
  const uint64_t cbase_idx = (uint64_t)chunk * per;     // the partial chunk's first element (nf * per)
  const bool full = chunk < nf;
  const uint32_t nc = full ? (uint32_t)per : (uint32_t)(ne - cbase_idx);
  const uint32_t nsteps = (nc + lanes - 1) / lanes;
  const uint32_t bsteps = lanes == 256 ? 4u : 8u;     // block_steps<K>()
  const uint32_t dense_plane = ((nsteps + bsteps - 1) / bsteps) * bsteps * lanes;
  const bool has_plane = mode == 1 || mode == 3;      // dense plane
  const bool split = region && full;                  // dense plane in the plane region
  const uint64_t pblk = (uint64_t)bsteps * lanes;      // plane bytes per block
  // stream: rANS nw 16-bit words; tANS nw bits (at most 12 per element, 20 with compact plane
  // bits; coder 2: the 12-bit states first). Coder 2 has no state array, and 256 bytes from the
  // chunk's start lie inside the blob (ring loads of lanes past a stream's end read there).
  const uint32_t sbytes = coder ? pad16(((nw + 31u) / 32u) * 4u) : pad16(nw * 2u);
  const uint64_t sarr = coder == 2 ? 0u : 4ull * lanes, hbits = coder == 2 ? 12ull * lanes : 0u;
  bool ok = (off % 16) == 0 && off + sarr + sbytes + (split ? 0u : pad16(np)) <= T.blob_bytes &&
            (coder != 2 || (off + 256u <= T.blob_bytes && nw >= hbits)) &&
            (coder ? (uint64_t)nw <= (uint64_t)nc * (mode == 2 ? 20u : 12u) + hbits : nw <= nsteps * lanes) &&
            T.out != nullptr && ((uintptr_t)T.out & 15u) == 0;
  if (has_plane) ok = ok && np == dense_plane;
  if (mode == 2) ok = ok && (coder ? np == 0 : np <= nc);
  if (mode == 0) ok = ok && np == 0;
  if (!ok) {
    report(status, BS_DEV_ERR_BOUNDS);
    if ((tid & (kWave - 1)) == 0) *(volatile LDS uint16_t*)((LDS uint8_t*)smem + kProgOff + 2 * wave) = 0xFFFFu;
    return;
  }
  const GLB uint8_t* cbase = b + off;
  LDS uint16_t* wring = (LDS uint16_t*)(s_wring + wave * kRingBytes);
  LDS uint8_t* pring = s_wring + wave * kRingBytes + Geo<1, 2>::kPRingOff;   // rANS compact chunks only
  LDS uint8_t* stage = s_stage + wave * kStageMax;
  GLB uint8_t* out = (GLB uint8_t*)T.out;
  const bool partial = !full;
  const GLB uint8_t* dplane = split ? b + preg + chunk * pblk : nullptr;   // nullptr: inline after the stream
  const uint64_t pstride = split ? nf * pblk : pblk;
  // version 3 interleaves the full chunks' 512-element units; version 2 (and
  // every partial chunk) holds its elements in order from chunk * per
  const bool inter = ver == kVersion && full;
  const uint64_t ubase = inter ? (uint64_t)chunk * kUnit : cbase_idx;
  const uint64_t ustride = inter ? nf * kUnit : kUnit;
  // bit 0: the later of its CU's two workgroups; bit 1: tANS states at the stream head
  const uint32_t fl = (blockIdx.x >= first_round ? 1u : 0u) | (coder == 2 ? 2u : 0u);
  if (lanes == 64)
    decode_chunk_k<1, COMPACT>(eb, partial, mode, coder, s_tbl, wring, pring, stage, cbase, nw, np, dplane, pstride,
                               out, ubase, ustride, nc, nsteps, status, fl);
  else if (lanes == 128)
    decode_chunk_k<2, COMPACT>(eb, partial, mode, coder, s_tbl, wring, pring, stage, cbase, nw, np, dplane, pstride,
                               out, ubase, ustride, nc, nsteps, status, fl);
  else
    decode_chunk_k<4, COMPACT>(eb, partial, mode, coder, s_tbl, wring, pring, stage, cbase, nw, np, dplane, pstride,
                               out, ubase, ustride, nc, nsteps, status, fl);
}

inline uint32_t groups_for(uint32_t n_chunks) { return (n_chunks + kWaves - 1) / kWaves; }

std::atomic<uint64_t> g_lds_plain{0}, g_lds_compact{0};   // devices configured, one bit each

// Compute units of the current device, asked once per device (devices 0..63);
// 2^32-1 when unknown, which marks no workgroup as the younger of its CU's two.
std::atomic<uint32_t> g_cus[64];
uint32_t device_cus() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0xFFFFFFFFu;
  uint32_t v = g_cus[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 0xFFFFFFFFu;
    v = (uint32_t)n;
    g_cus[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

int launch(const bs_chunk_task* tasks, uint32_t n_tasks, const bs_chunk_task& single, uint32_t groups,
           uint32_t max_mode, int32_t* status, void* stream) {
  const uint32_t first_round = device_cus();
  if (max_mode >= 2) {
    bs_internal::ensure_lds_limit((const void*)bsck_decode_kernel<true>, kLds, g_lds_compact);
    hipLaunchKernelGGL(bsck_decode_kernel<true>, dim3(groups), dim3(kThreads), kLds, (hipStream_t)stream,
                       tasks, n_tasks, single, status, first_round);
  } else {
    bs_internal::ensure_lds_limit((const void*)bsck_decode_kernel<false>, kLds, g_lds_plain);
    hipLaunchKernelGGL(bsck_decode_kernel<false>, dim3(groups), dim3(kThreads), kLds, (hipStream_t)stream,
                       tasks, n_tasks, single, status, first_round);
  }
  return hipGetLastError() == hipSuccess ? BS_OK : BS_ERR_HIP;
}

}  // namespace

extern "C" {

int bs_version(void) { return 300; }

int bs_chunk_chunks_per_group(void) { return kWaves; }

int bs_chunk_inspect(const uint8_t* h, uint64_t len, bs_chunk_info* info) {
  if (!h || !info) return BS_ERR_ARG;
  if (len < 32 || h[0] != 'B' || h[1] != 'S' || h[2] != 'C' || h[3] != 'K' || (h[4] != 2 && h[4] != kVersion))
    return BS_ERR_FORMAT;
  auto u32 = [&](int o) { return (uint32_t)h[o] | ((uint32_t)h[o + 1] << 8) | ((uint32_t)h[o + 2] << 16) | ((uint32_t)h[o + 3] << 24); };
  info->elem_bytes = h[5];
  info->plane_mode = h[6];
  info->n = (uint64_t)u32(8) | ((uint64_t)u32(12) << 32);
  info->steps = u32(16);
  info->lanes = (uint32_t)h[20] | ((uint32_t)h[21] << 8);
  info->n_syms = (uint32_t)h[22] | ((uint32_t)h[23] << 8);
  info->n_chunks = u32(24);
  info->coder = u32(28);
  const uint32_t mode = info->plane_mode, eb = info->elem_bytes;
  if (h[7] != 12 || (info->lanes != 64 && info->lanes != 128 && info->lanes != 256) || info->steps == 0 ||
      info->steps % (2 * kBlockMax) || info->n_syms == 0 || info->n_syms > 256 || (eb != 1 && eb != 2) || mode > 3 ||
      (eb == 1 ? (mode != 0 && mode != 3) : mode == 3) || info->coder > 2 ||
      (h[4] == 2 && (info->coder != 0 || mode == 3)) || (mode == 3 && (info->n & 1)))
    return BS_ERR_FORMAT;
  const uint64_t per = (uint64_t)info->lanes * info->steps;
  const uint64_t ne = mode == 3 ? info->n / 2 : info->n;
  if (per > kMaxChunk || info->n_chunks != (ne + per - 1) / per) return BS_ERR_FORMAT;
  return BS_OK;
}

int bs_chunk_decode(const uint8_t* d_blob, uint64_t blob_bytes, void* d_out, uint64_t n, uint32_t n_chunks,
                    uint32_t plane_mode, int32_t* d_status, void* stream) {
  if (!d_status || (n > 0 && (!d_blob || !d_out))) return BS_ERR_ARG;
  if (((uintptr_t)d_blob & 15u) != 0 || ((uintptr_t)d_out & 15u) != 0 || plane_mode > 3) return BS_ERR_ARG;
  if (n == 0 || n_chunks == 0) return BS_OK;
  bs_chunk_task t{d_blob, blob_bytes, d_out, n, 0u, n_chunks};
  return launch(nullptr, 0u, t, groups_for(n_chunks), plane_mode, d_status, stream);
}

int bs_chunk_decode_batch(const bs_chunk_task* d_tasks, uint32_t n_tasks, uint32_t total_groups,
                          uint32_t max_plane_mode, int32_t* d_status, void* stream) {
  if (!d_status || (n_tasks > 0 && !d_tasks) || max_plane_mode > 3) return BS_ERR_ARG;
  if (n_tasks == 0 || total_groups == 0) return BS_OK;
  bs_chunk_task dummy{};
  return launch(d_tasks, n_tasks, dummy, total_groups, max_plane_mode, d_status, stream);
}

}  // extern "C"
