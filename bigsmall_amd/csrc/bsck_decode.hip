// BSCK decode: the GPU-native chunked rANS format of the BigSmall decode
// engine, decoded on CDNA4 (gfx950).
//
// Format (little-endian; produced by bsck_encode.cpp):
//   [0]  "BSCK"  [4] u8 version=1  [5] u8 elem_bytes (1|2)  [6] u8 plane_mode
//   [7]  u8 prec_log2 = 12  [8] u64 n  [16] u32 steps  [20] u16 lanes = 64
//   [22] u16 n_syms  [24] u32 n_chunks  [28] u32 reserved
//   [32] n_syms x u32 symbol entries: bits 0..15 output value (bf16 word with
//        zero sign/mantissa for exponent symbols, or the exact word/byte),
//        bits 16..28 quantised frequency (sum 4096), bit 31 = reads one plane byte
//   pad to 16; n_chunks x {u64 offset, u32 n_words, u32 n_plane}
//   chunk (16-aligned): 64 x u32 initial states | n_words x u16 renorm words
//        (pad 16) | n_plane plane bytes (pad 16)
//
// Element j of chunk c is element c*64*steps + j of the tensor; lane j%64
// decodes it at step j/64, so one step of a wavefront produces 64 consecutive
// outputs (one 128-byte line for bf16). The 64 rANS states of a chunk share one
// 16-bit word stream: at each step the lanes whose state fell below L=2^16 take
// the next words in lane order, placed with a wavefront ballot + mbcnt prefix.
// Plane bytes (sign<<7 | mantissa) complete bf16 exponent symbols:
//   plane_mode 1 (dense): every element has one, stored per 8-step block with
//                         lane l's 8 bytes contiguous (one 8-byte load per lane
//                         per block, no prefix needed);
//   plane_mode 2 (compact): only elements whose symbol has bit 31 set have one,
//                         in decode order (ballot + mbcnt again);
//   plane_mode 0: no plane (every symbol is an exact value).
//
// rANS state machine (the same as the reference's, bigsmall/codecs/rans.py:165-207:
// 32-bit state, L = 2^16, 16-bit renormalisation, M = 2^12):
//   slot = x & 4095; s = sym(slot); x = f[s]*(x>>12) + slot - cf[s];
//   if x < L: x = (x << 16) | next_word
// A valid chunk ends with every lane back at x == L and every word and plane
// byte consumed; anything else is reported as BS_DEV_ERR_STREAM.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bigsmall_hip.h"

namespace {

#define LDS __attribute__((address_space(3)))
#define GLB __attribute__((address_space(1)))
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;                 // lanes of a wavefront
constexpr int kWaves = 8;                 // chunks (wavefronts) per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kBlock = 8;                 // steps per block (plane block, output flush, refill check)
constexpr uint32_t kRing = 2048;          // per-wave word ring (u16) and plane ring (bytes)
constexpr uint32_t kSeg = 256;            // refill segment: words (64 lanes x 8 B) / plane bytes (64 x 4 B)
constexpr uint32_t kL = 1u << 16;
// dynamic LDS layout (bytes): decode table | word rings | output staging | plane rings (compact launches)
constexpr uint32_t kTblBytes = 4096 * 8;
constexpr uint32_t kWringBytes = kWaves * kRing * 2;
constexpr uint32_t kStageMax = kBlock * 128 * 2;   // per wave: 8 steps x up to 128 states x 2 bytes
constexpr uint32_t kLdsLean = kTblBytes + kWringBytes + kWaves * kStageMax;
constexpr uint32_t kLdsCompact = kLdsLean + kWaves * kRing;

__device__ __forceinline__ uint32_t ld_u32(const GLB uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// rank of this lane among the set lanes of m, plus `base`
__device__ __forceinline__ uint32_t lane_rank(uint64_t m, uint32_t base) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, base));
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t pad16(uint32_t v) { return (v + 15u) & ~15u; }

__device__ __forceinline__ void report(int32_t* status, int32_t bits) {
  if (__lane_id() == 0) atomicOr(status, bits);
}

// A plane byte b = sign<<7 | mantissa completes an exponent symbol's value v:
// (b | b<<8) & 0x807F puts the sign at bit 15 and the mantissa at bits 0..6.
// `sel` picks byte q of the 8 plane bytes {hi:lo} into bytes 0 and 1.
__device__ __forceinline__ uint32_t plane_merge(uint32_t v, uint64_t bytes8, uint32_t sel) {
  const uint32_t bb = __builtin_amdgcn_perm((uint32_t)(bytes8 >> 32), (uint32_t)bytes8, sel);
  return (bb & 0x807Fu) | v;
}
__device__ __forceinline__ uint32_t byte_merge(uint32_t v, uint32_t b) { return ((b * 0x101u) & 0x807Fu) | v; }

// ---- ring refills: lane l moves 8 bytes (4 words) / 4 bytes of a 256-entry segment
__device__ __forceinline__ uint64_t load_wseg(const GLB uint64_t* src, uint32_t pos, uint32_t valid, uint32_t lane) {
  const uint32_t slot = pos / 4u + lane;
  return slot < valid ? src[slot] : 0ull;
}
// Unconditional variant for prefetches: out-of-range slots re-read `safe` (the
// chunk's state words: always inside the blob and in cache) so every block
// issues the same number of loads; a fixed count lets the compiler's waitcnt
// placement wait only for the data actually needed.
__device__ __forceinline__ uint64_t load_wseg_always(const GLB uint64_t* src, uint32_t pos, uint32_t valid, uint32_t lane,
                                                     const GLB uint64_t* safe) {
  const uint32_t slot = pos / 4u + lane;
  return *(slot < valid ? src + slot : safe + (lane & 31u));
}
__device__ __forceinline__ uint32_t load_pseg_always(const GLB uint32_t* src, uint32_t pos, uint32_t valid, uint32_t lane,
                                                     const GLB uint32_t* safe) {
  const uint32_t slot = pos / 4u + lane;
  return *(slot < valid ? src + slot : safe + lane);
}
__device__ __forceinline__ void store_wseg(LDS uint16_t* ring, uint32_t pos, uint64_t v, uint32_t lane) {
  *(LDS uint64_t*)(ring + ((pos + lane * 4u) & (kRing - 1u))) = v;
}
__device__ __forceinline__ uint32_t load_pseg(const GLB uint32_t* src, uint32_t pos, uint32_t valid, uint32_t lane) {
  const uint32_t slot = pos / 4u + lane;
  return slot < valid ? src[slot] : 0u;
}
__device__ __forceinline__ void store_pseg(LDS uint8_t* ring, uint32_t pos, uint32_t v, uint32_t lane) {
  *(LDS uint32_t*)(ring + ((pos + lane * 4u) & (kRing - 1u))) = v;
}

// Per-wavefront decode state of one chunk.
template <int K>
struct ChunkState {
  uint32_t x[K];
  uint32_t wptr, wld;    // word ring holds words [wptr, wld)
  uint32_t pptr, pld;    // plane ring (compact mode) holds bytes [pptr, pld)
  uint32_t wn, pn;       // segments prefetched for landing at the next block start
  uint64_t wp0, wp1;
  uint32_t pp0, pp1;
};

// Chunk-constant parameters.
struct ChunkParams {
  const GLB uint64_t* wsrc;     // renorm words, as 8-byte segments
  const GLB uint32_t* psrc;     // compact plane, as 4-byte segments
  const GLB uint64_t* dplane;   // dense plane, 8 bytes per lane per state group per block
  const GLB uint8_t* cbase;     // chunk start (its state words are a safe dummy address)
  GLB uint8_t* out8;
  uint64_t base;                // first element of the chunk
  uint32_t n_words, n_plane, wvalid, pvalid, nc, nsteps, nblk, lane;
};

// One block of kBlock steps: land prefetched ring segments, top up the rings
// if they hold less than a block of worst-case demand (rare), prefetch the
// next segments, decode into the LDS staging area, then store the staged block
// with one 16-byte store per lane per KiB.
template <int K, int MODE, int EB, bool PARTIAL>
__device__ __forceinline__ void decode_block(uint32_t blk, const uint64_t (&pl)[K], ChunkState<K>& S, const ChunkParams& C,
                                             const LDS uint64_t* __restrict__ tbl, LDS uint16_t* __restrict__ wring,
                                             LDS uint8_t* __restrict__ pring, LDS uint8_t* __restrict__ stage) {
  constexpr uint32_t kStates = kWave * K;
  constexpr uint32_t kBlkElems = kBlock * kStates;
  const uint32_t lane = C.lane;
  if (S.wn >= 1) { store_wseg(wring, S.wld, S.wp0, lane); S.wld += kSeg; }
  if (S.wn >= 2) { store_wseg(wring, S.wld, S.wp1, lane); S.wld += kSeg; }
  if (MODE == 2) {
    if (S.pn >= 1) { store_pseg(pring, S.pld, S.pp0, lane); S.pld += kSeg; }
    if (S.pn >= 2) { store_pseg(pring, S.pld, S.pp1, lane); S.pld += kSeg; }
  }
  {
    const uint32_t need_w = min(kBlkElems, C.n_words - S.wptr);
    while (S.wld - S.wptr < need_w && S.wld < C.n_words) {
      store_wseg(wring, S.wld, load_wseg(C.wsrc, S.wld, C.wvalid, lane), lane);
      S.wld += kSeg;
    }
    if (MODE == 2) {
      const uint32_t need_p = min(kBlkElems, C.n_plane - S.pptr);
      while (S.pld - S.pptr < need_p && S.pld < C.n_plane) {
        store_pseg(pring, S.pld, load_pseg(C.psrc, S.pld, C.pvalid, lane), lane);
        S.pld += kSeg;
      }
    }
  }
  wave_sync();
  // prefetch for the next block; always two loads per ring
  S.wn = 0;
  if (S.wld < C.n_words && S.wld - S.wptr + kSeg <= kRing) {
    S.wn = 1;
    if (S.wld + kSeg < C.n_words && S.wld - S.wptr + 2 * kSeg <= kRing) S.wn = 2;
  }
  S.wp0 = load_wseg_always(C.wsrc, S.wn >= 1 ? S.wld : 0u, C.wvalid, lane, (const GLB uint64_t*)C.cbase);
  S.wp1 = load_wseg_always(C.wsrc, S.wn >= 2 ? S.wld + kSeg : 0u, C.wvalid, lane, (const GLB uint64_t*)C.cbase);
  if (MODE == 2) {
    S.pn = 0;
    if (S.pld < C.n_plane && S.pld - S.pptr + kSeg <= kRing) {
      S.pn = 1;
      if (S.pld + kSeg < C.n_plane && S.pld - S.pptr + 2 * kSeg <= kRing) S.pn = 2;
    }
    S.pp0 = load_pseg_always(C.psrc, S.pn >= 1 ? S.pld : 0u, C.pvalid, lane, (const GLB uint32_t*)C.cbase);
    S.pp1 = load_pseg_always(C.psrc, S.pn >= 2 ? S.pld + kSeg : 0u, C.pvalid, lane, (const GLB uint32_t*)C.cbase);
  }

#pragma unroll
  for (int q = 0; q < kBlock; ++q) {
    const uint32_t t = blk * kBlock + q;
    if (PARTIAL && t >= C.nsteps) break;                 // wave-uniform
    const uint32_t sel = (uint32_t)q * 0x0101u | 0x0C0C0000u;
#pragma unroll
    for (int g = 0; g < K; ++g) {
      const uint32_t jl = t * kStates + g * kWave + lane;   // element index within the chunk
      const bool active = !PARTIAL || jl < C.nc;
      const uint64_t e = tbl[S.x[g] & 4095u];
      const uint32_t elo = (uint32_t)e, ehi = (uint32_t)(e >> 32);
      uint32_t xn = __umul24(elo & 0x1FFFu, S.x[g] >> 12) + (elo >> 13);
      if (PARTIAL && !active) xn = S.x[g];
      const bool need = xn < kL;
      const uint64_t m = __ballot(need);
      const uint32_t w = wring[lane_rank(m, S.wptr) & (kRing - 1u)];
      S.x[g] = need ? ((xn << 16) | w) : xn;
      S.wptr += (uint32_t)__popcll(m);
      uint32_t v = ehi;
      if (MODE == 1) {
        v = plane_merge(v, pl[g], sel);
      } else if (MODE == 2) {
        const bool cons = active && (ehi >> 31);
        const uint64_t bm = __ballot(cons);
        const uint32_t b = pring[lane_rank(bm, S.pptr) & (kRing - 1u)];
        S.pptr += (uint32_t)__popcll(bm);
        if (cons) v = byte_merge(v, b);
      }
      const uint32_t si = (uint32_t)q * kStates + g * kWave + lane;   // element index within the block
      if (EB == 2) ((LDS uint16_t*)stage)[si] = (uint16_t)v;
      else stage[si] = (uint8_t)v;
    }
  }
}

template <int K, int EB, bool PARTIAL>
__device__ __forceinline__ void flush_block(uint32_t blk, const ChunkParams& C, LDS uint8_t* __restrict__ stage) {
  constexpr uint32_t kBlkElems = kBlock * kWave * K;
  constexpr uint32_t kBlkBytes = kBlkElems * EB;
  wave_sync();
  const uint64_t blk_byte0 = (C.base + (uint64_t)blk * kBlkElems) * EB;
  const uint32_t valid_bytes = PARTIAL ? min(kBlkBytes, (C.nc - min(C.nc, blk * kBlkElems)) * EB) : kBlkBytes;
#pragma unroll
  for (uint32_t i = 0; i < (kBlkBytes + 1023) / 1024; ++i) {
    const uint32_t o = i * 1024u + C.lane * 16u;
    if (o + 16u <= valid_bytes) {
      const u32x4 d = *(const LDS u32x4*)(stage + o);
      *(GLB u32x4*)(C.out8 + blk_byte0 + o) = d;
    } else if (PARTIAL && o < valid_bytes) {
      for (uint32_t k = o; k < min(o + 16u, valid_bytes); ++k) C.out8[blk_byte0 + k] = stage[k];
    }
  }
}

// Decode one chunk with one wavefront: K interleaved states per lane (state
// v = g*64 + lane), MODE = plane mode, EB = element bytes, PARTIAL = chunk may
// be shorter than 64*K*steps (the tensor's last chunk).
template <int K, int MODE, int EB, bool PARTIAL>
__device__ __forceinline__ void decode_chunk(const LDS uint64_t* __restrict__ tbl, LDS uint16_t* __restrict__ wring,
                                             LDS uint8_t* __restrict__ pring, LDS uint8_t* __restrict__ stage,
                                             const GLB uint8_t* __restrict__ cbase, uint32_t n_words,
                                             uint32_t n_plane, GLB uint8_t* __restrict__ out8, uint64_t base,
                                             uint32_t nc, uint32_t nsteps, int32_t* status) {
  constexpr uint32_t kStates = kWave * K;
  constexpr uint32_t kBlkU64 = kBlock * kStates / 8;   // dense-plane u64s per block
  ChunkParams C;
  C.lane = __lane_id();
  const uint32_t wbytes = pad16(n_words * 2u);
  C.wsrc = (const GLB uint64_t*)(cbase + 4u * kStates);
  const GLB uint8_t* psrc8 = cbase + 4u * kStates + wbytes;
  C.psrc = (const GLB uint32_t*)psrc8;
  C.dplane = (const GLB uint64_t*)psrc8;
  C.cbase = cbase;
  C.out8 = out8;
  C.base = base;
  C.n_words = n_words;
  C.n_plane = n_plane;
  C.wvalid = wbytes / 8u;
  C.pvalid = pad16(n_plane) / 4u;
  C.nc = nc;
  C.nsteps = nsteps;
  C.nblk = (nsteps + kBlock - 1) / kBlock;

  ChunkState<K> S;
#pragma unroll
  for (int g = 0; g < K; ++g) S.x[g] = ((const GLB uint32_t*)cbase)[g * kWave + C.lane];
  S.wptr = S.wld = S.pptr = S.pld = 0;
  S.wn = S.pn = 0;
  S.wp0 = S.wp1 = 0;
  S.pp0 = S.pp1 = 0;

  // dense plane double buffer (blocks b and b+1), reloaded two blocks ahead
  uint64_t plA[K], plB[K];
#pragma unroll
  for (int g = 0; g < K; ++g) {
    plA[g] = 0;
    plB[g] = 0;
    if (MODE == 1) {
      plA[g] = C.dplane[C.lane * K + g];
      plB[g] = C.dplane[min(1u, C.nblk - 1) * kBlkU64 + C.lane * K + g];
    }
  }
  // Consume the prologue loads here, so the loop body never waits on them.
#pragma unroll
  for (int g = 0; g < K; ++g) asm volatile("" ::"v"(S.x[g]), "v"(plA[g]), "v"(plB[g]));

  // Two blocks per iteration so the dense-plane registers alternate without
  // copies. Full chunks have an even block count (steps % 16 == 0), so the
  // second half is unconditional and every iteration issues the same memory
  // operations.
  for (uint32_t blk = 0; blk < C.nblk; blk += 2) {
    decode_block<K, MODE, EB, PARTIAL>(blk, plA, S, C, tbl, wring, pring, stage);
    if (MODE == 1) {
      const uint32_t nb = min(blk + 2, C.nblk - 1);
#pragma unroll
      for (int g = 0; g < K; ++g) plA[g] = C.dplane[nb * kBlkU64 + C.lane * K + g];
    }
    flush_block<K, EB, PARTIAL>(blk, C, stage);
    if (PARTIAL && blk + 1 >= C.nblk) break;
    decode_block<K, MODE, EB, PARTIAL>(blk + 1, plB, S, C, tbl, wring, pring, stage);
    if (MODE == 1) {
      const uint32_t nb = min(blk + 3, C.nblk - 1);
#pragma unroll
      for (int g = 0; g < K; ++g) plB[g] = C.dplane[nb * kBlkU64 + C.lane * K + g];
    }
    flush_block<K, EB, PARTIAL>(blk + 1, C, stage);
  }

  bool bad_state = false;
#pragma unroll
  for (int g = 0; g < K; ++g) bad_state |= S.x[g] != kL;
  const bool bad = __ballot(bad_state) != 0 || S.wptr != n_words || (MODE == 2 && S.pptr != n_plane);
  if (bad) report(status, BS_DEV_ERR_STREAM);
}

template <int K, int EB, bool PARTIAL, bool COMPACT>
__device__ __forceinline__ void decode_chunk_mode(uint32_t mode, const LDS uint64_t* tbl, LDS uint16_t* wring,
                                                  LDS uint8_t* pring, LDS uint8_t* stage, const GLB uint8_t* cbase,
                                                  uint32_t nw, uint32_t np, GLB uint8_t* out, uint64_t base,
                                                  uint32_t nc, uint32_t nsteps, int32_t* status) {
  if (EB == 1 || mode == 0)
    decode_chunk<K, 0, EB, PARTIAL>(tbl, wring, pring, stage, cbase, nw, np, out, base, nc, nsteps, status);
  else if (mode == 1)
    decode_chunk<K, 1, EB, PARTIAL>(tbl, wring, pring, stage, cbase, nw, np, out, base, nc, nsteps, status);
  else if (COMPACT)
    decode_chunk<K, 2, EB, PARTIAL>(tbl, wring, pring, stage, cbase, nw, np, out, base, nc, nsteps, status);
}

template <int K, bool COMPACT>
__device__ __forceinline__ void decode_chunk_k(uint32_t eb, bool partial, uint32_t mode, const LDS uint64_t* tbl,
                                               LDS uint16_t* wring, LDS uint8_t* pring, LDS uint8_t* stage,
                                               const GLB uint8_t* cbase, uint32_t nw, uint32_t np, GLB uint8_t* out,
                                               uint64_t base, uint32_t nc, uint32_t nsteps, int32_t* status) {
  if (eb == 2) {
    if (partial) decode_chunk_mode<K, 2, true, COMPACT>(mode, tbl, wring, pring, stage, cbase, nw, np, out, base, nc, nsteps, status);
    else decode_chunk_mode<K, 2, false, COMPACT>(mode, tbl, wring, pring, stage, cbase, nw, np, out, base, nc, nsteps, status);
  } else {
    if (partial) decode_chunk_mode<K, 1, true, COMPACT>(0, tbl, wring, pring, stage, cbase, nw, np, out, base, nc, nsteps, status);
    else decode_chunk_mode<K, 1, false, COMPACT>(0, tbl, wring, pring, stage, cbase, nw, np, out, base, nc, nsteps, status);
  }
}

template <bool COMPACT>
__global__ __launch_bounds__(kThreads) void bsck_decode_kernel(const bs_chunk_task* __restrict__ tasks,
                                                               uint32_t n_tasks, bs_chunk_task single,
                                                               int32_t* __restrict__ status) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  LDS uint64_t* s_tbl = (LDS uint64_t*)smem;
  LDS uint16_t* s_wring = (LDS uint16_t*)(smem + kTblBytes);
  LDS uint8_t* s_stage = (LDS uint8_t*)(smem + kTblBytes + kWringBytes);
  LDS uint8_t* s_pring = (LDS uint8_t*)(smem + kLdsLean);
  // table-build scratch overlaps the staging area (unused until decoding starts)
  LDS uint32_t* s_cum = (LDS uint32_t*)s_stage;        // 257 entries
  LDS uint32_t* s_val = s_cum + 260;                    // 256 entries
  LDS uint32_t* s_flag = s_val + 256;                   // table-check flag

  // ---- which tensor does this workgroup serve (wave-uniform binary search)
  bs_chunk_task T = single;
  if (tasks != nullptr) {
    uint32_t lo = 0, hi = n_tasks;
    while (hi - lo > 1) {
      uint32_t mid = (lo + hi) >> 1;
      if (tasks[mid].wg_begin <= blockIdx.x) lo = mid; else hi = mid;
    }
    T = tasks[lo];
  }
  const uint32_t group = blockIdx.x - T.wg_begin;
  const GLB uint8_t* __restrict__ b = (const GLB uint8_t*)T.blob;

  // ---- header checks (uniform across the workgroup)
  if (T.blob_bytes < 32 || b[0] != 'B' || b[1] != 'S' || b[2] != 'C' || b[3] != 'K' || b[4] != 1 ||
      (b[5] != 1 && b[5] != 2) || b[6] > 2 || b[7] != 12 || (!COMPACT && b[6] == 2)) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  const uint32_t eb = b[5], mode = b[6];
  const uint64_t n = (uint64_t)ld_u32(b + 8) | ((uint64_t)ld_u32(b + 12) << 32);
  const uint32_t steps = ld_u32(b + 16);
  const uint32_t lanes = (uint32_t)b[20] | ((uint32_t)b[21] << 8);
  const uint32_t nsym = (uint32_t)b[22] | ((uint32_t)b[23] << 8);
  const uint32_t nch = ld_u32(b + 24);
  const uint64_t per = (uint64_t)lanes * steps;
  if ((lanes != 64 && lanes != 128) || steps == 0 || (steps % (2 * kBlock)) != 0 || nsym == 0 ||
      nsym > 256 || (eb == 1 && mode != 0) || nch != T.n_chunks || per == 0 || nch != (n + per - 1) / per) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  if (n != T.n) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_COUNT);
    return;
  }
  const uint32_t ctab = pad16(32u + 4u * nsym);
  if ((uint64_t)ctab + 16ull * nch > T.blob_bytes) {
    if (threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_BOUNDS);
    return;
  }

  // ---- decode table in LDS: slot -> {f | (slot-cf) << 13, value | consume << 31}
  const uint32_t tid = threadIdx.x;
  uint32_t f_own = 0;
  if (tid < nsym) {
    const uint32_t ent = ld_u32(b + 32 + 4 * tid);
    f_own = (ent >> 16) & 0x1FFFu;
    s_val[tid] = (ent & 0xFFFFu) | (ent & 0x80000000u);
  }
  if (tid < 256) s_cum[tid + 1] = f_own;
  if (tid == 0) { s_cum[0] = 0; *s_flag = 0; }
  __syncthreads();
  for (uint32_t d = 1; d < 256; d <<= 1) {        // inclusive scan of s_cum[1..256]
    uint32_t add = (tid < 256 && tid >= d) ? s_cum[tid + 1 - d] : 0u;
    __syncthreads();
    if (tid < 256) s_cum[tid + 1] += add;
    __syncthreads();
  }
  if ((tid == 0 && s_cum[256] != 4096u) || (tid < nsym && f_own == 0)) *s_flag = 1;
  __syncthreads();
  if (*s_flag) {
    if (tid == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  for (uint32_t slot = tid; slot < 4096u; slot += kThreads) {
    uint32_t lo = 0, hi = nsym;                      // cum[lo] <= slot < cum[hi]
    while (hi - lo > 1) {
      uint32_t mid = (lo + hi) >> 1;
      if (s_cum[mid] <= slot) lo = mid; else hi = mid;
    }
    const uint32_t f = s_cum[lo + 1] - s_cum[lo];
    s_tbl[slot] = (uint64_t)(f | ((slot - s_cum[lo]) << 13)) | ((uint64_t)s_val[lo] << 32);
  }
  __syncthreads();

  // ---- one chunk per wavefront
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);   // wave-uniform: keeps chunk state scalar
  const uint32_t chunk = group * kWaves + wave;
  if (chunk >= nch) return;
  const GLB uint8_t* ce = b + ctab + 16ull * chunk;
  const uint64_t off = (uint64_t)ld_u32(ce) | ((uint64_t)ld_u32(ce + 4) << 32);
  const uint32_t nw = ld_u32(ce + 8), np = ld_u32(ce + 12);
  const uint64_t cbase_idx = (uint64_t)chunk * per;
  const uint32_t nc = (uint32_t)((n - cbase_idx) < per ? (n - cbase_idx) : per);
  const uint32_t nsteps = (nc + lanes - 1) / lanes;
  const uint32_t dense_plane = ((nsteps + kBlock - 1) / kBlock) * kBlock * lanes;
  bool ok = (off % 16) == 0 && off + 4ull * lanes + pad16(nw * 2u) + pad16(np) <= T.blob_bytes &&
            nw <= nsteps * lanes && T.out != nullptr && ((uintptr_t)T.out & 15u) == 0;
  if (mode == 1) ok = ok && np == dense_plane;
  if (mode == 2) ok = ok && np <= nc;
  if (mode == 0) ok = ok && np == 0;
  if (!ok) {
    report(status, BS_DEV_ERR_BOUNDS);
    return;
  }
  const GLB uint8_t* cbase = b + off;
  LDS uint16_t* wring = s_wring + wave * kRing;
  LDS uint8_t* pring = s_pring + wave * kRing;
  LDS uint8_t* stage = s_stage + wave * kStageMax;
  GLB uint8_t* out = (GLB uint8_t*)T.out;
  const bool partial = nc != per;
  if (lanes == 64)
    decode_chunk_k<1, COMPACT>(eb, partial, mode, s_tbl, wring, pring, stage, cbase, nw, np, out, cbase_idx, nc, nsteps, status);
  else
    decode_chunk_k<2, COMPACT>(eb, partial, mode, s_tbl, wring, pring, stage, cbase, nw, np, out, cbase_idx, nc, nsteps, status);
}

inline uint32_t groups_for(uint32_t n_chunks) { return (n_chunks + kWaves - 1) / kWaves; }

bool g_attr_set = false;
void ensure_lds_attr() {
  if (g_attr_set) return;
  (void)hipFuncSetAttribute((const void*)bsck_decode_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLean);
  (void)hipFuncSetAttribute((const void*)bsck_decode_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsCompact);
  g_attr_set = true;
}

int launch(const bs_chunk_task* tasks, uint32_t n_tasks, const bs_chunk_task& single, uint32_t groups,
           uint32_t max_mode, int32_t* status, void* stream) {
  ensure_lds_attr();
  if (max_mode >= 2)
    hipLaunchKernelGGL(bsck_decode_kernel<true>, dim3(groups), dim3(kThreads), kLdsCompact, (hipStream_t)stream,
                       tasks, n_tasks, single, status);
  else
    hipLaunchKernelGGL(bsck_decode_kernel<false>, dim3(groups), dim3(kThreads), kLdsLean, (hipStream_t)stream,
                       tasks, n_tasks, single, status);
  return hipGetLastError() == hipSuccess ? BS_OK : BS_ERR_HIP;
}

}  // namespace

extern "C" {

int bs_version(void) { return 100; }

int bs_chunk_chunks_per_group(void) { return kWaves; }

int bs_chunk_inspect(const uint8_t* h, uint64_t len, bs_chunk_info* info) {
  if (!h || !info) return BS_ERR_ARG;
  if (len < 32 || h[0] != 'B' || h[1] != 'S' || h[2] != 'C' || h[3] != 'K' || h[4] != 1) return BS_ERR_FORMAT;
  auto u32 = [&](int o) { return (uint32_t)h[o] | ((uint32_t)h[o + 1] << 8) | ((uint32_t)h[o + 2] << 16) | ((uint32_t)h[o + 3] << 24); };
  info->elem_bytes = h[5];
  info->plane_mode = h[6];
  info->n = (uint64_t)u32(8) | ((uint64_t)u32(12) << 32);
  info->steps = u32(16);
  info->lanes = (uint32_t)h[20] | ((uint32_t)h[21] << 8);
  info->n_syms = (uint32_t)h[22] | ((uint32_t)h[23] << 8);
  info->n_chunks = u32(24);
  if (h[7] != 12 || (info->lanes != 64 && info->lanes != 128) || info->steps == 0 || info->steps % (2 * kBlock) || info->n_syms == 0 ||
      info->n_syms > 256 || (info->elem_bytes != 1 && info->elem_bytes != 2) || info->plane_mode > 2)
    return BS_ERR_FORMAT;
  const uint64_t per = (uint64_t)info->lanes * info->steps;
  if (info->n_chunks != (info->n + per - 1) / per) return BS_ERR_FORMAT;
  return BS_OK;
}

int bs_chunk_decode(const uint8_t* d_blob, uint64_t blob_bytes, void* d_out, uint64_t n, uint32_t n_chunks,
                    uint32_t plane_mode, int32_t* d_status, void* stream) {
  if (!d_status || (n > 0 && (!d_blob || !d_out))) return BS_ERR_ARG;
  if (((uintptr_t)d_blob & 15u) != 0 || ((uintptr_t)d_out & 15u) != 0 || plane_mode > 2) return BS_ERR_ARG;
  if (n == 0 || n_chunks == 0) return BS_OK;
  bs_chunk_task t{d_blob, blob_bytes, d_out, n, 0u, n_chunks};
  return launch(nullptr, 0u, t, groups_for(n_chunks), plane_mode, d_status, stream);
}

int bs_chunk_decode_batch(const bs_chunk_task* d_tasks, uint32_t n_tasks, uint32_t total_groups,
                          uint32_t max_plane_mode, int32_t* d_status, void* stream) {
  if (!d_status || (n_tasks > 0 && !d_tasks) || max_plane_mode > 2) return BS_ERR_ARG;
  if (n_tasks == 0 || total_groups == 0) return BS_OK;
  bs_chunk_task dummy{};
  return launch(d_tasks, n_tasks, dummy, total_groups, max_plane_mode, d_status, stream);
}

}  // extern "C"
