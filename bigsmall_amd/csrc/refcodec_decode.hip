// GPU decode of the reference's own rANS-family bf16 formats:
//   bf16_parallel_v1   (bigsmall/codecs/bf16_parallel.py:262-352, streams via rans.py:165-207)
//   bf16_se_tans       (bigsmall/codecs/bf16_tans.py:121-167, streams via numba_rans.py:168-192)
//   bf16_se_single_kernel (bigsmall/codecs/single_kernel.py:431-580)
//
// All three code a bf16 word as a sign+exponent ("SE", 9-bit) symbol with
// rANS M = 4096, plus the 7-bit mantissa with a per-exponent rANS table
// (M = 1024), in "buckets": the mantissas of the elements that share an
// exponent, in element order (a stable sort by exponent). The state machine is
// the same everywhere: 32-bit state, L = 2^16, 16-bit renormalisation,
//   slot = x & (M-1); s = sym(slot); x = f*(x >> log2 M) + slot - cf;
//   while (x < L && words remain) x = (x << 16) | next_word;
// The formats differ only in framing, which the host resolves into the
// stream descriptors below (initial state, word array, optional odd trailing
// byte that reads as one more word).
//
// Decoding is two launches on one stream:
//   1. se_kernel: one lane per SE stream (bf16_parallel_v1 has N interleaved
//      streams, the other two formats one). Writes sign<<15 | exp<<7 of every
//      element, and the element's index into `perm` at the next free position
//      of its (stream, exponent) bucket: per-lane cursors in LDS give the
//      stable-sort rank without any sort.
//   2. mant_kernel: one lane per bucket. Decodes the bucket's mantissas in
//      order and ORs mantissa r into element perm[bucket_begin + r].
// The SE decode tables sit in LDS; mantissa tables (1024 entries per
// exponent, up to 256 of them) are read through the caches.
#include <stdint.h>

#include "simt.h"

#include "../../include/bigsmall_hip.h"
#include "lds_limit.h"

namespace {


constexpr uint32_t kL = 1u << 16;
constexpr int kWave = 64;
constexpr int kSeLanes = 64;        // SE streams per workgroup (one wavefront)
constexpr int kMantThreads = 64;

__device__ __forceinline__ uint32_t word_at(const GLB uint8_t* w, uint32_t i) {
  return (uint32_t)w[2 * i] | ((uint32_t)w[2 * i + 1] << 8);   // byte loads: any alignment
}

// One renormalisation with the reference's loop: while the state is below L
// and words remain, shift one in. The optional tail is the last "word".
__device__ __forceinline__ void renorm(uint32_t& x, uint32_t& pos, uint32_t n_eff, const GLB uint8_t* w,
                                       uint32_t n_words, uint32_t tail) {
  while (x < kL && pos < n_eff) {
    const uint32_t v = pos < n_words ? word_at(w, pos) : (tail & 0xFFFFu);
    x = (x << 16) | v;
    ++pos;
  }
}

__device__ __forceinline__ void flag(int32_t* status, int32_t bits) { atomicOr(status, bits); }

// SE table (LDS): slot -> {f | (slot - cf) << 13, symbol}
__global__ __launch_bounds__(kSeLanes) void se_kernel(const bs_se_stream* __restrict__ streams, uint32_t n_streams,
                                                      const uint32_t* __restrict__ se_table,
                                                      const uint32_t* __restrict__ bstart, uint64_t n_out,
                                                      uint16_t* __restrict__ out, uint32_t* __restrict__ perm,
                                                      int32_t* __restrict__ status) {
  BS_DYNAMIC_LDS(smem);
  LDS uint64_t* s_tbl = (LDS uint64_t*)smem;                   // 4096 entries
  LDS uint32_t* s_cur = (LDS uint32_t*)(smem + 4096 * 8);      // cursor of exponent e for lane l at e*64 + l
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < 4096; i += kSeLanes)
    s_tbl[i] = (uint64_t)se_table[2 * i] | ((uint64_t)se_table[2 * i + 1] << 32);
  const uint32_t sid = blockIdx.x * kSeLanes + lane;
  const bool live = sid < n_streams;
  const GLB uint32_t* bs = (const GLB uint32_t*)bstart + (uint64_t)(live ? sid : 0) * 257;
  for (uint32_t e = 0; e < 256; ++e) s_cur[e * kSeLanes + lane] = live ? bs[e] : 0u;
  __syncthreads();
  if (!live) return;

  const bs_se_stream S = streams[sid];
  const GLB uint8_t* w = (const GLB uint8_t*)S.words;
  const uint32_t n_eff = S.n_words + ((S.tail >> 16) & 1u);
  uint32_t x = S.x0, pos = 0;
  uint64_t idx = S.first;
  const uint32_t pend = bs[256];   // the stream's perm region ends here: no write goes past it
  bool bad = false;
  for (uint32_t i = 0; i < S.n; ++i, idx += S.stride) {
    const uint64_t ent = s_tbl[x & 4095u];
    const uint32_t lo = (uint32_t)ent, sym = (uint32_t)(ent >> 32);
    x = (lo & 0x1FFFu) * (x >> 12) + (lo >> 13);
    renorm(x, pos, n_eff, w, S.n_words, S.tail);
    const uint32_t e = sym & 0xFFu;
    const uint32_t p = s_cur[e * kSeLanes + lane];
    if (idx < n_out && p < pend) {
      out[idx] = (uint16_t)((((sym >> 8) & 1u) << 15) | (e << 7));
      perm[p] = (uint32_t)idx;
      s_cur[e * kSeLanes + lane] = p + 1;
    } else {
      bad = true;   // more elements than the stream's buckets hold, or a bad index
    }
  }
  // every bucket must be exactly full: the header's bucket sizes match the
  // decoded exponents (a bucket overfilled into its neighbour leaves one short)
  for (uint32_t e = 0; e < 256; ++e) bad |= s_cur[e * kSeLanes + lane] != bs[e + 1];
  if (bad) flag(status, BS_DEV_ERR_COUNT);
  if (x != kL || pos != n_eff) flag(status, BS_DEV_ERR_STREAM);
}

// Mantissa table (global): table*1024 + slot -> f | (slot - cf) << 11 | symbol << 21
__global__ __launch_bounds__(kMantThreads) void mant_kernel(const bs_mant_bucket* __restrict__ buckets,
                                                            uint32_t n_buckets, const uint32_t* __restrict__ tables,
                                                            uint32_t n_tables, const uint32_t* __restrict__ perm,
                                                            uint64_t n_perm, uint64_t n_out,
                                                            uint16_t* __restrict__ out, int32_t* __restrict__ status) {
  const uint32_t bid = blockIdx.x * kMantThreads + threadIdx.x;
  if (bid >= n_buckets) return;
  const bs_mant_bucket B = buckets[bid];
  if (B.table >= n_tables || B.perm_begin + B.n > n_perm) {
    flag(status, BS_DEV_ERR_HEADER);
    return;
  }
  const GLB uint32_t* tbl = (const GLB uint32_t*)tables + (uint64_t)B.table * 1024;
  const GLB uint8_t* w = (const GLB uint8_t*)B.words;
  const uint32_t n_eff = B.n_words + ((B.tail >> 16) & 1u);
  uint32_t x = B.x0, pos = 0;
  bool bad = false;
  for (uint32_t r = 0; r < B.n; ++r) {
    const uint32_t ent = tbl[x & 1023u];
    x = (ent & 0x7FFu) * (x >> 10) + ((ent >> 11) & 0x3FFu);
    renorm(x, pos, n_eff, w, B.n_words, B.tail);
    const uint32_t idx = perm[B.perm_begin + r];
    if (idx < n_out) out[idx] |= (uint16_t)((ent >> 21) & 0x7Fu);
    else bad = true;
  }
  if (bad) flag(status, BS_DEV_ERR_COUNT);
  if (x != kL || pos != n_eff) flag(status, BS_DEV_ERR_STREAM);
}

// ---- wave-serial path: every SE stream (one for bf16_se_tans and
// bf16_se_single_kernel, N interleaved ones for bf16_parallel_v1) and every
// mantissa bucket is a chain decoded by its own wavefront.
//
// Each chain is decoded by one wavefront. The chain itself is uniform (every
// lane computes the same state; the compiler keeps it in scalar registers),
// the decode table sits in LDS, and the lanes cooperate on everything around
// it: they load the word stream 1 KB at a time into an LDS byte ring one
// segment ahead of use, hold a 128-word window of it in two registers (lane
// l: words base + l and base + 64 + l, moved on at most once per 64 steps) so
// that a renormalisation takes its word with a readlane and no branch, and
// they stage 64 consecutive outputs (lane j keeps step j) for one coalesced
// store. The SE chain writes sign<<15 | exp<<7 of
// every element and counts the exponents of each tile of kTile symbols of its
// stream; the mantissa chains, which do not depend on it, run at the same time
// in other workgroups and write their bucket's mantissas in bucket order. Two
// parallel passes then give every element its position in its (stream,
// exponent) bucket (a stable counting sort by exponent within each stream: a
// scan of the tile counts over the stream's tiles, then per-tile ranks by
// wavefront ballots) and OR in its mantissa.

constexpr uint32_t kRingB = 2048;     // word-stream byte ring per chain (two segments: one landed, one in flight)
constexpr uint32_t kSegB = 1024;      // bytes per cooperative load (64 lanes x 16 B)
constexpr uint32_t kTile = 16384;     // elements per tile of the placement passes
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// This lane's 16 bytes of ring segment q of a stream whose bytes are
// [s_off, e_off) relative to the 16-byte aligned address A. Bytes outside that
// range are never read (they come back as zero).
__device__ __forceinline__ u32x4 seg_block(const GLB uint8_t* A, uint64_t q, uint32_t lane, uint64_t s_off,
                                           uint64_t e_off) {
  const uint64_t b0 = q * kSegB + lane * 16u;
  if (b0 >= s_off && b0 + 16u <= e_off) return *(const GLB u32x4*)(A + b0);
  u32x4 r = {0u, 0u, 0u, 0u};
#pragma unroll
  for (uint32_t k = 0; k < 16; ++k) {
    const uint64_t b = b0 + k;
    if (b >= s_off && b < e_off) r[k >> 2] |= (uint32_t)A[b] << (8u * (k & 3u));
  }
  return r;
}

__device__ __forceinline__ void seg_land(LDS uint8_t* ring, uint64_t q, uint32_t lane, u32x4 v) {
  *(LDS u32x4*)(ring + ((q * kSegB + lane * 16u) & (kRingB - 1u))) = v;
}

// A stream descriptor every pass of the serial path may use: at most max_len
// symbols (what the placement tiles cover) and every element index inside the
// output. The chain and placement kernels check it alike, so a bad
// descriptor is reported and skipped, never followed.
__device__ __forceinline__ bool stream_ok(const bs_se_stream& S, uint64_t max_len, uint64_t n_out) {
  return S.n <= max_len && S.stride != 0 && (S.n == 0 || S.first + (uint64_t)(S.n - 1) * S.stride < n_out);
}

// Exponent counts of an SE chain, kept in the wave's own 256 LDS bins for
// the current tile of kTile symbols and written to ghist[tile][256] when the
// tile ends (symbols [i0, i0 + cnt) are this batch, lane j holding output
// word j; a stream of n symbols). Counting here, one LDS add per lane per 64
// steps, replaced a pass that read every output word back with a stride of
// n_streams elements (1.6 of 39 ms for an 8B layer in bf16_parallel_v1).
__device__ __forceinline__ void tile_count(LDS uint32_t* hist, GLB uint32_t* ghist, uint32_t word, uint32_t lane,
                                           uint32_t i0, uint32_t cnt, uint32_t n) {
  if (lane < cnt) BS_LDS_ADD(hist + ((word >> 7) & 0xFFu), 1u);
  const uint32_t end = i0 + cnt;
  if (end % kTile == 0 || end == n) {
    wave_sync();
    GLB uint32_t* g = ghist + (uint64_t)(i0 / kTile) * 256u;
    for (uint32_t b = lane; b < 256; b += kWave) {
      g[b] = hist[b];
      hist[b] = 0;
    }
    wave_sync();
  }
}
// Before an SE chain: empty bins. After it: zero counts for the tiles its n
// symbols do not reach (of the task's tps per stream).
__device__ __forceinline__ void tile_count_begin(LDS uint32_t* hist, uint32_t lane) {
  for (uint32_t b = lane; b < 256; b += kWave) hist[b] = 0;
  wave_sync();
}
__device__ __forceinline__ void tile_count_end(GLB uint32_t* ghist, uint32_t lane, uint32_t n, uint32_t tps) {
  for (uint64_t i = ((uint64_t)n + kTile - 1) / kTile * 256u + lane; i < (uint64_t)tps * 256u; i += kWave) ghist[i] = 0;
}

// Decode one chain of n symbols. The LDS table has one 16-byte entry per slot,
// {f, slot - cf, output, 0} (SE: M = 4096, output the word sign<<15 | exp<<7,
// stored as u16; mantissa: M = 1024, output one byte per symbol), so a step is
// one table read and one v_mad_u32_u24 on the state, which every lane holds.
// One wavefront issues about one instruction per four cycles, so the step is
// kept to a dozen instructions: the renormalisation is a scalar branch on the
// state, its word comes from a register window by readlane, and the output is
// staged with a lane select.
//
// Renormalisation: the reference loops `while x < L and words remain`. From a
// state x >= L one decode step leaves x >= 2^4 (SE) or 2^6 (mantissa), so one
// shifted-in word restores x >= L: a valid stream never takes the loop twice,
// and an initial state below L, which no encoder writes, is reported as a
// corrupt stream. A corrupt stream that runs out of words shifts in its tail
// word (zero when it has none) and fails the end-of-stream check.
template <bool SE>
__device__ __forceinline__ void serial_chain(const GLB uint8_t* words, uint32_t n_words, uint32_t tail, uint32_t x0,
                                             uint32_t n, const LDS u32x4* __restrict__ tbl,
                                             LDS uint8_t* ring, LDS uint16_t* stage, GLB uint8_t* __restrict__ out,
                                             uint32_t stride, LDS uint32_t* hist, GLB uint32_t* ghist, uint32_t tps,
                                             int32_t* status) {
  constexpr uint32_t kSlotMask = SE ? 4095u : 1023u;
  constexpr uint32_t kShift = SE ? 12u : 10u;
  const uint32_t lane = __lane_id();
  const uint64_t wa = (uint64_t)words;
  const GLB uint8_t* A = (const GLB uint8_t*)(wa & ~15ull);
  const uint32_t s_off = (uint32_t)(wa & 15u);
  const uint64_t e_off = s_off + 2ull * n_words;
  const uint32_t n_eff = n_words + ((tail >> 16) & 1u);
  const uint32_t tail_word = tail & 0xFFFFu;
  uint64_t landed = 0;        // stream bytes [.., landed) are in the ring (relative to A)
  bool inflight = false;      // segment `landed / kSegB` is being loaded into `seg`
  u32x4 seg = {0u, 0u, 0u, 0u};
  uint32_t x = x0, pos = 0;
  // Word window: lane l of w_lo / w_hi holds word base + l / base + 64 + l.
  // At a batch start pos - base < 64, so the batch's at most 64 words are in it.
  uint32_t base = 0, w_lo = 0, w_hi = 0;
  if (x0 < kL) {
    if (lane == 0) flag(status, BS_DEV_ERR_STREAM);
    return;
  }
  if (SE) tile_count_begin(hist, lane);
  auto ring_word = [&](uint32_t idx) {
    const uint32_t b = s_off + 2u * idx;
    return (uint32_t)ring[b & (kRingB - 1u)] | ((uint32_t)ring[(b + 1u) & (kRingB - 1u)] << 8);
  };
  // The state stays in a vector register (the empty asm hides its uniformity,
  // which would otherwise move the update to scalar instructions plus two
  // readfirstlanes); only the renormalisation test reads it back.
  BS_OPAQUE(x);
  auto step = [&](uint32_t j) {
    const u32x4 e = tbl[x & kSlotMask];
    uint32_t xn = __umul24(e.x, x >> kShift) + e.y;         // v_mad_u32_u24 (f <= 4096)
    if ((uint32_t)__builtin_amdgcn_readfirstlane((int)xn) < kL) {   // uniform: a scalar branch
      const uint32_t d = pos - base;                       // < 128
      const uint32_t w_a = __builtin_amdgcn_readlane(w_lo, d & 63u);
      const uint32_t w_b = __builtin_amdgcn_readlane(w_hi, d & 63u);
      uint32_t w = d < (uint32_t)kWave ? w_a : w_b;
      w = pos < n_words ? w : tail_word;
      xn = (xn << 16) | w;
      ++pos;
    }
    x = xn;
    BS_OPAQUE(x);
    // the step's output goes to slot j of the wave's 64-entry stage (every
    // lane writes the same value), read back by lane j after the batch: a
    // select per step (keep = lane == j ? out : keep) made the optimiser hold
    // the batch's 64 outputs, or its 64 lane masks, in registers
    *(volatile LDS uint16_t*)(stage + j) = (uint16_t)e.z;
  };
  for (uint32_t i0 = 0; i0 < n; i0 += kWave) {
    // ring upkeep: the window reaches at most 128 words (256 bytes) past pos
    const uint64_t consumed = s_off + 2ull * pos;
    if (inflight) {
      seg_land(ring, landed / kSegB, lane, seg);
      landed += kSegB;
      inflight = false;
    }
    while (landed < e_off && landed < consumed + 4u * kWave + 2u) {
      seg_land(ring, landed / kSegB, lane, seg_block(A, landed / kSegB, lane, s_off, e_off));
      landed += kSegB;
    }
    if (landed < e_off && landed + kSegB <= consumed + kRingB) {
      seg = seg_block(A, landed / kSegB, lane, s_off, e_off);
      inflight = true;
    }
    wave_sync();
    if (i0 == 0) {
      w_lo = ring_word(lane);
      w_hi = ring_word(kWave + lane);
    } else if (pos - base >= (uint32_t)kWave) {           // one move keeps pos - base < 64
      base += kWave;
      w_lo = w_hi;
      w_hi = ring_word(base + kWave + lane);
    }
    const uint32_t cnt = min((uint32_t)kWave, n - i0);
    if (cnt == (uint32_t)kWave) {
#pragma unroll
      for (uint32_t j = 0; j < (uint32_t)kWave; ++j) step(j);
    } else {
      for (uint32_t j = 0; j < cnt; ++j) step(j);
    }
    wave_sync();
    const uint32_t keep = stage[lane];
    if (lane < cnt) {
      if (SE) ((GLB uint16_t*)out)[(uint64_t)(i0 + lane) * stride] = (uint16_t)keep;
      else out[i0 + lane] = (uint8_t)keep;
    }
    if (SE) tile_count(hist, ghist, keep, lane, i0, cnt, n);
  }
  if (SE) tile_count_end(ghist, lane, n, tps);
  if (__builtin_amdgcn_readfirstlane(x) != kL || pos != n_eff) {
    if (lane == 0) flag(status, BS_DEV_ERR_STREAM);
  }
}

// The same chain with the state in scalar registers and the table read
// through the scalar cache (uniform loads, read-only): one s_load_dword and
// the update in SALU instructions; the step's output goes into one lane of a
// register. Tables of 4-byte entries: SE, {index | f << 8 | (slot - cf)
// << 20} (the 16 KB table of a tensor with at most 256 live sign/exponent
// symbols, none of frequency 4096; the index selects the output word from
// `out_words`, a 256-entry LDS map applied once per 64 outputs); mantissa,
// the global table itself {f | (slot - cf) << 11 | symbol << 21} (4 KB per
// bucket table). A scalar-cache hit comes back sooner than the LDS round
// trip, and the step issues fewer instructions (C0 in bf16_se_tans: 1.04
// against 1.22 s on one chain, before the register output). A 16 KB table
// stays in the scalar cache only while it has the cache of its CUs to
// itself (an 8B layer in bf16_parallel_v1, every tensor's SE groups spread
// over every XCD: 43-45 against 39-41 ms with LDS tables), so the host sets
// it per task and lays the SE groups out by XCD.
__device__ __forceinline__ uint32_t uni32(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ uint64_t uni64(uint64_t v) {
  return (uint64_t)uni32((uint32_t)v) | ((uint64_t)uni32((uint32_t)(v >> 32)) << 32);
}

template <bool SE>
__device__ __forceinline__ void serial_chain_scalar(const GLB uint8_t* words, uint32_t n_words, uint32_t tail,
                                                    uint32_t x0, uint32_t n, const CST uint32_t* t4_in,
                                                    const LDS uint32_t* out_words, LDS uint8_t* ring,
                                                    GLB uint8_t* __restrict__ out, uint32_t stride,
                                                    LDS uint32_t* hist, GLB uint32_t* ghist, uint32_t tps,
                                                    int32_t* status) {
  // the descriptor's fields are the same in every lane: say so, so that the
  // whole chain (state, word position, table address) stays scalar
  n_words = uni32(n_words);
  tail = uni32(tail);
  n = uni32(n);
  const CST uint32_t* __restrict__ t4 = (const CST uint32_t*)uni64((uint64_t)t4_in);
  constexpr uint32_t kSlotMask = SE ? 4095u : 1023u;
  constexpr uint32_t kShift = SE ? 12u : 10u;
  const uint32_t lane = __lane_id();
  const uint64_t wa = (uint64_t)words;
  const GLB uint8_t* A = (const GLB uint8_t*)(wa & ~15ull);
  const uint32_t s_off = (uint32_t)(wa & 15u);
  const uint64_t e_off = s_off + 2ull * n_words;
  const uint32_t n_eff = n_words + ((tail >> 16) & 1u);
  const uint32_t tail_word = tail & 0xFFFFu;
  uint64_t landed = 0;
  bool inflight = false;
  u32x4 seg = {0u, 0u, 0u, 0u};
  uint32_t x = __builtin_amdgcn_readfirstlane(x0), pos = 0;
  uint32_t base = 0, w_lo = 0, w_hi = 0;
  if (x < kL) {
    if (lane == 0) flag(status, BS_DEV_ERR_STREAM);
    return;
  }
  if (SE) tile_count_begin(hist, lane);
  auto ring_word = [&](uint32_t idx) {
    const uint32_t b = s_off + 2u * idx;
    return (uint32_t)ring[b & (kRingB - 1u)] | ((uint32_t)ring[(b + 1u) & (kRingB - 1u)] << 8);
  };
  uint32_t acc = 0;            // lane j: output j of the batch
  auto step = [&]() -> uint32_t {
    const uint32_t e = t4[x & kSlotMask];                  // s_load_dword: x is wave-uniform
    const uint32_t f = SE ? (e >> 8) & 0xFFFu : e & 0x7FFu;
    const uint32_t bias = SE ? e >> 20 : (e >> 11) & 0x3FFu;
    uint32_t xn = f * (x >> kShift) + bias;
    // uniform: a scalar branch, taken by about one step in five, so laid out
    // off the straight path
    if (__builtin_expect(xn < kL, 0)) {
      const uint32_t d = pos - base;                       // < 128
      const uint32_t w_a = __builtin_amdgcn_readlane(w_lo, d & 63u);
      const uint32_t w_b = __builtin_amdgcn_readlane(w_hi, d & 63u);
      uint32_t w = d < (uint32_t)kWave ? w_a : w_b;
      w = pos < n_words ? w : tail_word;
      xn = (xn << 16) | w;
      ++pos;
    }
    x = xn;
    // the SE index is the entry's low byte, kept as it is
    return SE ? e : (e >> 21) & 0x7Fu;
  };
  for (uint32_t i0 = 0; i0 < n; i0 += kWave) {
    // ring upkeep: the window reaches at most 128 words (256 bytes) past pos
    const uint64_t consumed = s_off + 2ull * pos;
    if (inflight) {
      seg_land(ring, landed / kSegB, lane, seg);
      landed += kSegB;
      inflight = false;
    }
    while (landed < e_off && landed < consumed + 4u * kWave + 2u) {
      seg_land(ring, landed / kSegB, lane, seg_block(A, landed / kSegB, lane, s_off, e_off));
      landed += kSegB;
    }
    if (landed < e_off && landed + kSegB <= consumed + kRingB) {
      seg = seg_block(A, landed / kSegB, lane, s_off, e_off);
      inflight = true;
    }
    wave_sync();
    if (i0 == 0) {
      w_lo = ring_word(lane);
      w_hi = ring_word(kWave + lane);
    } else if (pos - base >= (uint32_t)kWave) {           // one move keeps pos - base < 64
      base += kWave;
      w_lo = w_hi;
      w_hi = ring_word(base + kWave + lane);
    }
    // each step's output goes straight into lane j of acc (v_writelane): the
    // LDS stage of serial_chain cost a v_mov and a ds_write per step, and its
    // LDS count held up the wait for the next table load (a probe chain: 54.1
    // against 50.4 ns per step)
    const uint32_t cnt = min((uint32_t)kWave, n - i0);
    if (cnt == (uint32_t)kWave) {
#pragma unroll
      for (uint32_t j = 0; j < (uint32_t)kWave; ++j) {
        const uint32_t o = step();
        BS_WRITELANE_I(acc, o, j);
      }
    } else {
      for (uint32_t j = 0; j < cnt; ++j) {                 // the last, partial batch
        const uint32_t o = step();
        acc = lane == j ? o : acc;
      }
    }
    const uint32_t keep = acc & 0xFFu;
    const uint32_t word = SE ? out_words[keep] : keep;
    if (lane < cnt) {
      if (SE) ((GLB uint16_t*)out)[(uint64_t)(i0 + lane) * stride] = (uint16_t)word;
      else out[i0 + lane] = (uint8_t)keep;
    }
    if (SE) tile_count(hist, ghist, word, lane, i0, cnt, n);
  }
  if (SE) tile_count_end(ghist, lane, n, tps);
  if (x != kL || pos != n_eff) {
    if (lane == 0) flag(status, BS_DEV_ERR_STREAM);
  }
}

// ---- tasks of a wave-serial launch. Every tensor of a batch is one task; its
// chain groups, tiles and streams occupy consecutive workgroups of the grids
// (se_group_begin, mant_group_begin, tile_begin, stream_begin), so one launch
// of each kernel covers the whole batch and the chains of all its tensors run
// side by side. The single-tensor entry point passes its one task by value
// (tasks == nullptr).

__host__ __device__ inline uint64_t serial_max_len(uint64_t n_out, uint32_t n_streams) {
  return (n_out + n_streams - 1) / n_streams;
}
__host__ __device__ inline uint32_t serial_tiles(uint64_t n_out, uint32_t n_streams) {
  return (uint32_t)((serial_max_len(n_out, n_streams) + kTile - 1) / kTile);
}
__host__ __device__ inline uint64_t serial_work(uint64_t n_out, uint32_t n_streams) {
  return ((n_out + 255) & ~255ull) + (uint64_t)n_streams * serial_tiles(n_out, n_streams) * 256 * 4;
}

// A task every kernel may follow: 1 <= n_out < 2^32, at least one stream, a
// tile count that fits 32 bits, and its scratch inside the work buffer. Every
// kernel checks it alike, so a bad task is reported once and skipped by all.
__device__ __forceinline__ bool task_ok(const bs_ref_task& T, uint64_t work_bytes) {
  if (T.n_out == 0 || T.n_out > 0xFFFFFFFFull || T.n_streams == 0 || (T.work_offset & 255u)) return false;
  if ((uint64_t)T.n_streams * serial_tiles(T.n_out, T.n_streams) > 0xFFFFFFFFull) return false;
  return T.work_offset <= work_bytes && serial_work(T.n_out, T.n_streams) <= work_bytes - T.work_offset;
}

enum { kSeGrid = 0, kMantGrid = 1, kTileGrid = 2, kStreamGrid = 3 };
template <int G>
__device__ __forceinline__ uint32_t grid_begin(const bs_ref_task& t) {
  return G == kSeGrid ? t.se_group_begin : G == kMantGrid ? t.mant_group_begin
                                         : G == kTileGrid ? t.tile_begin : t.stream_begin;
}
// The task whose range of grid G holds workgroup b (binary search over the
// ascending begins; wave-uniform).
template <int G>
__device__ __forceinline__ bs_ref_task pick_task(const bs_ref_task* __restrict__ tasks, uint32_t n_tasks,
                                                 const bs_ref_task& single, uint32_t b) {
  if (tasks == nullptr) return single;
  uint32_t lo = 0, hi = n_tasks;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (grid_begin<G>(tasks[mid]) <= b) lo = mid; else hi = mid;
  }
  return tasks[lo];
}

// Chain grid: workgroups of kSerWaves wavefronts, one chain each. The first
// xcd_slots(se_groups) workgroups serve the SE groups (task by
// se_group_begin; their order is below): wave w of group j decodes SE stream
// j*kSerWaves + w (element first + i*stride for symbol i) with the task's SE
// table, built once per workgroup and shared.
// The rest are mantissa groups (task by mant_group_begin): wave w decodes
// bucket j*kSerWaves + w into mant[perm_begin ...] with its own bucket table.
// Sharing the 64 KB SE table lets a CU hold eight chains instead of two. The
// host lists buckets longest first, so the four buckets of a group end at
// about the same time and the longest start first.
//
// The SE part of the grid has xcd_slots(se_groups) workgroups, a multiple of
// kXcds: workgroup p serves SE group (p % kXcds) * (slots / kXcds) + p / kXcds
// (none past the last group). Workgroups go to the XCDs round-robin, so each
// XCD decodes one contiguous run of groups, which covers one or two tasks: the
// scalar-cache form of an SE table (16 KB) then meets at most two tables in an
// XCD's scalar caches, where seven interleaved tasks' tables missed often
// enough to make each step ~40 % slower.
constexpr uint32_t kSerWaves = 4;
constexpr uint32_t kXcds = 8;
// A grid part of `count` workgroups dealt to the XCDs in contiguous blocks:
// count rounded up to a multiple of kXcds.
__host__ __device__ constexpr uint64_t xcd_slots(uint32_t count) {
  return ((uint64_t)count + kXcds - 1) / kXcds * kXcds;
}
constexpr uint32_t kStageB = 128;      // per chain: 64 u16 outputs of a batch
constexpr uint32_t kHistB = 256 * 4;   // per SE chain: the exponent counts of its current tile
// 78336: rings | SE table or kSerWaves mantissa tables | stages | tile counts.
// Two groups fit the 160 KB of a CU (two of 81,920 B did not).
constexpr uint32_t kSerLds = kSerWaves * kRingB + 4096 * 16 + kSerWaves * kStageB + kSerWaves * kHistB;
static_assert(2 * kSerLds <= 160 * 1024 - 4096, "two chain groups per CU");
static_assert(kSerWaves * 1024 * 16 <= 4096 * 16, "mantissa tables exceed the table area");

__global__ __launch_bounds__(kSerWaves * kWave) void serial_kernel(const bs_ref_task* __restrict__ tasks,
                                                                   uint32_t n_tasks, bs_ref_task single,
                                                                   uint32_t se_groups, uint8_t* __restrict__ work,
                                                                   uint64_t work_bytes, int32_t* __restrict__ status) {
  BS_DYNAMIC_LDS(smem);
  const uint32_t tid = threadIdx.x, lane = tid % kWave;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  LDS uint8_t* ring = (LDS uint8_t*)smem + wave * kRingB;
  LDS u32x4* tbl_area = (LDS u32x4*)(smem + kSerWaves * kRingB);
  LDS uint16_t* stage = (LDS uint16_t*)(smem + kSerWaves * kRingB + 4096 * 16 + wave * kStageB);
  LDS uint32_t* hist = (LDS uint32_t*)(smem + kSerWaves * kRingB + 4096 * 16 + kSerWaves * kStageB + wave * kHistB);
  const uint32_t slots = (uint32_t)xcd_slots(se_groups);  // the launch checked that it fits
  const bool se = blockIdx.x < slots;                     // uniform over the workgroup
  const uint32_t g = se ? (blockIdx.x % kXcds) * (slots / kXcds) + blockIdx.x / kXcds : blockIdx.x - slots;
  if (se && g >= se_groups) return;
  const bs_ref_task T = se ? pick_task<kSeGrid>(tasks, n_tasks, single, g)
                           : pick_task<kMantGrid>(tasks, n_tasks, single, g);
  const uint32_t begin = se ? T.se_group_begin : T.mant_group_begin;
  if (g < begin) return;
  const uint32_t local = g - begin, count = se ? T.n_streams : T.n_buckets;
  if ((uint64_t)local * kSerWaves >= count) return;
  if (!task_ok(T, work_bytes)) {
    if (local == 0 && tid == 0) flag(status, BS_DEV_ERR_HEADER);
    return;
  }
  const uint32_t c = local * kSerWaves + wave;            // this wave's stream or bucket (none when >= count)
  const uint64_t max_len = (uint64_t)serial_tiles(T.n_out, T.n_streams) * kTile;
  uint8_t* mant = work + T.work_offset;
  const bool scalar_se = (T.flags & BS_REF_FLAG_SE_SCALAR) != 0;
  if (se) {
    LDS uint32_t* out_words = (LDS uint32_t*)tbl_area;    // scalar-cache form: the 256 output words
    if (scalar_se) {
      for (uint32_t i = tid; i < 256; i += kSerWaves * kWave) out_words[i] = T.se_table[8192 + 4096 + i];
    } else {
      for (uint32_t i = tid; i < 4096; i += kSerWaves * kWave) {
        const uint32_t lo = T.se_table[2 * i], sym = T.se_table[2 * i + 1];
        const uint32_t word = (((sym >> 8) & 1u) << 15) | ((sym & 0xFFu) << 7);
        tbl_area[i] = u32x4{lo & 0x1FFFu, lo >> 13, word, 0u};
      }
    }
    __syncthreads();
    if (c >= count) return;
    const bs_se_stream S = T.streams[c];
    if (!stream_ok(S, max_len, T.n_out)) {
      if (lane == 0) flag(status, BS_DEV_ERR_HEADER);
      return;
    }
    // the stream's tile counts: tps x 256 after the task's mantissa area
    const uint32_t tps = serial_tiles(T.n_out, T.n_streams);
    GLB uint32_t* ghist = (GLB uint32_t*)(work + T.work_offset + ((T.n_out + 255) & ~255ull)) + (uint64_t)c * tps * 256u;
    if (scalar_se)
      serial_chain_scalar<true>((const GLB uint8_t*)S.words, S.n_words, S.tail, S.x0, S.n,
                                (const CST uint32_t*)(T.se_table + 8192), out_words, ring,
                                (GLB uint8_t*)(T.out + S.first), S.stride, hist, ghist, tps, status);
    else
      serial_chain<true>((const GLB uint8_t*)S.words, S.n_words, S.tail, S.x0, S.n, tbl_area, ring, stage,
                         (GLB uint8_t*)(T.out + S.first), S.stride, hist, ghist, tps, status);
  } else {
    if (c >= count) return;
    const bs_mant_bucket B = T.buckets[c];
    if (B.table >= T.n_tables || B.perm_begin + B.n > T.n_out) {
      if (lane == 0) flag(status, BS_DEV_ERR_HEADER);
      return;
    }
    const GLB uint32_t* t = (const GLB uint32_t*)T.mant_tables + (uint64_t)B.table * 1024u;
    if (T.flags & BS_REF_FLAG_MANT_SCALAR) {
      serial_chain_scalar<false>((const GLB uint8_t*)B.words, B.n_words, B.tail, B.x0, B.n, (const CST uint32_t*)t,
                                 nullptr, ring, (GLB uint8_t*)(mant + B.perm_begin), 1u, nullptr, nullptr, 0u,
                                 status);
      return;
    }
    LDS u32x4* tbl = tbl_area + wave * 1024u;
    for (uint32_t i = lane; i < 1024; i += kWave) {
      const uint32_t e = t[i];
      tbl[i] = u32x4{e & 0x7FFu, (e >> 11) & 0x3FFu, (e >> 21) & 0x7Fu, 0u};
    }
    wave_sync();
    serial_chain<false>((const GLB uint8_t*)B.words, B.n_words, B.tail, B.x0, B.n, tbl, ring, stage,
                        (GLB uint8_t*)(mant + B.perm_begin), 1u, nullptr, nullptr, 0u, status);
  }
}

// Stream grid, one workgroup per stream k of a task, thread e: turn stream
// k's tile counts of exponent e into each tile's first position in the
// bucket (bstart[k][e] + counts of the earlier tiles), and check that the
// decoded exponents fill every bucket exactly.
__global__ __launch_bounds__(256) void scan_kernel(const bs_ref_task* __restrict__ tasks, uint32_t n_tasks,
                                                   bs_ref_task single, uint8_t* __restrict__ work,
                                                   uint64_t work_bytes, int32_t* __restrict__ status) {
  const uint32_t e = threadIdx.x;
  const bs_ref_task T = pick_task<kStreamGrid>(tasks, n_tasks, single, blockIdx.x);
  if (blockIdx.x < T.stream_begin || !task_ok(T, work_bytes)) return;
  const uint32_t k = blockIdx.x - T.stream_begin;
  if (k >= T.n_streams) return;
  const uint32_t tps = serial_tiles(T.n_out, T.n_streams);
  const uint32_t* bs = T.bstart + (uint64_t)k * 257;
  uint32_t* hk = (uint32_t*)(work + T.work_offset + ((T.n_out + 255) & ~255ull)) + (uint64_t)k * tps * 256;
  uint32_t run = bs[e];
  for (uint32_t t = 0; t < tps; ++t) {
    const uint32_t c = hk[(uint64_t)t * 256 + e];
    hk[(uint64_t)t * 256 + e] = run;
    run += c;
  }
  if (run != bs[e + 1]) flag(status, BS_DEV_ERR_COUNT);
}

// Tile grid, one wavefront per (stream k, tile t) of a task: the position of
// each element in its bucket, from the tile's first positions plus its rank
// among the equal exponents before it (64 elements at a time: lanes with the
// same exponent found with eight ballots); then OR the element's mantissa
// into it.
//
// A 128-byte line of output holds one symbol of 64 streams, so the waves of
// one tile column (tile t of every stream of a task) share their lines. The
// grid (a multiple of kXcds workgroups) is dealt like the SE part of the
// chain grid: workgroup p takes tile slot (p % kXcds) * (grid / kXcds) + p /
// kXcds of the tile grid, in which a task's tiles run streams fastest, so
// each XCD works through whole columns one after another and a line's 64
// writers meet in one L2. Tile order (stream, tile) spread every column
// over all XCDs: the batched 8B layer placed in 4.5 ms against 2.4 ms in
// column order (loading up to eight batches of 64 words at once, instead of
// one, made no difference in column order).
__global__ __launch_bounds__(kWave) void place_kernel(const bs_ref_task* __restrict__ tasks, uint32_t n_tasks,
                                                      bs_ref_task single, uint32_t n_tiles, uint8_t* __restrict__ work,
                                                      uint64_t work_bytes, int32_t* __restrict__ status) {
  __shared__ uint32_t cnt[256];
  const uint32_t lane = threadIdx.x;
  const uint32_t v = (blockIdx.x % kXcds) * (gridDim.x / kXcds) + blockIdx.x / kXcds;
  if (v >= n_tiles) return;
  const bs_ref_task T = pick_task<kTileGrid>(tasks, n_tasks, single, v);
  if (v < T.tile_begin || !task_ok(T, work_bytes)) return;
  const uint32_t tps = serial_tiles(T.n_out, T.n_streams), local = v - T.tile_begin;
  if (local >= T.n_streams * tps) return;
  const uint32_t t = local / T.n_streams, k = local % T.n_streams;
  const uint64_t n = T.n_out;
  const uint8_t* mant = work + T.work_offset;
  const uint32_t* first = (const uint32_t*)(mant + ((n + 255) & ~255ull));
  uint16_t* out = T.out;
  const bs_se_stream S = T.streams[k];
  if (!stream_ok(S, (uint64_t)tps * kTile, n)) return;     // reported by serial_kernel
  const uint64_t kt = (uint64_t)k * tps + t;               // the scan's (stream, tile) order
  for (uint32_t e = lane; e < 256; e += kWave) cnt[e] = first[kt * 256 + e];
  wave_sync();
  const uint32_t lo = t * kTile, hi = (uint32_t)min((uint64_t)S.n, (uint64_t)lo + kTile);
  const uint64_t lt = (1ull << lane) - 1ull;
  bool bad = false;
  for (uint32_t k0 = lo; k0 < hi; k0 += kWave) {
    const uint32_t i = k0 + lane;
    const bool valid = i < hi;
    const uint64_t el = S.first + (uint64_t)i * S.stride;
    const uint32_t word = valid ? out[el] : 0u;
    const uint32_t e = (word >> 7) & 0xFFu;
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (e >> b) & 1u;
      const uint64_t bb = __ballot(bit);
      m &= bit ? bb : ~bb;
    }
    const uint32_t rank = (uint32_t)__popcll(m & lt), total = (uint32_t)__popcll(m);
    const uint32_t base = cnt[e];
    wave_sync();
    if (valid && rank == 0) cnt[e] = base + total;
    if (valid) {
      const uint32_t p = base + rank;
      if (p < n) out[el] = (uint16_t)(word | mant[p]);
      else bad = true;
    }
    wave_sync();
  }
  if (__ballot(bad) != 0 && lane == 0) flag(status, BS_DEV_ERR_COUNT);
}

std::atomic<uint64_t> g_serial_lds{0};

int launch_serial(const bs_ref_task* tasks, uint32_t n_tasks, const bs_ref_task& single, uint32_t se_groups,
                  uint32_t mant_groups, uint32_t tiles, uint32_t streams, uint8_t* work, uint64_t work_bytes,
                  int32_t* status, hipStream_t s) {
  if (xcd_slots(se_groups) + mant_groups > 0xFFFFFFFFull || xcd_slots(tiles) > 0xFFFFFFFFull) return BS_ERR_ARG;
  bs_internal::ensure_lds_limit((const void*)serial_kernel, kSerLds, g_serial_lds);
  hipLaunchKernelGGL(serial_kernel, dim3((uint32_t)xcd_slots(se_groups) + mant_groups), dim3(kSerWaves * kWave),
                     kSerLds, s, tasks, n_tasks, single, se_groups, work, work_bytes, status);
  if (hipGetLastError() != hipSuccess) return BS_ERR_HIP;
  hipLaunchKernelGGL(scan_kernel, dim3(streams), dim3(256), 0, s, tasks, n_tasks, single, work, work_bytes, status);
  if (hipGetLastError() != hipSuccess) return BS_ERR_HIP;
  hipLaunchKernelGGL(place_kernel, dim3((uint32_t)xcd_slots(tiles)), dim3(kWave), 0, s, tasks, n_tasks, single, tiles,
                     work, work_bytes, status);
  return hipGetLastError() == hipSuccess ? BS_OK : BS_ERR_HIP;
}

}  // namespace

extern "C" {

int bs_refcodec_decode(const bs_se_stream* d_streams, uint32_t n_streams, const uint32_t* d_se_table,
                       const uint32_t* d_bstart, const bs_mant_bucket* d_buckets, uint32_t n_buckets,
                       const uint32_t* d_mant_tables, uint32_t n_tables, uint16_t* d_out, uint64_t n_out,
                       uint32_t* d_perm, int32_t* d_status, void* stream) {
  if (!d_status || (n_streams && (!d_streams || !d_se_table || !d_bstart)) ||
      (n_buckets && (!d_buckets || !d_mant_tables)) || (n_out && (!d_out || !d_perm)))
    return BS_ERR_ARG;
  if (n_out == 0 || n_streams == 0) return BS_OK;
  hipStream_t s = (hipStream_t)stream;
  constexpr uint32_t kSeLds = 4096 * 8 + 256 * kSeLanes * 4;
  static std::atomic<uint64_t> lds_set{0};
  bs_internal::ensure_lds_limit((const void*)se_kernel, kSeLds, lds_set);
  hipLaunchKernelGGL(se_kernel, dim3((n_streams + kSeLanes - 1) / kSeLanes), dim3(kSeLanes), kSeLds, s, d_streams,
                     n_streams, d_se_table, d_bstart, n_out, d_out, d_perm, d_status);
  if (hipGetLastError() != hipSuccess) return BS_ERR_HIP;
  if (n_buckets) {
    hipLaunchKernelGGL(mant_kernel, dim3((n_buckets + kMantThreads - 1) / kMantThreads), dim3(kMantThreads), 0, s,
                       d_buckets, n_buckets, d_mant_tables, n_tables, d_perm, n_out, n_out, d_out, d_status);
    if (hipGetLastError() != hipSuccess) return BS_ERR_HIP;
  }
  return BS_OK;
}

uint64_t bs_refcodec_serial_work_bytes(uint64_t n_out, uint32_t n_streams) {
  if (n_streams == 0) return 0;
  return serial_work(n_out, n_streams);
}

uint32_t bs_refcodec_serial_tiles(uint64_t n_out, uint32_t n_streams) {
  if (n_streams == 0 || n_out == 0) return 0;
  return serial_tiles(n_out, n_streams);
}

int bs_refcodec_decode_serial(const bs_se_stream* d_streams, uint32_t n_streams, const uint32_t* d_se_table,
                              const uint32_t* d_bstart, const bs_mant_bucket* d_buckets, uint32_t n_buckets,
                              const uint32_t* d_mant_tables, uint32_t n_tables, uint16_t* d_out, uint64_t n_out,
                              void* d_work, uint64_t work_bytes, int32_t* d_status, void* stream) {
  if (!d_status || (n_out && (!d_streams || !d_se_table || !d_bstart || !d_out || !d_work || !n_streams)) ||
      (n_buckets && (!d_buckets || !d_mant_tables)) || n_out > 0xFFFFFFFFull)
    return BS_ERR_ARG;
  if (n_out == 0) return BS_OK;
  if (work_bytes < bs_refcodec_serial_work_bytes(n_out, n_streams) || ((uintptr_t)d_work & 255u)) return BS_ERR_ARG;
  const uint64_t tiles = (uint64_t)n_streams * serial_tiles(n_out, n_streams);
  if ((uint64_t)n_streams + n_buckets > 0xFFFFFFFFull || tiles > 0xFFFFFFFFull) return BS_ERR_ARG;
  bs_ref_task t{};
  t.streams = d_streams;
  t.se_table = d_se_table;
  t.bstart = d_bstart;
  t.buckets = d_buckets;
  t.mant_tables = d_mant_tables;
  t.out = d_out;
  t.n_out = n_out;
  t.work_offset = 0;
  t.n_streams = n_streams;
  t.n_buckets = n_buckets;
  t.n_tables = n_tables;
  return launch_serial(nullptr, 0u, t, (n_streams + kSerWaves - 1) / kSerWaves,
                       (uint32_t)(((uint64_t)n_buckets + kSerWaves - 1) / kSerWaves), (uint32_t)tiles, n_streams,
                       (uint8_t*)d_work, work_bytes, d_status, (hipStream_t)stream);
}

uint32_t bs_refcodec_serial_chains_per_group(void) { return kSerWaves; }

int bs_refcodec_decode_serial_batch(const bs_ref_task* d_tasks, uint32_t n_tasks, uint32_t total_se_groups,
                                    uint32_t total_mant_groups, uint32_t total_tiles, uint32_t total_streams,
                                    void* d_work, uint64_t work_bytes, int32_t* d_status, void* stream) {
  if (!d_status || (n_tasks && (!d_tasks || !d_work)) || ((uintptr_t)d_work & 255u)) return BS_ERR_ARG;
  if (n_tasks == 0) return BS_OK;
  if (total_se_groups == 0 || total_tiles == 0 || total_streams == 0) return BS_ERR_ARG;
  bs_ref_task dummy{};
  return launch_serial(d_tasks, n_tasks, dummy, total_se_groups, total_mant_groups, total_tiles, total_streams,
                       (uint8_t*)d_work, work_bytes, d_status, (hipStream_t)stream);
}

}  // extern "C"
