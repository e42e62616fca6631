// GPU encoder for BSCK (bf16_chunked_v1), dense plane mode, 128 states per
// chunk: the device-side counterpart of bsck_encode.cpp for tensors that are
// already in HBM (KV-cache blocks), so compressing them needs no copy to the
// host. Its blobs are byte-identical to bsck_encode.cpp with plane mode 1
// forced (same symbol order, integer quantiser, state walk and layout).
//
// A batch of tensors ("tasks") is encoded by six launches on one stream:
//   clear     zero the per-task exponent histograms;
//   hist      per chunk: exponent histogram (16 interleaved copies in LDS),
//             added into its task's;
//   plan      per task (one wavefront): symbols = exponents present, in
//             ascending order; frequencies by the quantiser of bsck_encode.cpp
//             (rounding, then greedy +-1 corrections, the argmax taken across
//             the wavefront); writes the blob header and symbol table;
//   chunk     per chunk (one wavefront, lane l owns states l and 64 + l):
//             walks the steps backwards, renormalising before each encode as
//             the decoder renormalises after each decode; renorm words of a
//             (step, state group) are placed by ballot rank so the decoder
//             reads them lane-ascending; words go to the chunk's scratch from
//             its end backwards, final states to its head; a full chunk also
//             stores its dense sign|mantissa plane in the plane region
//             (interleaved per block), from the words it loads to encode;
//   layout    per task: chunk offsets (prefix sum of chunk sizes), chunk table,
//             blob length (or a capacity error);
//   assemble  per chunk: states and renorm words at the chunk's offset in
//             the blob; the partial chunk's plane after its words.
// Chunk k's elements follow the layout's interleave: a full chunk (k < nf)
// takes 512-element units k, nf + k, 2nf + k, ...; the partial chunk the tail.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/bigsmall_hip.h"

namespace {

#define LDS __attribute__((address_space(3)))
#define GLB __attribute__((address_space(1)))
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kWave = 64;
constexpr uint32_t kLanes = 128;       // states per chunk (two per wavefront lane)
constexpr uint32_t kBlock = 8;         // steps per dense-plane block
constexpr uint32_t kM = 4096;
constexpr uint32_t kL = 1u << 16;
constexpr uint8_t kVersion = 3;
constexpr uint32_t kUnit = 512;        // elements per output interleave unit

// Per-task plan in the work area.
struct Plan {
  uint32_t hist[256];         // elements per exponent
  uint32_t sym_of_exp[256];   // exponent -> symbol index
  uint32_t freq[256];         // per symbol
  uint32_t cum[256];          // per symbol
  uint32_t rcp[256];          // per symbol: multiplier for x / freq (see div_constants)
  uint32_t shf[256];          // per symbol: its two shifts (s1 | s2 << 8)
  uint32_t nsym, ok, pad0, pad1;
};
constexpr uint64_t kPlanBytes = (sizeof(Plan) + 255) & ~uint64_t(255);
// Per-chunk record in the work area.
struct ChunkRec {
  uint64_t off;               // byte offset of the chunk in the blob
  uint32_t nw, pad;
};

__host__ __device__ inline uint64_t pad16(uint64_t v) { return (v + 15) & ~uint64_t(15); }
__host__ __device__ inline uint64_t pad256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

// Tensor element holding element j of chunk k (nf full chunks of `per` elements).
__device__ __forceinline__ uint64_t chunk_elem(uint64_t k, uint64_t j, uint64_t nf, uint64_t per) {
  return k < nf ? ((j / kUnit) * nf + k) * kUnit + j % kUnit : nf * per + j;
}

// Constants for x / f with a fixed divisor 1 <= f <= 4096 and any 32-bit x, without a divide
// instruction: Granlund and Montgomery, "Division by Invariant Integers using
// Multiplication" (PLDI 1994), Figure 4.1. With l = ceil(log2 f),
//   m = floor(2^32 * (2^l - f) / f) + 1,  s1 = min(l, 1),  s2 = max(l - 1, 0),
//   t = mulhi(m, x),  x / f = (t + ((x - t) >> s1)) >> s2.
__device__ __forceinline__ void div_constants(uint32_t f, uint32_t& m, uint32_t& shf) {
  const uint32_t l = f > 1 ? 32u - (uint32_t)__clz(f - 1) : 0u;
  m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - f)) / f + 1);
  shf = (l ? 1u : 0u) | ((l ? l - 1 : 0u) << 8);
}
__host__ __device__ inline uint64_t scratch_bytes(uint32_t steps) { return 4ull * kLanes + 2ull * kLanes * steps; }

__device__ __forceinline__ void flag(int32_t* status, int32_t bits) { atomicOr(status, bits); }

// task serving global chunk c (tasks sorted by chunk_begin)
__device__ __forceinline__ uint32_t task_of(const bs_encode_task* tasks, uint32_t n_tasks, uint32_t c) {
  uint32_t lo = 0, hi = n_tasks;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (tasks[mid].chunk_begin <= c) lo = mid; else hi = mid;
  }
  return lo;
}

// Checks every kernel repeats: the task's fields agree with each other. A
// segmented task's segments hold whole 512-element units, start 16-byte
// aligned relative to src, and reach no word 2^32 or more past src.
__device__ __forceinline__ bool task_ok(const bs_encode_task& T, uint64_t per) {
  return T.n > 0 && T.n <= 0xFFFFFFFFull && ((uintptr_t)T.src & 3u) == 0 && ((uintptr_t)T.dst & 15u) == 0 &&
         (uint64_t)T.n_chunks == (T.n + per - 1) / per &&
         (T.seg_len == 0 ||
          (T.seg_len % kUnit == 0 && T.seg_stride >= T.seg_len && T.seg_stride % 8 == 0 &&
           ((T.n - 1) / T.seg_len) * T.seg_stride + (T.n - 1) % T.seg_len <= 0xFFFFFFFFull));
}

// Word offset of tensor element e from the task's src: e itself, or its
// segment's start plus its place in the segment.
__device__ __forceinline__ uint64_t src_word(const bs_encode_task& T, uint64_t e) {
  return T.seg_len ? (e / T.seg_len) * T.seg_stride + e % T.seg_len : e;
}

// The same for whole 512-element units, wave-uniform and without a divide:
// us units per segment (0: contiguous), inv = floor((2^32 - 1) / us). For a
// unit index u < 2^23, mulhi(u, inv) is u / us or one less, and one test
// settles it.
struct SegMap {
  uint32_t us, inv;
  uint64_t stride;             // words from one segment's start to the next's
};
__device__ __forceinline__ SegMap seg_map(const bs_encode_task& T) {
  SegMap m;
  m.us = (uint32_t)(T.seg_len / kUnit);
  m.inv = m.us ? 0xFFFFFFFFu / m.us : 0u;
  m.stride = T.seg_stride;
  return m;
}
__device__ __forceinline__ uint64_t unit_word(const SegMap& m, uint32_t u) {
  if (!m.us) return (uint64_t)u * kUnit;
  uint32_t q = __umulhi(u, m.inv);
  if ((q + 1u) * m.us <= u) ++q;
  return (uint64_t)q * m.stride + (uint64_t)(u - q * m.us) * kUnit;
}

__global__ __launch_bounds__(256) void enc_clear_kernel(uint8_t* __restrict__ plans) {
  Plan* P = (Plan*)(plans + blockIdx.x * kPlanBytes);
  P->hist[threadIdx.x] = 0;
  if (threadIdx.x == 0) { P->nsym = 0; P->ok = 0; }
}

// Per chunk (256 threads): the exponent histogram of its slice, added into
// its task's. The slice is read with 16-byte loads (the 0-6 elements before
// the first 16-byte boundary and the tail one at a time) and counted into 16
// interleaved copies of the histogram in LDS (bin b, copy c at b * 16 + c;
// thread t counts into copy t mod 16). Most lanes of a wavefront hit one of a
// few exponents; with one histogram their LDS adds to a word serialise, here
// at most 4 lanes of a wavefront share a copy, and the copies of a bin lie in
// 16 different banks.
__global__ __launch_bounds__(256) void enc_hist_kernel(const bs_encode_task* __restrict__ tasks, uint32_t n_tasks,
                                                       uint32_t steps, uint8_t* __restrict__ plans) {
  constexpr uint32_t kCopies = 16;
  __shared__ __attribute__((aligned(16))) uint32_t h[256 * kCopies];
  const uint32_t tid = threadIdx.x, c = blockIdx.x;
  const uint32_t ti = task_of(tasks, n_tasks, c);
  const bs_encode_task T = tasks[ti];
  const uint64_t per = (uint64_t)kLanes * steps;
  if (!task_ok(T, per) || c < T.chunk_begin || c - T.chunk_begin >= T.n_chunks) return;
  for (uint32_t i = tid; i < 256 * kCopies; i += 256) h[i] = 0;
  __syncthreads();
  const uint64_t base = (uint64_t)(c - T.chunk_begin) * per;   // the slices cover the tensor once
  const uint32_t nc = (uint32_t)min(per, T.n - base);
  const uint32_t cp = tid & (kCopies - 1);
  auto count = [&](uint32_t w) { atomicAdd(&h[((w >> 7) & 0xFFu) * kCopies + cp], 1u); };
  // the slice in pieces that each lie inside one segment (a contiguous task: one piece)
  for (uint64_t e = base, end = base + nc; e < end;) {
    const uint64_t stop = T.seg_len ? min(end, (e / T.seg_len + 1) * T.seg_len) : end;
    const uint32_t m = (uint32_t)(stop - e);
    const GLB uint16_t* src = (const GLB uint16_t*)T.src + src_word(T, e);
    const uint32_t head = min(m, (uint32_t)(((16u - ((uintptr_t)src & 15u)) & 15u) / 2u));   // src is 4-byte aligned
    if (tid < head) count(src[tid]);
    const uint32_t nv = (m - head) / 8u;
    const GLB u32x4* vsrc = (const GLB u32x4*)(src + head);
    for (uint32_t v = tid; v < nv; v += 256) {
      const u32x4 q = vsrc[v];
      count(q.x); count(q.x >> 16); count(q.y); count(q.y >> 16);
      count(q.z); count(q.z >> 16); count(q.w); count(q.w >> 16);
    }
    for (uint32_t j = head + 8u * nv + tid; j < m; j += 256) count(src[j]);
    e = stop;
  }
  __syncthreads();
  uint32_t sum = 0;
#pragma unroll
  for (uint32_t i = 0; i < kCopies; ++i) sum += h[tid * kCopies + i];
  if (sum) atomicAdd(&((Plan*)(plans + ti * kPlanBytes))->hist[tid], sum);
}

// is candidate (c1, d1, i1) better than (c0, d0, i0)? up: larger c/d; down: smaller c/d; ties: lower index.
// c < 2^32 (elements of one tensor) and d <= 8193, so the products fit in 64 bits.
__device__ __forceinline__ bool better(bool up, uint64_t c1, uint64_t d1, uint32_t i1, uint64_t c0, uint64_t d0,
                                       uint32_t i0) {
  const uint64_t a = c1 * d0, b = c0 * d1;
  if (a != b) return up ? a > b : a < b;
  return i1 < i0;
}

__device__ __forceinline__ uint64_t shfl64(uint64_t v, uint32_t src_lane) {
  const uint32_t lo = __shfl((uint32_t)v, src_lane), hi = __shfl((uint32_t)(v >> 32), src_lane);
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

// One wavefront per task. Lane l holds exponents 4l .. 4l+3, so symbol indices
// (exponents present, ascending) increase with lane and slot.
__global__ __launch_bounds__(kWave) void enc_plan_kernel(const bs_encode_task* __restrict__ tasks, uint32_t steps,
                                                         uint8_t* __restrict__ plans, int32_t* __restrict__ status) {
  const uint32_t lane = threadIdx.x, ti = blockIdx.x;
  const bs_encode_task T = tasks[ti];
  const uint64_t per = (uint64_t)kLanes * steps;
  Plan* P = (Plan*)(plans + ti * kPlanBytes);
  if (!task_ok(T, per)) {
    if (lane == 0) flag(status, BS_DEV_ERR_HEADER);
    return;
  }
  uint64_t c[4];
  uint32_t present = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    c[r] = P->hist[lane * 4 + r];
    present += c[r] != 0;
  }
  // exclusive scan of `present` across lanes -> first symbol index of this lane
  uint32_t incl = present;
  for (uint32_t d = 1; d < kWave; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  const uint32_t nsym = __shfl(incl, kWave - 1);
  uint32_t sidx[4];
  uint32_t s = incl - present;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    sidx[r] = s;
    s += c[r] != 0;
  }
  uint64_t total = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) total += c[r];
  for (uint32_t d = 1; d < kWave; d <<= 1) total += shfl64(total, lane ^ d);
  // proportional rounding, half up, at least 1
  int64_t f[4];
  int64_t sum = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    f[r] = 0;
    if (c[r]) {
      int64_t v = (int64_t)((2 * c[r] * kM + total) / (2 * total));
      f[r] = v < 1 ? 1 : v;
    }
    sum += f[r];
  }
  for (uint32_t d = 1; d < kWave; d <<= 1) sum += (int64_t)shfl64((uint64_t)sum, lane ^ d);
  // greedy corrections, one symbol per iteration (the same sequence as bsck_encode.cpp)
  while (sum != (int64_t)kM) {
    const bool up = sum < (int64_t)kM;
    uint64_t bc = 0, bd = 1;
    uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (!c[r] || (!up && f[r] <= 1)) continue;
      const uint64_t d = up ? 2 * f[r] + 1 : 2 * f[r] - 1;
      if (bi == 0xFFFFFFFFu || better(up, c[r], d, sidx[r], bc, bd, bi)) { bc = c[r]; bd = d; bi = sidx[r]; }
    }
    for (uint32_t d = 1; d < kWave; d <<= 1) {
      const uint64_t oc = shfl64(bc, lane ^ d), od = shfl64(bd, lane ^ d);
      const uint32_t oi = __shfl(bi, lane ^ d);
      if (oi != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || better(up, oc, od, oi, bc, bd, bi))) { bc = oc; bd = od; bi = oi; }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (c[r] && sidx[r] == bi) f[r] += up ? 1 : -1;
    sum += up ? 1 : -1;
  }
  // cumulative frequencies in symbol order
  int64_t fl = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) fl += f[r];
  int64_t finc = fl;
  for (uint32_t d = 1; d < kWave; d <<= 1) {
    const int64_t o = (int64_t)shfl64((uint64_t)finc, lane - d < kWave ? lane - d : lane);
    if (lane >= d) finc += o;
  }
  int64_t cum = finc - fl;
  const uint64_t nch = T.n_chunks;
  const uint64_t ctab = pad16(32 + 4ull * nsym);
  const uint64_t preg = pad256(ctab + 16 * nch);   // plane region (or the first chunk)
  const bool fits = preg <= T.cap && nsym >= 1;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t e = lane * 4 + r;
    P->sym_of_exp[e] = c[r] ? sidx[r] : 0u;
    if (c[r]) {
      P->freq[sidx[r]] = (uint32_t)f[r];
      P->cum[sidx[r]] = (uint32_t)cum;
      uint32_t dm, ds;
      div_constants((uint32_t)max(f[r], (int64_t)1), dm, ds);
      P->rcp[sidx[r]] = dm;
      P->shf[sidx[r]] = ds;
      if (fits)
        *(GLB uint32_t*)(T.dst + 32 + 4ull * sidx[r]) = (e << 7) | ((uint32_t)f[r] << 16) | 0x80000000u;
      cum += f[r];
    }
  }
  if (!fits) {
    if (lane == 0) flag(status, BS_DEV_ERR_BOUNDS);
    return;
  }
  // header, and zeros from the symbol table's end to the chunk table and from
  // the chunk table's end to the plane region (the chunk table itself is
  // written by the layout pass)
  for (uint64_t b = 32 + 4ull * nsym + lane; b < ctab; b += kWave) T.dst[b] = 0;
  for (uint64_t b = ctab + 16 * nch + lane; b < preg; b += kWave) T.dst[b] = 0;
  if (lane == 0) {
    P->nsym = nsym;
    uint8_t* d = T.dst;
    d[0] = 'B'; d[1] = 'S'; d[2] = 'C'; d[3] = 'K';
    d[4] = kVersion; d[5] = 2; d[6] = 1; d[7] = 12;
    *(GLB uint32_t*)(d + 8) = (uint32_t)T.n;
    *(GLB uint32_t*)(d + 12) = (uint32_t)(T.n >> 32);
    *(GLB uint32_t*)(d + 16) = steps;
    *(GLB uint32_t*)(d + 20) = kLanes | (nsym << 16);
    *(GLB uint32_t*)(d + 24) = (uint32_t)nch;
    *(GLB uint32_t*)(d + 28) = 0;
    P->ok = 1;
  }
}

// The steps of one chunk, last to first, in blocks of kBlock steps; the next
// block's words are loaded while the current block is encoded, so the loads'
// latency is not on the encode chain. FULL: a full chunk (every element
// present, its 512-element units k, nf + k, 2nf + k, ...), which needs no
// per-element bounds; else the partial chunk (contiguous from nf * per). Element
// indices fit 32 bits (a task has fewer than 2^32 elements), and at each step
// all but the lane's own offset is the same in every lane.
template <bool FULL>
__device__ __forceinline__ void encode_steps(const GLB uint32_t* src2, const GLB uint16_t* src1, const SegMap& sm,
                                             uint32_t lane, uint32_t nc, uint32_t nsteps, uint32_t k, uint32_t nf,
                                             uint32_t per, const uint32_t* s_fc, const uint32_t* s_m,
                                             GLB uint16_t* words, uint32_t& wpos, uint32_t (&x)[2], bool plane_here,
                                             GLB uint8_t* plane, uint64_t pstride) {
  // this lane's two words of step t, packed (first | second << 16); 0 past the
  // end. A step's 128 elements lie in one unit, so their words are contiguous.
  auto load_step = [&](uint32_t t) -> uint32_t {
    // element of the step's first word: full chunks take unit (t/4)*nf + k at
    // quarter t mod 4, the partial chunk runs on from nf * per
    const uint32_t e0 = FULL ? ((t >> 2) * nf + k) * kUnit + (t & 3u) * kLanes : nf * per + t * kLanes;
    const uint64_t w0 = unit_word(sm, e0 / kUnit) + e0 % kUnit;   // wave-uniform, even
    if (FULL) return src2[(w0 >> 1) + lane];
    const uint32_t j0 = t * kLanes + 2 * lane;
    if (j0 + 1 < nc) return src2[(w0 >> 1) + lane];
    return j0 < nc ? (uint32_t)src1[w0 + 2 * lane] : 0u;
  };
  const uint32_t nblk = (nsteps + kBlock - 1) / kBlock;
  uint32_t cur[kBlock];
#pragma unroll
  for (uint32_t q = 0; q < kBlock; ++q) cur[q] = load_step((nblk - 1) * kBlock + q);
  for (uint32_t b = nblk; b-- > 0;) {
    uint32_t nxt[kBlock];
#pragma unroll
    for (uint32_t q = 0; q < kBlock; ++q) nxt[q] = b > 0 ? load_step((b - 1) * kBlock + q) : 0u;
    if (FULL && plane_here) {
      // sign | mantissa bytes: word pair (q, g = 0, 1) -> bytes 0 and 2, then two steps per word
      uint32_t pw[kBlock / 2];
#pragma unroll
      for (uint32_t i = 0; i < kBlock / 2; ++i) {
        const uint32_t a = cur[2 * i], c2 = cur[2 * i + 1];
        const uint32_t pa = (a & 0x007F007Fu) | ((a >> 8) & 0x00800080u);
        const uint32_t pb = (c2 & 0x007F007Fu) | ((c2 >> 8) & 0x00800080u);
        pw[i] = __builtin_amdgcn_perm(pb, pa, 0x06040200u);
      }
      *(GLB u32x4*)(plane + (uint64_t)b * pstride) = u32x4{pw[0], pw[1], pw[2], pw[3]};
    }
#pragma unroll
    for (int q = (int)kBlock - 1; q >= 0; --q) {
      const uint32_t t = b * kBlock + (uint32_t)q;
      if (!FULL && t >= nsteps) continue;                      // uniform: the last block may be short
      const uint32_t j0 = t * kLanes + 2 * lane;
      const uint32_t wv[2] = {cur[q] & 0xFFFFu, cur[q] >> 16};
#pragma unroll
      for (int g = 1; g >= 0; --g) {
        const bool active = FULL || j0 + g < nc;
        const uint32_t ex = (wv[g] >> 7) & 0xFFu;
        const uint32_t fc = s_fc[ex], f = (fc >> 5) & 0x1FFFu, cm = (fc >> 18) & 0xFFFu;
        uint32_t xv = x[g];
        // renormalise while x >= f * 2^20 (never for f = 4096): f * 2^20 is a
        // multiple of 2^20, so the test is x >> 20 >= f, in 32 bits
        const bool emit = active && (xv >> 20) >= f;
        const uint64_t m = __ballot(emit);
        // the emitting lanes' words, lane-descending from wpos - 1: a lane's slot
        // is the new wpos plus the emitting lanes below it
        wpos -= (uint32_t)__popcll(m);
        if (emit) {
          words[wpos + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u))] =
              (uint16_t)(xv & 0xFFFFu);
          xv >>= 16;
        }
        if (active) {
          // q = xv / f (Granlund-Montgomery with div_constants' m, s1, s2; the
          // second shift by fc, whose bits 0..4 are s2), then xv' = (q << 12) + xv mod f + cum
          // = xv + cum + q * (4096 - f): q < 2^20 (xv < f * 2^20 after the
          // renormalisation) and 4096 - f < 2^13, a 24-bit product
          const uint32_t mh = __umulhi(s_m[ex], xv);
          const uint32_t q2 = (mh + ((xv - mh) >> ((fc >> 30) & 1u))) >> fc;
          xv = xv + cm + __umul24(q2, 4096u - f);
        }
        x[g] = xv;
      }
    }
#pragma unroll
    for (uint32_t q = 0; q < kBlock; ++q) cur[q] = nxt[q];
  }
}

// One wavefront per chunk: lane l owns states l (group 0) and 64 + l (group 1);
// state (g, l) codes element t*128 + 2l + g at step t.
__global__ __launch_bounds__(kWave) void enc_chunk_kernel(const bs_encode_task* __restrict__ tasks, uint32_t n_tasks,
                                                          uint32_t steps, const uint8_t* __restrict__ plans,
                                                          ChunkRec* __restrict__ recs, uint8_t* __restrict__ scratch) {
  // per exponent: {s2:5, f:13, cum:12, s1:1} of its symbol (s2 in bits 0..4, where a
  // shift reads its amount), and the divisor's multiplier
  __shared__ uint32_t s_fc[256], s_m[256];
  const uint32_t lane = threadIdx.x, cg = blockIdx.x;
  const uint32_t ti = task_of(tasks, n_tasks, cg);
  const bs_encode_task T = tasks[ti];
  const uint64_t per = (uint64_t)kLanes * steps;
  const Plan* P = (const Plan*)(plans + ti * kPlanBytes);
  if (!task_ok(T, per) || cg < T.chunk_begin || cg - T.chunk_begin >= T.n_chunks || !P->ok) return;
  for (uint32_t i = lane; i < 256; i += kWave) {
    const uint32_t sym = P->sym_of_exp[i], shf = P->shf[sym];
    s_fc[i] = (shf >> 8) | (P->freq[sym] << 5) | (P->cum[sym] << 18) | ((shf & 1u) << 30);
    s_m[i] = P->rcp[sym];
  }
  __syncthreads();
  const uint64_t k = cg - T.chunk_begin, nf = T.n / per;
  const uint32_t nc = (uint32_t)min(per, T.n - k * per);
  const uint32_t nsteps = (nc + kLanes - 1) / kLanes;
  // A full chunk stores its dense plane here, from the words it loads for the
  // encode: per block of kBlock steps, lane l's 16 bytes hold (q, g) at q*2 + g
  // for chunk element (blk*kBlock + q)*128 + 2l + g, at block blk*nf + k of
  // the plane region (which starts after the chunk table, a place the plan
  // fixes). The partial chunk's plane follows its words, whose count is known
  // only after the encode: the assemble pass writes that one. A region past
  // the capacity is not written (the layout pass reports the capacity error).
  constexpr uint64_t kBlkBytes = (uint64_t)kBlock * kLanes;
  const uint64_t preg = pad256(pad16(32 + 4ull * P->nsym) + 16ull * T.n_chunks);
  const bool plane_here = k < nf && preg + nf * per <= T.cap;
  GLB uint8_t* plane = (GLB uint8_t*)T.dst + preg + k * kBlkBytes + 16u * lane;
  const uint64_t pstride = nf * kBlkBytes;
  const GLB uint32_t* src2 = (const GLB uint32_t*)T.src;   // two words per lane-step (even elements)
  const GLB uint16_t* src1 = (const GLB uint16_t*)T.src;
  uint8_t* chunk = scratch + (uint64_t)cg * scratch_bytes(steps);
  GLB uint16_t* words = (GLB uint16_t*)(chunk + 4u * kLanes);   // capacity per; filled from the end
  uint32_t x[2] = {kL, kL};
  uint32_t wpos = (uint32_t)per;
  const SegMap sm = seg_map(T);
  if (k < nf)
    encode_steps<true>(src2, src1, sm, lane, nc, nsteps, (uint32_t)k, (uint32_t)nf, (uint32_t)per, s_fc, s_m, words,
                       wpos, x, plane_here, plane, pstride);
  else
    encode_steps<false>(src2, src1, sm, lane, nc, nsteps, (uint32_t)k, (uint32_t)nf, (uint32_t)per, s_fc, s_m,
                        words, wpos, x, false, plane, pstride);
  GLB uint32_t* st = (GLB uint32_t*)chunk;
  st[lane] = x[0];
  st[kWave + lane] = x[1];
  if (lane == 0) recs[cg].nw = (uint32_t)per - wpos;
}

// Bytes of a chunk's region: states, words and, for the partial chunk, its plane.
__device__ __forceinline__ uint64_t chunk_bytes(uint32_t nc, uint32_t nw, bool full) {
  const uint32_t nsteps = (nc + kLanes - 1) / kLanes;
  const uint64_t np = (uint64_t)((nsteps + kBlock - 1) / kBlock) * kBlock * kLanes;
  return 4ull * kLanes + pad16(2ull * nw) + (full ? 0ull : np);
}

// One wavefront per task: chunk offsets, chunk table, blob length.
__global__ __launch_bounds__(kWave) void enc_layout_kernel(const bs_encode_task* __restrict__ tasks, uint32_t steps,
                                                           uint8_t* __restrict__ plans, ChunkRec* __restrict__ recs,
                                                           uint64_t* __restrict__ out_len,
                                                           int32_t* __restrict__ status) {
  const uint32_t lane = threadIdx.x, ti = blockIdx.x;
  const bs_encode_task T = tasks[ti];
  const uint64_t per = (uint64_t)kLanes * steps;
  Plan* P = (Plan*)(plans + ti * kPlanBytes);
  if (lane == 0) out_len[ti] = 0;
  if (!task_ok(T, per) || !P->ok) return;
  const uint64_t ctab = pad16(32 + 4ull * P->nsym);
  const uint64_t nf = T.n / per;
  uint64_t run = pad256(ctab + 16ull * T.n_chunks) + nf * per;   // after the plane region
  for (uint32_t b0 = 0; b0 < T.n_chunks; b0 += kWave) {
    const uint32_t k = b0 + lane;
    const bool live = k < T.n_chunks;
    uint32_t nw = 0, nc = 0;
    uint64_t sz = 0;
    if (live) {
      nw = recs[T.chunk_begin + k].nw;
      nc = (uint32_t)min(per, T.n - (uint64_t)k * per);
      sz = chunk_bytes(nc, nw, k < nf);
    }
    uint64_t inc = sz;
    for (uint32_t d = 1; d < kWave; d <<= 1) {
      const uint64_t o = shfl64(inc, lane >= d ? lane - d : lane);
      if (lane >= d) inc += o;
    }
    if (live) {
      const uint64_t off = run + inc - sz;
      recs[T.chunk_begin + k].off = off;
      const uint32_t nsteps = (nc + kLanes - 1) / kLanes;
      const uint32_t np = ((nsteps + kBlock - 1) / kBlock) * kBlock * kLanes;
      GLB uint32_t* e = (GLB uint32_t*)(T.dst + ctab + 16ull * k);
      e[0] = (uint32_t)off;
      e[1] = (uint32_t)(off >> 32);
      e[2] = nw;
      e[3] = np;
    }
    run += shfl64(inc, kWave - 1);
  }
  const uint64_t total = pad256(run);                              // blob lengths are multiples of 256
  if (total > T.cap) {
    if (lane == 0) {
      flag(status, BS_DEV_ERR_BOUNDS);
      P->ok = 0;
    }
    return;
  }
  for (uint64_t b = run + lane; b < total; b += kWave) T.dst[b] = 0;
  if (lane == 0) out_len[ti] = total;
}

// One wavefront per chunk: states, words (zero-padded to 16), dense plane.
__global__ __launch_bounds__(kWave) void enc_assemble_kernel(const bs_encode_task* __restrict__ tasks, uint32_t n_tasks,
                                                             uint32_t steps, const uint8_t* __restrict__ plans,
                                                             const ChunkRec* __restrict__ recs,
                                                             const uint8_t* __restrict__ scratch) {
  const uint32_t lane = threadIdx.x, cg = blockIdx.x;
  const uint32_t ti = task_of(tasks, n_tasks, cg);
  const bs_encode_task T = tasks[ti];
  const uint64_t per = (uint64_t)kLanes * steps;
  const Plan* P = (const Plan*)(plans + ti * kPlanBytes);
  if (!task_ok(T, per) || cg < T.chunk_begin || cg - T.chunk_begin >= T.n_chunks || !P->ok) return;
  const ChunkRec R = recs[cg];
  const uint64_t k = cg - T.chunk_begin, nf = T.n / per;
  const uint32_t nc = (uint32_t)min(per, T.n - k * per);
  const uint8_t* chunk = scratch + (uint64_t)cg * scratch_bytes(steps);
  GLB uint8_t* out = (GLB uint8_t*)(T.dst + R.off);
  // states: 512 bytes
  if (lane < 32) *(GLB u32x4*)(out + 16u * lane) = *(const GLB u32x4*)(chunk + 16u * lane);
  // words [per - nw, per) of the scratch, then zeros up to a multiple of 8
  // words, in 16-byte vectors: output vector i holds words s0 + 8i .. +7, taken
  // from the two aligned vectors around them (s0 mod 8 words into the first;
  // indices clamped to the word area, whose words past `per` would land only
  // in the zeroed tail)
  const GLB u32x4* wsrc = (const GLB u32x4*)(chunk + 4u * kLanes);
  GLB u32x4* wdst = (GLB u32x4*)(out + 4u * kLanes);
  const uint32_t nw_pad = (uint32_t)(pad16(2ull * R.nw) / 2);
  const uint32_t s0 = (uint32_t)per - R.nw, dw = (s0 & 7u) >> 1, bsh = (s0 & 1u) * 16u;
  const uint32_t last = (uint32_t)(per / 8) - 1u;
  for (uint32_t i = lane; i < nw_pad / 8u; i += kWave) {
    const uint32_t va = (s0 >> 3) + i;
    const u32x4 a = wsrc[min(va, last)], b = wsrc[min(va + 1u, last)];
    // dwords dw .. dw + 4 of a:b (dw is the same in every lane)
    const uint32_t d0 = dw == 0 ? a.x : dw == 1 ? a.y : dw == 2 ? a.z : a.w;
    const uint32_t d1 = dw == 0 ? a.y : dw == 1 ? a.z : dw == 2 ? a.w : b.x;
    const uint32_t d2 = dw == 0 ? a.z : dw == 1 ? a.w : dw == 2 ? b.x : b.y;
    const uint32_t d3 = dw == 0 ? a.w : dw == 1 ? b.x : dw == 2 ? b.y : b.z;
    const uint32_t d4 = dw == 0 ? b.x : dw == 1 ? b.y : dw == 2 ? b.z : b.w;
    uint32_t o[4] = {__builtin_amdgcn_alignbit(d1, d0, bsh), __builtin_amdgcn_alignbit(d2, d1, bsh),
                     __builtin_amdgcn_alignbit(d3, d2, bsh), __builtin_amdgcn_alignbit(d4, d3, bsh)};
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {                   // zeros from word nw on
      const uint32_t w = 8u * i + 2u * j;
      o[j] = w + 1u < R.nw ? o[j] : w < R.nw ? (o[j] & 0xFFFFu) : 0u;
    }
    wdst[i] = u32x4{o[0], o[1], o[2], o[3]};
  }
  // the partial chunk's dense plane, after its words (full chunks stored
  // theirs in the plane region during the encode): per 8-step block, lane l's
  // 16 bytes hold (q, g) at q*2 + g for chunk element (blk*8 + q)*128 + 2l + g
  if (k < nf) return;
  constexpr uint64_t kBlkBytes = (uint64_t)kBlock * kLanes;
  GLB uint8_t* plane = out + 4u * kLanes + 2ull * nw_pad;
  const uint64_t pstride = kBlkBytes;
  const uint32_t nsteps = (nc + kLanes - 1) / kLanes;
  const uint32_t nblk = (nsteps + kBlock - 1) / kBlock;
  const GLB uint16_t* src = (const GLB uint16_t*)T.src;
  for (uint32_t blk = 0; blk < nblk; ++blk) {
    uint32_t b[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (uint32_t q = 0; q < kBlock; ++q) {
#pragma unroll
      for (uint32_t g = 0; g < 2; ++g) {
        const uint32_t j = (blk * kBlock + q) * kLanes + 2 * lane + g;
        const uint32_t w = j < nc ? src[src_word(T, chunk_elem(k, j, nf, per))] : 0u;
        const uint32_t byte = ((w >> 8) & 0x80u) | (w & 0x7Fu);
        const uint32_t k = q * 2 + g;
        b[k >> 2] |= byte << (8 * (k & 3));
      }
    }
    *(GLB u32x4*)(plane + (uint64_t)blk * pstride + 16u * lane) = u32x4{b[0], b[1], b[2], b[3]};
  }
}

// Span j of the batch: blockIdx.y strides over its 16-byte vectors.
__global__ __launch_bounds__(256) void copy_spans_kernel(const bs_span* __restrict__ spans, int32_t* __restrict__ status) {
  const bs_span S = spans[blockIdx.x];
  if (((uintptr_t)S.src | (uintptr_t)S.dst | S.len) & 15u) {
    if (blockIdx.y == 0 && threadIdx.x == 0) flag(status, BS_DEV_ERR_HEADER);
    return;
  }
  const uint64_t nv = S.len / 16;
  const GLB u32x4* src = (const GLB u32x4*)S.src;
  GLB u32x4* dst = (GLB u32x4*)S.dst;
  // four 16-byte vectors per thread in flight, loaded and then stored with
  // streaming hints (each byte is read once and written once): a 2 GiB copy
  // measured 5.73 TB/s this way against 5.55 TB/s one vector at a time
  constexpr uint32_t kU = 4;
  for (uint64_t i = (uint64_t)blockIdx.y * 256u * kU + threadIdx.x; i < nv; i += 256ull * kU * gridDim.y) {
    u32x4 v[kU];
#pragma unroll
    for (uint32_t u = 0; u < kU; ++u) {
      const uint64_t j = i + 256ull * u;
      v[u] = j < nv ? __builtin_nontemporal_load(src + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (uint32_t u = 0; u < kU; ++u) {
      const uint64_t j = i + 256ull * u;
      if (j < nv) __builtin_nontemporal_store(v[u], dst + j);
    }
  }
}

}  // namespace

extern "C" {

uint64_t bs_chunk_encode_gpu_work_bytes(uint32_t n_tasks, uint64_t total_chunks, uint32_t steps) {
  return (uint64_t)n_tasks * kPlanBytes + ((total_chunks * sizeof(ChunkRec) + 255) & ~255ull) +
         total_chunks * scratch_bytes(steps);
}

int bs_chunk_encode_gpu(const bs_encode_task* d_tasks, uint32_t n_tasks, uint32_t total_chunks, uint32_t steps,
                        void* d_work, uint64_t work_bytes, uint64_t* d_out_len, int32_t* d_status, void* stream) {
  if (!d_status || (n_tasks && (!d_tasks || !d_work || !d_out_len)) || steps == 0 || steps % 16 ||
      128ull * steps > (1ull << 24) || ((uintptr_t)d_work & 255u))   // chunks of at most 2^24 elements
    return BS_ERR_ARG;
  if (n_tasks == 0) return BS_OK;
  if (work_bytes < bs_chunk_encode_gpu_work_bytes(n_tasks, total_chunks, steps)) return BS_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  uint8_t* plans = (uint8_t*)d_work;
  ChunkRec* recs = (ChunkRec*)(plans + (uint64_t)n_tasks * kPlanBytes);
  uint8_t* scratch = (uint8_t*)recs + ((total_chunks * sizeof(ChunkRec) + 255) & ~255ull);
  hipLaunchKernelGGL(enc_clear_kernel, dim3(n_tasks), dim3(256), 0, s, plans);
  if (total_chunks)
    hipLaunchKernelGGL(enc_hist_kernel, dim3(total_chunks), dim3(256), 0, s, d_tasks, n_tasks, steps, plans);
  hipLaunchKernelGGL(enc_plan_kernel, dim3(n_tasks), dim3(kWave), 0, s, d_tasks, steps, plans, d_status);
  if (total_chunks)
    hipLaunchKernelGGL(enc_chunk_kernel, dim3(total_chunks), dim3(kWave), 0, s, d_tasks, n_tasks, steps, plans, recs,
                       scratch);
  hipLaunchKernelGGL(enc_layout_kernel, dim3(n_tasks), dim3(kWave), 0, s, d_tasks, steps, plans, recs, d_out_len,
                     d_status);
  if (total_chunks)
    hipLaunchKernelGGL(enc_assemble_kernel, dim3(total_chunks), dim3(kWave), 0, s, d_tasks, n_tasks, steps, plans,
                       recs, scratch);
  return hipGetLastError() == hipSuccess ? BS_OK : BS_ERR_HIP;
}

int bs_copy_spans(const bs_span* d_spans, uint32_t n_spans, uint64_t max_len, int32_t* d_status, void* stream) {
  if (!d_status || (n_spans && !d_spans) || n_spans > 0x7FFFFFFFu) return BS_ERR_ARG;
  if (n_spans == 0 || max_len == 0) return BS_OK;
  // one pass of four 16-byte vectors per thread over the longest span, at most
  // 8192 workgroups per span (a 2 GiB copy ran fastest with 8192)
  const uint64_t per_block = 256ull * 16ull * 4ull;
  const uint32_t gy = (uint32_t)std::min<uint64_t>((max_len + per_block - 1) / per_block, 8192ull);
  hipLaunchKernelGGL(copy_spans_kernel, dim3(n_spans, gy), dim3(256), 0, (hipStream_t)stream, d_spans, d_status);
  return hipGetLastError() == hipSuccess ? BS_OK : BS_ERR_HIP;
}

}  // extern "C"
