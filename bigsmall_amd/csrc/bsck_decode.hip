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

constexpr int kLanes = 64;
constexpr int kWaves = 8;                 // chunks (wavefronts) per workgroup
constexpr int kThreads = kWaves * kLanes;
constexpr int kBlock = 8;                 // steps per refill block
constexpr uint32_t kRing = 2048;          // per-wave word ring (u16) and plane ring (bytes)
constexpr uint32_t kSeg = 256;            // refill segment: words (64 lanes x 8 B) / plane bytes (64 x 4 B)
constexpr uint32_t kL = 1u << 16;
// dynamic LDS layout: decode table | word rings | plane rings (compact-capable launches only)
constexpr uint32_t kTblBytes = 4096 * 8;
constexpr uint32_t kWringBytes = kWaves * kRing * 2;
constexpr uint32_t kPringBytes = kWaves * kRing;
constexpr uint32_t kLdsLean = kTblBytes + kWringBytes;
constexpr uint32_t kLdsCompact = kLdsLean + kPringBytes;

__device__ __forceinline__ uint32_t ld_u32(const GLB uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__device__ __forceinline__ uint32_t lane_rank(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t pad16(uint32_t v) { return (v + 15u) & ~15u; }

// Combine a bf16 exponent symbol's value with its plane byte (sign<<7 | mant).
__device__ __forceinline__ uint32_t with_plane(uint32_t v, uint32_t b) {
  return v | (b & 0x7Fu) | ((b & 0x80u) << 8);
}

__device__ __forceinline__ void report(int32_t* status, int32_t bits) {
  if (__lane_id() == 0) atomicOr(status, bits);
}

// ring segment load/store: lane l moves 8 bytes (4 words) / 4 bytes of a 256-entry segment
__device__ __forceinline__ uint64_t load_wseg(const GLB uint64_t* src, uint32_t pos, uint32_t valid, uint32_t lane) {
  const uint32_t slot = pos / 4u + lane;
  return slot < valid ? src[slot] : 0ull;
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

// Decode one chunk with one wavefront. MODE = plane mode, EB = element bytes,
// PARTIAL = chunk may be shorter than 64*steps (the tensor's last chunk).
template <int MODE, int EB, bool PARTIAL>
__device__ __forceinline__ void decode_chunk(const LDS uint64_t* __restrict__ tbl, LDS uint16_t* __restrict__ wring,
                                             LDS uint8_t* __restrict__ pring, const GLB uint8_t* __restrict__ cbase,
                                             uint32_t n_words, uint32_t n_plane, GLB uint8_t* __restrict__ out8,
                                             uint64_t base, uint32_t nc, uint32_t nsteps, int32_t* status) {
  const uint32_t lane = __lane_id();
  const uint32_t wbytes = pad16(n_words * 2u);
  const GLB uint64_t* __restrict__ wsrc = (const GLB uint64_t*)(cbase + 4u * kLanes);
  const GLB uint8_t* psrc8 = cbase + 4u * kLanes + wbytes;
  const GLB uint32_t* __restrict__ psrc = (const GLB uint32_t*)psrc8;
  const GLB uint64_t* __restrict__ dplane = (const GLB uint64_t*)psrc8;
  const uint32_t wvalid = wbytes / 8u;           // readable uint2 slots in the word section
  const uint32_t pvalid = pad16(n_plane) / 4u;   // readable u32 slots in the plane section

  uint32_t x = ((const GLB uint32_t*)cbase)[lane];
  uint32_t wptr = 0, wld = 0;   // word ring holds words [wptr, wld)
  uint32_t pptr = 0, pld = 0;   // plane ring (compact mode) holds bytes [pptr, pld)

  for (int s = 0; s < 2; ++s) {   // prologue: >= one block of worst-case demand
    if (wld < n_words) { store_wseg(wring, wld, load_wseg(wsrc, wld, wvalid, lane), lane); wld += kSeg; }
    if (MODE == 2 && pld < n_plane) { store_pseg(pring, pld, load_pseg(psrc, pld, pvalid, lane), lane); pld += kSeg; }
  }
  wave_sync();

  const uint32_t nblk = (nsteps + kBlock - 1) / kBlock;
  uint64_t pnext = 0;
  if (MODE == 1) pnext = dplane[lane];
  GLB uint16_t* out16 = (GLB uint16_t*)out8;

  for (uint32_t blk = 0; blk < nblk; ++blk) {
    // refills issued now, written to the rings after this block (<= 2 segments each)
    uint64_t wp0 = 0, wp1 = 0;
    int wn = 0;
    if (wld < n_words && wld - wptr + kSeg <= kRing) {
      wp0 = load_wseg(wsrc, wld, wvalid, lane); wn = 1;
      if (wld + kSeg < n_words && wld - wptr + 2 * kSeg <= kRing) { wp1 = load_wseg(wsrc, wld + kSeg, wvalid, lane); wn = 2; }
    }
    uint32_t pp0 = 0, pp1 = 0;
    int pn = 0;
    if (MODE == 2 && pld < n_plane && pld - pptr + kSeg <= kRing) {
      pp0 = load_pseg(psrc, pld, pvalid, lane); pn = 1;
      if (pld + kSeg < n_plane && pld - pptr + 2 * kSeg <= kRing) { pp1 = load_pseg(psrc, pld + kSeg, pvalid, lane); pn = 2; }
    }
    const uint64_t pcur = pnext;
    if (MODE == 1 && blk + 1 < nblk) pnext = dplane[(blk + 1) * kLanes + lane];

#pragma unroll
    for (int q = 0; q < kBlock; ++q) {
      const uint32_t t = blk * kBlock + q;
      if (PARTIAL && t >= nsteps) break;                 // wave-uniform
      const uint32_t j = t * kLanes + lane;
      const bool active = !PARTIAL || j < nc;
      const uint64_t e = tbl[x & 4095u];
      const uint32_t elo = (uint32_t)e, ehi = (uint32_t)(e >> 32);
      uint32_t xn = __umul24(elo & 0x1FFFu, x >> 12) + (elo >> 13);
      if (PARTIAL && !active) xn = x;
      const bool need = xn < kL;
      const uint64_t m = __ballot(need);
      const uint32_t w = wring[(wptr + lane_rank(m)) & (kRing - 1u)];
      x = need ? ((xn << 16) | w) : xn;
      wptr += (uint32_t)__popcll(m);
      uint32_t v = ehi;
      if (MODE == 1) {
        v = with_plane(v, (uint32_t)(pcur >> (8 * q)) & 0xFFu);
      } else if (MODE == 2) {
        const bool cons = active && (ehi >> 31);
        const uint64_t bm = __ballot(cons);
        const uint32_t b = pring[(pptr + lane_rank(bm)) & (kRing - 1u)];
        pptr += (uint32_t)__popcll(bm);
        if (cons) v = with_plane(v, b);
      }
      if (active) {
        if (EB == 2) out16[base + j] = (uint16_t)v;
        else out8[base + j] = (uint8_t)v;
      }
    }

    if (wn >= 1) { store_wseg(wring, wld, wp0, lane); wld += kSeg; }
    if (wn >= 2) { store_wseg(wring, wld, wp1, lane); wld += kSeg; }
    if (MODE == 2) {
      if (pn >= 1) { store_pseg(pring, pld, pp0, lane); pld += kSeg; }
      if (pn >= 2) { store_pseg(pring, pld, pp1, lane); pld += kSeg; }
    }
    wave_sync();
  }

  const bool bad_state = x != kL;
  const bool bad = __ballot(bad_state) != 0 || wptr != n_words || (MODE == 2 && pptr != n_plane);
  if (bad) report(status, BS_DEV_ERR_STREAM);
}

template <int EB, bool PARTIAL, bool COMPACT>
__device__ __forceinline__ void decode_chunk_mode(uint32_t mode, const LDS uint64_t* tbl, LDS uint16_t* wring, LDS uint8_t* pring,
                                                  const GLB uint8_t* cbase, uint32_t nw, uint32_t np, GLB uint8_t* out,
                                                  uint64_t base, uint32_t nc, uint32_t nsteps, int32_t* status) {
  if (EB == 1 || mode == 0)
    decode_chunk<0, EB, PARTIAL>(tbl, wring, pring, cbase, nw, np, out, base, nc, nsteps, status);
  else if (mode == 1)
    decode_chunk<1, EB, PARTIAL>(tbl, wring, pring, cbase, nw, np, out, base, nc, nsteps, status);
  else if (COMPACT)
    decode_chunk<2, EB, PARTIAL>(tbl, wring, pring, cbase, nw, np, out, base, nc, nsteps, status);
}

template <bool COMPACT>
__global__ __launch_bounds__(kThreads) void bsck_decode_kernel(const bs_chunk_task* __restrict__ tasks,
                                                               uint32_t n_tasks, bs_chunk_task single,
                                                               int32_t* __restrict__ status) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t s_cum[257];
  __shared__ uint32_t s_val[256];
  LDS uint64_t* s_tbl = (LDS uint64_t*)smem;
  LDS uint16_t* s_wring = (LDS uint16_t*)(smem + kTblBytes);
  LDS uint8_t* s_pring = (LDS uint8_t*)(smem + kLdsLean);

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
  const uint64_t per = (uint64_t)kLanes * steps;
  if (lanes != kLanes || steps == 0 || (steps % kBlock) != 0 || nsym == 0 || nsym > 256 ||
      (eb == 1 && mode != 0) || nch != T.n_chunks || per == 0 || nch != (n + per - 1) / per) {
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
  if (tid == 0) s_cum[0] = 0;
  __syncthreads();
  for (uint32_t d = 1; d < 256; d <<= 1) {        // inclusive scan of s_cum[1..256]
    uint32_t add = (tid < 256 && tid >= d) ? s_cum[tid + 1 - d] : 0u;
    __syncthreads();
    if (tid < 256) s_cum[tid + 1] += add;
    __syncthreads();
  }
  bool bad_tbl = s_cum[256] != 4096u;
  if (tid < nsym && f_own == 0) bad_tbl = true;
  if (__syncthreads_or(bad_tbl)) {
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
  const uint32_t wave = tid / kLanes;
  const uint32_t chunk = group * kWaves + wave;
  if (chunk >= nch) return;
  const GLB uint8_t* ce = b + ctab + 16ull * chunk;
  const uint64_t off = (uint64_t)ld_u32(ce) | ((uint64_t)ld_u32(ce + 4) << 32);
  const uint32_t nw = ld_u32(ce + 8), np = ld_u32(ce + 12);
  const uint64_t cbase_idx = (uint64_t)chunk * per;
  const uint32_t nc = (uint32_t)((n - cbase_idx) < per ? (n - cbase_idx) : per);
  const uint32_t nsteps = (nc + kLanes - 1) / kLanes;
  const uint32_t dense_plane = ((nsteps + kBlock - 1) / kBlock) * kBlock * kLanes;
  bool ok = (off % 16) == 0 && off + 4ull * kLanes + pad16(nw * 2u) + pad16(np) <= T.blob_bytes &&
            nw <= nsteps * kLanes;
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
  GLB uint8_t* out = (GLB uint8_t*)T.out;
  const bool partial = nc != per;
  if (eb == 2) {
    if (partial) decode_chunk_mode<2, true, COMPACT>(mode, s_tbl, wring, pring, cbase, nw, np, out, cbase_idx, nc, nsteps, status);
    else decode_chunk_mode<2, false, COMPACT>(mode, s_tbl, wring, pring, cbase, nw, np, out, cbase_idx, nc, nsteps, status);
  } else {
    if (partial) decode_chunk_mode<1, true, COMPACT>(0, s_tbl, wring, pring, cbase, nw, np, out, cbase_idx, nc, nsteps, status);
    else decode_chunk_mode<1, false, COMPACT>(0, s_tbl, wring, pring, cbase, nw, np, out, cbase_idx, nc, nsteps, status);
  }
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
  if (h[7] != 12 || info->lanes != kLanes || info->steps == 0 || info->steps % kBlock || info->n_syms == 0 ||
      info->n_syms > 256 || (info->elem_bytes != 1 && info->elem_bytes != 2) || info->plane_mode > 2)
    return BS_ERR_FORMAT;
  const uint64_t per = (uint64_t)kLanes * info->steps;
  if (info->n_chunks != (info->n + per - 1) / per) return BS_ERR_FORMAT;
  return BS_OK;
}

int bs_chunk_decode(const uint8_t* d_blob, uint64_t blob_bytes, void* d_out, uint64_t n, uint32_t n_chunks,
                    uint32_t plane_mode, int32_t* d_status, void* stream) {
  if (!d_status || (n > 0 && (!d_blob || !d_out))) return BS_ERR_ARG;
  if (((uintptr_t)d_blob & 15u) != 0 || plane_mode > 2) return BS_ERR_ARG;
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
