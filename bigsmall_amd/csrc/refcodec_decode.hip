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
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bigsmall_hip.h"

namespace {

#define LDS __attribute__((address_space(3)))
#define GLB __attribute__((address_space(1)))

constexpr uint32_t kL = 1u << 16;
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
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
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
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)se_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kSeLds);
    attr = true;
  }
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

}  // extern "C"
