// Zstandard decoding on the GPU, for the reference's zstd-coded container
// entries:
//   codec "zstd"            the whole tensor is one zstd frame
//                           (bigsmall/codecs/generic.py:15-18, bigsmall/decoder.py:80-81);
//   codec "special/lowcard" a table of <= 255 distinct element values and a
//                           zstd frame of one uint8 index per element
//                           (bigsmall/codecs/special.py:23-85);
//   codec "zstd_xor_delta"  a zstd frame of XOR differences to a base tensor
//                           (bigsmall/decoder.py:88-90, 190-198); with a base
//                           given, the kernel XORs it into the output.
//
// One 64-lane workgroup per task decodes all frames of its input with the
// team-parallel decoder of zstd_core.h: tables and the current compressed
// block (when it is at most 24 KB) in LDS, about 39 KB in all; literals
// of the current block in a 128 KiB slice of the work buffer, matches copied
// by all lanes. Zstandard is a sequential format (each match may copy bytes
// of the one before), so a frame is not split across workgroups; the
// reference's zstd entries are small (norm-weight indices, integer buffers)
// and many of them go in one launch.
//
// lut_expand_kernel turns lowcard indices into element bytes.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "../../include/bigsmall_hip.h"
#include "zstd_core.h"

// Work area of bs_zstd_decode_static: BS_ZSTD_STATIC_MAX_TASKS literal slices
// of 128 KiB (8 MiB) in a file-scope device array, so that entry point
// allocates nothing. Each GPU the library runs on holds its own copy until the
// process ends; host code reaches it only through the address
// hipGetSymbolAddress returns on that device (the array's name is a host-side
// stand-in, not a device address). Every call on one GPU shares it: the
// kernel writes each literal before reading it, so nothing needs clearing.
// The library orders the calls on one GPU itself: each call's stream first
// waits for an event recorded after the previous call's launch (one event per
// device, created with the address lookup), so calls on different streams or
// host threads run one after another instead of racing on the array.
static __device__ __align__(256) uint8_t scratch[(uint64_t)BS_ZSTD_STATIC_MAX_TASKS * bs_zstd::kBlockMax];

namespace {

struct DevTeam {
  static constexpr uint32_t size = 64;
  __device__ uint32_t lane() const { return threadIdx.x; }
  __device__ void sync() const { __syncthreads(); }
};

__device__ int32_t status_bits(int32_t e) {
  switch (e) {
    case bs_zstd::kOk: return 0;
    case bs_zstd::kErrTruncated: return BS_DEV_ERR_BOUNDS;
    case bs_zstd::kErrFormat: return BS_DEV_ERR_HEADER;
    case bs_zstd::kErrOutput: return BS_DEV_ERR_COUNT;
    default: return BS_DEV_ERR_STREAM;
  }
}

__global__ __launch_bounds__(64) void zstd_kernel(const bs_zstd_task* __restrict__ tasks, uint8_t* __restrict__ work,
                                                  uint64_t* __restrict__ out_len, int32_t* __restrict__ status) {
  __shared__ bs_zstd::ZState z;
  const bs_zstd_task T = tasks[blockIdx.x];
  uint8_t* lit = work + (uint64_t)blockIdx.x * bs_zstd::kBlockMax;
  uint64_t got = 0;
  int32_t e = bs_zstd::kErrFormat;
  if (T.src && (T.dst || T.dst_len == 0)) {
    e = bs_zstd::zstd_frames(DevTeam{}, z, T.src, T.src_len, T.dst, T.dst_len, lit, got);
    if (e == bs_zstd::kOk && got != T.dst_len) e = bs_zstd::kErrOutput;
  }
  if (e == bs_zstd::kOk && T.xor_src) {        // a delta: dst ^= base (the frames are all written)
    for (uint64_t i = threadIdx.x; i < T.dst_len; i += 64) T.dst[i] ^= T.xor_src[i];
  }
  if (threadIdx.x == 0) {
    out_len[blockIdx.x] = e ? 0 : got;
    if (e) atomicOr(status, status_bits(e));
  }
}

// Task blockIdx.y; blockIdx.x strides over its elements.
__global__ __launch_bounds__(256) void lut_expand_kernel(const bs_lut_task* __restrict__ tasks,
                                                         int32_t* __restrict__ status) {
  const bs_lut_task T = tasks[blockIdx.y];
  if (T.item_bytes == 0 || T.item_bytes > 8 || T.n_lut > 256) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(status, BS_DEV_ERR_HEADER);
    return;
  }
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  bool bad = false;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < T.n; i += stride) {
    const uint32_t v = T.idx[i];
    if (v >= T.n_lut) {
      bad = true;
      continue;
    }
    for (uint32_t b = 0; b < T.item_bytes; ++b) T.out[i * T.item_bytes + b] = T.lut[v * T.item_bytes + b];
  }
  if (__any(bad) && (threadIdx.x & 63u) == 0) atomicOr(status, BS_DEV_ERR_COUNT);
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;                  // guards the tables below and orders the launches
void* g_scratch_ptr[kMaxDevices] = {};
hipEvent_t g_scratch_done[kMaxDevices] = {};   // recorded after each call's launch on that device

// Set-up of the current device, once (with that device current): the address
// of `scratch` and the ordering event. Called with g_scratch_mu held.
int scratch_setup(int* dev_out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return BS_ERR_HIP;
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return BS_ERR_HIP;
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return BS_ERR_HIP;
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = p;
  }
  *dev_out = dev;
  return BS_OK;
}

}  // namespace

extern "C" {

uint64_t bs_zstd_work_bytes(uint32_t n_tasks) { return (uint64_t)n_tasks * bs_zstd::kBlockMax; }

int bs_zstd_decode(const bs_zstd_task* d_tasks, uint32_t n_tasks, void* d_work, uint64_t work_bytes,
                   uint64_t* d_out_len, int32_t* d_status, void* stream) {
  if (!d_status || (n_tasks && (!d_tasks || !d_work || !d_out_len)) || n_tasks > 0x7FFFFFFFu) return BS_ERR_ARG;
  if (n_tasks == 0) return BS_OK;
  if (work_bytes < bs_zstd_work_bytes(n_tasks)) return BS_ERR_ARG;
  hipLaunchKernelGGL(zstd_kernel, dim3(n_tasks), dim3(64), 0, (hipStream_t)stream, d_tasks, (uint8_t*)d_work,
                     d_out_len, d_status);
  return hipGetLastError() == hipSuccess ? BS_OK : BS_ERR_HIP;
}

int bs_zstd_decode_static(const bs_zstd_task* d_tasks, uint32_t n_tasks, uint64_t* d_out_len, int32_t* d_status,
                          void* stream) {
  if (!d_status || (n_tasks && (!d_tasks || !d_out_len))) return BS_ERR_ARG;
  if (n_tasks > BS_ZSTD_STATIC_MAX_TASKS) return BS_ERR_CAP;
  if (n_tasks == 0) return BS_OK;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  int dev = -1;
  const int rc = scratch_setup(&dev);
  if (rc != BS_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  // Under stream capture the graph's own order applies (an event recorded
  // outside the capture cannot be waited on inside it): the event is neither
  // waited on nor recorded, and launches of two graphs that overlap race.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess) return BS_ERR_HIP;
  const bool order = cap == hipStreamCaptureStatusNone;
  // the previous call's launch (on any stream) has finished with the array;
  // an event never recorded is complete
  if (order && hipStreamWaitEvent(s, g_scratch_done[dev], 0) != hipSuccess) return BS_ERR_HIP;
  hipLaunchKernelGGL(zstd_kernel, dim3(n_tasks), dim3(64), 0, s, d_tasks, (uint8_t*)g_scratch_ptr[dev], d_out_len,
                     d_status);
  if (hipGetLastError() != hipSuccess) return BS_ERR_HIP;
  if (order && hipEventRecord(g_scratch_done[dev], s) != hipSuccess) return BS_ERR_HIP;
  return BS_OK;
}

int bs_lut_expand(const bs_lut_task* d_tasks, uint32_t n_tasks, uint64_t max_n, int32_t* d_status, void* stream) {
  if (!d_status || (n_tasks && !d_tasks) || n_tasks > 65535u) return BS_ERR_ARG;
  if (n_tasks == 0 || max_n == 0) return BS_OK;
  const uint64_t blocks = std::min<uint64_t>((max_n + 255) / 256, 1024);
  hipLaunchKernelGGL(lut_expand_kernel, dim3((uint32_t)blocks, n_tasks), dim3(256), 0, (hipStream_t)stream, d_tasks,
                     d_status);
  return hipGetLastError() == hipSuccess ? BS_OK : BS_ERR_HIP;
}

}  // extern "C"
