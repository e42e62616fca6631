// Raising a kernel's dynamic-LDS limit above the 64 KiB default, once per
// device, safely from any number of host threads.
#pragma once

#include "simt.h"
#include <stdint.h>

#include <atomic>

namespace bs_internal {

// Bit d of `done` records that `fn` was configured on device d. The attribute
// call is idempotent, so two threads racing on the first launch both set it;
// the mask only saves the call on later launches. Devices beyond 63 set it on
// every launch. A failure is left to the launch itself, which then reports
// the error through hipGetLastError.
inline void ensure_lds_limit(const void* fn, uint32_t bytes, std::atomic<uint64_t>& done) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  const uint64_t bit = (dev >= 0 && dev < 64) ? (1ull << dev) : 0ull;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess && bit)
    done.fetch_or(bit, std::memory_order_acq_rel);
}

}  // namespace bs_internal
