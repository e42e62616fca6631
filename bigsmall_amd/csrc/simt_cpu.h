// Host execution of this library's HIP kernels, for AddressSanitizer / UBSan
// runs on the CPU (tests/native/). Every lane of a workgroup is a fiber (its
// own stack, switched by a few instructions), all on the calling thread:
// a lane runs until it reaches a barrier, then the next lane runs.
// Wavefront operations exchange values through a per-wave slot array between
// two barrier phases of the wave's lanes; __syncthreads is a barrier of the
// workgroup's lanes; a lane that returns from the kernel leaves both barriers.
// Workgroups of a launch run one after another. Dynamic LDS is a per-workgroup
// buffer filled with 0xA5, as LDS holds no defined value at launch;
// __shared__ arrays are static (workgroups never overlap). Because lanes run
// in a fixed order between barriers, a read of LDS that another lane writes
// without a barrier in between sees the launch fill, not the written value.
// x86-64 only; requires clang (ext_vector_type) and C++17.
#pragma once

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <memory>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define BS_SIMT_ASAN 1
#endif
#endif
#ifdef BS_SIMT_ASAN
#include <sanitizer/common_interface_defs.h>
#endif

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static

struct dim3 {
  uint32_t x, y, z;
  dim3(uint32_t x_ = 1, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
};
typedef void* hipStream_t;
typedef int hipError_t;
enum { hipSuccess = 0 };
enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
inline hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute, int) { return hipSuccess; }
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 63 };
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {   // an MI355X's compute units
  *v = 256;
  return hipSuccess;
}

// Saves the callee-saved registers and the stack pointer of the running
// context in *from_sp and resumes the context whose stack pointer is to_sp
// (a weak symbol: every translation unit that includes this header emits it).
extern "C" void bs_simt_switch(void** from_sp, void* to_sp);
asm(R"(
.text
.p2align 4
.weak bs_simt_switch
.type bs_simt_switch,@function
bs_simt_switch:
  pushq %rbp
  pushq %rbx
  pushq %r12
  pushq %r13
  pushq %r14
  pushq %r15
  movq %rsp, (%rdi)
  movq %rsi, %rsp
  popq %r15
  popq %r14
  popq %r13
  popq %r12
  popq %rbx
  popq %rbp
  ret
.size bs_simt_switch, .-bs_simt_switch
)");

namespace bs_simt {

constexpr uint32_t kLanes = 64;
constexpr size_t kStack = 512 * 1024;

// A barrier of cooperating lanes: arriving lanes yield until the phase's
// last participant arrives.
struct Barrier {
  explicit Barrier(uint32_t n) : expected(n) {}
  uint32_t expected, arrived = 0;
  uint64_t phase = 0;
  void complete() {
    arrived = 0;
    ++phase;
  }
  void arrive_and_wait();
  void arrive_and_drop() {
    --expected;
    if (expected > 0 && arrived >= expected) complete();
  }
};

struct Wave {
  explicit Wave(uint32_t n) : bar(n), lanes(n), alive(n == 64 ? ~0ull : ((1ull << n) - 1)) {}
  Barrier bar;
  uint32_t lanes;
  uint64_t alive;
  uint64_t slot[kLanes] = {};
};

struct Block {
  Block(uint32_t n, size_t lds_bytes) : bar(n), lds(lds_bytes + 16, 0xA5) {}
  Barrier bar;
  std::vector<uint8_t> lds;
  std::vector<std::unique_ptr<Wave>> waves;
};

struct Ctx {
  dim3 tid, bid, bdim, gdim;
  uint32_t lane = 0;
  Block* blk = nullptr;
  Wave* wave = nullptr;
};

struct Fiber {
  uint8_t* stack = nullptr;                   // kStack bytes, kept for later launches
  void* sp = nullptr;
  bool done = false;
  Ctx ctx;
  void* fake = nullptr;
};

// Fiber stacks are allocated once per thread and reused by every launch.
inline std::vector<std::unique_ptr<uint8_t[]>>& stack_pool() {
  static thread_local std::vector<std::unique_ptr<uint8_t[]>> pool;
  return pool;
}

struct Sched {
  std::vector<std::unique_ptr<Fiber>> fibers;
  Fiber* cur = nullptr;
  void* main_sp = nullptr;
  void* main_fake = nullptr;
  const void* main_bottom = nullptr;
  size_t main_size = 0;
  std::function<void()> body;
};
inline thread_local Sched* sched = nullptr;

inline Ctx& ctx() { return sched->cur->ctx; }

// Back to the scheduler (the fiber resumes here when it is next run).
inline void yield() {
  Sched& S = *sched;
  Fiber* f = S.cur;
#ifdef BS_SIMT_ASAN
  __sanitizer_start_switch_fiber(f->done ? nullptr : &f->fake, S.main_bottom, S.main_size);
#endif
  bs_simt_switch(&f->sp, S.main_sp);
#ifdef BS_SIMT_ASAN
  __sanitizer_finish_switch_fiber(f->fake, &S.main_bottom, &S.main_size);
#endif
}

inline void Barrier::arrive_and_wait() {
  const uint64_t p = phase;
  if (++arrived >= expected) {
    complete();
    return;
  }
  while (phase == p) yield();
}

[[noreturn]] inline void fiber_start() {
  Sched& S = *sched;
#ifdef BS_SIMT_ASAN
  __sanitizer_finish_switch_fiber(nullptr, &S.main_bottom, &S.main_size);
#endif
  S.body();
  Fiber* f = S.cur;
  f->ctx.wave->alive &= ~(1ull << f->ctx.lane);
  f->ctx.wave->bar.arrive_and_drop();
  f->ctx.blk->bar.arrive_and_drop();
  f->done = true;
  yield();
  abort();   // a finished fiber is never resumed
}

inline void resume(Fiber* f) {
  Sched& S = *sched;
  S.cur = f;
#ifdef BS_SIMT_ASAN
  __sanitizer_start_switch_fiber(&S.main_fake, f->stack, kStack);
#endif
  bs_simt_switch(&S.main_sp, f->sp);
#ifdef BS_SIMT_ASAN
  __sanitizer_finish_switch_fiber(S.main_fake, nullptr, nullptr);
#endif
}

inline uint8_t* dynamic_lds() {
  uint8_t* p = ctx().blk->lds.data();
  return p + ((16 - ((uintptr_t)p & 15)) & 15);
}

// One value per lane in, every lane's value visible to all (between two barriers).
template <class F>
inline auto exchange(uint64_t mine, F read) {
  Wave& w = *ctx().wave;
  w.slot[ctx().lane] = mine;
  w.bar.arrive_and_wait();
  auto r = read(w);
  w.bar.arrive_and_wait();
  return r;
}

template <class K, class... A>
inline void launch(K kernel, dim3 g, dim3 b, size_t lds, hipStream_t, A... args) {
  const uint32_t n = b.x * b.y * b.z;
  if (n == 0) return;
  Sched S;
  Sched* outer = sched;
  sched = &S;
  S.body = [&] { kernel(args...); };
  auto& pool = stack_pool();
  while (pool.size() < n) pool.emplace_back(new uint8_t[kStack]);
  for (uint32_t t = 0; t < n; ++t) {
    S.fibers.emplace_back(new Fiber);
    S.fibers.back()->stack = pool[t].get();
  }
  for (uint32_t by = 0; by < g.y; ++by)
    for (uint32_t bx = 0; bx < g.x; ++bx) {
      Block blk(n, lds);
      for (uint32_t w = 0; w * kLanes < n; ++w) blk.waves.emplace_back(new Wave(std::min(kLanes, n - w * kLanes)));
      for (uint32_t t = 0; t < n; ++t) {
        Fiber& f = *S.fibers[t];
        f.done = false;
        f.ctx = Ctx{dim3(t), dim3(bx, by), b, g, t % kLanes, &blk, blk.waves[t / kLanes].get()};
        // a fresh stack: fiber_start as the return address of the switch,
        // below it the six callee-saved registers it pops
        uintptr_t top = ((uintptr_t)f.stack + kStack) & ~(uintptr_t)15;
        void** sp = (void**)(top - 16);
        sp[0] = (void*)&fiber_start;
        for (int r = 1; r <= 6; ++r) sp[-r] = nullptr;
        f.sp = (void*)(sp - 6);
      }
      for (uint32_t left = n; left > 0;) {
        left = 0;
        for (uint32_t t = 0; t < n; ++t)
          if (!S.fibers[t]->done) {
            resume(S.fibers[t].get());
            left += !S.fibers[t]->done;
          }
      }
    }
  sched = outer;
}

}  // namespace bs_simt

#define hipLaunchKernelGGL(k, g, b, lds, s, ...) bs_simt::launch(k, g, b, lds, s, __VA_ARGS__)
#define threadIdx (bs_simt::ctx().tid)
#define blockIdx (bs_simt::ctx().bid)
#define blockDim (bs_simt::ctx().bdim)
#define gridDim (bs_simt::ctx().gdim)

// HIP's integer min / max of device code
inline uint32_t min(uint32_t a, uint32_t b) { return b < a ? b : a; }
inline uint64_t min(uint64_t a, uint64_t b) { return b < a ? b : a; }
inline int min(int a, int b) { return b < a ? b : a; }
inline uint32_t max(uint32_t a, uint32_t b) { return a < b ? b : a; }
inline uint64_t max(uint64_t a, uint64_t b) { return a < b ? b : a; }
inline int max(int a, int b) { return a < b ? b : a; }

inline void __syncthreads() { bs_simt::ctx().blk->bar.arrive_and_wait(); }
inline uint32_t __lane_id() { return bs_simt::ctx().lane; }
inline uint64_t __ballot(int pred) {
  return bs_simt::exchange(pred ? 1u : 0u, [](bs_simt::Wave& w) {
    uint64_t m = 0;
    for (uint32_t l = 0; l < w.lanes; ++l) m |= (w.slot[l] & 1ull) << l;
    return m & w.alive;
  });
}
inline int __any(int pred) { return __ballot(pred) != 0; }
inline int __popcll(uint64_t v) { return __builtin_popcountll(v); }
inline uint32_t __umul24(uint32_t a, uint32_t b) { return (a & 0xFFFFFFu) * (b & 0xFFFFFFu); }
inline int32_t atomicOr(int32_t* p, int32_t v) {
  const int32_t o = *p;
  *p = o | v;
  return o;
}
inline uint32_t atomicAdd(uint32_t* p, uint32_t v) {
  const uint32_t o = *p;
  *p = o + v;
  return o;
}

// The gfx9 builtins the kernels use, with the instructions' semantics.
inline uint32_t __builtin_amdgcn_mbcnt_lo(uint32_t m, uint32_t acc) {
  const uint32_t l = bs_simt::ctx().lane;
  return acc + __builtin_popcount(m & (l >= 32 ? 0xFFFFFFFFu : ((1u << l) - 1u)));
}
inline uint32_t __builtin_amdgcn_mbcnt_hi(uint32_t m, uint32_t acc) {
  const uint32_t l = bs_simt::ctx().lane;
  return acc + __builtin_popcount(m & (l <= 32 ? 0u : ((1u << (l - 32)) - 1u)));
}
// readfirstlane is only applied to wave-uniform values here, so every lane's
// copy is the first lane's; readlane exchanges through the wave. Both return
// int, as the GPU builtins do, so that a widening cast sign-extends here too.
inline int __builtin_amdgcn_readfirstlane(int x) { return x; }
inline int __builtin_amdgcn_readlane(int x, int lane) {
  return (int)(uint32_t)bs_simt::exchange((uint32_t)x, [lane](bs_simt::Wave& w) { return w.slot[lane & 63]; });
}
inline void __builtin_amdgcn_wave_barrier() { bs_simt::ctx().wave->bar.arrive_and_wait(); }
// ds_bpermute: each lane reads the value of lane (index / 4) mod 64
inline int __builtin_amdgcn_ds_bpermute(int index, int v) {
  const uint32_t src = ((uint32_t)index >> 2) & 63u;
  return (int)(uint32_t)bs_simt::exchange((uint32_t)v, [src](bs_simt::Wave& w) { return w.slot[src]; });
}
inline void __builtin_amdgcn_s_setprio(int) {}   // issue priority: no effect on results
inline void __builtin_amdgcn_fence(int, const char*) {}
inline void __builtin_amdgcn_fence(int, const char*, const char*) {}
inline void __builtin_amdgcn_s_barrier() { bs_simt::ctx().blk->bar.arrive_and_wait(); }
inline void __builtin_amdgcn_s_waitcnt(int) {}
// v_bfe_u32: `width` bits of src from bit `offset` (both taken mod 32; width 0 gives 0)
inline uint32_t __builtin_amdgcn_ubfe(uint32_t src, uint32_t offset, uint32_t width) {
  offset &= 31u;
  width &= 31u;
  return width ? (uint32_t)((src >> offset) & ((1ull << width) - 1ull)) : 0u;
}
// v_alignbit_b32: the 32 bits of {hi, lo} from bit (shift mod 32)
inline uint32_t __builtin_amdgcn_alignbit(uint32_t hi, uint32_t lo, uint32_t shift) {
  return (uint32_t)((((uint64_t)hi << 32) | lo) >> (shift & 31u));
}
// DPP data movement of a 32-bit value, for the controls the kernels use:
// row_shr:n (0x111-0x11F: the lane n below in the same 16-lane row),
// row_bcast:15 (0x142: lane 15 of the previous row), row_bcast:31 (0x143:
// lane 31). A lane of a row that row_mask leaves out, or whose source lies
// outside its row (row_shr) or before row 1 / row 2 (the broadcasts),
// returns `old` (bound_ctrl = 0) or 0 (bound_ctrl = 1); the kernels pass 0
// for old, so either reads as 0. bank_mask must be 0xF.
inline int __builtin_amdgcn_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
  const uint32_t l = bs_simt::ctx().lane, row = l / 16u;
  int src_lane = -1;
  if (ctrl >= 0x111 && ctrl <= 0x11F) {
    const uint32_t k = (uint32_t)ctrl - 0x110u;
    if (l % 16u >= k) src_lane = (int)(l - k);
  } else if (ctrl == 0x142) {
    if (row >= 1) src_lane = (int)(row * 16u - 1u);
  } else if (ctrl == 0x143) {
    if (row >= 2) src_lane = 31;
  } else {
    abort();                                     // a control this emulation does not cover
  }
  if (bank_mask != 0xF) abort();
  const uint32_t v = (uint32_t)bs_simt::exchange((uint32_t)src, [src_lane](bs_simt::Wave& w) {
    return src_lane >= 0 ? w.slot[src_lane] : 0ull;
  });
  if (!((row_mask >> row) & 1)) return old;
  if (src_lane < 0) return bound_ctrl ? 0 : old;
  return (int)v;
}
// v_perm_b32: byte i of the result is selected by byte i of sel from the
// 8 bytes {a, b} (b the low dword): 0-7 that byte, 8-11 the sign of bytes
// 1, 3, 5, 7 spread to 0x00 / 0xFF, 12 zero, 13-255 0xFF.
inline uint32_t __builtin_amdgcn_perm(uint32_t a, uint32_t b, uint32_t sel) {
  const uint64_t in = ((uint64_t)a << 32) | b;
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i) {
    const uint32_t s = (sel >> (8 * i)) & 0xFFu;
    uint32_t v;
    if (s < 8) v = (uint32_t)(in >> (8 * s)) & 0xFFu;
    else if (s < 12) v = ((in >> (16 * (s - 8) + 15)) & 1u) ? 0xFFu : 0u;
    else if (s == 12) v = 0;
    else v = 0xFFu;
    r |= v << (8 * i);
  }
  return r;
}
