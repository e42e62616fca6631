// What the decode kernels need from the compiler beyond plain C++: the HIP
// runtime and kernel language, the LDS / global / constant address spaces, and empty asm
// statements that pin values in vector registers at chosen points. The
// library is built for gfx950 by hipcc; the same kernel sources also build as
// host C++ for sanitizer runs on the CPU (BS_SIMT_CPU, simt_cpu.h), where the
// address spaces and register pins are empty and every lane is a thread.
#pragma once

#ifdef BS_SIMT_CPU
#include "simt_cpu.h"
#define LDS
#define GLB
#define CST
#define BS_DYNAMIC_LDS(name) uint8_t* name = bs_simt::dynamic_lds()
#define BS_KEEP1(a) ((void)(a))
#define BS_KEEP2(a, b) ((void)(a), (void)(b))
#define BS_KEEP4(a, b, c, d) ((void)(a), (void)(b), (void)(c), (void)(d))
#define BS_OPAQUE(x) ((void)(x))
#define BS_WRITELANE_I(acc, v, j) ((acc) = __lane_id() == (uint32_t)(j) ? (uint32_t)(v) : (acc))
#define BS_LDS_ADD(p, v) ((void)atomicAdd((p), (v)))
#define BS_BFE_U32(dst, x, off, width) ((dst) = ((uint32_t)(x) >> (off)) & ((1u << (width)) - 1u))
#else
#include <hip/hip_runtime.h>
#define LDS __attribute__((address_space(3)))
#define GLB __attribute__((address_space(1)))
// Read-only global memory at wave-uniform addresses: loads through the scalar
// cache into scalar registers (reads only; nothing stores through it).
#define CST __attribute__((address_space(4)))
#define BS_DYNAMIC_LDS(name) extern __shared__ __attribute__((aligned(16))) uint8_t name[]
// Makes the values available at this point: every load producing them is
// issued before it, and nothing can sink them under a later branch.
#define BS_KEEP1(a) asm volatile("" ::"v"(a))
#define BS_KEEP2(a, b) asm volatile("" ::"v"(a), "v"(b))
#define BS_KEEP4(a, b, c, d) asm volatile("" ::"v"(a), "v"(b), "v"(c), "v"(d))
// Hides a value's provenance from the optimiser (it stays in a vector register).
#define BS_OPAQUE(x) asm volatile("" : "+v"(x))
// Lane j of the 32-bit register acc takes the wave-uniform value v (one
// v_writelane_b32; v in a scalar register); j must be a constant once the
// caller's loop is unrolled (a compile error otherwise).
#define BS_WRITELANE_I(acc, v, j) asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(acc) : "s"(v), "i"(j))
// dst = bits [off, off + width) of x in one v_bfe_u32 the optimiser cannot
// rewrite (it turns a field extract followed by a scale into a shift and a
// mask; kept whole, an LDS address from it is one v_lshl_add). off and width
// are literal constants.
#define BS_BFE_U32(dst, x, off, width) asm("v_bfe_u32 %0, %1, " #off ", " #width : "=v"(dst) : "v"(x))
// Atomic add to a 32-bit LDS word (ds_add_u32), ordered only within the wave.
#define BS_LDS_ADD(p, v) ((void)__hip_atomic_fetch_add((p), (v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT))
#endif
