// Shared device and host helpers for the gfx950 QSA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "fastdiv.h"

namespace qsa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Host-side error reporting shared by every entry point (qsa_errors.hip).
// ---------------------------------------------------------------------------
void set_error(const std::string& message);
int fail(int status, const std::string& message);
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  // v_perm_b32: byte i of the result is byte sel.byte[i] of the 8 bytes
  // (hi_src:lo_src), lo_src supplying bytes 0-3.
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const __bf16 a = (__bf16)lo;  // round to nearest even
  const __bf16 b = (__bf16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ float bf16_lo(uint32_t pair) {
  return __builtin_bit_cast(float, pair << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t pair) {
  return __builtin_bit_cast(float, pair & 0xffff0000u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier that orders LDS accesses only. __syncthreads() also waits
// for every outstanding global load of the wave (vmcnt(0)); this one leaves
// them in flight, so loads issued early (prefetches) overlap barrier-heavy
// phases. Use it only where threads communicate through LDS alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

// v[lane] + v[lane ^ 32] in every lane, without the LDS crossbar.
// v_permlane32_swap a, b exchanges the upper half of a with the lower half of
// b; with a and b both holding v, a becomes (v[0..31], v[0..31]) and b
// (v[32..63], v[32..63]), so a + b adds each lane to its partner (lower half
// first in every lane, so both halves get the same bits). The builtin ties
// both operands to its results, so they get distinct registers (a swap of a
// register with itself would be a rotation), and the compiler places the
// hazard nops and may schedule it like any other VALU op.
__device__ __forceinline__ float sum_wave_halves(float v) {
  const uint32_t a = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Load of a wave-uniform address through the scalar memory path (the
// constant address space: the data must not change during the kernel). Its
// wait is on the scalar counter, so it never queues behind vector loads.
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ u32x4 load_u32x4(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x2 load_u32x2(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}

}  // namespace qsa

// A block of zeros in device memory (one copy per translation unit). Gathers of
// invalid slots are redirected here so masked K/V rows read as exact zeros.
static __device__ __attribute__((aligned(256))) uint32_t g_qsa_zero_rows[256];
// A -1 page-table entry: loads of entries that do not exist read it, so the
// loaded value needs no select afterwards (a select right after a load makes
// the compiler wait for that load, and with it every older one, at once).
static __device__ int32_t g_qsa_no_page[1] = {-1};  // never written
