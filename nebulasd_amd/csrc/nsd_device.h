// Device-side helpers for the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "nsd_common.h"

namespace nsd {

typedef _Float16 f16;
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// The QK-norm's x_d^2 + x_{d+64}^2 and the rotate-half RoPE pair with the
// fused multiply-adds spelled out, so that every kernel computing them (the
// prologue, the attention that runs it fused) rounds identically, whatever
// the compiler would contract on its own.
__device__ inline float sq_pair(float a, float b) { return __builtin_fmaf(a, a, b * b); }
__device__ inline float rope_lo(float x0, float x1, float c, float s) { return __builtin_fmaf(x0, c, -(x1 * s)); }
__device__ inline float rope_hi(float x0, float x1, float c, float s) { return __builtin_fmaf(x0, s, x1 * c); }
// fp32 value x rounded to fp16.  The empty asm pins x as an fp32 register, so
// the conversion stays a separate step: left alone, the compiler folds it into
// a mixed-precision FMA (v_fma_mixlo_f16 / v_fma_mixhi_f16) in some kernels
// and not in others, and the two can differ in the last place.  (Not
// volatile: a volatile asm would also order the memory operations around it.)
__device__ inline f16 f16_of(float x) {
  asm("" : "+v"(x));
  return (f16)x;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ inline void flag_status(int32_t* status, int32_t bit) {
  if (status != nullptr) atomicOr(status, bit);
}

// Launch-status helper for the C ABI.
inline int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(NSD_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(err));
  return NSD_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) f16x8 lds_f16x8;
typedef __fp16 fp16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4;

// v_mfma_f32_16x16x32_f16: lane (i = lane % 16, g = lane / 16) holds
// A[i][8g .. 8g+7] and B[8g .. 8g+7][i]; it receives C[4g .. 4g+3][i].
__device__ inline f32x4 mfma_k32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_16x16x16_f16: as above with k = 16 (A[i][4g .. 4g+3]).
__device__ inline f32x4 mfma_k16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Transposing LDS read: lane j of each 16-lane group receives, in slot m,
// 16-bit element (j % 4) of the 8 bytes addressed by lane 4*m + j/4.
__device__ inline f16x4 ds_read_tr16(const lds_char* p) {
  fp16x4_t t = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)p);
  return __builtin_bit_cast(f16x4, t);
}

// Calls f(integral_constant<int, i>) for i = 0 .. N-1 (compile-time unrolled).
template <int N, typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

}  // namespace nsd
