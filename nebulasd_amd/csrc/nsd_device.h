// Device-side helpers for the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nsd_common.h"

namespace nsd {

typedef _Float16 f16;
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

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

}  // namespace nsd
