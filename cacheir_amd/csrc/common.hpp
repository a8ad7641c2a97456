// Shared helpers for the gfx950 decode-step kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "cacheir_hip.h"

namespace cir {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per-thread text of the last argument error (read by cir_last_error_string).
void set_error(const char* fmt, ...);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Launch-status helper: returns the launch error of the most recent launch.
inline int launch_status() { return static_cast<int>(hipGetLastError()); }

#define CIR_CHECK_ARG(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      ::cir::set_error(__VA_ARGS__);             \
      return static_cast<int>(hipErrorInvalidValue); \
    }                                            \
  } while (0)

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<f16>(f16 v) { return static_cast<float>(v); }

// Materialise v as an fp32 value: stops the compiler contracting the operation that
// produced it with a following conversion (e.g. a multiply and an fp16 conversion
// into one mixed-precision FMA, which rounds once instead of twice), so every kernel
// that computes the same expression stores the same bits.
__device__ __forceinline__ float as_f32_value(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }

// Wavefront (64-lane) reductions through DPP/swizzle-backed shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Greedy-sampling order (numpy argmax, scheduler.py:535-543): the larger value wins,
// NaN counts as larger than every number, and equal values go to the smaller index.
__device__ __forceinline__ void argmax_better(float& bv, int& bi, float v, int i) {
  const bool vn = v != v, bn = bv != bv;
  const bool take = vn ? (!bn || i < bi) : (!bn && (v > bv || (v == bv && i < bi)));
  bv = take ? v : bv;  // selects, not a branch: callers run this between lane shuffles
  bi = take ? i : bi;
}

}  // namespace cir
