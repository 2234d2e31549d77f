// Shared device helpers for the FlashDP MI355X (gfx950) kernels.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, MFMA operand
// vectors, and bf16/fp16 bit-level conversions.  No CUDA or dual-path code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flashdp_hip.h"

namespace fdp {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kWave = 64;

// ---------------------------------------------------------------- dtype tags
struct F32 {
  using storage = float;
  static constexpr int code = FDP_F32;
  __device__ static inline float to_f32(float v) { return v; }
  __device__ static inline float from_f32(float v) { return v; }
};
struct BF16 {
  using storage = uint16_t;
  static constexpr int code = FDP_BF16;
  __device__ static inline float to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
  }
  // round-to-nearest-even, NaN stays NaN
  __device__ static inline uint16_t from_f32(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
  }
};
struct F16 {
  using storage = uint16_t;
  static constexpr int code = FDP_F16;
  __device__ static inline float to_f32(uint16_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};

// Load one element of any storage dtype as fp32 / store fp32 into a dtype code.
__device__ inline float load_as_f32(const void* p, int64_t i, int dtype) {
  if (dtype == FDP_F32) return static_cast<const float*>(p)[i];
  uint16_t v = static_cast<const uint16_t*>(p)[i];
  return dtype == FDP_BF16 ? BF16::to_f32(v) : F16::to_f32(v);
}
__device__ inline void store_from_f32(void* p, int64_t i, int dtype, float v) {
  if (dtype == FDP_F32) {
    static_cast<float*>(p)[i] = v;
  } else {
    static_cast<uint16_t*>(p)[i] = dtype == FDP_BF16 ? BF16::from_f32(v) : F16::from_f32(v);
  }
}

// ------------------------------------------------------------ reductions
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// min(clamp, C / (n + 1e-10)) with the reference's epsilon
// (flashdp/core/clip_fn.py:6-8).
__device__ inline float clip_factor(float norm, float C, float clamp) {
  float c = C / (norm + 1e-10f);
  return c < clamp ? c : clamp;
}

}  // namespace fdp
