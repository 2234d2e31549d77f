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
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;

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
  // round-to-nearest-even (gfx950's v_cvt_pk_bf16_f32), NaN stays NaN
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
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

// Device-coherent word access for values exchanged between workgroups that may
// sit on different XCDs (whose L2 caches are not coherent with each other):
// relaxed agent-scope atomics, ordered by wait_stores() and a ticket atomic.
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this wave's stores have completed.
__device__ __forceinline__ void wait_stores() {
  __builtin_amdgcn_s_waitcnt((0 & 0xf) | (0x7 << 4) | (0xf << 8));  // vmcnt(0)
}

constexpr int kCoherent = 0x10;               // buffer cache policy bit sc1: agent-coherent
constexpr uint32_t kRawBufferWord3 = 0x00020000u;  // raw buffer resource, 32-bit records

// 16-byte agent-coherent loads/stores of fp32 data through a buffer resource
// over [base, base + bytes) (bytes < 2^32; accesses past the end read zero
// and are not written).
struct CoherentSpan {
  __amdgpu_buffer_rsrc_t r;
  __device__ CoherentSpan(const float* base, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                            static_cast<int>(bytes), kRawBufferWord3)) {}
  __device__ f32x4 load4(uint32_t byte_off) const {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCoherent));
  }
  __device__ void store4(uint32_t byte_off, f32x4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, kCoherent);
  }
};

}  // namespace fdp
