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

// Whether `extra + rows * ld` 16-bit elements fit one 32-bit buffer record
// (fewer than 2^31 bytes), with `rows` rounded up to 128, the deepest padding
// of a sample's rows in any tile: the padding rows' byte offsets (rows * ld * 2
// and up, which read as zeros past the record) then stay below 2^32 and cannot
// wrap back into it.  Every factor is bounded first, so the products cannot
// overflow for any caller-supplied size.
inline bool fits_record(int64_t rows, int64_t ld, int64_t extra = 0) {
  constexpr int64_t lim = int64_t(1) << 30;  // elements of 2 bytes
  if (rows < 0 || ld < 0 || extra < 0 || rows >= lim || ld >= lim || extra >= lim) return false;
  const int64_t padded = (rows + 127) / 128 * 128;
  return extra + padded * ld < lim;
}

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
  // lo | hi << 16, both rounded as from_f32, in one v_cvt_pk_bf16_f32
  __device__ static inline uint32_t pack2(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{lo, hi}), h2));
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
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return uint32_t(from_f32(lo)) | (uint32_t(from_f32(hi)) << 16);
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

// ------------------------------------------------------------ Gaussian noise
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC 2011): ten rounds, each multiplying counter words 0 and 2 by
// the round constants (32x32 -> 64 bits) and mixing the halves with the other
// words and the key; the key is bumped by the Weyl constants between rounds.
struct U32x4 {
  uint32_t w[4];
};
__device__ __forceinline__ U32x4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                               uint32_t k0, uint32_t k1) {
  constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
  constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += kW0;
      k1 += kW1;
    }
    // one v_mad_u64_u32 per product (both halves at once)
    const uint64_t p0 = static_cast<uint64_t>(kM0) * c0, p1 = static_cast<uint64_t>(kM1) * c2;
    const uint32_t lo0 = static_cast<uint32_t>(p0), hi0 = static_cast<uint32_t>(p0 >> 32);
    const uint32_t lo1 = static_cast<uint32_t>(p1), hi1 = static_cast<uint32_t>(p1 >> 32);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return U32x4{{c0, c1, c2, c3}};
}

// Box-Muller: r = sqrt(-2 ln u_a), (r cos 2 pi u_b, r sin 2 pi u_b), with the
// radius uniform u_a = (a + 1/2) 2^-32 built from the whole 32-bit word (its
// smallest value 2^-33 bounds |z| by sqrt(66 ln 2) = 6.76) and the angle
// uniform u_b = ((b >> 8) + 1/2) 2^-24.  v_log_f32 is log2; v_sin/v_cos_f32
// take their argument in revolutions.  (float)a rounds to nearest: for a
// within 128 of 2^32, u_a rounds to 1 and r to 0 instead of about 1e-5.
__device__ __forceinline__ void box_muller(uint32_t a, uint32_t b, float& z0, float& z1) {
  constexpr float kInv32 = 2.3283064365386963e-10f;   // 2^-32
  constexpr float kHalf32 = 1.16415321826934814e-10f;  // 2^-33
  constexpr float kInv24 = 5.9604644775390625e-08f;   // 2^-24
  const float ua = __builtin_fmaf(static_cast<float>(a), kInv32, kHalf32);
  const float ub = (static_cast<float>(b >> 8) + 0.5f) * kInv24;
  const float r = __builtin_sqrtf(-1.3862943611198906f * __builtin_amdgcn_logf(ua));  // -2 ln 2 log2
  z0 = r * __builtin_amdgcn_cosf(ub);
  z1 = r * __builtin_amdgcn_sinf(ub);
}

// Noise of one output: an injected tensor z (row-major, dtype `dtype`) or, when
// `draw`, the Philox stream of fdp_noise_key (counter block offset (+ *ctr) +
// e/4, counter word 2 = stream).  ctr: the key's device counter (read when the
// kernel runs; nullptr: none).
struct NoiseSrc {
  const void* z;
  int dtype;
  bool draw;
  uint32_t k0, k1, stream;
  uint64_t offset;
  const uint64_t* ctr;
  __device__ __forceinline__ bool on() const { return z != nullptr || draw; }
  // A copy with the device counter added to the offset (one read per copy:
  // kernels take it once for their main output).
  __device__ __forceinline__ NoiseSrc resolved() const {
    NoiseSrc n = *this;
    if (n.draw && n.ctr != nullptr) {
      n.offset += *n.ctr;
      n.ctr = nullptr;
    }
    return n;
  }
  __device__ __forceinline__ void block(int64_t q, float (&o)[4]) const {
    const uint64_t c = offset + (ctr != nullptr ? *ctr : 0ull) + static_cast<uint64_t>(q);
    const U32x4 r = philox4x32_10(static_cast<uint32_t>(c), static_cast<uint32_t>(c >> 32), stream,
                                  0u, k0, k1);
    box_muller(r.w[0], r.w[1], o[0], o[1]);
    box_muller(r.w[2], r.w[3], o[2], o[3]);
  }
  // z[e] (a single element)
  __device__ __forceinline__ float at(int64_t e) const;
  // z[e .. e+n-1] for any e: whole blocks around the window, then a select
  // network on e mod 4 (no dynamically indexed register arrays)
  template <int n>
  __device__ __forceinline__ void window(int64_t e, float (&o)[n]) const {
    static_assert(n % 4 == 0, "whole Philox blocks");
    float w[n + 4];
#pragma unroll
    for (int i = 0; i <= n / 4; ++i) {
      float b[4];
      block(e / 4 + i, b);
#pragma unroll
      for (int j = 0; j < 4; ++j) w[4 * i + j] = b[j];
    }
    const int sh = static_cast<int>(e & 3);
#pragma unroll
    for (int j = 0; j < n; ++j)
      o[j] = sh == 0 ? w[j] : sh == 1 ? w[j + 1] : sh == 2 ? w[j + 2] : w[j + 3];
  }
  // z[e .. e+n-1] for n a multiple of 4 and e a multiple of 4
  template <int n>
  __device__ __forceinline__ void run(int64_t e, float (&o)[n]) const {
    static_assert(n % 4 == 0, "whole Philox blocks");
#pragma unroll
    for (int i = 0; i < n / 4; ++i) {
      float b[4];
      block(e / 4 + i, b);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[4 * i + j] = b[j];
    }
  }
};

__device__ __forceinline__ float NoiseSrc::at(int64_t e) const {
  if (z != nullptr) return load_as_f32(z, e, dtype);
  float b[4];
  block(e / 4, b);
  const int j = static_cast<int>(e & 3);
  return j == 0 ? b[0] : j == 1 ? b[1] : j == 2 ? b[2] : b[3];
}

// How the E-element chunk at row-major index e (e % E == 0, whole chunk inside
// a row of length N) can be read: 2 = one 16-byte load of the injected
// tensor, 1 = whole Philox blocks, 0 = element by element, -1 = no noise.
template <int E>
__device__ __forceinline__ int noise_chunks(const NoiseSrc& nz, int64_t N) {
  if (!nz.on()) return -1;
  if (nz.z != nullptr)
    return (reinterpret_cast<uintptr_t>(nz.z) % 16 == 0 && N % (16 / (nz.dtype == FDP_F32 ? 4 : 2)) == 0 &&
            E == 16 / (nz.dtype == FDP_F32 ? 4 : 2))
               ? 2
               : 0;
  return N % 4 == 0 ? 1 : 0;
}
// v[j] += scale * z[e + j], j < E, read as noise_chunks() allows; the injected
// tensor has the output's storage type OT.
template <class OT, int E>
__device__ __forceinline__ void add_noise_chunk(const NoiseSrc& nz, int how, int64_t e, float scale,
                                                float (&v)[E]) {
  static_assert(E % 4 == 0, "16-byte chunks of 16- or 32-bit values");
  if (how < 0) return;
  if (how == 2) {
    using S = typename OT::storage;
    const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const S*>(nz.z) + e);
    const S* zs = reinterpret_cast<const S*>(&raw);
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] += scale * OT::to_f32(zs[j]);
  } else if (how == 1) {
    float z[E];
    nz.run(e, z);
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] += scale * z[j];
  } else {
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] += scale * nz.at(e + j);
  }
}

// Host side: the noise of output `stream` of a call.
inline NoiseSrc make_noise(const void* z, int dtype, const fdp_noise_key* key, uint32_t stream) {
  NoiseSrc n{};
  n.z = z;
  n.dtype = dtype;
  n.draw = z == nullptr && key != nullptr;
  n.stream = stream;
  if (key != nullptr) {
    n.k0 = static_cast<uint32_t>(key->seed);
    n.k1 = static_cast<uint32_t>(key->seed >> 32);
    n.offset = key->offset;
    n.ctr = key->counter;
  }
  return n;
}

// ------------------------------------------------------------ reductions
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// The same sum through DPP lane moves only (no LDS round trips): butterflies
// within each row of 16 lanes (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror), then row_bcast:15 and row_bcast:31 carry the row sums into
// lane 63, which is broadcast.  Every lane of the wavefront must be active.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf,
                                                        false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_add<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror
  v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
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

// Argument checks shared by fdp_wgrad_clip and fdp_wgrad_clip_noalloc (host
// only, touches no device): FDP_OK or the status the entry point returns.
int wgrad_check_args(const void* a, const void* b, int64_t B, int64_t K, int64_t M, int64_t N,
                     int64_t lda, int64_t ldb, int layout, int dtype, const void* out,
                     int64_t ldo, int out_dtype, const float* norms, int flags);

}  // namespace fdp
