// Bandwidth-bound per-sample kernels on gfx950: clipped column sums (bias
// gradients, LayerNorm gamma/beta gradients) and the LayerNorm forward/backward.
//
// Reference math:
//   bias:      flashdp/core/linear_clip.py:116-123 (norm of the flattened g_b,
//              mean over B*T of the clipped g)
//   LN dw/db:  flashdp/core/layernorm_clip.py:163-198 (per-sample sums over T,
//              norm, clip, mean over B)
//   LN fwd:    flashdp/core/layernorm_clip.py:26-60 (mean, biased variance,
//              rstd = 1/sqrt(var+eps), y = x_hat*w + b)
//   LN dx:     flashdp/core/layernorm_clip.py:98-107
//
// All reductions are fixed-order (no float atomics): the row kernel writes
// per-(sample, row-chunk) partial vectors to the workspace, chunk_sum_block
// adds each sample's chunks in chunk order (and the squares for the norm), and
// combine_block derives the clip factors and adds the clipped samples in
// sample order into the output -- in two launches (chunk_sum_kernel,
// combine_kernel), or in one (reduce_kernel) when the per-stream sums are
// small.  Rows are read with 16-byte loads, one
// wavefront per row for the LayerNorm kernels (row statistics are wavefront
// shuffles, no LDS), 64..256 threads across the columns for the column sums.
#include <atomic>
#include <type_traits>
#include <chrono>

#include "fdp_common.hpp"
#include "host_cache.hpp"

namespace fdp {
namespace rw {

constexpr int NT = 256;

// ------------------------------------------------------------ row access
template <class DT, int VEC>
struct Vec;
template <class DT>
struct Vec<DT, 1> {
  using S = typename DT::storage;
  __device__ static inline void load(const S* p, float* o) { o[0] = DT::to_f32(p[0]); }
  __device__ static inline void store(S* p, const float* v) { p[0] = DT::from_f32(v[0]); }
};
template <class DT>
struct Vec<DT, 8> {  // 8 x 16-bit = 16 bytes
  __device__ static inline void load(const uint16_t* p, float* o) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = DT::to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
      o[2 * j + 1] = DT::to_f32(static_cast<uint16_t>(w[j] >> 16));
    }
  }
  __device__ static inline void store(uint16_t* p, const float* v) {
    uint4 o;
    o.x = DT::from_f32(v[0]) | (uint32_t(DT::from_f32(v[1])) << 16);
    o.y = DT::from_f32(v[2]) | (uint32_t(DT::from_f32(v[3])) << 16);
    o.z = DT::from_f32(v[4]) | (uint32_t(DT::from_f32(v[5])) << 16);
    o.w = DT::from_f32(v[6]) | (uint32_t(DT::from_f32(v[7])) << 16);
    *reinterpret_cast<uint4*>(p) = o;
  }
};
template <>
struct Vec<F32, 4> {  // 4 x fp32 = 16 bytes
  __device__ static inline void load(const float* p, float* o) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
    o[3] = v.w;
  }
  __device__ static inline void store(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

// Element e of thread `lane` in a row handled by LANES threads (one
// wavefront, or LANES/64 wavefronts sharing a long row): vector
// v = lane + LANES*i covers elements v*VEC .. v*VEC+VEC-1.
template <int EPL, int VEC, int LANES = 64>
__device__ __forceinline__ int wave_elem(int lane, int i) {
  return (lane + LANES * i) * VEC;  // < 2^31: a row (or a long row's segment) holds <= 16384
}

// LDS position of element e of a wave's row in the LayerNorm backward fold.
// A lane parks 8 consecutive elements, 32 bytes from the next lane's, so each
// group of 8 is XOR-permuted by its lane's bits 3..5: every store of one
// element per lane then covers the 64 banks once, and the fold's reads of 64
// consecutive elements stay a permutation of one 64-float span.
__host__ __device__ __forceinline__ int64_t fold_pos(int64_t e) {
  return (e & ~int64_t(7)) | ((e & 7) ^ ((e >> 6) & 7));
}
// Floats per wave slice: the row rounded up to whole 128-float blocks, so that
// every permuted group of 8 stays inside the slice.
__host__ __device__ __forceinline__ int64_t fold_slice(int64_t H) { return (H + 127) / 128 * 128; }

// Parameter vectors (gamma/beta) in an arbitrary dtype, default `dflt` if NULL.
// One uniform branch on the dtype, then straight-line loads: all EPL loads are
// in flight together (a per-element dtype switch made each load wait for the
// previous one, EPL round trips at every workgroup's start).
template <int EPL, int VEC, int LANES, class S, class Cvt>
__device__ inline void load_param_as(const S* p, int64_t H, int lane, Cvt cvt, float (&o)[EPL]) {
  S raw[EPL];
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e = wave_elem<EPL, VEC, LANES>(lane, i) + j;
      const S v = p[e < static_cast<int>(H) ? e : 0];  // clamped: no branch around the load
      raw[i * VEC + j] = e < static_cast<int>(H) ? v : S(0);
    }
#pragma unroll
  for (int k = 0; k < EPL; ++k) o[k] = cvt(raw[k]);
}
template <int EPL, int VEC, int LANES = 64>
__device__ inline void load_param(const void* p, int dtype, int64_t H, int lane, float dflt,
                                  float (&o)[EPL]) {
  if (p == nullptr) {
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        o[i * VEC + j] = wave_elem<EPL, VEC, LANES>(lane, i) + j < static_cast<int>(H) ? dflt : 0.f;
  } else if (dtype == FDP_F32) {
    load_param_as<EPL, VEC, LANES>(static_cast<const float*>(p), H, lane,
                                   [](float v) { return v; }, o);
  } else if (dtype == FDP_BF16) {
    load_param_as<EPL, VEC, LANES>(static_cast<const uint16_t*>(p), H, lane,
                                   [](uint16_t v) { return BF16::to_f32(v); }, o);
  } else {
    load_param_as<EPL, VEC, LANES>(static_cast<const uint16_t*>(p), H, lane,
                                   [](uint16_t v) { return F16::to_f32(v); }, o);
  }
}

// ========================================================== column sums
// grid (col_blocks, chunks, B); thread owns VEC consecutive columns of one
// 16-byte vector and walks `rows` rows of one sample.  Writes the chunk's
// partial column sums partials[b][chunk][h] and, for FDP_NORM_FROB, the
// workgroup's sum of u^2 to frob[b][chunk * col_blocks + col_block].
// Workgroup (0,0,0) zeroes the reduction's ticket.
template <class DT, int VEC>
__global__ __launch_bounds__(NT) void colsum_kernel(const typename DT::storage* u,
                                                    const typename DT::storage* v, int64_t T,
                                                    int64_t H, int64_t rows, int chunks,
                                                    float* partials, float* frob,
                                                    unsigned* tickets) {
  __shared__ float red[NT / kWave];
  if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0)
    __hip_atomic_store(tickets, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int64_t b = blockIdx.z;
  const int chunk = blockIdx.y;
  const int64_t vi = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t h = vi * VEC;
  const int64_t t0 = int64_t(chunk) * rows;
  const int64_t t1 = t0 + rows < T ? t0 + rows : T;
  float acc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) acc[j] = 0.f;
  float sq = 0.f;
  if (h < H) {
    const typename DT::storage* pu = u + (b * T + t0) * H + h;
    const typename DT::storage* pv = v ? v + (b * T + t0) * H + h : nullptr;
    int64_t t = t0;
    for (; t + 4 <= t1; t += 4) {
      float x[4][VEC], y[4][VEC];
#pragma unroll
      for (int r = 0; r < 4; ++r) Vec<DT, VEC>::load(pu + r * H, x[r]);
      if (pv) {
#pragma unroll
        for (int r = 0; r < 4; ++r) Vec<DT, VEC>::load(pv + r * H, y[r]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          sq += x[r][j] * x[r][j];
          acc[j] += pv ? x[r][j] * y[r][j] : x[r][j];
        }
      pu += 4 * H;
      if (pv) pv += 4 * H;
    }
    for (; t < t1; ++t) {
      float x[VEC], y[VEC];
      Vec<DT, VEC>::load(pu, x);
      if (pv) Vec<DT, VEC>::load(pv, y);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        sq += x[j] * x[j];
        acc[j] += pv ? x[j] * y[j] : x[j];
      }
      pu += H;
      if (pv) pv += H;
    }
    float* dst = partials + (b * chunks + chunk) * H + h;
#pragma unroll
    for (int j = 0; j < VEC; ++j) dst[j] = acc[j];
  }
  if (frob) {
    sq = wave_sum(sq);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int w = 0; w < int(blockDim.x >> 6); ++w) t += red[w];
      frob[(b * chunks + chunk) * gridDim.x + blockIdx.x] = t;
    }
  }
}

// ====================================================== per-sample reductions
// Items: 4 consecutive columns (V4, H % 4 == 0) or one column.  A workgroup
// takes 64 items of one stream; its four waves each sum one contiguous quarter
// of the chunks (loads in flight together, additions in chunk order) and the
// quarters are added in order through LDS: fixed order, no atomics.
template <bool V4>
struct Item {
  static constexpr int W = V4 ? 4 : 1;
  f32x4 v;
  __device__ void zero() { v = f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ void load(const float* p) {
    if constexpr (V4) v = *reinterpret_cast<const f32x4*>(p);
    else v = f32x4{p[0], 0.f, 0.f, 0.f};
  }
  __device__ void store(float* p) const {
    if constexpr (V4) *reinterpret_cast<f32x4*>(p) = v;
    else p[0] = v[0];
  }
  __device__ float sq() const {
    return (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
  }
};

constexpr int kItemsPerBlock = 64;

// Loads and stores of the per-sample sums: element `off` of the region at
// `base` (uniform across the workgroup; `bytes` long, < 2^32).  COH:
// agent-coherent (sc1) accesses, for values exchanged between workgroups of
// one launch that may sit on different XCDs; otherwise plain ones (values from
// an earlier launch).
template <bool V4, bool COH>
__device__ __forceinline__ f32x4 ld_item(const float* base, int64_t off, uint32_t bytes) {
  if constexpr (COH) {
    if constexpr (V4) return CoherentSpan(base, bytes).load4(static_cast<uint32_t>(off * 4));
    else return f32x4{ld_coherent(base + off), 0.f, 0.f, 0.f};
  } else {
    if constexpr (V4) return *reinterpret_cast<const f32x4*>(base + off);
    else return f32x4{base[off], 0.f, 0.f, 0.f};
  }
}
template <bool V4, bool COH>
__device__ __forceinline__ void st_item(float* base, int64_t off, uint32_t bytes, f32x4 v) {
  if constexpr (COH) {
    if constexpr (V4) CoherentSpan(base, bytes).store4(static_cast<uint32_t>(off * 4), v);
    else st_coherent(base + off, v[0]);
  } else {
    if constexpr (V4) *reinterpret_cast<f32x4*>(base + off) = v;
    else base[off] = v[0];
  }
}
template <bool COH>
__device__ __forceinline__ float ld_word(const float* p) {
  if constexpr (COH) return ld_coherent(p);
  else return *p;
}

// Item block ib of stream s: sums[s][h] = sum_c partials[s][c][h];
// sq_part[s][ib] = sum of squares of this block's sums.
template <bool V4, bool COH>
__device__ inline void chunk_sum_block(const float* partials, int64_t H, int chunks, float* sums,
                                       float* sq_part, int64_t s, int ib, int nib) {
  __shared__ f32x4 grp[NT / kWave][kItemsPerBlock];
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t items = (H + Item<V4>::W - 1) / Item<V4>::W;
  const int64_t it = int64_t(ib) * kItemsPerBlock + lane;
  const int per = (chunks + NT / kWave - 1) / (NT / kWave);
  const int c0 = g * per < chunks ? g * per : chunks;
  const int c1 = c0 + per < chunks ? c0 + per : chunks;
  Item<V4> acc;
  acc.zero();
  if (it < items) {
    const float* src = partials + s * chunks * H + it * Item<V4>::W;
    // batches of 8 chunks, the last one masked: its loads are in flight together
    for (int c = c0; c < c1; c += 8) {
      Item<V4> x[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (c + q < c1) x[q].load(src + int64_t(c + q) * H);
        else x[q].zero();
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (c + q < c1) acc.v += x[q].v;
    }
  }
  grp[g][lane] = acc.v;
  __syncthreads();
  if (g == 0) {
    Item<V4> tot;
    tot.v = ((grp[0][lane] + grp[1][lane]) + grp[2][lane]) + grp[3][lane];
    float q = 0.f;
    if (it < items) {
      st_item<V4, COH>(sums + s * H, it * Item<V4>::W, static_cast<uint32_t>(H * 4), tot.v);
      q = tot.sq();
    }
    q = wave_sum(q);
    if (lane == 0) {
      if constexpr (COH) st_coherent(sq_part + s * nib + ib, q);
      else sq_part[s * nib + ib] = q;
    }
  }
}

// grid (item_blocks, S): chunk_sum_block of every (stream, item block).
template <bool V4>
__global__ __launch_bounds__(NT) void chunk_sum_kernel(const float* partials, int64_t H,
                                                       int chunks, float* sums, float* sq_part) {
  chunk_sum_block<V4, false>(partials, H, chunks, sums, sq_part, blockIdx.y, blockIdx.x,
                             gridDim.x);
}

constexpr int kFacChunk = 1024;  // clip factors staged in LDS per pass

// What the clipped sum of stream k needs besides the sums.
struct CombineArgs {
  const float* parts;  // per-sample norm parts [S][nparts]
  int nparts;
  int64_t B, H;
  float C, clamp;
  const float* clip_args_dev;
  float out_scale;
  NoiseSrc noise0, noise1;
  float noise_scale;
  void* out0;
  void* out1;
  int out_dtype;
  float* norms;
  float* factors;
};

// Item block ib of stream k: the clip factors c_{k,b} from the norm parts
// (nparts per sample, summed in order), then
//   out_k[h] = out_scale * sum_b c_{k,b} sums[k*B+b][h] + noise_scale * noise_k[h]
// with the four waves each taking a contiguous quarter of the samples, added
// in order.  write_stats: also write norms / factors.
template <bool V4, bool COH>
__device__ inline void combine_block(const float* sums, const CombineArgs& a, int k, int ib,
                                     bool write_stats) {
  __shared__ float fac[kFacChunk];
  __shared__ f32x4 grp[NT / kWave][kItemsPerBlock];
  float C = a.C, clamp = a.clamp;
  if (a.clip_args_dev != nullptr) {
    C = a.clip_args_dev[0];
    clamp = a.clip_args_dev[1];
  }
  const int64_t B = a.B, H = a.H;
  void* out = k == 0 ? a.out0 : a.out1;
  const NoiseSrc noise = k == 0 ? a.noise0 : a.noise1;
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t items = (H + Item<V4>::W - 1) / Item<V4>::W;
  const int64_t it = int64_t(ib) * kItemsPerBlock + lane;
  const int64_t per = (B + NT / kWave - 1) / (NT / kWave);
  const int64_t g0 = g * per < B ? g * per : B;
  const int64_t g1 = g0 + per < B ? g0 + per : B;
  Item<V4> acc;
  acc.zero();
  for (int64_t bc = 0; bc < B; bc += kFacChunk) {
    const int64_t nb = B - bc < kFacChunk ? B - bc : kFacChunk;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < nb; i += NT) {
      const int64_t s = k * B + bc + i;
      const float* src = a.parts + s * a.nparts;
      float q = 0.f;
      int j = 0;
      for (; j + 4 <= a.nparts; j += 4) {
        const float a0 = ld_word<COH>(src + j), a1 = ld_word<COH>(src + j + 1);
        const float a2 = ld_word<COH>(src + j + 2), a3 = ld_word<COH>(src + j + 3);
        q = (((q + a0) + a1) + a2) + a3;
      }
      for (; j < a.nparts; ++j) q += ld_word<COH>(src + j);
      const float n = sqrtf(q);
      const float c = clip_factor(n, C, clamp);
      fac[i] = c;
      if (write_stats) {
        if (a.norms) a.norms[s] = n;
        if (a.factors) a.factors[s] = c;
      }
    }
    __syncthreads();
    if (out != nullptr && it < items) {
      const int64_t lo = g0 > bc ? g0 : bc;
      const int64_t hi = g1 < bc + nb ? g1 : bc + nb;
      // the stream's sums: [B][H] at base (B * H * 4 bytes < 2^32 where COH)
      const float* base = sums + (k * B) * H;
      const uint32_t bytes = static_cast<uint32_t>(COH ? B * H * 4 : 0);
      const int64_t col = it * Item<V4>::W;
      int64_t b = lo;
      for (; b + 8 <= hi; b += 8) {
        f32x4 x[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = ld_item<V4, COH>(base, (b + q) * H + col, bytes);
#pragma unroll
        for (int q = 0; q < 8; ++q) acc.v += fac[b + q - bc] * x[q];
      }
      for (; b < hi; ++b) acc.v += fac[b - bc] * ld_item<V4, COH>(base, b * H + col, bytes);
    }
  }
  if (out == nullptr) return;
  grp[g][lane] = acc.v;
  __syncthreads();
  if (g == 0 && it < items) {
    const f32x4 tot = ((grp[0][lane] + grp[1][lane]) + grp[2][lane]) + grp[3][lane];
    constexpr int W = Item<V4>::W;
    float z[4] = {0.f, 0.f, 0.f, 0.f};
    if (noise.z != nullptr) {
#pragma unroll
      for (int e = 0; e < W; ++e)
        if (it * W + e < H) z[e] = noise.at(it * W + e);
    } else if (noise.draw) {
      noise.window(it * W, z);
    }
#pragma unroll
    for (int e = 0; e < W; ++e) {
      const int64_t h = it * W + e;
      if (h < H) store_from_f32(out, h, a.out_dtype, tot[e] * a.out_scale + a.noise_scale * z[e]);
    }
  }
}

// grid (item_blocks, nstreams): combine_block of every (stream, item block);
// workgroup 0 of each stream writes norms / factors.
template <bool V4>
__global__ __launch_bounds__(NT) void combine_kernel(const float* sums, CombineArgs a) {
  combine_block<V4, false>(sums, a, blockIdx.y, blockIdx.x, blockIdx.x == 0);
}

// The clipped sum of stream k by one workgroup: every thread takes whole items
// and adds the samples in sample order, 16 loads in flight at a time (a fixed
// order, not combine_block's quarters).  B <= kFacChunk.  Reads agent-coherent
// sums and parts.
template <bool V4>
__device__ inline void combine_stream(const float* sums, const CombineArgs& a, int k) {
  __shared__ float fac[kFacChunk];
  float C = a.C, clamp = a.clamp;
  if (a.clip_args_dev != nullptr) {
    C = a.clip_args_dev[0];
    clamp = a.clip_args_dev[1];
  }
  const int64_t B = a.B, H = a.H;
  void* out = k == 0 ? a.out0 : a.out1;
  constexpr int W = Item<V4>::W;
  const int64_t items = (H + W - 1) / W;
  const float* base = sums + (k * B) * H;
  const uint32_t bytes = static_cast<uint32_t>(B * H * 4);
  // the first batch of this thread's first item is loaded before the factors
  // are formed: the two round trips overlap
  f32x4 x[16];
  const bool pre = out != nullptr && static_cast<int64_t>(threadIdx.x) < items;
  if (pre) {
#pragma unroll
    for (int q = 0; q < 16; ++q)
      x[q] = q < B ? ld_item<V4, true>(base, q * H + int64_t(threadIdx.x) * W, bytes)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int64_t i = threadIdx.x; i < B; i += NT) {
    const int64_t s = k * B + i;
    const float* src = a.parts + s * a.nparts;
    float q = 0.f;
    int j = 0;
    for (; j + 4 <= a.nparts; j += 4) {
      const float a0 = ld_coherent(src + j), a1 = ld_coherent(src + j + 1);
      const float a2 = ld_coherent(src + j + 2), a3 = ld_coherent(src + j + 3);
      q = (((q + a0) + a1) + a2) + a3;
    }
    for (; j < a.nparts; ++j) q += ld_coherent(src + j);
    const float n = sqrtf(q);
    const float c = clip_factor(n, C, clamp);
    fac[i] = c;
    if (a.norms) a.norms[s] = n;
    if (a.factors) a.factors[s] = c;
  }
  __syncthreads();
  if (out == nullptr) return;
  const NoiseSrc noise = k == 0 ? a.noise0 : a.noise1;
  for (int64_t it = threadIdx.x; it < items; it += NT) {
    const int64_t col = it * W;
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int64_t b = 0; b < B; b += 16) {
      if (b > 0 || it != static_cast<int64_t>(threadIdx.x)) {
#pragma unroll
        for (int q = 0; q < 16; ++q)
          x[q] = b + q < B ? ld_item<V4, true>(base, (b + q) * H + col, bytes)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int q = 0; q < 16; ++q)
        if (b + q < B) tot += fac[b + q] * x[q];
    }
    float z[4] = {0.f, 0.f, 0.f, 0.f};
    if (noise.z != nullptr) {
#pragma unroll
      for (int e = 0; e < W; ++e)
        if (col + e < H) z[e] = noise.at(col + e);
    } else if (noise.draw) {
      noise.window(col, z);
    }
#pragma unroll
    for (int e = 0; e < W; ++e)
      if (col + e < H)
        store_from_f32(out, col + e, a.out_dtype, tot[e] * a.out_scale + a.noise_scale * z[e]);
  }
}

// Both steps in one launch, for small per-stream sums: grid (item_blocks, S)
// runs chunk_sum_block, and the last workgroup of stream k to finish (a ticket
// per stream, zeroed by the row kernel that wrote the partials) runs
// combine_stream.  The sums and squares it reads are agent-coherent; every
// workgroup's stores have completed before it takes its ticket.
template <bool V4>
__global__ __launch_bounds__(NT) void reduce_kernel(const float* partials, int chunks,
                                                    float* sums, float* sq_part,
                                                    unsigned* tickets, CombineArgs a) {
  __shared__ int last;
  const int64_t s = blockIdx.y;
  const int k = static_cast<int>(s / a.B);
  chunk_sum_block<V4, true>(partials, a.H, chunks, sums, sq_part, s, blockIdx.x, gridDim.x);
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned n = static_cast<unsigned>(a.B) * gridDim.x;
    const unsigned old =
        __hip_atomic_fetch_add(tickets + k, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old + 1 == n;
  }
  __syncthreads();
  if (last) combine_stream<V4>(sums, a, k);
}

// ================================================================= LayerNorm
constexpr int kLnThreads = 512;  // forward: 8 wavefronts, one row each at a time
// Backward: rows in flight per row group.  On cfg4 (16x1024x1024 bf16, one
// launch) 1, 2 and 4 measured 27.5, 28.2 and 29.8 us per call.
constexpr int kLnLookahead = 1;

// Row I/O goes through a raw buffer resource over the row's bytes: accesses
// past the end read zero and are dropped, so loads and stores need no branch.
// (With a branch around each load or store the compiler could not count the
// memory operations in flight at the loop's back edge and waited for all of
// them -- the next row's prefetch included -- at every row.)
// A value known to be the same in every lane of the wavefront, read from the
// first lane (so it lives in scalar registers and feeds scalar loads).
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Every caller's row and range are the same across the wavefront: reading
// them from the first lane puts the resource in scalar registers (otherwise
// the compiler loops over the lanes' values around every access).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* row, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(row);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  void* base = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(base, static_cast<short>(0),
                                           static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)),
                                           kRawBufferWord3);
}

// Raw (undecoded) row fragment of one thread: lets the next row's loads be in
// flight while the current row is processed.  `on` false issues the loads
// against a zero-length range: they read zero and touch no memory.
template <class DT, int EPL, int VEC, int LANES = 64>
struct RawRow;
template <class DT, int EPL, int LANES>
struct RawRow<DT, EPL, 8, LANES> {  // 16-bit, 16-byte vectors
  u32x4 q[EPL / 8];
  // hides the held bytes from the optimiser, so that a later decode is
  // recomputed instead of an earlier one being kept live
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int i = 0; i < EPL / 8; ++i) __asm__ volatile("" : "+v"(q[i]));
  }
  __device__ __forceinline__ void load(const uint16_t* row, int64_t H, int lane, bool on = true) {
    const auto r = row_rsrc(row, on ? static_cast<uint32_t>(H * 2) : 0u);
#pragma unroll
    for (int i = 0; i < EPL / 8; ++i)
      q[i] = __builtin_amdgcn_raw_buffer_load_b128(r, wave_elem<EPL, 8, LANES>(lane, i) * 2, 0, 0);
  }
  __device__ __forceinline__ void decode(float (&o)[EPL]) const {
#pragma unroll
    for (int i = 0; i < EPL / 8; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[i * 8 + 2 * j] = DT::to_f32(static_cast<uint16_t>(q[i][j] & 0xffffu));
        o[i * 8 + 2 * j + 1] = DT::to_f32(static_cast<uint16_t>(q[i][j] >> 16));
      }
    }
  }
};
template <int EPL, int LANES>
struct RawRow<F32, EPL, 4, LANES> {  // fp32, 16-byte vectors
  u32x4 q[EPL / 4];
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int i = 0; i < EPL / 4; ++i) __asm__ volatile("" : "+v"(q[i]));
  }
  __device__ __forceinline__ void load(const float* row, int64_t H, int lane, bool on = true) {
    const auto r = row_rsrc(row, on ? static_cast<uint32_t>(H * 4) : 0u);
#pragma unroll
    for (int i = 0; i < EPL / 4; ++i)
      q[i] = __builtin_amdgcn_raw_buffer_load_b128(r, wave_elem<EPL, 4, LANES>(lane, i) * 4, 0, 0);
  }
  __device__ __forceinline__ void decode(float (&o)[EPL]) const {
#pragma unroll
    for (int i = 0; i < EPL / 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) o[4 * i + j] = __uint_as_float(q[i][j]);
  }
};
template <class DT, int EPL, int LANES>
struct RawRow<DT, EPL, 1, LANES> {  // any dtype, element loads (unaligned rows)
  uint32_t q[EPL];
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int i = 0; i < EPL; ++i) __asm__ volatile("" : "+v"(q[i]));
  }
  __device__ __forceinline__ void load(const typename DT::storage* row, int64_t H, int lane,
                                      bool on = true) {
    constexpr int ES = sizeof(typename DT::storage);
    const auto r = row_rsrc(row, on ? static_cast<uint32_t>(H * ES) : 0u);
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int off = wave_elem<EPL, 1, LANES>(lane, i) * ES;
      if constexpr (ES == 4) q[i] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
      else q[i] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    }
  }
  __device__ __forceinline__ void decode(float (&o)[EPL]) const {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      if constexpr (sizeof(typename DT::storage) == 4) o[i] = __uint_as_float(q[i]);
      else o[i] = DT::to_f32(static_cast<uint16_t>(q[i]));
    }
  }
};

// Row store: `on` false drops the whole row (a zero-length resource).
template <class DT, int EPL, int VEC, int LANES = 64>
__device__ inline void store_row(typename DT::storage* row, int64_t H, int lane,
                                 const float (&v)[EPL], bool on = true) {
  constexpr int ES = sizeof(typename DT::storage);
  const auto r = row_rsrc(row, on ? static_cast<uint32_t>(H * ES) : 0u);
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i) {
    const int off = wave_elem<EPL, VEC, LANES>(lane, i) * ES;
    if constexpr (VEC == 8) {  // 16-bit
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = DT::pack2(v[i * 8 + 2 * j], v[i * 8 + 2 * j + 1]);
      __builtin_amdgcn_raw_buffer_store_b128(o, r, off, 0, 0);
    } else if constexpr (VEC == 4) {  // fp32
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = __float_as_uint(v[i * 4 + j]);
      __builtin_amdgcn_raw_buffer_store_b128(o, r, off, 0, 0);
    } else if constexpr (ES == 4) {
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[i]), r, off, 0, 0);
    } else {
      __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(DT::from_f32(v[i])), r, off, 0,
                                            0);
    }
  }
}

// One wavefront per row, rows dealt grid-stride to the wavefronts, the next
// row's loads issued before the current row is normalised.
template <class DT, int EPL, int VEC>
__global__ __launch_bounds__(kLnThreads) void ln_fwd_kernel(const typename DT::storage* x,
                                                            const void* w, const void* bias,
                                                            int w_dtype, int64_t rows, int64_t H,
                                                            float eps, typename DT::storage* y,
                                                            float* mean, float* rstd) {
  constexpr int W = kLnThreads / kWave;
  const int lane = threadIdx.x & 63;
  const int64_t wid = int64_t(blockIdx.x) * W + (threadIdx.x >> 6);
  const int64_t nw = int64_t(gridDim.x) * W;
  float wv[EPL], bv[EPL];
  load_param<EPL, VEC>(w, w_dtype, H, lane, 1.f, wv);
  load_param<EPL, VEC>(bias, w_dtype, H, lane, 0.f, bv);
  const float inv_h = 1.f / static_cast<float>(H);
  RawRow<DT, EPL, VEC> rx;
  rx.load(x + (wid < rows ? wid : 0) * H, H, lane, wid < rows);
  for (int64_t r = wid; r < rows; r += nw) {
    float xv[EPL];
    rx.decode(xv);
    const bool more = r + nw < rows;
    rx.load(x + (more ? r + nw : r) * H, H, lane, more);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) s += xv[i];
    const float mu = wave_sum_dpp(s) * inv_h;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float d = wave_elem<EPL, VEC>(lane, i) + j < static_cast<int>(H) ? xv[i * VEC + j] - mu : 0.f;
        q += d * d;
      }
    const float var = wave_sum_dpp(q) * inv_h;
    const float rs = 1.f / sqrtf(var + eps);
    float yv[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) yv[i] = (xv[i] - mu) * rs * wv[i] + bv[i];
    store_row<DT, EPL, VEC>(y + r * H, H, lane, yv);
    if (lane == 0) {
      if (mean) mean[r] = mu;
      if (rstd) rstd[r] = rs;
    }
  }
}

// One (chunk, sample) workgroup of the LayerNorm backward.  Rows are shared by
// NWR wavefronts (L = 64*NWR threads, EPL elements each); the workgroup's
// G = NTH/L row groups take rows t = t0 + g, t0 + g + G, ... < t1 of sample b,
// with the next row's x / dy / mean / rstd loads in flight while the current
// row is processed: writes dx and accumulates P = sum dy*x_hat, Q = sum dy in
// registers.  With NWR > 1 a row's two sums are wavefront sums added in
// wavefront order through LDS (double-buffered by parity; every thread runs
// the same trip count, so the barrier is uniform).  The G row groups are then
// folded in order through LDS (`lds`: G * fold_slice(H) floats), and
// put(0, e, P_e) / put(1, e, Q_e) receives the chunk's sums.
template <class DT, int EPL, int VEC, int NTH, int NWR, int LA, class Put>
__device__ inline void ln_bwd_chunk(const typename DT::storage* dy,
                                    const typename DT::storage* x, const void* w, int w_dtype,
                                    const float* mean, const float* rstd, int64_t T, int64_t H,
                                    int64_t b, int64_t t0, int64_t t1,
                                    typename DT::storage* dx, float* lds, Put put) {
  constexpr int L = NWR * kWave;
  constexpr int G = NTH / L;
  static_assert(G >= 1 && G * L == NTH, "whole row groups");
  __shared__ float red[2][G][NWR][2];
  const int lid = threadIdx.x % L, g = threadIdx.x / L;
  const int lane = threadIdx.x & 63, wig = lid >> 6;
  float wv[EPL];
  load_param<EPL, VEC, L>(w, w_dtype, H, lid, 1.f, wv);
  float P[EPL], Q[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    P[i] = 0.f;
    Q[i] = 0.f;
  }
  const float inv_h = 1.f / static_cast<float>(H);
  // LA rows per row group are in flight: the loop is unrolled by LA with one
  // register slot per row (a slot is refilled right after it is decoded, so no
  // registers are copied across iterations), and every group runs the same
  // number of iterations, padded to a multiple of LA.  Rows past t1 are loaded
  // against zero-length ranges (no memory touched) with the statistics of row
  // t0, and their dx stores are dropped: no branch around any load or store,
  // so the compiler can count the memory operations in flight.  An empty
  // chunk (T = 0) touches no row and no statistic.
  if (t1 > t0) {
    RawRow<DT, EPL, VEC, L> rx[LA], rg[LA];
    float mu_n[LA], rs_n[LA];
    const int64_t base = b * T;
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int64_t t = t0 + g + int64_t(j) * G;
      const bool on = t < t1;
      const int64_t row = uniform_i64(base + (on ? t : t0));
      rx[j].load(x + row * H, H, lid, on);
      rg[j].load(dy + row * H, H, lid, on);
      mu_n[j] = mean[row];
      rs_n[j] = rstd[row];
    }
    const int64_t trips = (t1 - t0 + G - 1) / G;
    const int64_t padded = (trips + LA - 1) / LA * LA;
    for (int64_t it = 0; it < padded; it += LA) {
#pragma unroll
      for (int j = 0; j < LA; ++j) {
        const int64_t t = t0 + g + (it + j) * G;
        const bool valid = t < t1;  // uniform within a row group
        const int par = static_cast<int>((it + j) & 1);  // consecutive rows alternate
        const int64_t r = uniform_i64(base + (valid ? t : t0));
        float xv[EPL], gv[EPL];
        rx[j].decode(xv);
        rg[j].decode(gv);
        const float mu = mu_n[j], rs = rs_n[j];
        const int64_t tn = t + int64_t(LA) * G;
        const bool more = tn < t1;
        const int64_t rn = uniform_i64(base + (more ? tn : t0));
        rx[j].load(x + rn * H, H, lid, more);
        rg[j].load(dy + rn * H, H, lid, more);
        mu_n[j] = mean[rn];
        rs_n[j] = rstd[rn];
        // Elements past H read dy = 0 and w = 0 (x_hat stays finite), so they
        // add nothing to s1, s2, P and Q, and their dx stores are dropped: no
        // per-element range test.  Rows past t1 read zeros and skip the sums.
        float s1 = 0.f, s2 = 0.f;
        float wdy[EPL];
#pragma unroll
        for (int k = 0; k < EPL; ++k) {
          xv[k] = (xv[k] - mu) * rs;  // x_hat
          wdy[k] = wv[k] * gv[k];
        }
        if (valid) {
#pragma unroll
          for (int k = 0; k < EPL; ++k) {
            s1 = fmaf(xv[k], wdy[k], s1);
            s2 += wdy[k];
            P[k] = fmaf(gv[k], xv[k], P[k]);
            Q[k] += gv[k];
          }
          s1 = wave_sum_dpp(s1);
          s2 = wave_sum_dpp(s2);
        }
        if constexpr (NWR > 1) {
          if (lane == 0) {
            red[par][g][wig][0] = s1;
            red[par][g][wig][1] = s2;
          }
          __syncthreads();
          s1 = 0.f;
          s2 = 0.f;
#pragma unroll
          for (int q = 0; q < NWR; ++q) {
            s1 += red[par][g][q][0];
            s2 += red[par][g][q][1];
          }
        }
        // dx = rs (w dy - x_hat c1 - c2), c1 = s1 / H, c2 = s2 / H
        const float b1 = -rs * (s1 * inv_h), b2 = -rs * (s2 * inv_h);
#pragma unroll
        for (int k = 0; k < EPL; ++k) gv[k] = fmaf(rs, wdy[k], fmaf(xv[k], b1, b2));
        store_row<DT, EPL, VEC, L>(dx + r * H, H, lid, gv, valid);
      }
    }
  }
  // Fold the row groups in order 0..G-1: every group parks its P (then Q) in
  // its own LDS slice (fold_slice(H) floats, element e at fold_pos(e)), and all
  // threads sum the slices element-wise.
  const int64_t slice = fold_slice(H);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    float* mine = lds + g * slice;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int e = wave_elem<EPL, VEC, L>(lid, i) + j;
        if (e < H) mine[fold_pos(e)] = half == 0 ? P[i * VEC + j] : Q[i * VEC + j];
      }
    __syncthreads();
    for (int64_t e = threadIdx.x; e < H; e += NTH) {
      const int64_t at = fold_pos(e);
      float v = lds[at];
#pragma unroll
      for (int gg = 1; gg < G; ++gg) v += lds[gg * slice + at];
      put(half, e, v);
    }
    __syncthreads();
  }
}

// grid (chunks, B): ln_bwd_chunk of every (chunk, sample), the chunk's sums
// written as partials (stream b: P, stream B+b: Q).  Workgroup (0,0) zeroes
// the reduction's two tickets.
template <class DT, int EPL, int VEC, int NTH, int NWR>
__global__ __launch_bounds__(NTH) void ln_bwd_kernel(const typename DT::storage* dy,
                                                    const typename DT::storage* x, const void* w,
                                                    int w_dtype, const float* mean,
                                                    const float* rstd, int64_t T, int64_t H,
                                                    int64_t rows, int chunks,
                                                    typename DT::storage* dx, float* partials,
                                                    int64_t B, unsigned* tickets) {
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 2)
    __hip_atomic_store(tickets + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  const int64_t b = blockIdx.y;
  const int chunk = blockIdx.x;
  const int64_t t0 = int64_t(chunk) * rows;
  const int64_t t1 = t0 + rows < T ? t0 + rows : T;
  float* pP = partials + (b * chunks + chunk) * H;
  float* pQ = partials + ((B + b) * chunks + chunk) * H;
  ln_bwd_chunk<DT, EPL, VEC, NTH, NWR, kLnLookahead>(dy, x, w, w_dtype, mean, rstd, T, H, b,
                                                     t0, t1, dx,
                                                     reinterpret_cast<float*>(smem_raw),
                                                     [&](int half, int64_t e, float v) {
                                                       (half == 0 ? pP : pQ)[e] = v;
                                                     });
}

// Tickets shared by the workgroups of one launch: word = (tag << 32) | count,
// where tag is unique to the launch (the host's call counter), so a word left
// by an earlier launch -- or never written -- is recognised as stale and the
// workspace needs no clearing.  Every workgroup claims the word at its start
// (ticket_claim: if the tag is stale, swap in (tag, 0)); a failed swap means
// the word has changed, and only this launch's workgroups change it, always
// to this tag.  So when a workgroup arrives (ticket_arrive, a single
// fetch-and-add after its rows), the word holds this launch's tag and counts
// only this launch's arrivals.  No workgroup waits for another, and neither
// step retries.  ticket_arrive is true for the n-th (last) arrival.
__device__ inline void ticket_claim(unsigned long long* word, uint32_t tag) {
  unsigned long long old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (static_cast<uint32_t>(old >> 32) != tag)
    __hip_atomic_compare_exchange_strong(word, &old, static_cast<unsigned long long>(tag) << 32,
                                         __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline bool ticket_arrive(unsigned long long* word, uint32_t n) {
  const unsigned long long prev =
      __hip_atomic_fetch_add(word, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return static_cast<uint32_t>(prev) + 1u == n;
}

// What the one-launch LayerNorm backward needs beyond the rows.
struct LnFusedArgs {
  float* partials;             // [B][chunks][2H]: the chunk sums (P then Q)
  float* sums;                 // [B][2H]: the per-sample sums
  float* fac;                  // [2B]: clip factors (gamma then beta)
  unsigned long long* tickets; // [B + 1]: per-sample, then the last sample's
  uint32_t tag;
  CombineArgs e;               // clip, scale, noise, outputs (parts unused)
};

// The LayerNorm backward in one launch, for B*H <= 65536 and B <= kFacChunk.
// grid (chunks, B), NTH threads.  Every workgroup runs ln_bwd_chunk and
// publishes its chunk sums (agent-coherent stores); the last chunk of sample
// b to arrive adds the sample's chunks in chunk order, forms the two norms
// and clip factors and publishes the sums; the last sample to arrive forms
// out = out_scale * sum_b c_b * sums_b + noise_scale * z in sample order for
// dgamma and dbeta.  No workgroup waits for another.
template <class DT, int EPL, int VEC, int NTH, int NWR, bool V4, int LA = kLnLookahead>
__global__ __launch_bounds__(NTH) void ln_bwd_fused_kernel(
    const typename DT::storage* dy, const typename DT::storage* x, const void* w, int w_dtype,
    const float* mean, const float* rstd, int64_t T, int64_t H, int64_t rows, int chunks,
    typename DT::storage* dx, LnFusedArgs f) {
  constexpr int W = NTH / kWave;
  constexpr int IW = Item<V4>::W;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  __shared__ float red[W][2];
  __shared__ int role;
  const int64_t b = blockIdx.y;
  const int chunk = blockIdx.x;
  const int64_t B = f.e.B;
  const int64_t t0 = int64_t(chunk) * rows;
  const int64_t t1 = t0 + rows < T ? t0 + rows : T;
  const int64_t per = 2 * H;  // floats per (sample, chunk)
  float* mine = f.partials + (b * chunks + chunk) * per;
  if (threadIdx.x == 0) {
    ticket_claim(f.tickets + b, f.tag);
    ticket_claim(f.tickets + B, f.tag);
  }
  ln_bwd_chunk<DT, EPL, VEC, NTH, NWR, LA>(dy, x, w, w_dtype, mean, rstd, T, H, b, t0, t1, dx,
                                           reinterpret_cast<float*>(smem_raw),
                                           [&](int half, int64_t e, float v) {
                                             st_coherent(mine + half * H + e, v);
                                           });
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0)
    role = ticket_arrive(f.tickets + b, static_cast<uint32_t>(chunks)) ? 1 : 0;
  __syncthreads();
  if (role == 0) return;

  // ---- the sample's sums, norms and clip factors (last chunk of sample b)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t items = per / IW;
  const uint32_t pbytes = static_cast<uint32_t>(B * chunks * per * 4);
  const uint32_t sbytes = static_cast<uint32_t>(B * per * 4);
  const int64_t pbase = b * chunks * per;
  float ssp = 0.f, ssq = 0.f;
  for (int64_t it = threadIdx.x; it < items; it += NTH) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < chunks; c += 16) {
      f32x4 v[16];
#pragma unroll
      for (int q = 0; q < 16; ++q)
        v[q] = c + q < chunks
                   ? ld_item<V4, true>(f.partials, pbase + int64_t(c + q) * per + it * IW, pbytes)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 16; ++q)
        if (c + q < chunks) acc += v[q];
    }
    st_item<V4, true>(f.sums, b * per + it * IW, sbytes, acc);
    Item<V4> item;
    item.v = acc;
    if (it * IW < H) ssp += item.sq();
    else ssq += item.sq();
  }
  ssp = wave_sum_dpp(ssp);
  ssq = wave_sum_dpp(ssq);
  if (lane == 0) {
    red[wave][0] = ssp;
    red[wave][1] = ssq;
  }
  __syncthreads();
  float C = f.e.C, clamp = f.e.clamp;
  if (f.e.clip_args_dev != nullptr) {
    C = f.e.clip_args_dev[0];
    clamp = f.e.clip_args_dev[1];
  }
  if (threadIdx.x == 0) {
    float qp = 0.f, qq = 0.f;
#pragma unroll
    for (int q = 0; q < W; ++q) {
      qp += red[q][0];
      qq += red[q][1];
    }
    const float np = sqrtf(qp), nq = sqrtf(qq);
    const float cp = clip_factor(np, C, clamp), cq = clip_factor(nq, C, clamp);
    st_coherent(f.fac + b, cp);
    st_coherent(f.fac + B + b, cq);
    if (f.e.norms) {
      f.e.norms[b] = np;
      f.e.norms[B + b] = nq;
    }
    if (f.e.factors) {
      f.e.factors[b] = cp;
      f.e.factors[B + b] = cq;
    }
  }
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0)
    role = ticket_arrive(f.tickets + B, static_cast<uint32_t>(B)) ? 2 : 0;
  __syncthreads();
  if (role != 2) return;

  // ---- dgamma, dbeta (last sample): the clipped sum in sample order
  float* fac = reinterpret_cast<float*>(smem_raw);  // [2B] (B <= kFacChunk)
  for (int64_t i = threadIdx.x; i < 2 * B; i += NTH) fac[i] = ld_coherent(f.fac + i);
  __syncthreads();
  for (int64_t it = threadIdx.x; it < items; it += NTH) {
    const int k = it * IW < H ? 0 : 1;
    const int64_t col = it * IW - k * H;
    const float* fk = fac + k * B;
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int64_t s0 = 0; s0 < B; s0 += 16) {
      f32x4 v[16];
#pragma unroll
      for (int q = 0; q < 16; ++q)
        v[q] = s0 + q < B ? ld_item<V4, true>(f.sums, (s0 + q) * per + it * IW, sbytes)
                          : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 16; ++q)
        if (s0 + q < B) tot += fk[s0 + q] * v[q];
    }
    void* out = k == 0 ? f.e.out0 : f.e.out1;
    if (out == nullptr) continue;
    const NoiseSrc noise = k == 0 ? f.e.noise0 : f.e.noise1;
    float z[4] = {0.f, 0.f, 0.f, 0.f};
    if (noise.z != nullptr) {
#pragma unroll
      for (int e = 0; e < IW; ++e) z[e] = noise.at(col + e);
    } else if (noise.draw) {
      noise.window(col, z);
    }
#pragma unroll
    for (int e = 0; e < IW; ++e)
      store_from_f32(out, col + e, f.e.out_dtype, tot[e] * f.e.out_scale + f.e.noise_scale * z[e]);
  }
}

// ------------------------------------------------- rows shared by wavefronts
// Rows of more than 1024 elements: several wavefronts share each row, every
// thread holding EPL <= 16 elements (element e of thread l at
// (l + L*i)*VEC + j, L threads per row), which keeps the per-thread arrays in
// registers.  A row's statistics are wavefront sums added in wavefront order
// through LDS, double-buffered by row parity.  The workgroup walks its rows
// one at a time with the next row's loads in flight; all threads run the same
// trip count, so the barriers are uniform.
constexpr int kSplitWaves = 16;              // wavefronts per long row
constexpr int kSplitLanes = kSplitWaves * kWave;

// grid-stride over rows, one row per workgroup of NW wavefronts at a time
template <class DT, int EPL, int VEC, int NW>
__global__ __launch_bounds__(NW * kWave) void ln_fwd_split_kernel(
    const typename DT::storage* x, const void* w, const void* bias, int w_dtype, int64_t rows,
    int64_t H, float eps, typename DT::storage* y, float* mean, float* rstd) {
  constexpr int L = NW * kWave;
  __shared__ float red[2][2][NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float wv[EPL], bv[EPL];
  load_param<EPL, VEC, L>(w, w_dtype, H, tid, 1.f, wv);
  load_param<EPL, VEC, L>(bias, w_dtype, H, tid, 0.f, bv);
  const float inv_h = 1.f / static_cast<float>(H);
  const int64_t step = gridDim.x;
  RawRow<DT, EPL, VEC, L> rx;
  int64_t r = blockIdx.x;
  rx.load(x + (r < rows ? r : 0) * H, H, tid, r < rows);
  for (int par = 0; r < rows; r += step, par ^= 1) {
    float xv[EPL];
    rx.decode(xv);
    const bool more = r + step < rows;
    rx.load(x + (more ? r + step : r) * H, H, tid, more);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) sum += xv[i];
    sum = wave_sum_dpp(sum);
    if (lane == 0) red[par][0][wave] = sum;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) tot += red[par][0][q];
    const float mu = tot * inv_h;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float d = wave_elem<EPL, VEC, L>(tid, i) + j < static_cast<int>(H) ? xv[i * VEC + j] - mu : 0.f;
        sq += d * d;
      }
    sq = wave_sum_dpp(sq);
    if (lane == 0) red[par][1][wave] = sq;
    __syncthreads();
    float var = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) var += red[par][1][q];
    const float rs = 1.f / sqrtf(var * inv_h + eps);
    float yv[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) yv[i] = (xv[i] - mu) * rs * wv[i] + bv[i];
    store_row<DT, EPL, VEC, L>(y + r * H, H, tid, yv);
    if (tid == 0) {
      if (mean) mean[r] = mu;
      if (rstd) rstd[r] = rs;
    }
  }
}

// grid (chunks, B): the workgroup walks the chunk's rows of sample b; every
// thread accumulates P = sum dy*x_hat and Q = sum dy of its own columns in
// LDS (the 128 registers a 1024-thread workgroup allows hold gamma, x_hat, dy
// and the raw rows; P and Q in registers spilled) and writes them as the
// chunk's partials (no fold: the columns are disjoint).  Workgroup (0,0)
// zeroes the reduction's two tickets.
template <class DT, int EPL, int VEC>
__global__ __launch_bounds__(kSplitLanes) void ln_bwd_split_kernel(
    const typename DT::storage* dy, const typename DT::storage* x, const void* w, int w_dtype,
    const float* mean, const float* rstd, int64_t T, int64_t H, int64_t rows, int chunks,
    typename DT::storage* dx, float* partials, int64_t B, unsigned* tickets) {
  constexpr int NW = kSplitWaves, L = kSplitLanes;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 2)
    __hip_atomic_store(tickets + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __shared__ float red[2][2][NW];
  __shared__ float accP[L * EPL], accQ[L * EPL];  // element e at e (own columns only)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int Hn = static_cast<int>(H);
  const int64_t b = blockIdx.y;
  const int chunk = blockIdx.x;
  const int64_t t0 = int64_t(chunk) * rows;
  const int64_t t1 = t0 + rows < T ? t0 + rows : T;
  float wv[EPL];
  load_param<EPL, VEC, L>(w, w_dtype, H, tid, 1.f, wv);
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e = wave_elem<EPL, VEC, L>(tid, i) + j;
      accP[e] = 0.f;
      accQ[e] = 0.f;
    }
  const float inv_h = 1.f / static_cast<float>(H);
  RawRow<DT, EPL, VEC, L> rx, rg;
  int64_t t = t0;
  float mu_n = 0.f, rs_n = 0.f;
  if (t0 < t1) {  // (an empty chunk, T = 0, touches no row and no statistic)
    rx.load(x + (b * T + t0) * H, H, tid);
    rg.load(dy + (b * T + t0) * H, H, tid);
    mu_n = mean[b * T + t0];
    rs_n = rstd[b * T + t0];
  }
  for (int par = 0; t < t1; ++t, par ^= 1) {
    const int64_t r = b * T + t;
    float xv[EPL], gv[EPL];
    rx.decode(xv);
    rg.decode(gv);
    const float mu = mu_n, rs = rs_n;
    const bool more = t + 1 < t1;
    const int64_t rn = more ? r + 1 : r;
    rx.load(x + rn * H, H, tid, more);
    rg.load(dy + rn * H, H, tid, more);
    mu_n = mean[rn];
    rs_n = rstd[rn];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int k = i * VEC + j;
        const int e = wave_elem<EPL, VEC, L>(tid, i) + j;
        const bool in = e < Hn;
        xv[k] = in ? (xv[k] - mu) * rs : 0.f;  // x_hat
        const float wdy = wv[k] * gv[k];
        s1 += xv[k] * wdy;
        s2 += wdy;
        accP[e] += gv[k] * xv[k];
        accQ[e] += gv[k];
      }
    s1 = wave_sum_dpp(s1);
    s2 = wave_sum_dpp(s2);
    if (lane == 0) {
      red[par][0][wave] = s1;
      red[par][1][wave] = s2;
    }
    __syncthreads();
    float a1 = 0.f, a2 = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      a1 += red[par][0][q];
      a2 += red[par][1][q];
    }
    const float c1 = a1 * inv_h, c2 = a2 * inv_h;
#pragma unroll
    for (int k = 0; k < EPL; ++k) gv[k] = (wv[k] * gv[k] - (xv[k] * c1 + c2)) * rs;
    store_row<DT, EPL, VEC, L>(dx + r * H, H, tid, gv);
  }
  float* pP = partials + (b * chunks + chunk) * H;
  float* pQ = partials + ((B + b) * chunks + chunk) * H;
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e = wave_elem<EPL, VEC, L>(tid, i) + j;
      if (e < Hn) {
        pP[e] = accP[e];
        pQ[e] = accQ[e];
      }
    }
}

// ----------------------------------------------------------- very long rows
// Rows of more than 16384 elements do not fit the registers of one
// workgroup, so they are swept in segments of kLongSeg elements (1024
// threads, 8 each; element e of a segment at wave_elem<8, VEC, 1024>), with
// the next segment's loads in flight while one is used.  Every sweep adds in
// a fixed order: per thread over the segments, then wavefronts in order.
constexpr int kLongLanes = kSplitLanes;
constexpr int kLongEpt = 8;
constexpr int64_t kLongSeg = int64_t(kLongLanes) * kLongEpt;

// Workgroup sums of two values, wavefronts added in order through LDS
// (`red` double-buffered by `par`: consecutive calls alternate it, so one
// barrier per call suffices).
template <int NW>
__device__ __forceinline__ void block_sum2(float& a, float& b, float (&red)[2][2][NW], int par) {
  a = wave_sum_dpp(a);
  b = wave_sum_dpp(b);
  if ((threadIdx.x & 63) == 0) {
    red[par][0][threadIdx.x >> 6] = a;
    red[par][1][threadIdx.x >> 6] = b;
  }
  __syncthreads();
  a = 0.f;
  b = 0.f;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    a += red[par][0][q];
    b += red[par][1][q];
  }
}

// Length of segment `sg` of a long row (it starts at element sg * kLongSeg).
__device__ __forceinline__ int64_t seg_len(int64_t H, int64_t sg) {
  const int64_t n = H - sg * kLongSeg;
  return n < kLongSeg ? n : kLongSeg;
}

// A parameter vector's segment: the pointer moved to element h0 (NULL stays
// NULL, load_param then supplies the default).
__device__ __forceinline__ const void* param_at(const void* p, int dtype, int64_t h0) {
  if (p == nullptr) return nullptr;
  return static_cast<const char*>(p) + h0 * (dtype == FDP_F32 ? 4 : 2);
}

// A long row's parameter segment (hn elements from p; NULL: `dflt`), in the
// element layout of RawRow<DT, 8, VEC, LANES>: raw buffer loads, so elements
// past the segment read zero with no clamping and one offset register.
template <int E, int VEC, int LANES>
__device__ inline void load_param_seg(const void* p, int dtype, int64_t hn, int lane, float dflt,
                                      float (&o)[E]) {
  if (p == nullptr) {
#pragma unroll
    for (int i = 0; i < E / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        o[i * VEC + j] = wave_elem<E, VEC, LANES>(lane, i) + j < hn ? dflt : 0.f;
    return;
  }
  const int es = dtype == FDP_F32 ? 4 : 2;
  const auto r = row_rsrc(p, static_cast<uint32_t>(hn * es));
  if constexpr (VEC > 1) {
    // VEC consecutive elements per vector: 16-byte (or, 16-bit with VEC = 4,
    // 8-byte) loads when the segment is 16-byte aligned.  Rows taken with
    // VEC > 1 hold a multiple of VEC elements, so no vector straddles the end.
    if (reinterpret_cast<uintptr_t>(p) % 16 == 0) {
#pragma unroll
      for (int i = 0; i < E / VEC; ++i) {
        const int e0 = wave_elem<E, VEC, LANES>(lane, i);
        if (dtype == FDP_F32) {
#pragma unroll
          for (int v = 0; v < VEC / 4; ++v) {
            const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, (e0 + 4 * v) * 4, 0, 0);
#pragma unroll
            for (int k = 0; k < 4; ++k) o[i * VEC + 4 * v + k] = __uint_as_float(q[k]);
          }
        } else {
          uint32_t q[VEC / 2];
          if constexpr (VEC == 8) {
            const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(r, e0 * 2, 0, 0);
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = t[k];
          } else {
            const auto t = __builtin_amdgcn_raw_buffer_load_b64(r, e0 * 2, 0, 0);
            q[0] = t[0];
            q[1] = t[1];
          }
#pragma unroll
          for (int k = 0; k < VEC / 2; ++k) {
            const uint16_t lo = static_cast<uint16_t>(q[k] & 0xffffu);
            const uint16_t hi = static_cast<uint16_t>(q[k] >> 16);
            o[i * VEC + 2 * k] = dtype == FDP_BF16 ? BF16::to_f32(lo) : F16::to_f32(lo);
            o[i * VEC + 2 * k + 1] = dtype == FDP_BF16 ? BF16::to_f32(hi) : F16::to_f32(hi);
          }
        }
      }
      return;
    }
  }
  if (dtype == FDP_F32) {
#pragma unroll
    for (int i = 0; i < E / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        o[i * VEC + j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            r, (wave_elem<E, VEC, LANES>(lane, i) + j) * 4, 0, 0));
  } else {
    uint16_t raw[E];
#pragma unroll
    for (int i = 0; i < E / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        raw[i * VEC + j] = __builtin_amdgcn_raw_buffer_load_b16(
            r, (wave_elem<E, VEC, LANES>(lane, i) + j) * 2, 0, 0);
    if (dtype == FDP_BF16) {
#pragma unroll
      for (int k = 0; k < E; ++k) o[k] = BF16::to_f32(raw[k]);
    } else {
#pragma unroll
      for (int k = 0; k < E; ++k) o[k] = F16::to_f32(raw[k]);
    }
  }
}

// The same pointer, opaque to the optimiser: parameter loads through it stay
// where they are written (once per row, L2 hits) instead of being hoisted out
// of the row loop, where every segment's gamma and beta would stay live in
// registers (2 * NS * 8 per thread) and spill.
__device__ __forceinline__ const void* per_row(const void* p) {
  __asm__ volatile("" : "+s"(p));
  return p;
}

// Forward, grid-stride over rows, one row per 1024-thread workgroup at a time:
// three sweeps over the row (sum; centred sum of squares; output), the second
// and third mostly from L2.
template <class DT, int VEC>
__global__ __launch_bounds__(kLongLanes) void ln_fwd_long_kernel(
    const typename DT::storage* x, const void* w, const void* bias, int w_dtype, int64_t rows,
    int64_t H, float eps, typename DT::storage* y, float* mean, float* rstd) {
  constexpr int NW = kLongLanes / kWave, E = kLongEpt, L = kLongLanes;
  __shared__ float red[2][2][NW];
  const int tid = threadIdx.x;
  const int64_t nseg = (H + kLongSeg - 1) / kLongSeg;
  const float inv_h = 1.f / static_cast<float>(H);
  int par = 0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const typename DT::storage* xr = x + r * H;
    RawRow<DT, E, VEC, L> cur, nxt;
    // sweep 1: the sum (elements past the row read zero)
    float s = 0.f, unused = 0.f;
    cur.load(xr, seg_len(H, 0), tid);
    for (int64_t sg = 0; sg < nseg; ++sg) {
      const bool more = sg + 1 < nseg;
      nxt.load(xr + (more ? sg + 1 : sg) * kLongSeg, seg_len(H, more ? sg + 1 : sg), tid, more);
      float xv[E];
      cur.decode(xv);
#pragma unroll
      for (int k = 0; k < E; ++k) s += xv[k];
      cur = nxt;
    }
    block_sum2<NW>(s, unused, red, par);
    par ^= 1;
    const float mu = s * inv_h;
    // sweep 2: the centred sum of squares, elements past the row masked
    float q = 0.f;
    unused = 0.f;
    cur.load(xr, seg_len(H, 0), tid);
    for (int64_t sg = 0; sg < nseg; ++sg) {
      const bool more = sg + 1 < nseg;
      nxt.load(xr + (more ? sg + 1 : sg) * kLongSeg, seg_len(H, more ? sg + 1 : sg), tid, more);
      const int64_t hn = seg_len(H, sg);
      float xv[E];
      cur.decode(xv);
#pragma unroll
      for (int i = 0; i < E / VEC; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const float d = wave_elem<E, VEC, L>(tid, i) + j < hn ? xv[i * VEC + j] - mu : 0.f;
          q += d * d;
        }
      cur = nxt;
    }
    block_sum2<NW>(q, unused, red, par);
    par ^= 1;
    const float rs = 1.f / sqrtf(q * inv_h + eps);
    // sweep 3: y = (x - mu) * rs * w + b
    cur.load(xr, seg_len(H, 0), tid);
    for (int64_t sg = 0; sg < nseg; ++sg) {
      const bool more = sg + 1 < nseg;
      nxt.load(xr + (more ? sg + 1 : sg) * kLongSeg, seg_len(H, more ? sg + 1 : sg), tid, more);
      const int64_t h0 = sg * kLongSeg, hn = seg_len(H, sg);
      float xv[E], wv[E], bv[E], yv[E];
      load_param_seg<E, VEC, L>(param_at(w, w_dtype, h0), w_dtype, hn, tid, 1.f, wv);
      load_param_seg<E, VEC, L>(param_at(bias, w_dtype, h0), w_dtype, hn, tid, 0.f, bv);
      cur.decode(xv);
#pragma unroll
      for (int k = 0; k < E; ++k) yv[k] = (xv[k] - mu) * rs * wv[k] + bv[k];
      store_row<DT, E, VEC, L>(y + r * H + h0, hn, tid, yv);
      cur = nxt;
    }
    if (tid == 0) {
      if (mean) mean[r] = mu;
      if (rstd) rstd[r] = rs;
    }
  }
}

// Rows of at most NS segments (NS * 8192 elements): the row's raw bytes are
// loaded into registers once, every segment's loads in flight together, and
// the three sweeps read the registers.  Segments past the row load nothing
// and hold zeros, so the sums are those of ln_fwd_long_kernel.
template <class DT, int VEC, int NS>
__global__ __launch_bounds__(kLongLanes) void ln_fwd_held_kernel(
    const typename DT::storage* x, const void* w, const void* bias, int w_dtype, int64_t rows,
    int64_t H, float eps, typename DT::storage* y, float* mean, float* rstd) {
  constexpr int NW = kLongLanes / kWave, E = kLongEpt, L = kLongLanes;
  __shared__ float red[2][2][NW];
  const int tid = threadIdx.x;
  const int nseg = static_cast<int>((H + kLongSeg - 1) / kLongSeg);  // <= NS
  const float inv_h = 1.f / static_cast<float>(H);
  int par = 0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const typename DT::storage* xr = x + r * H;
    RawRow<DT, E, VEC, L> seg[NS];
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) {
      const bool on = sg < nseg;
      seg[sg].load(xr + (on ? sg : 0) * kLongSeg, on ? seg_len(H, sg) : 0, tid, on);
    }
    float s = 0.f, unused = 0.f;
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) {
      float xv[E];
      seg[sg].decode(xv);
#pragma unroll
      for (int k = 0; k < E; ++k) s += xv[k];
    }
    block_sum2<NW>(s, unused, red, par);
    par ^= 1;
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) seg[sg].opaque();
    const float mu = s * inv_h;
    float q = 0.f;
    unused = 0.f;
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) {
      const int64_t hn = sg < nseg ? seg_len(H, sg) : 0;
      float xv[E];
      seg[sg].decode(xv);
#pragma unroll
      for (int i = 0; i < E / VEC; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const float d = wave_elem<E, VEC, L>(tid, i) + j < hn ? xv[i * VEC + j] - mu : 0.f;
          q += d * d;
        }
    }
    block_sum2<NW>(q, unused, red, par);
    par ^= 1;
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) seg[sg].opaque();
    const float rs = 1.f / sqrtf(q * inv_h + eps);
    const void* wr = per_row(w);
    const void* br = per_row(bias);
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) {
      if (sg < nseg) {
        const int64_t h0 = sg * kLongSeg, hn = seg_len(H, sg);
        float xv[E], wv[E], bv[E], yv[E];
        load_param_seg<E, VEC, L>(param_at(wr, w_dtype, h0), w_dtype, hn, tid, 1.f, wv);
        load_param_seg<E, VEC, L>(param_at(br, w_dtype, h0), w_dtype, hn, tid, 0.f, bv);
        seg[sg].decode(xv);
#pragma unroll
        for (int k = 0; k < E; ++k) yv[k] = (xv[k] - mu) * rs * wv[k] + bv[k];
        store_row<DT, E, VEC, L>(y + r * H + h0, hn, tid, yv);
      }
    }
    if (tid == 0) {
      if (mean) mean[r] = mu;
      if (rstd) rstd[r] = rs;
    }
  }
}

// Backward, first launch: for every row (grid-stride, one row per 1024-thread
// workgroup at a time) c1 = sum(x_hat w dy) / H and c2 = sum(w dy) / H into
// cst[r].  Elements past the row read dy = 0 and w = 0, so they add nothing.
// NS > 0: rows of at most NS segments, every segment of x and dy loaded at
// once; NS = 0: any row, streamed one segment ahead.
template <class DT, int VEC, int NS>
__global__ __launch_bounds__(kLongLanes) void ln_rowstat_long_kernel(
    const typename DT::storage* dy, const typename DT::storage* x, const void* w, int w_dtype,
    const float* mean, const float* rstd, int64_t rows, int64_t H, float2* cst) {
  constexpr int NW = kLongLanes / kWave, E = kLongEpt, L = kLongLanes;
  __shared__ float red[2][2][NW];
  const int tid = threadIdx.x;
  const int64_t nseg = (H + kLongSeg - 1) / kLongSeg;
  const float inv_h = 1.f / static_cast<float>(H);
  int par = 0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const float mu = mean[r], rs = rstd[r];
    const typename DT::storage* xr = x + r * H;
    const typename DT::storage* gr = dy + r * H;
    float s1 = 0.f, s2 = 0.f;
    const void* wr = per_row(w);
    // one segment's contribution (elements past the row add nothing)
    auto add = [&](const RawRow<DT, E, VEC, L>& sx, const RawRow<DT, E, VEC, L>& sgr,
                   int64_t sg) {
      float xv[E], gv[E], wv[E];
      load_param_seg<E, VEC, L>(param_at(wr, w_dtype, sg * kLongSeg), w_dtype, seg_len(H, sg), tid,
                            1.f, wv);
      sx.decode(xv);
      sgr.decode(gv);
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const float wdy = wv[k] * gv[k];
        s1 = fmaf((xv[k] - mu) * rs, wdy, s1);
        s2 += wdy;
      }
    };
    if constexpr (NS > 0) {
      RawRow<DT, E, VEC, L> sx[NS], sg_[NS];
#pragma unroll
      for (int sg = 0; sg < NS; ++sg) {
        const bool on = sg < nseg;
        const int64_t off = (on ? sg : 0) * kLongSeg, n = on ? seg_len(H, sg) : 0;
        sx[sg].load(xr + off, n, tid, on);
        sg_[sg].load(gr + off, n, tid, on);
      }
#pragma unroll
      for (int sg = 0; sg < NS; ++sg)
        if (sg < nseg) add(sx[sg], sg_[sg], sg);
    } else {
      RawRow<DT, E, VEC, L> cx, cg, nx, ng;
      cx.load(xr, seg_len(H, 0), tid);
      cg.load(gr, seg_len(H, 0), tid);
      for (int64_t sg = 0; sg < nseg; ++sg) {
        const bool more = sg + 1 < nseg;
        const int64_t sn = more ? sg + 1 : sg;
        nx.load(xr + sn * kLongSeg, seg_len(H, sn), tid, more);
        ng.load(gr + sn * kLongSeg, seg_len(H, sn), tid, more);
        add(cx, cg, sg);
        cx = nx;
        cg = ng;
      }
    }
    block_sum2<NW>(s1, s2, red, par);
    par ^= 1;
    if (tid == 0) cst[r] = make_float2(s1 * inv_h, s2 * inv_h);
  }
}

// Backward, second launch: grid (column blocks, chunks, B).  A 256-thread
// workgroup owns kColsBlock columns (8 per thread) of one chunk's rows of
// sample b: it writes their dx and the chunk's partial column sums P and Q
// in ln_bwd_kernel's layout, with the next row's loads in flight.
// Workgroup (0,0,0) zeroes the reduction's two tickets.
constexpr int kColsThreads = 256;
constexpr int64_t kColsBlock = int64_t(kColsThreads) * kLongEpt;

template <class DT, int VEC>
__global__ __launch_bounds__(kColsThreads) void ln_bwd_cols_kernel(
    const typename DT::storage* dy, const typename DT::storage* x, const void* w, int w_dtype,
    const float* mean, const float* rstd, const float2* cst, int64_t T, int64_t H, int64_t rows,
    int chunks, typename DT::storage* dx, float* partials, int64_t B, unsigned* tickets) {
  constexpr int E = kLongEpt, L = kColsThreads;
  if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x < 2)
    __hip_atomic_store(tickets + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int tid = threadIdx.x;
  const int64_t h0 = int64_t(blockIdx.x) * kColsBlock;
  const int64_t hn = H - h0 < kColsBlock ? H - h0 : kColsBlock;
  const int chunk = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int64_t t0 = int64_t(chunk) * rows;
  const int64_t t1 = t0 + rows < T ? t0 + rows : T;
  float wv[E], P[E], Q[E];
  load_param_seg<E, VEC, L>(param_at(w, w_dtype, h0), w_dtype, hn, tid, 1.f, wv);
#pragma unroll
  for (int k = 0; k < E; ++k) {
    P[k] = 0.f;
    Q[k] = 0.f;
  }
  if (t1 > t0) {  // (an empty chunk, T = 0, touches no row and no statistic)
    RawRow<DT, E, VEC, L> rx, rg;
    int64_t r = b * T + t0;
    rx.load(x + r * H + h0, hn, tid);
    rg.load(dy + r * H + h0, hn, tid);
    float mu_n = mean[r], rs_n = rstd[r];
    float2 c_n = cst[r];
    for (int64_t t = t0; t < t1; ++t, ++r) {
      float xv[E], gv[E];
      rx.decode(xv);
      rg.decode(gv);
      const float mu = mu_n, rs = rs_n, c1 = c_n.x, c2 = c_n.y;
      const bool more = t + 1 < t1;
      const int64_t rn = more ? r + 1 : r;
      rx.load(x + rn * H + h0, hn, tid, more);
      rg.load(dy + rn * H + h0, hn, tid, more);
      mu_n = mean[rn];
      rs_n = rstd[rn];
      c_n = cst[rn];
      // dx = rs (w dy - x_hat c1 - c2); columns past H read dy = 0, w = 0
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const float xh = (xv[k] - mu) * rs;
        P[k] = fmaf(gv[k], xh, P[k]);
        Q[k] += gv[k];
        gv[k] = rs * (wv[k] * gv[k] - fmaf(xh, c1, c2));
      }
      store_row<DT, E, VEC, L>(dx + r * H + h0, hn, tid, gv);
    }
  }
  float* pP = partials + (b * chunks + chunk) * H + h0;
  float* pQ = partials + ((B + b) * chunks + chunk) * H + h0;
#pragma unroll
  for (int i = 0; i < E / VEC; ++i)
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e = wave_elem<E, VEC, L>(tid, i) + j;
      if (e < hn) {
        pP[e] = P[i * VEC + j];
        pQ[e] = Q[i * VEC + j];
      }
    }
}

}  // namespace rw
}  // namespace fdp

// ====================================================================== host
using namespace fdp;
using namespace fdp::rw;

namespace {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
bool valid_dtype(int d) { return d == FDP_F32 || d == FDP_F16 || d == FDP_BF16; }
int esize(int d) { return d == FDP_F32 ? 4 : 2; }

int num_cus() { return fdp::host::device_cus(); }

// Workspace of both reductions (offsets in bytes), S = streams * B:
//   off_part   partials [S][chunks][H] (fp32)
//   off_frob   per-(sample, workgroup) sums of u^2 [B][parts] (FDP_NORM_FROB)
//   off_sums   per-sample sums [S][H] (fp32)
//   off_sq     per-(stream, item block) sums of squares [S][item_blocks]
//   off_ticket one arrival ticket per stream (reduce_kernel; zeroed by the row
//              kernel of the same call)
struct RedPlan {
  int vec, bs, cblocks, chunks, parts, iblocks;
  bool v4;
  bool one_launch;  // reduce_kernel instead of chunk_sum_kernel + combine_kernel
  bool fused;       // LayerNorm: ln_bwd_fused_kernel (the reduction in the row launch)
  bool long_rows;   // LayerNorm rows of more than kMaxLnH: ln_rowstat_long + ln_bwd_cols
  int64_t rows;
  size_t off_part, off_frob, off_sums, off_sq, off_ticket, total;
  size_t off_fac;   // fused: clip factors [2B]
  size_t off_cst;   // long rows: per-row (c1, c2) [B*T]
};

// Per-stream sums of at most this many elements are combined by one workgroup
// (reduce_kernel): there the saved launch outweighs the serial combine.
constexpr int64_t kOneLaunchElems = 65536;

void finish_plan(RedPlan& p, int64_t B, int64_t H, int streams) {
  const size_t S = size_t(streams) * B;
  p.parts = p.chunks * p.cblocks;
  p.v4 = H % 4 == 0;
  const int64_t items = p.v4 ? H / 4 : H;
  p.iblocks = static_cast<int>((items + kItemsPerBlock - 1) / kItemsPerBlock);
  p.off_part = 0;
  p.off_frob = align_up(sizeof(float) * S * p.chunks * H);
  p.off_sums = p.off_frob + align_up(sizeof(float) * size_t(B) * p.parts);
  p.off_sq = p.off_sums + align_up(sizeof(float) * S * H);
  p.off_ticket = p.off_sq + align_up(sizeof(float) * S * p.iblocks);
  p.total = p.off_ticket + align_up(sizeof(unsigned) * streams);
  p.one_launch = B * H <= kOneLaunchElems && B <= kFacChunk;
}

// Rows per chunk so that there are about `per_cu` workgroups per CU, with at
// least `min_rows` rows per chunk.
void split_rows(RedPlan& p, int64_t B, int64_t T, int cus, int per_cu, int64_t min_rows) {
  int64_t want = (per_cu * int64_t(cus) + B * p.cblocks - 1) / (B * p.cblocks);
  int64_t max_chunks = (T + min_rows - 1) / min_rows;
  if (max_chunks < 1) max_chunks = 1;
  if (want > max_chunks) want = max_chunks;
  if (want < 1) want = 1;
  p.rows = T > 0 ? (T + want - 1) / want : 1;
  p.chunks = static_cast<int>(T > 0 ? (T + p.rows - 1) / p.rows : 1);
}

// Column sums: about four workgroups per CU, with chunks of at least 64 rows.
// A chunk's fp32 partials cost 4H bytes against its 2·rows·H bytes of 16-bit
// rows; on 8x1024xH bf16 bias gradients (H = 2048 .. 8192) minimums of 8 and
// 128 rows measured 5-18% and 0-45% slower than 64.
RedPlan col_plan(int64_t B, int64_t T, int64_t H, int dtype, int cus, bool aligned) {
  RedPlan p{};
  p.vec = aligned ? 16 / esize(dtype) : 1;
  const int64_t nvec = (H + p.vec - 1) / p.vec;
  int64_t bs = ((nvec + 63) / 64) * 64;
  if (bs > NT) bs = NT;
  p.bs = static_cast<int>(bs);
  p.cblocks = static_cast<int>((nvec + bs - 1) / bs);
  split_rows(p, B, T, cus, 4, 64);
  finish_plan(p, B, H, 1);
  return p;
}

// How a LayerNorm row of H elements is spread over threads, at most 16
// elements per thread (the backward kernel's per-thread columns, x_hat, dy
// and gamma stay in registers; 32 or 64 per lane spilled):
//   H <= 512: one wavefront, 8 each;   H <= 1024: one wavefront, 16 each;
//   H <= 2048: 2 wavefronts, 16 each;  H <= 4096: 4 wavefronts, 16 each;
//   H <= 8192: 16 wavefronts (a 1024-thread workgroup per row), 8 each;
//   H <= 16384: 16 wavefronts, 16 each.
// Rows of up to 4096 elements are processed several to a workgroup, longer
// ones one per workgroup (ln_*_split_kernel).
struct LnShape {
  int nwr, epl;
};
constexpr int64_t kMaxWaveH = 4096;
constexpr int64_t kMaxLnH = int64_t(kSplitLanes) * 16;  // longer rows: the *_long kernels
// Longest row accepted: per-row offsets and the partials' indices stay in
// range well beyond it.
constexpr int64_t kMaxRowH = int64_t(1) << 30;

LnShape ln_shape(int64_t H) {
  if (H <= 512) return {1, 8};
  if (H <= 1024) return {1, 16};
  if (H <= 2048) return {2, 16};
  if (H <= kMaxWaveH) return {4, 16};
  if (H <= 8192) return {kSplitWaves, 8};
  return {kSplitWaves, 16};
}

// f(NWR, EPL) with both as compile-time constants.
template <class F>
void with_ln_shape(LnShape sh, F&& f) {
  using std::integral_constant;
  if (sh.nwr == 1 && sh.epl == 8) f(integral_constant<int, 1>{}, integral_constant<int, 8>{});
  else if (sh.nwr == 1) f(integral_constant<int, 1>{}, integral_constant<int, 16>{});
  else if (sh.nwr == 2) f(integral_constant<int, 2>{}, integral_constant<int, 16>{});
  else if (sh.nwr == 4) f(integral_constant<int, 4>{}, integral_constant<int, 16>{});
  else if (sh.epl == 8) f(integral_constant<int, kSplitWaves>{}, integral_constant<int, 8>{});
  else f(integral_constant<int, kSplitWaves>{}, integral_constant<int, 16>{});
}


// LayerNorm backward workgroup of the two-launch path: 8 waves, about one
// workgroup per CU, chunks of at least 16 rows (ln_plan).  A chunk's partials
// cost 8H bytes against its 6·rows·H bytes of rows, and more chunks also mean
// more partials for the reduction to read.
constexpr int ln_bwd_threads(int) { return 512; }

// The one-launch LayerNorm backward: 8-wave workgroups, one per CU, chunks of
// at least 32 rows; taken when the last-arriving workgroups' serial work stays
// small: at most 16 chunks per sample for the per-sample sums and B*H <= 65536
// (B <= 1024) for the sum over samples.  Per call (bf16, T=1024) against the
// two-launch path: 16x1024: 27.5 / 27.1 us; 32x1024: 42.6 / 44.6 us;
// 8x2048 (32 chunks per sample, left to the two-launch path): 33.8 / 30.0 us.
constexpr int kLnFusedThreads = 512;
constexpr int kLnFusedMaxChunks = 16;

RedPlan ln_plan(int64_t B, int64_t T, int64_t H, int cus) {
  RedPlan p{};
  p.cblocks = 1;
  if (H <= kMaxWaveH && B * H <= kOneLaunchElems && B <= kFacChunk) {
    split_rows(p, B, T, cus, 1, 32);
    const size_t per = size_t(2) * H;
    const size_t part = sizeof(float) * size_t(B) * p.chunks * per;
    if (p.chunks <= kLnFusedMaxChunks && part < (size_t(1) << 31)) {
      p.fused = true;
      p.v4 = H % 4 == 0;
      p.off_part = 0;
      p.off_sums = align_up(part);
      p.off_fac = p.off_sums + align_up(sizeof(float) * size_t(B) * per);
      p.off_ticket = p.off_fac + align_up(sizeof(float) * 2 * size_t(B));
      p.total = p.off_ticket + align_up(sizeof(unsigned long long) * size_t(B + 1));
      return p;
    }
  }
  if (H > kMaxLnH) {
    // 2048-column blocks of 256 threads, about eight workgroups per CU
    p.long_rows = true;
    p.cblocks = static_cast<int>((H + kColsBlock - 1) / kColsBlock);
    split_rows(p, B, T, cus, 8, 32);
    finish_plan(p, B, H, 2);
    p.off_cst = p.total;
    p.total += align_up(sizeof(float2) * size_t(B) * size_t(T));
    return p;
  }
  // Rows of more than kMaxWaveH take one 1024-thread workgroup per CU; shorter
  // ones one 512-thread workgroup (ln_bwd_threads) per CU, with chunks of at
  // least 16 rows so that small batches still fill the CUs.  T = 1024 bf16,
  // against 256-thread workgroups, two per CU, chunks of at least 32 rows:
  // B x H = 8 x 2048 29.1 / 31.2 us, 4 x 4096 32.8 / 44.4, 8 x 3072 38.4 /
  // 44.5, 2 x 2048 19.4 / 27.8, 8 x 1024 19.0 / 19.7, 16 x 2048 44.5 / 45.0.
  split_rows(p, B, T, cus, 1, H > kMaxWaveH ? 32 : 16);
  finish_plan(p, B, H, 2);
  return p;
}

// Launch tag of the one-launch LayerNorm backward: unique per call in this
// process (its tickets count only arrivals carrying the same tag), starting
// from a clock-derived value so that a stale word in reused memory is unlikely
// to carry it either.
uint32_t next_ln_tag() {
  static std::atomic<uint32_t> counter{static_cast<uint32_t>(
      std::chrono::steady_clock::now().time_since_epoch().count() * 2654435761u)};
  uint32_t t = counter.fetch_add(1, std::memory_order_relaxed) + 1;
  if (t == 0) t = counter.fetch_add(1, std::memory_order_relaxed) + 1;
  return t;
}

// chunk sums -> per-sample norms, clip factors and the clipped, scaled sum.
struct Epilogue {
  float C, clamp;
  const float* clip_args_dev;
  float out_scale, noise_scale;
  NoiseSrc noise0, noise1;
  void* out0;
  void* out1;
  int out_dtype;
  float* norms;
  float* factors;
};

void launch_reduce(const RedPlan& p, char* ws, int64_t B, int64_t H, int streams, bool frob,
                   const Epilogue& e, hipStream_t s) {
  const float* part = reinterpret_cast<const float*>(ws + p.off_part);
  float* sums = reinterpret_cast<float*>(ws + p.off_sums);
  float* sq = reinterpret_cast<float*>(ws + p.off_sq);
  unsigned* tickets = reinterpret_cast<unsigned*>(ws + p.off_ticket);
  const CombineArgs a{frob ? reinterpret_cast<const float*>(ws + p.off_frob) : sq,
                      frob ? p.parts : p.iblocks,
                      B, H, e.C, e.clamp, e.clip_args_dev, e.out_scale, e.noise0, e.noise1,
                      e.noise_scale, e.out0, e.out1, e.out_dtype, e.norms, e.factors};
  const dim3 rgrid(static_cast<unsigned>(p.iblocks), static_cast<unsigned>(streams * B));
  const dim3 cgrid(static_cast<unsigned>(p.iblocks), static_cast<unsigned>(streams));
  if (p.one_launch) {
    if (p.v4)
      hipLaunchKernelGGL(reduce_kernel<true>, rgrid, dim3(NT), 0, s, part, p.chunks, sums, sq,
                         tickets, a);
    else
      hipLaunchKernelGGL(reduce_kernel<false>, rgrid, dim3(NT), 0, s, part, p.chunks, sums, sq,
                         tickets, a);
  } else if (p.v4) {
    hipLaunchKernelGGL(chunk_sum_kernel<true>, rgrid, dim3(NT), 0, s, part, H, p.chunks, sums, sq);
    hipLaunchKernelGGL(combine_kernel<true>, cgrid, dim3(NT), 0, s, sums, a);
  } else {
    hipLaunchKernelGGL(chunk_sum_kernel<false>, rgrid, dim3(NT), 0, s, part, H, p.chunks, sums,
                       sq);
    hipLaunchKernelGGL(combine_kernel<false>, cgrid, dim3(NT), 0, s, sums, a);
  }
}

template <class DT, int VEC>
void launch_colsum(const RedPlan& p, const void* u, const void* v, int64_t B, int64_t T,
                   int64_t H, char* ws, bool frob, hipStream_t s) {
  using S = typename DT::storage;
  hipLaunchKernelGGL((colsum_kernel<DT, VEC>), dim3(p.cblocks, p.chunks, B), dim3(p.bs), 0, s,
                     static_cast<const S*>(u), static_cast<const S*>(v), T, H, p.rows, p.chunks,
                     reinterpret_cast<float*>(ws + p.off_part),
                     frob ? reinterpret_cast<float*>(ws + p.off_frob) : nullptr,
                     reinterpret_cast<unsigned*>(ws + p.off_ticket));
}

template <class DT>
void launch_colsum_dt(const RedPlan& p, const void* u, const void* v, int64_t B, int64_t T,
                      int64_t H, char* ws, bool frob, hipStream_t s) {
  if (p.vec == 1) launch_colsum<DT, 1>(p, u, v, B, T, H, ws, frob, s);
  else if constexpr (DT::code == FDP_F32) launch_colsum<DT, 4>(p, u, v, B, T, H, ws, frob, s);
  else launch_colsum<DT, 8>(p, u, v, B, T, H, ws, frob, s);
}

// Rows of up to 1024 elements: ln_fwd_kernel, enough wavefronts for ~4 rows
// each, at most 2 workgroups per CU.  Longer rows: one row per workgroup of
// NWR wavefronts, grid-stride, about 512 threads per CU for rows of 2 or 4
// wavefronts and 2048 for 16 (each workgroup then walks more rows with the
// next row's loads in flight).  8192 rows of bf16, threads per CU 2048 / 1024
// / 512 / 256: H = 2048 22.7 / 17.0 / 15.7 / 19.9 us, H = 4096 27.7 / 26.6 /
// 25.1 / 31.4 us, H = 8192 49.0 / 50.2 / 50.2 / 50.3 us.
template <class DT, int VEC>
void launch_ln_fwd(LnShape sh, const void* x, const void* w, const void* b, int w_dtype,
                   int64_t rows, int64_t H, float eps, void* y, float* mean, float* rstd, int cus,
                   hipStream_t s) {
  using S = typename DT::storage;
  with_ln_shape(sh, [&](auto nwr_c, auto epl_c) {
    constexpr int NWR = decltype(nwr_c)::value, EPL = decltype(epl_c)::value;
    if constexpr (NWR == 1) {
      constexpr int W = kLnThreads / kWave;
      int64_t grid = (rows + 4 * W - 1) / (4 * W);
      const int64_t cap = int64_t(cus) * 2;
      if (grid > cap) grid = cap;
      if (grid < 1) grid = 1;
      hipLaunchKernelGGL((ln_fwd_kernel<DT, EPL, VEC>), dim3(static_cast<unsigned>(grid)),
                         dim3(kLnThreads), 0, s, static_cast<const S*>(x), w, b, w_dtype, rows, H,
                         eps, static_cast<S*>(y), mean, rstd);
    } else {
      constexpr int kThreadsPerCu = NWR == kSplitWaves ? 2048 : 512;
      int64_t grid = int64_t(cus) * (kThreadsPerCu / (NWR * kWave));
      if (grid > rows) grid = rows;
      hipLaunchKernelGGL((ln_fwd_split_kernel<DT, EPL, VEC, NWR>),
                         dim3(static_cast<unsigned>(grid)), dim3(NWR * kWave), 0, s,
                         static_cast<const S*>(x), w, b, w_dtype, rows, H, eps,
                         static_cast<S*>(y), mean, rstd);
    }
  });
}

// Rows of more than kMaxLnH elements: one row per 1024-thread workgroup,
// grid-stride, two workgroups per CU; rows of up to 4 segments held in
// registers (8 spilled), longer ones swept three times.
template <class DT, int VEC>
void launch_ln_fwd_long(const void* x, const void* w, const void* b, int w_dtype, int64_t rows,
                        int64_t H, float eps, void* y, float* mean, float* rstd, int cus,
                        hipStream_t s) {
  using S = typename DT::storage;
  int64_t grid = int64_t(cus) * 2;
  if (grid > rows) grid = rows;
  const int64_t nseg = (H + kLongSeg - 1) / kLongSeg;
  const dim3 g(static_cast<unsigned>(grid)), t(kLongLanes);
  const S* xs = static_cast<const S*>(x);
  S* ys = static_cast<S*>(y);
  if (nseg <= 4)
    hipLaunchKernelGGL((ln_fwd_held_kernel<DT, VEC, 4>), g, t, 0, s, xs, w, b, w_dtype, rows, H,
                       eps, ys, mean, rstd);
  else
    hipLaunchKernelGGL((ln_fwd_long_kernel<DT, VEC>), g, t, 0, s, xs, w, b, w_dtype, rows, H, eps,
                       ys, mean, rstd);
}

template <class DT>
void launch_ln_fwd_dt(bool vec, LnShape sh, const void* x, const void* w, const void* b,
                      int w_dtype, int64_t rows, int64_t H, float eps, void* y, float* mean,
                      float* rstd, int cus, hipStream_t s) {
  if (H > kMaxLnH) {
    if (!vec) launch_ln_fwd_long<DT, 1>(x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
    else if constexpr (DT::code == FDP_F32)
      launch_ln_fwd_long<DT, 4>(x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
    else launch_ln_fwd_long<DT, 8>(x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
    return;
  }
  if (!vec) launch_ln_fwd<DT, 1>(sh, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else if constexpr (DT::code == FDP_F32)
    launch_ln_fwd<DT, 4>(sh, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else launch_ln_fwd<DT, 8>(sh, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
}

struct LnBwdIo {
  const void* dy;
  const void* x;
  const void* w;
  int w_dtype;
  const float* mean;
  const float* rstd;
  int64_t B, T, H;
  void* dx;
};

// Two-launch backward (rows, then launch_reduce): rows of up to 4096 elements
// in 4-wave workgroups, longer ones in one 1024-thread workgroup per row.
template <class DT, int VEC>
void launch_ln_bwd(LnShape sh, const RedPlan& p, const LnBwdIo& io, float* part,
                   unsigned* tickets, hipStream_t s) {
  using S = typename DT::storage;
  with_ln_shape(sh, [&](auto nwr_c, auto epl_c) {
    constexpr int NWR = decltype(nwr_c)::value, EPL = decltype(epl_c)::value;
    if constexpr (NWR == kSplitWaves) {
      hipLaunchKernelGGL((ln_bwd_split_kernel<DT, EPL, VEC>), dim3(p.chunks, io.B),
                         dim3(kSplitLanes), 0, s, static_cast<const S*>(io.dy),
                         static_cast<const S*>(io.x), io.w, io.w_dtype, io.mean, io.rstd, io.T,
                         io.H, p.rows, p.chunks, static_cast<S*>(io.dx), part, io.B, tickets);
    } else {
      constexpr int NTH = ln_bwd_threads(EPL);
      constexpr int G = NTH / (NWR * kWave);
      hipLaunchKernelGGL((ln_bwd_kernel<DT, EPL, VEC, NTH, NWR>), dim3(p.chunks, io.B),
                         dim3(NTH), sizeof(float) * G * fold_slice(io.H), s,
                         static_cast<const S*>(io.dy), static_cast<const S*>(io.x), io.w,
                         io.w_dtype, io.mean, io.rstd, io.T, io.H, p.rows, p.chunks,
                         static_cast<S*>(io.dx), part, io.B, tickets);
    }
  });
}

template <class DT>
void launch_ln_bwd_dt(bool vec, LnShape sh, const RedPlan& p, const LnBwdIo& io, float* part,
                      unsigned* tickets, hipStream_t s) {
  if (!vec) launch_ln_bwd<DT, 1>(sh, p, io, part, tickets, s);
  else if constexpr (DT::code == FDP_F32) launch_ln_bwd<DT, 4>(sh, p, io, part, tickets, s);
  else launch_ln_bwd<DT, 8>(sh, p, io, part, tickets, s);
}

// Rows of more than kMaxLnH elements: the per-row statistics (one row per
// 1024-thread workgroup, two per CU), then the column blocks; launch_reduce
// follows as for the other two-launch shapes.
template <class DT, int VEC>
void launch_ln_bwd_long(const RedPlan& p, const LnBwdIo& io, float2* cst, float* part,
                        unsigned* tickets, int cus, hipStream_t s) {
  using S = typename DT::storage;
  const int64_t rows = io.B * io.T;
  if (rows > 0) {
    int64_t grid = int64_t(cus) * 2;
    if (grid > rows) grid = rows;
    const dim3 g(static_cast<unsigned>(grid)), t(kLongLanes);
    const S* dys = static_cast<const S*>(io.dy);
    const S* xs = static_cast<const S*>(io.x);
    bool held = false;  // 16-bit rows of at most four segments: x and dy loaded at once
    if constexpr (VEC == 8) {
      held = io.H <= 4 * kLongSeg;
      if (held)
        hipLaunchKernelGGL((ln_rowstat_long_kernel<DT, VEC, 4>), g, t, 0, s, dys, xs, io.w,
                           io.w_dtype, io.mean, io.rstd, rows, io.H, cst);
    }
    if (!held)
      hipLaunchKernelGGL((ln_rowstat_long_kernel<DT, VEC, 0>), g, t, 0, s, dys, xs, io.w,
                         io.w_dtype, io.mean, io.rstd, rows, io.H, cst);
  }
  hipLaunchKernelGGL((ln_bwd_cols_kernel<DT, VEC>),
                     dim3(static_cast<unsigned>(p.cblocks), static_cast<unsigned>(p.chunks),
                          static_cast<unsigned>(io.B)),
                     dim3(kColsThreads), 0, s, static_cast<const S*>(io.dy),
                     static_cast<const S*>(io.x), io.w, io.w_dtype, io.mean, io.rstd, cst, io.T,
                     io.H, p.rows, p.chunks, static_cast<S*>(io.dx), part, io.B, tickets);
}

template <class DT>
void launch_ln_bwd_long_dt(bool vec, const RedPlan& p, const LnBwdIo& io, float2* cst,
                           float* part, unsigned* tickets, int cus, hipStream_t s) {
  if (!vec) launch_ln_bwd_long<DT, 1>(p, io, cst, part, tickets, cus, s);
  else if constexpr (DT::code == FDP_F32) launch_ln_bwd_long<DT, 4>(p, io, cst, part, tickets, cus, s);
  else launch_ln_bwd_long<DT, 8>(p, io, cst, part, tickets, cus, s);
}

// One-launch backward (rows of up to 4096 elements).
template <class DT, int VEC, bool V4>
void launch_ln_fused(LnShape sh, const RedPlan& p, const LnBwdIo& io, const LnFusedArgs& f,
                     hipStream_t s) {
  using S = typename DT::storage;
  with_ln_shape(sh, [&](auto nwr_c, auto epl_c) {
    constexpr int NWR = decltype(nwr_c)::value, EPL = decltype(epl_c)::value;
    if constexpr (NWR < kSplitWaves) {
      constexpr int G = kLnFusedThreads / (NWR * kWave);
      size_t lds = sizeof(float) * G * fold_slice(io.H);
      if (lds < sizeof(float) * 2 * size_t(io.B)) lds = sizeof(float) * 2 * size_t(io.B);
      hipLaunchKernelGGL((ln_bwd_fused_kernel<DT, EPL, VEC, kLnFusedThreads, NWR, V4>),
                         dim3(p.chunks, io.B), dim3(kLnFusedThreads), lds, s,
                         static_cast<const S*>(io.dy), static_cast<const S*>(io.x), io.w,
                         io.w_dtype, io.mean, io.rstd, io.T, io.H, p.rows, p.chunks,
                         static_cast<S*>(io.dx), f);
    }
  });
}

// Aligned 16-byte rows imply H % 4 == 0 (V4); element rows take either.
template <class DT>
void launch_ln_fused_dt(bool vec, LnShape sh, const RedPlan& p, const LnBwdIo& io,
                        const LnFusedArgs& f, hipStream_t s) {
  if (!vec) {
    if (p.v4) launch_ln_fused<DT, 1, true>(sh, p, io, f, s);
    else launch_ln_fused<DT, 1, false>(sh, p, io, f, s);
  } else if constexpr (DT::code == FDP_F32) {
    launch_ln_fused<DT, 4, true>(sh, p, io, f, s);
  } else {
    launch_ln_fused<DT, 8, true>(sh, p, io, f, s);
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

// ------------------------------------------------------------ C ABI
extern "C" int fdp_colsum_clip_workspace_size(int64_t B, int64_t T, int64_t H, int dtype,
                                              size_t* bytes) {
  if (bytes == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || T < 0 || H < 1) return FDP_ERR_SHAPE;
  // The aligned plan has the most chunk partials; size for the larger of both.
  const RedPlan a = col_plan(B, T, H, dtype, num_cus(), true);
  const RedPlan u = col_plan(B, T, H, dtype, num_cus(), false);
  *bytes = a.total > u.total ? a.total : u.total;
  return FDP_OK;
}

extern "C" int fdp_colsum_clip(const void* u, const void* v, int64_t B, int64_t T, int64_t H,
                               int dtype, int norm_kind, float C, float clamp,
                               const float* clip_args_dev, float out_scale, const void* noise,
                               float noise_scale, const fdp_noise_key* noise_key, void* out,
                               int out_dtype, float* norms, float* factors, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return FDP_ERR_DTYPE;
  if (norm_kind != FDP_NORM_SUM && norm_kind != FDP_NORM_FROB) return FDP_ERR_ARG;
  if (B < 1 || T < 0 || H < 1) return FDP_ERR_SHAPE;
  // samples index grid.y / grid.z (at most 65535)
  if (B > 65535 || H > (int64_t(1) << 31)) return FDP_ERR_SHAPE;
  if ((T > 0 && u == nullptr) || out == nullptr) return FDP_ERR_ARG;
  const bool aligned = aligned16(u) && (v == nullptr || aligned16(v)) &&
                       (H * esize(dtype)) % 16 == 0;
  const int cus = num_cus();
  const RedPlan p = col_plan(B, T, H, dtype, cus, aligned);
  if (workspace == nullptr || workspace_bytes < p.total) return FDP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return FDP_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  const bool frob = norm_kind == FDP_NORM_FROB;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FDP_BF16) launch_colsum_dt<BF16>(p, u, v, B, T, H, ws, frob, s);
  else if (dtype == FDP_F16) launch_colsum_dt<F16>(p, u, v, B, T, H, ws, frob, s);
  else launch_colsum_dt<F32>(p, u, v, B, T, H, ws, frob, s);
  const fdp_noise_key* key = noise_scale != 0.f ? noise_key : nullptr;
  const Epilogue e{C,         clamp,
                   clip_args_dev,
                   out_scale, noise_scale,
                   make_noise(noise, out_dtype, key, 0),
                   make_noise(nullptr, out_dtype, nullptr, 1),
                   out,       nullptr,
                   out_dtype, norms,
                   factors};
  launch_reduce(p, ws, B, H, 1, frob, e, s);
  return hipGetLastError() == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}

extern "C" int fdp_layernorm_fwd(const void* x, const void* w, const void* b, int64_t rows,
                                 int64_t H, float eps, int dtype, int w_dtype, void* y,
                                 float* mean, float* rstd, void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(w_dtype)) return FDP_ERR_DTYPE;
  if (rows < 0 || H < 1 || H > kMaxRowH) return FDP_ERR_SHAPE;
  if (rows == 0) return FDP_OK;
  if (x == nullptr || y == nullptr) return FDP_ERR_ARG;
  const bool vec = aligned16(x) && aligned16(y) && (H * esize(dtype)) % 16 == 0;
  const LnShape sh = ln_shape(H);
  const int cus = num_cus();
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FDP_BF16) launch_ln_fwd_dt<BF16>(vec, sh, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else if (dtype == FDP_F16) launch_ln_fwd_dt<F16>(vec, sh, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else launch_ln_fwd_dt<F32>(vec, sh, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  return hipGetLastError() == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}

extern "C" int fdp_layernorm_bwd_clip_workspace_size(int64_t B, int64_t T, int64_t H, int dtype,
                                                     size_t* bytes) {
  if (bytes == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || T < 0 || H < 1 || H > kMaxRowH) return FDP_ERR_SHAPE;
  *bytes = ln_plan(B, T, H, num_cus()).total;
  return FDP_OK;
}

extern "C" int fdp_layernorm_bwd_clip(const void* dy, const void* x, const void* w,
                                      const float* mean, const float* rstd, int64_t B, int64_t T,
                                      int64_t H, int dtype, int w_dtype, float C, float clamp,
                                      const float* clip_args_dev, float out_scale,
                                      const void* noise_w, const void* noise_b,
                                      float noise_scale, const fdp_noise_key* noise_key,
                                      void* dx, void* dw, void* db, float* norms, float* factors,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(w_dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || T < 0 || H < 1 || H > kMaxRowH) return FDP_ERR_SHAPE;
  if (B > 32767) return FDP_ERR_SHAPE;  // the 2B streams index grid.y
  if (T > 0 && (dy == nullptr || x == nullptr || dx == nullptr || mean == nullptr ||
                rstd == nullptr))
    return FDP_ERR_ARG;
  const int cus = num_cus();
  const RedPlan p = ln_plan(B, T, H, cus);
  if (workspace == nullptr || workspace_bytes < p.total) return FDP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return FDP_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = aligned16(dy) && aligned16(x) && aligned16(dx) && (H * esize(dtype)) % 16 == 0;
  const LnShape sh = ln_shape(H);
  const LnBwdIo io{dy, x, w, w_dtype, mean, rstd, B, T, H, dx};
  float* part = reinterpret_cast<float*>(ws + p.off_part);
  const fdp_noise_key* key = noise_scale != 0.f ? noise_key : nullptr;
  if (p.fused) {
    LnFusedArgs f{};
    f.partials = part;
    f.sums = reinterpret_cast<float*>(ws + p.off_sums);
    f.fac = reinterpret_cast<float*>(ws + p.off_fac);
    f.tickets = reinterpret_cast<unsigned long long*>(ws + p.off_ticket);
    f.tag = next_ln_tag();
    f.e = CombineArgs{nullptr, 0, B, H, C, clamp, clip_args_dev, out_scale,
                      make_noise(noise_w, w_dtype, key, 0), make_noise(noise_b, w_dtype, key, 1),
                      noise_scale, dw, db, w_dtype, norms, factors};
    if (dtype == FDP_BF16) launch_ln_fused_dt<BF16>(vec, sh, p, io, f, s);
    else if (dtype == FDP_F16) launch_ln_fused_dt<F16>(vec, sh, p, io, f, s);
    else launch_ln_fused_dt<F32>(vec, sh, p, io, f, s);
    return hipGetLastError() == hipSuccess ? FDP_OK : FDP_ERR_HIP;
  }
  unsigned* tickets = reinterpret_cast<unsigned*>(ws + p.off_ticket);
  if (p.long_rows) {
    float2* cst = reinterpret_cast<float2*>(ws + p.off_cst);
    if (dtype == FDP_BF16) launch_ln_bwd_long_dt<BF16>(vec, p, io, cst, part, tickets, cus, s);
    else if (dtype == FDP_F16) launch_ln_bwd_long_dt<F16>(vec, p, io, cst, part, tickets, cus, s);
    else launch_ln_bwd_long_dt<F32>(vec, p, io, cst, part, tickets, cus, s);
  } else if (dtype == FDP_BF16) {
    launch_ln_bwd_dt<BF16>(vec, sh, p, io, part, tickets, s);
  } else if (dtype == FDP_F16) {
    launch_ln_bwd_dt<F16>(vec, sh, p, io, part, tickets, s);
  } else {
    launch_ln_bwd_dt<F32>(vec, sh, p, io, part, tickets, s);
  }
  const Epilogue e{C,        clamp,
                   clip_args_dev,
                   out_scale, noise_scale,
                   make_noise(noise_w, w_dtype, key, 0),
                   make_noise(noise_b, w_dtype, key, 1),
                   dw,       db,
                   w_dtype,  norms,
                   factors};
  launch_reduce(p, ws, B, H, 2, false, e, s);
  return hipGetLastError() == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}

extern "C" const char* fdp_strerror(int status) {
  switch (status) {
    case FDP_OK: return "ok";
    case FDP_ERR_DTYPE: return "unsupported dtype";
    case FDP_ERR_SHAPE: return "unsupported or inconsistent sizes";
    case FDP_ERR_ARG: return "invalid argument";
    case FDP_ERR_WORKSPACE: return "workspace missing or too small";
    case FDP_ERR_HIP: return "HIP launch failed";
    case FDP_ERR_ALIGN: return "pointer alignment violated";
    case FDP_ERR_TOO_LARGE: return "problem needs more than the no-allocation scratch array";
    default: return "unknown status";
  }
}

extern "C" int fdp_version(void) { return 200; }
