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

// Element e of lane `lane` in a row handled by one wavefront: vector
// v = lane + 64*i covers elements v*VEC .. v*VEC+VEC-1.
template <int EPL, int VEC>
__device__ __forceinline__ int64_t wave_elem(int lane, int i) {
  return (int64_t(lane) + 64 * i) * VEC;
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

template <class DT, int EPL, int VEC>
__device__ inline void load_row(const typename DT::storage* row, int64_t H, int lane,
                                float (&o)[EPL]) {
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i) {
    const int64_t e = wave_elem<EPL, VEC>(lane, i);
    if (e < H) {
      Vec<DT, VEC>::load(row + e, o + i * VEC);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) o[i * VEC + j] = 0.f;
    }
  }
}
template <class DT, int EPL, int VEC>
__device__ inline void store_row(typename DT::storage* row, int64_t H, int lane,
                                 const float (&v)[EPL]) {
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i) {
    const int64_t e = wave_elem<EPL, VEC>(lane, i);
    if (e < H) Vec<DT, VEC>::store(row + e, v + i * VEC);
  }
}
// Parameter vectors (gamma/beta) in an arbitrary dtype, default `dflt` if NULL.
template <int EPL, int VEC>
__device__ inline void load_param(const void* p, int dtype, int64_t H, int lane, float dflt,
                                  float (&o)[EPL]) {
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int64_t e = wave_elem<EPL, VEC>(lane, i) + j;
      o[i * VEC + j] = (p != nullptr && e < H) ? load_as_f32(p, e, dtype) : (e < H ? dflt : 0.f);
    }
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

// Raw (undecoded) row fragment of one lane: lets the next row's loads be in
// flight while the current row is processed.
template <class DT, int EPL, int VEC>
struct RawRow;
template <class DT, int EPL>
struct RawRow<DT, EPL, 8> {  // 16-bit, 16-byte vectors
  uint4 q[EPL / 8];
  __device__ __forceinline__ void load(const uint16_t* row, int64_t H, int lane) {
#pragma unroll
    for (int i = 0; i < EPL / 8; ++i) {
      const int64_t e = wave_elem<EPL, 8>(lane, i);
      q[i] = e < H ? *reinterpret_cast<const uint4*>(row + e) : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void decode(float (&o)[EPL]) const {
#pragma unroll
    for (int i = 0; i < EPL / 8; ++i) {
      const uint32_t w[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[i * 8 + 2 * j] = DT::to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
        o[i * 8 + 2 * j + 1] = DT::to_f32(static_cast<uint16_t>(w[j] >> 16));
      }
    }
  }
};
template <int EPL>
struct RawRow<F32, EPL, 4> {  // fp32, 16-byte vectors
  float4 q[EPL / 4];
  __device__ __forceinline__ void load(const float* row, int64_t H, int lane) {
#pragma unroll
    for (int i = 0; i < EPL / 4; ++i) {
      const int64_t e = wave_elem<EPL, 4>(lane, i);
      q[i] = e < H ? *reinterpret_cast<const float4*>(row + e) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __device__ __forceinline__ void decode(float (&o)[EPL]) const {
#pragma unroll
    for (int i = 0; i < EPL / 4; ++i) {
      o[4 * i] = q[i].x;
      o[4 * i + 1] = q[i].y;
      o[4 * i + 2] = q[i].z;
      o[4 * i + 3] = q[i].w;
    }
  }
};
template <class DT, int EPL>
struct RawRow<DT, EPL, 1> {  // any dtype, element loads (unaligned rows)
  typename DT::storage q[EPL];
  __device__ __forceinline__ void load(const typename DT::storage* row, int64_t H, int lane) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int64_t e = wave_elem<EPL, 1>(lane, i);
      q[i] = e < H ? row[e] : typename DT::storage(0);
    }
  }
  __device__ __forceinline__ void decode(float (&o)[EPL]) const {
#pragma unroll
    for (int i = 0; i < EPL; ++i) o[i] = DT::to_f32(q[i]);
  }
};

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
  if (wid < rows) rx.load(x + wid * H, H, lane);
  for (int64_t r = wid; r < rows; r += nw) {
    float xv[EPL];
    rx.decode(xv);
    if (r + nw < rows) rx.load(x + (r + nw) * H, H, lane);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) s += xv[i];
    const float mu = wave_sum_dpp(s) * inv_h;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float d = wave_elem<EPL, VEC>(lane, i) + j < H ? xv[i * VEC + j] - mu : 0.f;
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

// grid (chunks, B).  Wave w handles rows t = chunk*rows + w, +W, ... with the
// next row's x / dy / mean / rstd loads in flight while the current row is
// processed: writes dx and accumulates P = sum dy*x_hat, Q = sum dy in
// registers; the W = NTH/64 waves are folded in wave order through LDS into
// the chunk's partials (stream b: P, stream B+b: Q).  Workgroup (0,0) zeroes
// the reduction's two tickets.
template <class DT, int EPL, int VEC, int NTH>
__global__ __launch_bounds__(NTH) void ln_bwd_kernel(const typename DT::storage* dy,
                                                    const typename DT::storage* x, const void* w,
                                                    int w_dtype, const float* mean,
                                                    const float* rstd, int64_t T, int64_t H,
                                                    int64_t rows, int chunks,
                                                    typename DT::storage* dx, float* partials,
                                                    int64_t B, unsigned* tickets) {
  constexpr int W = NTH / kWave;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 2)
    __hip_atomic_store(tickets + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  float* lds = reinterpret_cast<float*>(smem_raw);  // [W][H]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t b = blockIdx.y;
  const int chunk = blockIdx.x;
  const int64_t t0 = int64_t(chunk) * rows;
  const int64_t t1 = t0 + rows < T ? t0 + rows : T;
  float wv[EPL];
  load_param<EPL, VEC>(w, w_dtype, H, lane, 1.f, wv);
  float P[EPL], Q[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    P[i] = 0.f;
    Q[i] = 0.f;
  }
  const float inv_h = 1.f / static_cast<float>(H);
  RawRow<DT, EPL, VEC> rx, rg;
  float mu_n = 0.f, rs_n = 0.f;
  int64_t t = t0 + wave;
  if (t < t1) {
    rx.load(x + (b * T + t) * H, H, lane);
    rg.load(dy + (b * T + t) * H, H, lane);
    mu_n = mean[b * T + t];
    rs_n = rstd[b * T + t];
  }
  for (; t < t1; t += W) {
    const int64_t r = b * T + t;
    float xv[EPL], gv[EPL];
    rx.decode(xv);
    rg.decode(gv);
    const float mu = mu_n, rs = rs_n;
    const int64_t tn = t + W;
    if (tn < t1) {
      rx.load(x + (b * T + tn) * H, H, lane);
      rg.load(dy + (b * T + tn) * H, H, lane);
      mu_n = mean[b * T + tn];
      rs_n = rstd[b * T + tn];
    }
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int k = i * VEC + j;
        const bool in = wave_elem<EPL, VEC>(lane, i) + j < H;
        xv[k] = in ? (xv[k] - mu) * rs : 0.f;  // x_hat
        const float wdy = wv[k] * gv[k];
        s1 += xv[k] * wdy;
        s2 += wdy;
        P[k] += gv[k] * xv[k];
        Q[k] += gv[k];
      }
    const float c1 = wave_sum_dpp(s1) * inv_h;
    const float c2 = wave_sum_dpp(s2) * inv_h;
#pragma unroll
    for (int k = 0; k < EPL; ++k) gv[k] = (wv[k] * gv[k] - (xv[k] * c1 + c2)) * rs;
    store_row<DT, EPL, VEC>(dx + r * H, H, lane, gv);
  }
  // Fold the waves in order 0..W-1: every wave parks its row of P (then of
  // Q) in its own LDS slice (fold_slice(H) floats, element e at fold_pos(e)),
  // and all threads sum the slices element-wise.
  float* pP = partials + (b * chunks + chunk) * H;
  float* pQ = partials + ((B + b) * chunks + chunk) * H;
  const int64_t slice = fold_slice(H);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    float* mine = lds + wave * slice;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const int64_t e = wave_elem<EPL, VEC>(lane, i) + j;
        if (e < H) mine[fold_pos(e)] = half == 0 ? P[i * VEC + j] : Q[i * VEC + j];
      }
    __syncthreads();
    float* dst = half == 0 ? pP : pQ;
    for (int64_t e = threadIdx.x; e < H; e += NTH) {
      const int64_t at = fold_pos(e);
      float v = lds[at];
#pragma unroll
      for (int ww = 1; ww < W; ++ww) v += lds[ww * slice + at];
      dst[e] = v;
    }
    __syncthreads();
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
  int64_t rows;
  size_t off_part, off_frob, off_sums, off_sq, off_ticket, total;
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

constexpr int64_t kMaxLnH = 4096;  // 64 elements per lane, one wave per row

// Elements per lane for a row of H (EPL in {8,16,32,64}).
int ln_epl(int64_t H) {
  int epl = 8;
  while (int64_t(epl) * 64 < H) epl *= 2;
  return epl;
}


// LayerNorm backward workgroup: 4 waves, about two workgroups per CU, with
// chunks of at least 32 rows.  On a 16x1024x1024 problem one, two and four
// per CU (chunks of 64, 32 and 16 rows) measured 28.6, 28.1 and 33.8 us per
// call: a chunk's partials cost 8H bytes against its 6·rows·H bytes of rows,
// and more chunks also mean more partials for the reduction to read.
constexpr int ln_bwd_threads(int) { return 256; }

RedPlan ln_plan(int64_t B, int64_t T, int64_t H, int cus) {
  RedPlan p{};
  p.cblocks = 1;
  split_rows(p, B, T, cus, 2, 32);
  finish_plan(p, B, H, 2);
  return p;
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

template <class DT, int EPL, int VEC>
void launch_ln_fwd_t(const void* x, const void* w, const void* b, int w_dtype, int64_t rows,
                     int64_t H, float eps, void* y, float* mean, float* rstd, int cus,
                     hipStream_t s) {
  using S = typename DT::storage;
  constexpr int W = kLnThreads / kWave;
  // enough wavefronts for ~4 rows each, at most 2 workgroups per CU
  int64_t grid = (rows + 4 * W - 1) / (4 * W);
  const int64_t cap = int64_t(cus) * 2;
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((ln_fwd_kernel<DT, EPL, VEC>), dim3(static_cast<unsigned>(grid)),
                     dim3(kLnThreads), 0, s, static_cast<const S*>(x), w, b, w_dtype, rows, H, eps,
                     static_cast<S*>(y), mean, rstd);
}

template <class DT, int VEC>
void launch_ln_fwd_v(int epl, const void* x, const void* w, const void* b, int w_dtype,
                     int64_t rows, int64_t H, float eps, void* y, float* mean, float* rstd,
                     int cus, hipStream_t s) {
  switch (epl) {
    case 8: launch_ln_fwd_t<DT, 8, VEC>(x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s); break;
    case 16: launch_ln_fwd_t<DT, 16, VEC>(x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s); break;
    case 32: launch_ln_fwd_t<DT, 32, VEC>(x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s); break;
    default: launch_ln_fwd_t<DT, 64, VEC>(x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s); break;
  }
}

template <class DT>
void launch_ln_fwd(bool vec, int epl, const void* x, const void* w, const void* b, int w_dtype,
                   int64_t rows, int64_t H, float eps, void* y, float* mean, float* rstd, int cus,
                   hipStream_t s) {
  if (!vec) launch_ln_fwd_v<DT, 1>(epl, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else if constexpr (DT::code == FDP_F32)
    launch_ln_fwd_v<DT, 4>(epl, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else launch_ln_fwd_v<DT, 8>(epl, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
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

template <class DT, int EPL, int VEC>
void launch_ln_bwd_t(const RedPlan& p, const LnBwdIo& io, float* part, unsigned* tickets,
                     hipStream_t s) {
  using S = typename DT::storage;
  constexpr int NTH = ln_bwd_threads(EPL);
  hipLaunchKernelGGL((ln_bwd_kernel<DT, EPL, VEC, NTH>), dim3(p.chunks, io.B), dim3(NTH),
                     sizeof(float) * (NTH / kWave) * fold_slice(io.H), s, static_cast<const S*>(io.dy),
                     static_cast<const S*>(io.x), io.w, io.w_dtype, io.mean, io.rstd, io.T, io.H,
                     p.rows, p.chunks, static_cast<S*>(io.dx), part, io.B, tickets);
}

template <class DT, int VEC>
void launch_ln_bwd_v(int epl, const RedPlan& p, const LnBwdIo& io, float* part,
                     unsigned* tickets, hipStream_t s) {
  switch (epl) {
    case 8: launch_ln_bwd_t<DT, 8, VEC>(p, io, part, tickets, s); break;
    case 16: launch_ln_bwd_t<DT, 16, VEC>(p, io, part, tickets, s); break;
    case 32: launch_ln_bwd_t<DT, 32, VEC>(p, io, part, tickets, s); break;
    default: launch_ln_bwd_t<DT, 64, VEC>(p, io, part, tickets, s); break;
  }
}

template <class DT>
void launch_ln_bwd(bool vec, int epl, const RedPlan& p, const LnBwdIo& io, float* part,
                   unsigned* tickets, hipStream_t s) {
  if (!vec) launch_ln_bwd_v<DT, 1>(epl, p, io, part, tickets, s);
  else if constexpr (DT::code == FDP_F32) launch_ln_bwd_v<DT, 4>(epl, p, io, part, tickets, s);
  else launch_ln_bwd_v<DT, 8>(epl, p, io, part, tickets, s);
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
  if (rows < 0 || H < 1 || H > kMaxLnH) return FDP_ERR_SHAPE;
  if (rows == 0) return FDP_OK;
  if (x == nullptr || y == nullptr) return FDP_ERR_ARG;
  const bool vec = aligned16(x) && aligned16(y) && (H * esize(dtype)) % 16 == 0;
  const int epl = ln_epl(H);
  const int cus = num_cus();
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FDP_BF16) launch_ln_fwd<BF16>(vec, epl, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else if (dtype == FDP_F16) launch_ln_fwd<F16>(vec, epl, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  else launch_ln_fwd<F32>(vec, epl, x, w, b, w_dtype, rows, H, eps, y, mean, rstd, cus, s);
  return hipGetLastError() == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}

extern "C" int fdp_layernorm_bwd_clip_workspace_size(int64_t B, int64_t T, int64_t H, int dtype,
                                                     size_t* bytes) {
  if (bytes == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || T < 0 || H < 1 || H > kMaxLnH) return FDP_ERR_SHAPE;
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
  if (B < 1 || T < 0 || H < 1 || H > kMaxLnH) return FDP_ERR_SHAPE;
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
  const int epl = ln_epl(H);
  const LnBwdIo io{dy, x, w, w_dtype, mean, rstd, B, T, H, dx};
  float* part = reinterpret_cast<float*>(ws + p.off_part);
  unsigned* tickets = reinterpret_cast<unsigned*>(ws + p.off_ticket);
  if (dtype == FDP_BF16) launch_ln_bwd<BF16>(vec, epl, p, io, part, tickets, s);
  else if (dtype == FDP_F16) launch_ln_bwd<F16>(vec, epl, p, io, part, tickets, s);
  else launch_ln_bwd<F32>(vec, epl, p, io, part, tickets, s);
  const fdp_noise_key* key = noise_scale != 0.f ? noise_key : nullptr;
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

extern "C" int fdp_version(void) { return 100; }
