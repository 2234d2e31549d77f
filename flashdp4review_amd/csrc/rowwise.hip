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
// All reductions are fixed-order (no float atomics): per-(sample, row-chunk)
// partial vectors go to a workspace, a per-sample kernel sums the chunks in
// chunk order and derives the clip factor, and a combine kernel sums the
// clipped samples in sample order.  Rows are read with 16-byte loads, one
// wavefront per row for the LayerNorm kernels (row statistics are wavefront
// shuffles, no LDS), 64..256 threads across the columns for the column sums.
#include "fdp_common.hpp"

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

// ======================================================= column-sum partials
// grid (col_blocks, chunks, B); thread owns VEC consecutive columns of one
// 16-byte vector and walks `rows` rows of one sample.
template <class DT, int VEC>
__global__ __launch_bounds__(NT) void colsum_partials_kernel(
    const typename DT::storage* u, const typename DT::storage* v, int64_t T, int64_t H,
    int64_t rows, int chunks, float* partials, float* frob) {
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
    __shared__ float red[NT / kWave];
    sq = wave_sum(sq);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
      float s = 0.f;
      for (int w = 0; w < int(blockDim.x >> 6); ++w) s += red[w];
      frob[(b * chunks + chunk) * gridDim.x + blockIdx.x] = s;
    }
  }
}

// ============================================================ per-stream reduce
// grid (ceil(H/NT), S): column h of stream s is summed over the chunk partials
// in chunk order (loads unrolled for memory-level parallelism, additions kept
// in order) into sums[s, h]; each block also writes the sum of squares of its
// columns to sq_part[s, block] for the ||S_s|| norm.
__global__ __launch_bounds__(NT) void chunk_reduce_kernel(const float* partials, int64_t H,
                                                          int chunks, float* sums, float* sq_part) {
  __shared__ float red[NT / kWave];
  const int64_t s = blockIdx.y;
  const int64_t h = int64_t(blockIdx.x) * NT + threadIdx.x;
  float acc = 0.f;
  if (h < H) {
    const float* src = partials + s * chunks * H + h;
    int c = 0;
    for (; c + 8 <= chunks; c += 8) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = src[int64_t(c + q) * H];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc += v[q];
    }
    for (; c < chunks; ++c) acc += src[int64_t(c) * H];
    sums[s * H + h] = acc;
  }
  const float sq = wave_sum(acc * acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
  __syncthreads();
  if (threadIdx.x == 0) sq_part[s * gridDim.x + blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// One wavefront per stream: n_s = sqrt(sum of its squared-norm parts), c_s.
// The parts are the per-block sums of squares of S_s (FDP_NORM_SUM) or the
// per-(chunk, column block) sums of u^2 (FDP_NORM_FROB), nparts per stream.
__global__ __launch_bounds__(NT) void stream_factor_kernel(const float* parts, int64_t S,
                                                           int nparts, float C, float clamp,
                                                           const float* clip_args_dev, float* fac,
                                                           float* norms, float* factors) {
  if (clip_args_dev != nullptr) {
    C = clip_args_dev[0];
    clamp = clip_args_dev[1];
  }
  const int lane = threadIdx.x & 63;
  const int64_t s = int64_t(blockIdx.x) * (NT / kWave) + (threadIdx.x >> 6);
  if (s >= S) return;
  float q = 0.f;
  for (int i = lane; i < nparts; i += kWave) q += parts[s * nparts + i];
  const float n = sqrtf(wave_sum(q));
  if (lane == 0) {
    const float c = clip_factor(n, C, clamp);
    fac[s] = c;
    if (norms) norms[s] = n;
    if (factors) factors[s] = c;
  }
}

// out_k[h] = out_scale * sum_b fac[kB+b] * sums[kB+b, h] + noise_scale * noise_k[h]
// for k = 0 (out0) and, when out1 != NULL, k = 1.
__global__ __launch_bounds__(NT) void combine_kernel(const float* sums, const float* fac,
                                                     int64_t B, int64_t H, float out_scale,
                                                     const void* noise0, const void* noise1,
                                                     float noise_scale, void* out0, void* out1,
                                                     int out_dtype) {
  const int64_t h = int64_t(blockIdx.x) * NT + threadIdx.x;
  if (h >= H) return;
  for (int k = 0; k < 2; ++k) {
    void* out = k == 0 ? out0 : out1;
    if (out == nullptr) continue;
    const void* noise = k == 0 ? noise0 : noise1;
    float acc = 0.f;
    for (int64_t b = 0; b < B; ++b) acc += fac[k * B + b] * sums[(k * B + b) * H + h];
    float v = acc * out_scale;
    if (noise) v += noise_scale * load_as_f32(noise, h, out_dtype);
    store_from_f32(out, h, out_dtype, v);
  }
}

// Zero-fill used instead of hipMemsetAsync so that callers may capture the
// entry points in a HIP graph.
__global__ __launch_bounds__(NT) void fill_zero_kernel(float* p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * NT + threadIdx.x; i < n; i += int64_t(gridDim.x) * NT)
    p[i] = 0.f;
}

// ================================================================= LayerNorm
// One wavefront per row; 4 rows in flight per workgroup.
template <class DT, int EPL, int VEC>
__global__ __launch_bounds__(NT) void ln_fwd_kernel(const typename DT::storage* x, const void* w,
                                                    const void* bias, int w_dtype, int64_t rows,
                                                    int64_t H, float eps,
                                                    typename DT::storage* y, float* mean,
                                                    float* rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = int64_t(blockIdx.x) * (NT / kWave) + (threadIdx.x >> 6);
  const int64_t nw = int64_t(gridDim.x) * (NT / kWave);
  float wv[EPL], bv[EPL];
  load_param<EPL, VEC>(w, w_dtype, H, lane, 1.f, wv);
  load_param<EPL, VEC>(bias, w_dtype, H, lane, 0.f, bv);
  const float inv_h = 1.f / static_cast<float>(H);
  for (int64_t r = wid; r < rows; r += nw) {
    float xv[EPL];
    load_row<DT, EPL, VEC>(x + r * H, H, lane, xv);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) s += xv[i];
    const float mu = wave_sum(s) * inv_h;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float d = wave_elem<EPL, VEC>(lane, i) + j < H ? xv[i * VEC + j] - mu : 0.f;
        q += d * d;
      }
    const float var = wave_sum(q) * inv_h;
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

// grid (chunks, B).  Each wave handles rows t = chunk*rows + wave, +4, ...
// with the next row's x / dy loads issued before the current row is used:
// writes dx and accumulates P = sum dy*x_hat, Q = sum dy in registers; the four
// waves are then folded in wave order through LDS into one partial per chunk.
template <class DT, int EPL, int VEC>
__global__ __launch_bounds__(NT) void ln_bwd_kernel(const typename DT::storage* dy,
                                                    const typename DT::storage* x, const void* w,
                                                    int w_dtype, const float* mean,
                                                    const float* rstd, int64_t T, int64_t H,
                                                    int64_t rows, int chunks,
                                                    typename DT::storage* dx, float* partials,
                                                    int64_t B) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  float* lds = reinterpret_cast<float*>(smem_raw);  // [2][H]
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
  int64_t t = t0 + wave;
  if (t < t1) {
    rx.load(x + (b * T + t) * H, H, lane);
    rg.load(dy + (b * T + t) * H, H, lane);
  }
  for (; t < t1; t += NT / kWave) {
    const int64_t r = b * T + t;
    float xv[EPL], gv[EPL];
    rx.decode(xv);
    rg.decode(gv);
    const float mu = mean[r], rs = rstd[r];
    const int64_t tn = t + NT / kWave;
    if (tn < t1) {  // next row in flight while this one is processed
      rx.load(x + (b * T + tn) * H, H, lane);
      rg.load(dy + (b * T + tn) * H, H, lane);
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
    const float c1 = wave_sum(s1) * inv_h;
    const float c2 = wave_sum(s2) * inv_h;
    float dv[EPL];
#pragma unroll
    for (int k = 0; k < EPL; ++k) dv[k] = (wv[k] * gv[k] - (xv[k] * c1 + c2)) * rs;
    store_row<DT, EPL, VEC>(dx + r * H, H, lane, dv);
  }
  // Fold the four waves in order 0,1,2,3.
  for (int wsel = 0; wsel < NT / kWave; ++wsel) {
    if (wave == wsel) {
#pragma unroll
      for (int i = 0; i < EPL / VEC; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const int64_t e = wave_elem<EPL, VEC>(lane, i) + j;
          if (e < H) {
            const int k = i * VEC + j;
            lds[e] = wsel == 0 ? P[k] : lds[e] + P[k];
            lds[H + e] = wsel == 0 ? Q[k] : lds[H + e] + Q[k];
          }
        }
    }
    __syncthreads();
  }
  float* pP = partials + (b * chunks + chunk) * H;
  float* pQ = partials + ((B + b) * chunks + chunk) * H;
  for (int64_t e = threadIdx.x; e < H; e += NT) {
    pP[e] = lds[e];
    pQ[e] = lds[H + e];
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

int num_cus() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      cus = v;
  }
  return cus;
}

// ---------------------------------------------------------- column sums
struct ColPlan {
  int vec, bs, cblocks, chunks, nblk;
  int64_t rows;
  size_t off_part, off_frob, off_sums, off_fac, off_sq, total;
};

ColPlan col_plan(int64_t B, int64_t T, int64_t H, int dtype, int cus, bool aligned) {
  ColPlan p{};
  p.vec = aligned ? 16 / esize(dtype) : 1;
  const int64_t nvec = (H + p.vec - 1) / p.vec;
  int64_t bs = ((nvec + 63) / 64) * 64;
  if (bs > NT) bs = NT;
  p.bs = static_cast<int>(bs);
  p.cblocks = static_cast<int>((nvec + bs - 1) / bs);
  // Aim for ~4 workgroups per CU, at least 8 rows per chunk.
  int64_t want = (4 * int64_t(cus) + B * p.cblocks - 1) / (B * p.cblocks);
  int64_t max_chunks = (T + 7) / 8;
  if (max_chunks < 1) max_chunks = 1;
  if (want > max_chunks) want = max_chunks;
  if (want < 1) want = 1;
  p.rows = (T + want - 1) / want;
  if (p.rows < 1) p.rows = 1;
  p.chunks = static_cast<int>(T > 0 ? (T + p.rows - 1) / p.rows : 1);
  p.off_part = 0;
  p.off_frob = align_up(sizeof(float) * size_t(B) * p.chunks * H);
  p.off_sums = p.off_frob + align_up(sizeof(float) * size_t(B) * p.chunks * p.cblocks);
  p.off_fac = p.off_sums + align_up(sizeof(float) * size_t(B) * H);
  p.nblk = static_cast<int>((H + NT - 1) / NT);
  p.off_sq = p.off_fac + align_up(sizeof(float) * size_t(B));
  p.total = p.off_sq + align_up(sizeof(float) * size_t(B) * p.nblk);
  return p;
}

template <class DT, int VEC>
void launch_colsum(const ColPlan& p, const void* u, const void* v, int64_t B, int64_t T,
                   int64_t H, float* part, float* frob, hipStream_t s) {
  using S = typename DT::storage;
  hipLaunchKernelGGL((colsum_partials_kernel<DT, VEC>), dim3(p.cblocks, p.chunks, B), dim3(p.bs),
                     0, s, static_cast<const S*>(u), static_cast<const S*>(v), T, H, p.rows,
                     p.chunks, part, frob);
}

template <class DT>
void launch_colsum_dt(const ColPlan& p, const void* u, const void* v, int64_t B, int64_t T,
                      int64_t H, float* part, float* frob, hipStream_t s) {
  if (p.vec == 1) launch_colsum<DT, 1>(p, u, v, B, T, H, part, frob, s);
  else if constexpr (DT::code == FDP_F32) launch_colsum<DT, 4>(p, u, v, B, T, H, part, frob, s);
  else launch_colsum<DT, 8>(p, u, v, B, T, H, part, frob, s);
}

// ------------------------------------------------------------ LayerNorm
constexpr int64_t kMaxLnH = 4096;  // 64 elements per lane, one wave per row

// Elements per lane for a row of H (EPL in {8,16,32,64}).
int ln_epl(int64_t H) {
  int epl = 8;
  while (int64_t(epl) * 64 < H) epl *= 2;
  return epl;
}

template <class DT, int EPL, int VEC>
void launch_ln_fwd_t(const void* x, const void* w, const void* b, int w_dtype, int64_t rows,
                     int64_t H, float eps, void* y, float* mean, float* rstd, int cus,
                     hipStream_t s) {
  using S = typename DT::storage;
  int64_t grid = (rows + 3) / 4;
  const int64_t cap = int64_t(cus) * 8;
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((ln_fwd_kernel<DT, EPL, VEC>), dim3(static_cast<unsigned>(grid)), dim3(NT),
                     0, s, static_cast<const S*>(x), w, b, w_dtype, rows, H, eps,
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

struct LnPlan {
  int chunks, nblk;
  int64_t rows;
  size_t off_part, off_sums, off_fac, off_sq, total;
};

LnPlan ln_plan(int64_t B, int64_t T, int64_t H, int cus) {
  LnPlan p{};
  // ~2 workgroups per CU, >= 16 rows (4 per wave) per chunk.
  int64_t want = (2 * int64_t(cus) + B - 1) / B;
  int64_t max_chunks = (T + 15) / 16;
  if (max_chunks < 1) max_chunks = 1;
  if (want > max_chunks) want = max_chunks;
  if (want < 1) want = 1;
  p.rows = T > 0 ? (T + want - 1) / want : 1;
  p.chunks = static_cast<int>(T > 0 ? (T + p.rows - 1) / p.rows : 1);
  p.off_part = 0;
  p.off_sums = align_up(sizeof(float) * size_t(2 * B) * p.chunks * H);
  p.off_fac = p.off_sums + align_up(sizeof(float) * size_t(2 * B) * H);
  p.nblk = static_cast<int>((H + NT - 1) / NT);
  p.off_sq = p.off_fac + align_up(sizeof(float) * size_t(2 * B));
  p.total = p.off_sq + align_up(sizeof(float) * size_t(2 * B) * p.nblk);
  return p;
}

template <class DT, int EPL, int VEC>
void launch_ln_bwd_t(const LnPlan& p, const void* dy, const void* x, const void* w, int w_dtype,
                     const float* mean, const float* rstd, int64_t B, int64_t T, int64_t H,
                     void* dx, float* part, hipStream_t s) {
  using S = typename DT::storage;
  hipLaunchKernelGGL((ln_bwd_kernel<DT, EPL, VEC>), dim3(p.chunks, B), dim3(NT),
                     sizeof(float) * 2 * H, s, static_cast<const S*>(dy),
                     static_cast<const S*>(x), w, w_dtype, mean, rstd, T, H, p.rows, p.chunks,
                     static_cast<S*>(dx), part, B);
}

template <class DT, int VEC>
void launch_ln_bwd_v(int epl, const LnPlan& p, const void* dy, const void* x, const void* w,
                     int w_dtype, const float* mean, const float* rstd, int64_t B, int64_t T,
                     int64_t H, void* dx, float* part, hipStream_t s) {
  switch (epl) {
    case 8: launch_ln_bwd_t<DT, 8, VEC>(p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s); break;
    case 16: launch_ln_bwd_t<DT, 16, VEC>(p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s); break;
    case 32: launch_ln_bwd_t<DT, 32, VEC>(p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s); break;
    default: launch_ln_bwd_t<DT, 64, VEC>(p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s); break;
  }
}

template <class DT>
void launch_ln_bwd(bool vec, int epl, const LnPlan& p, const void* dy, const void* x,
                   const void* w, int w_dtype, const float* mean, const float* rstd, int64_t B,
                   int64_t T, int64_t H, void* dx, float* part, hipStream_t s) {
  if (!vec) launch_ln_bwd_v<DT, 1>(epl, p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s);
  else if constexpr (DT::code == FDP_F32)
    launch_ln_bwd_v<DT, 4>(epl, p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s);
  else launch_ln_bwd_v<DT, 8>(epl, p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s);
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

void zero_fill(float* p, int64_t n, hipStream_t s) {
  int64_t g = (n + NT - 1) / NT;
  if (g > 1024) g = 1024;
  if (g < 1) g = 1;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(g)), dim3(NT), 0, s, p, n);
}

}  // namespace

// ------------------------------------------------------------ C ABI
extern "C" int fdp_colsum_clip_workspace_size(int64_t B, int64_t T, int64_t H, int dtype,
                                              size_t* bytes) {
  if (bytes == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || T < 0 || H < 1) return FDP_ERR_SHAPE;
  // The aligned plan has the most chunk partials; size for the larger of both.
  const ColPlan a = col_plan(B, T, H, dtype, num_cus(), true);
  const ColPlan u = col_plan(B, T, H, dtype, num_cus(), false);
  *bytes = a.total > u.total ? a.total : u.total;
  return FDP_OK;
}

extern "C" int fdp_colsum_clip(const void* u, const void* v, int64_t B, int64_t T, int64_t H,
                               int dtype, int norm_kind, float C, float clamp,
                               const float* clip_args_dev, float out_scale, const void* noise,
                               float noise_scale, void* out, int out_dtype, float* norms,
                               float* factors, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return FDP_ERR_DTYPE;
  if (norm_kind != FDP_NORM_SUM && norm_kind != FDP_NORM_FROB) return FDP_ERR_ARG;
  if (B < 1 || T < 0 || H < 1) return FDP_ERR_SHAPE;
  // samples index grid.y / grid.z (at most 65535)
  if (B > 32767 || H > (int64_t(1) << 31)) return FDP_ERR_SHAPE;
  if ((T > 0 && u == nullptr) || out == nullptr) return FDP_ERR_ARG;
  const bool aligned = aligned16(u) && (v == nullptr || aligned16(v)) &&
                       (H * esize(dtype)) % 16 == 0;
  const int cus = num_cus();
  const ColPlan p = col_plan(B, T, H, dtype, cus, aligned);
  if (workspace == nullptr || workspace_bytes < p.total) return FDP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return FDP_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws + p.off_part);
  float* frob = norm_kind == FDP_NORM_FROB ? reinterpret_cast<float*>(ws + p.off_frob) : nullptr;
  float* sums = reinterpret_cast<float*>(ws + p.off_sums);
  float* fac = reinterpret_cast<float*>(ws + p.off_fac);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T > 0) {
    if (dtype == FDP_BF16) launch_colsum_dt<BF16>(p, u, v, B, T, H, part, frob, s);
    else if (dtype == FDP_F16) launch_colsum_dt<F16>(p, u, v, B, T, H, part, frob, s);
    else launch_colsum_dt<F32>(p, u, v, B, T, H, part, frob, s);
  } else {
    zero_fill(part, int64_t(B) * p.chunks * H, s);
    if (frob) zero_fill(frob, int64_t(B) * p.chunks * p.cblocks, s);
  }
  float* sq = reinterpret_cast<float*>(ws + p.off_sq);
  hipLaunchKernelGGL(chunk_reduce_kernel, dim3(static_cast<unsigned>(p.nblk), static_cast<unsigned>(B)),
                     dim3(NT), 0, s, part, H, p.chunks, sums, sq);
  hipLaunchKernelGGL(stream_factor_kernel, dim3(static_cast<unsigned>((B + 3) / 4)), dim3(NT), 0, s,
                     frob ? static_cast<const float*>(frob) : static_cast<const float*>(sq), B,
                     frob ? p.chunks * p.cblocks : p.nblk, C, clamp, clip_args_dev, fac, norms,
                     factors);
  hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>((H + NT - 1) / NT)), dim3(NT), 0,
                     s, sums, fac, B, H, out_scale, noise, static_cast<const void*>(nullptr),
                     noise_scale, out, static_cast<void*>(nullptr), out_dtype);
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
                                      float noise_scale, void* dx, void* dw, void* db,
                                      float* norms, float* factors, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(w_dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || T < 0 || H < 1 || H > kMaxLnH) return FDP_ERR_SHAPE;
  if (B > 32767) return FDP_ERR_SHAPE;  // 2B streams index grid.y
  if (T > 0 && (dy == nullptr || x == nullptr || dx == nullptr || mean == nullptr ||
                rstd == nullptr))
    return FDP_ERR_ARG;
  const int cus = num_cus();
  const LnPlan p = ln_plan(B, T, H, cus);
  if (workspace == nullptr || workspace_bytes < p.total) return FDP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return FDP_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws + p.off_part);
  float* sums = reinterpret_cast<float*>(ws + p.off_sums);
  float* fac = reinterpret_cast<float*>(ws + p.off_fac);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = aligned16(dy) && aligned16(x) && aligned16(dx) && (H * esize(dtype)) % 16 == 0;
  const int epl = ln_epl(H);
  if (T > 0) {
    if (dtype == FDP_BF16) launch_ln_bwd<BF16>(vec, epl, p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s);
    else if (dtype == FDP_F16) launch_ln_bwd<F16>(vec, epl, p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s);
    else launch_ln_bwd<F32>(vec, epl, p, dy, x, w, w_dtype, mean, rstd, B, T, H, dx, part, s);
  } else {
    zero_fill(part, int64_t(2 * B) * p.chunks * H, s);
  }
  float* sq = reinterpret_cast<float*>(ws + p.off_sq);
  hipLaunchKernelGGL(chunk_reduce_kernel,
                     dim3(static_cast<unsigned>(p.nblk), static_cast<unsigned>(2 * B)), dim3(NT), 0,
                     s, part, H, p.chunks, sums, sq);
  hipLaunchKernelGGL(stream_factor_kernel, dim3(static_cast<unsigned>((2 * B + 3) / 4)), dim3(NT),
                     0, s, static_cast<const float*>(sq), 2 * B, p.nblk, C, clamp, clip_args_dev,
                     fac, norms, factors);
  if (dw != nullptr || db != nullptr) {
    // combine_kernel writes out0 from streams [0,B) and out1 from [B,2B).
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>((H + NT - 1) / NT)), dim3(NT),
                       0, s, sums, fac, B, H, out_scale, noise_w, noise_b, noise_scale, dw, db,
                       w_dtype);
  }
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
    default: return "unknown status";
  }
}

extern "C" int fdp_version(void) { return 100; }
