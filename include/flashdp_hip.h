/*
 * flashdp_hip.h - C ABI of libflashdp_hip.so, the MI355X (gfx950) kernels
 * behind the FlashDP DP-SGD hot path.
 *
 * The reference exposes only a Python operator API (flashdp/core/__init__.py:1-11)
 * whose functions launch Triton kernels; these entry points are the device work
 * those operators stand for.  Each declaration names the reference function it
 * replaces.  The host side (flashdp4review_amd/_lib.py) binds them with ctypes.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are device pointers (HBM) of contiguous row-major
 *     tensors unless a stride argument says otherwise.  Sizes are elements.
 *   - The caller owns every buffer, including the workspace; the library never
 *     allocates device memory and never synchronises the host.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream)
 *     in stream order.  Entry points keep no global mutable state, so calls on
 *     different streams may run concurrently with distinct workspaces.
 *   - Return 0 (FDP_OK) or a positive fdp_status; fdp_strerror() names it.
 *   - Clip factor: c = min(clamp, C / (norm + 1e-10))      (clip_fn.py:6-8).
 *     When `clip_args_dev` is non-NULL it points at two device floats
 *     {C, clamp} and overrides the scalar C/clamp arguments, the same device
 *     layout the reference's Triton kernels read (clip_fn.py:21-25).
 *   - Optional outputs (norms, factors, noise) may be NULL.
 *   - Noise (the layers' torch.normal draw + add_, flashdp/layers/linear.py:74-92):
 *     out += noise_scale * z with z either an injected tensor (`noise`), or,
 *     when `noise` is NULL and `noise_key` is not, standard normals drawn in
 *     the kernels (fdp_noise_key below); neither: no noise.
 */
#ifndef FLASHDP_HIP_H
#define FLASHDP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fdp_dtype {
  FDP_F32 = 0,
  FDP_F16 = 1,
  FDP_BF16 = 2
} fdp_dtype;

typedef enum fdp_status {
  FDP_OK = 0,
  FDP_ERR_DTYPE = 1,     /* unsupported dtype            -> KeyError     */
  FDP_ERR_SHAPE = 2,     /* bad / unsupported sizes       -> ValueError   */
  FDP_ERR_ARG = 3,       /* NULL pointer, bad flag        -> ValueError   */
  FDP_ERR_WORKSPACE = 4, /* workspace too small           -> RuntimeError */
  FDP_ERR_HIP = 5,       /* HIP launch error              -> RuntimeError */
  FDP_ERR_ALIGN = 6,     /* pointer alignment violated    -> ValueError   */
  FDP_ERR_TOO_LARGE = 7  /* needs more than the no-allocation scratch -> ValueError */
} fdp_status;

/* Operand layouts of the per-sample product G_b (b = 0..B-1).
 *   FDP_LAYOUT_TN: a is [B, K, M], b is [B, K, N]:  G_b = a_b^T b_b
 *                  (bmtm_clip, flashdp/core/bmtm_clip_loop.py:162-173;
 *                   Linear weight grad g^T x, flashdp/core/linear_clip.py:94-113)
 *   FDP_LAYOUT_NN: a is [B, M, K], b is [B, K, N]:  G_b = a_b b_b
 *                  (bmm_clip, flashdp/core/bmm_clip_loop.py:150-162)          */
typedef enum fdp_layout {
  FDP_LAYOUT_TN = 0,
  FDP_LAYOUT_NN = 1
} fdp_layout;

/* In-kernel Gaussian noise.  Output k of a call (k = 0; the LayerNorm entry
 * point's db is k = 1) gets, at its row-major element e, the (e mod 4)-th of
 * four normals made from the Philox4x32-10 block (Salmon et al., SC'11)
 *   counter {lo32(q), hi32(q), k, 0}, key {lo32(seed), hi32(seed)},
 *   q = offset + e/4 (+ *counter when `counter` is set)
 * whose words (w0, w1) and (w2, w3) each give two normals by Box-Muller:
 *   r = sqrt(-2 ln u_first), z = (r cos 2 pi u_second, r sin 2 pi u_second),
 *   u_first = (w_first + 0.5) / 2^32, u_second = ((w_second >> 8) + 0.5) / 2^24,
 * so |z| <= sqrt(-2 ln 2^-33) = 6.76 (the tail beyond holds about 1.4e-11 of
 * a normal's mass).
 * A call uses counter blocks [offset, offset + ceil(numel / 4)) of each output
 * (shifted by *counter); callers advance `offset` (or change `seed`) between
 * calls.  The struct is read on the host during the call.
 * counter: NULL, or a device pointer to a 64-bit block count that the kernels
 * read when they run (not when the call is made).  Work captured once into a
 * HIP graph and replayed then draws fresh noise on every replay if the
 * caller enqueues fdp_noise_advance(counter, blocks) after the call, in the
 * same capture (the reference's torch.normal on the device generator does the
 * same through the generator's offset, flashdp/layers/linear.py:74-80). */
typedef struct fdp_noise_key {
  uint64_t seed;
  uint64_t offset;
  const uint64_t* counter;
} fdp_noise_key;

/* *counter += blocks, stream-ordered (a one-thread kernel; no memset, so it
 * may be captured into a HIP graph).  No counterpart in the reference: the
 * device-side advance of a noise key's counter (see fdp_noise_key). */
int fdp_noise_advance(uint64_t* counter, uint64_t blocks, void* stream);

/* Which per-sample norm drives the clip of a column-sum reduction.
 *   FDP_NORM_SUM:  || sum_t u_bt (.* v_bt) ||_2       (LayerNorm dgamma/dbeta,
 *                  flashdp/core/layernorm_clip.py:163-198)
 *   FDP_NORM_FROB: || u_b ||_F over all T*H entries   (Linear/Conv1D bias,
 *                  flashdp/core/linear_clip.py:116-123)                     */
typedef enum fdp_norm_kind {
  FDP_NORM_SUM = 0,
  FDP_NORM_FROB = 1
} fdp_norm_kind;

const char* fdp_strerror(int status);
/* Library version, e.g. 100 for 0.1.0. */
int fdp_version(void);

/* ------------------------------------------------------------------------
 * Clipped per-sample product sum (the DP-SGD weight-gradient hot path):
 *
 *   out[m,n] = out_scale * sum_b c_b * G_b[m,n] + noise_scale * noise[m,n]
 *   c_b      = min(clamp, C / (||G_b||_F + 1e-10))
 *
 * Replaces: bmtm_clip_triton / mtm_clip (flashdp/core/bmtm_clip_loop.py:137-173),
 *           bmm_clip_triton / mm_clip (flashdp/core/bmm_clip_loop.py:129-162),
 *           mm_clip_triton (flashdp/core/mm_clip_loop.py:127-139, as B=K, K=1),
 *           _weight_grad_block_clip + linear_weight_flashdp
 *           (flashdp/core/linear_clip.py:94-113) and the .div_(B) + noise add_
 *           of _DPLinearFunc.backward (flashdp/layers/linear.py:72-80).
 *
 * a, b     : input dtype `dtype` (F32, F16 or BF16), batch strides
 *            stride_ab / stride_bb and row strides lda / ldb in elements
 *            (row = the contiguous dimension's parent: for TN, a row of a_b
 *            is one k; for NN, one m).  The innermost dimension must be
 *            contiguous.  The single-pass and streamed kernels address one
 *            sample's operand through a 32-bit buffer record: a sample whose
 *            K (rounded up to 128) times its row stride reaches 2^30 elements
 *            takes the generic two-pass schedule (64-bit addressing) instead.
 * out      : [M, N] row-major with row stride ldo, dtype `out_dtype`.
 * noise    : NULL or [M, N] contiguous, dtype `out_dtype`.
 * noise_key: NULL, or the in-kernel draw used when `noise` is NULL.
 * norms    : NULL or [B] fp32, ||G_b||_F.
 * factors  : NULL or [B] fp32, c_b.
 * flags    : bit 0 (FDP_WGRAD_NOCLIP) skips the norm pass and uses c_b = clamp
 *            (a plain batched product sum; `norms` must then be NULL);
 *            bit 1 (FDP_WGRAD_TWO_PASS) forces the two-pass schedule (norm
 *            pass, then clipped-sum pass) instead of the single-pass kernel
 *            the library uses whenever the problem fits it (16-bit TN
 *            operands, aligned rows, at most two 128x128 output tiles per
 *            CU); larger layers always take the two-pass schedule, whose norm
 *            pass uses the per-sample Gram matrices when that is cheaper;
 *            bit 2 (FDP_WGRAD_PLAIN_LAUNCH) dispatches the single-pass kernel
 *            as an ordinary launch instead of a cooperative one, saving the
 *            runtime's cooperative-launch synchronisation (about 15 us per
 *            call on MI355X).  The grid is sized to the kernel's occupancy,
 *            so it is resident at once when nothing else occupies the device;
 *            work on other streams only delays it.  The caller must not run
 *            concurrently a kernel that waits on this one.  Should a bounded
 *            grid wait (seconds) still expire, the affected outputs (and
 *            norms/factors) are NaN and the status word below is set;
 *            bits 4 and 5 choose between the two single-pass kernels for
 *            16-bit TN operands: by default the wide kernel (one 384x192 or
 *            192x384 output tile of one sample per CU, eight waves) is used
 *            when the layer's tiles times the batch fit the CUs and fill at
 *            least 70% of them, and the grouped kernel (128x128 tiles, several
 *            samples per workgroup) otherwise; bit 4 (FDP_WGRAD_WIDE) takes the
 *            wide kernel whenever the products fit the CUs at all, bit 5
 *            (FDP_WGRAD_NARROW) never takes it.  Where the batch is even
 *            (6 <= B <= 72) and K is a multiple of 32, the wide schedule
 *            holds two samples' 192x192 tiles per CU and adds them inside
 *            the CU (a quarter to a half of the exchanged bytes), with or
 *            without a bias; bit 7 (FDP_WGRAD_UNPAIRED) keeps one sample per
 *            CU;
 *            bit 3 (FDP_WGRAD_CLEAN_WORKSPACE) states that the workspace's
 *            control words (its first 2048 bytes) are valid -- a zero-filled
 *            buffer, or one whose last use was a completed fdp_wgrad_clip call
 *            of any shape, which always leaves them valid -- so the library
 *            skips clearing them.
 * workspace: device buffer of at least fdp_wgrad_clip_workspace_size() bytes,
 *            16-byte aligned.  Its first int is a status word: nonzero after
 *            the call completes means a bounded inter-workgroup wait of the
 *            single-pass kernel expired in this call or an earlier one since
 *            the caller last zeroed the word (results of the call whose wait
 *            expired are NaN).  The word is sticky: the library only sets it,
 *            the caller reads and zeroes it.  An expiry affects only the
 *            launch it happened in: the other control words carry a
 *            per-launch tag (word 2 counts launches), so later calls on the
 *            same workspace are exact whether or not the word was zeroed.
 * ---------------------------------------------------------------------- */
#define FDP_WGRAD_NOCLIP 1
#define FDP_WGRAD_TWO_PASS 2
#define FDP_WGRAD_PLAIN_LAUNCH 4
#define FDP_WGRAD_CLEAN_WORKSPACE 8
#define FDP_WGRAD_WIDE 16
#define FDP_WGRAD_NARROW 32
#define FDP_WGRAD_UNPAIRED 128

int fdp_wgrad_clip_workspace_size(int64_t B, int64_t K, int64_t M, int64_t N,
                                  int dtype, int flags, size_t* bytes);

int fdp_wgrad_clip(const void* a, const void* b, int64_t B, int64_t K, int64_t M,
                   int64_t N, int64_t stride_ab, int64_t lda, int64_t stride_bb,
                   int64_t ldb, int layout, int dtype, float C, float clamp,
                   const float* clip_args_dev, float out_scale, const void* noise,
                   float noise_scale, const fdp_noise_key* noise_key, void* out,
                   int64_t ldo, int out_dtype, float* norms, float* factors, int flags,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * The weight and bias gradients of a DP Linear or Conv1D layer in one call
 * (replaces the pair linear_weight_flashdp + linear_bias_grad_clip in the
 * reference's DPLinear backward, flashdp/layers/linear.py:72-92, with
 * flashdp/core/linear_clip.py:107-123; and conv1d_weight_flashdp +
 * conv1d_bias_grad_clip, flashdp/core/transformers_conv1d_clip.py:22-39, as
 * DPConv1D's backward intends them, flashdp/layers/transformers_conv1d.py:59-66):
 *
 *   out  = as fdp_wgrad_clip (layout FDP_LAYOUT_TN),
 *   bias[c] = bias->out_scale * sum_b c'_b sum_k op_b[k,c] + bias->noise_scale * zb[c],
 *   c'_b = min(clamp, C / (||op_b||_F + 1e-10))   (the weight's C, clamp),
 *
 * where op is operand a ([B,K,M]: a Linear's grad_output, G_b = g_b^T x_b),
 * or, with flags bit 6 (FDP_WGRAD_BIAS_OF_B), operand b ([B,K,N]: a Conv1D's
 * grad_output, G_b = x_b^T g_b).  This is linear_bias_grad_clip with
 * out_scale = 1/(B*K) (its mean over B*T) and noise_scale = sigma/sqrt(B).
 * zb is bias->noise (len values of bias->out_dtype, len = M or N) or, without
 * one, the in-kernel draw of bias->noise_key (stream 0, as fdp_colsum_clip).
 * The bias operand must be contiguous (stride K*len, row stride len);
 * FDP_WGRAD_NOCLIP is not accepted.  The 16-bit TN kernels (wide, grouped and
 * streamed schedules) form the bias from the operand fragments they already
 * hold, so grad_output is read once; the generic schedule (fp32 operands,
 * unaligned rows) runs fdp_colsum_clip (FDP_NORM_FROB) after the weight
 * gradient.  bias->norms / bias->factors (optional, B floats) receive
 * ||op_b||_F and c'_b.
 * Workspace: fdp_wgrad_bias_clip_workspace_size bytes (pass the same flags,
 * FDP_WGRAD_BIAS_OF_B included); its first fdp_wgrad_clip_workspace_size
 * bytes (rounded up to 256) are the weight gradient's workspace, with the
 * same rules (FDP_WGRAD_CLEAN_WORKSPACE); the rest needs no clearing.
 * ---------------------------------------------------------------------- */
#define FDP_WGRAD_BIAS_OF_B 64

typedef struct fdp_bias_out {
  void* out;
  int out_dtype;
  float out_scale;
  const void* noise;
  float noise_scale;
  const fdp_noise_key* noise_key;
  float* norms;
  float* factors;
} fdp_bias_out;

int fdp_wgrad_bias_clip_workspace_size(int64_t B, int64_t K, int64_t M, int64_t N, int dtype,
                                       int flags, size_t* bytes);
int fdp_wgrad_bias_clip(const void* a, const void* b, int64_t B, int64_t K, int64_t M, int64_t N,
                        int64_t stride_ab, int64_t lda, int64_t stride_bb, int64_t ldb,
                        int layout, int dtype, float C, float clamp, const float* clip_args_dev,
                        float out_scale, const void* noise, float noise_scale,
                        const fdp_noise_key* noise_key, void* out, int64_t ldo, int out_dtype,
                        float* norms, float* factors, int flags, const fdp_bias_out* bias,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * fdp_wgrad_clip for callers that cannot allocate device memory.
 *
 * No counterpart in the reference: it serves callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as fdp_wgrad_clip, without the
 * workspace: the library uses a file-scope device array of
 * FDP_NOALLOC_SCRATCH_BYTES (64 MiB) that each GPU it runs on holds until the
 * process ends (its address is resolved per device on the first call).  The
 * call allocates nothing and uses the ordinary launch (FDP_WGRAD_PLAIN_LAUNCH
 * is implied; FDP_WGRAD_CLEAN_WORKSPACE is ignored: every call clears the
 * array's control words with a fill kernel).  Problems whose
 * fdp_wgrad_clip_workspace_size exceeds the array return FDP_ERR_TOO_LARGE
 * without launching.  All calls on one GPU share the array: calls that
 * overlap on one GPU race, so the caller serialises them.  The array's
 * status word is not visible to the caller: an expired bounded wait shows
 * only as NaN outputs.  `stream` must belong to the current device (its
 * copy of the array and its CU count are used): FDP_ERR_ARG otherwise.  The
 * call may be captured into a HIP graph (it records kernels only, no memset);
 * a noise key with a device counter plus fdp_noise_advance then draws fresh
 * noise on every replay.
 * ---------------------------------------------------------------------- */
#define FDP_NOALLOC_SCRATCH_BYTES (64u << 20)

int fdp_wgrad_clip_noalloc(const void* a, const void* b, int64_t B, int64_t K, int64_t M,
                           int64_t N, int64_t stride_ab, int64_t lda, int64_t stride_bb,
                           int64_t ldb, int layout, int dtype, float C, float clamp,
                           const float* clip_args_dev, float out_scale, const void* noise,
                           float noise_scale, const fdp_noise_key* noise_key, void* out,
                           int64_t ldo, int out_dtype, float* norms, float* factors, int flags,
                           void* stream);

/* ------------------------------------------------------------------------
 * Input gradient of a DP Linear or Conv1D layer (the unclipped product of its
 * backward that reads the same grad_output as the clipped weight gradient):
 *
 *   dx[m, n] = sum_k g[m, k] * W(k, n)
 *
 *   FDP_DGRAD_NN: W(k, n) = w[k, n], w [K, N] row stride ldw -- a Linear
 *                 weight [out, in]: grad_input = grad_output @ weight
 *                 (flashdp/layers/linear.py:62-67);
 *   FDP_DGRAD_NT: W(k, n) = w[n, k], w [N, K] row stride ldw -- a Conv1D
 *                 weight [in, out]: grad_input = grad_output @ weight.t()
 *                 (flashdp/layers/transformers_conv1d.py:70-77).
 *
 * g  : [M, K] (M = B*T rows of grad_output, K = out features), row stride ldg.
 * dx : [M, N], row stride ldo.  g, w and dx share `dtype` (FDP_F16 or
 *      FDP_BF16); products accumulate in fp32 and dx is rounded once.
 * Requirements (FDP_ERR_SHAPE / FDP_ERR_ALIGN otherwise, nothing launched):
 *      K a multiple of 64; ldg and ldw multiples of 8 elements; g and w
 *      16-byte aligned; g and w each span less than 2 GiB.
 * No workspace: each workgroup forms whole output tiles and waits for no
 * other, so the call only enqueues one kernel on `stream` (it may be
 * captured into a HIP graph).  The result is deterministic (fixed summation
 * order).
 * ---------------------------------------------------------------------- */
typedef enum fdp_dgrad_layout {
  FDP_DGRAD_NN = 0,
  FDP_DGRAD_NT = 1
} fdp_dgrad_layout;

int fdp_dgrad(const void* g, const void* w, void* dx, int64_t M, int64_t N, int64_t K,
              int64_t ldg, int64_t ldw, int64_t ldo, int layout, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Clipped per-sample column sums over the middle axis:
 *
 *   S_b[h]  = sum_t u[b,t,h] * (v ? v[b,t,h] : 1)
 *   n_b     = ||S_b||_2 (FDP_NORM_SUM) or ||u_b||_F (FDP_NORM_FROB)
 *   out[h]  = out_scale * sum_b c_b S_b[h] + noise_scale * noise[h]
 *
 * Replaces: linear_bias_grad_clip (flashdp/core/linear_clip.py:116-123, with
 *           out_scale = 1/(B*T), without its in-place write to grad_output),
 *           conv1d_bias_grad_clip (flashdp/core/transformers_conv1d_clip.py:31-39),
 *           layernorm_dw_clip (v = x_hat) and layernorm_db_clip (v = NULL)
 *           (flashdp/core/layernorm_clip.py:163-198, out_scale = 1/B) and the
 *           noise add_ of the layers (flashdp/layers/linear.py:84-92,
 *           flashdp/layers/layernorm.py:139-155).
 * u, v     : [B, T, H] contiguous, dtype `dtype`; v may be NULL.
 * out      : [H], dtype `out_dtype`; noise NULL or [H] of `out_dtype`;
 *            noise_key as for fdp_wgrad_clip.
 * ---------------------------------------------------------------------- */
int fdp_colsum_clip_workspace_size(int64_t B, int64_t T, int64_t H, int dtype,
                                   size_t* bytes);

int fdp_colsum_clip(const void* u, const void* v, int64_t B, int64_t T, int64_t H,
                    int dtype, int norm_kind, float C, float clamp,
                    const float* clip_args_dev, float out_scale, const void* noise,
                    float noise_scale, const fdp_noise_key* noise_key, void* out,
                    int out_dtype, float* norms, float* factors, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * LayerNorm forward over the last axis, fp32 statistics:
 *   mean_r = mean(x_r), rstd_r = 1/sqrt(var_r + eps) (biased var),
 *   y_r = (x_r - mean_r) * rstd_r * w + b
 * Replaces: layernorm_fwd_fused_triton / _layer_norm_fwd_fused
 *           (flashdp/core/layernorm_clip.py:11-60,201-239).
 * x, y     : [rows, H] contiguous, dtype `dtype`; 1 <= H <= 2^30 (rows of more
 *            than 64 KB, which the reference's fused kernel rejects, included).
 * w, b     : [H] of `w_dtype`; either may be NULL (weight 1 / bias 0).
 * mean,rstd: [rows] fp32 (either may be NULL).
 * ---------------------------------------------------------------------- */
int fdp_layernorm_fwd(const void* x, const void* w, const void* b, int64_t rows,
                      int64_t H, float eps, int dtype, int w_dtype, void* y,
                      float* mean, float* rstd, void* stream);

/* ------------------------------------------------------------------------
 * LayerNorm backward with per-sample clipped gamma/beta gradients:
 *   x_hat = (x - mean) * rstd
 *   dx    = rstd * (w.dy - mean_h(w.dy) - x_hat * mean_h(w.dy.x_hat))
 *   P_b   = sum_t dy.x_hat,  Q_b = sum_t dy                  (per sample)
 *   dw    = out_scale * sum_b clip(||P_b||) P_b + noise_scale * noise_w
 *   db    = out_scale * sum_b clip(||Q_b||) Q_b + noise_scale * noise_b
 * Replaces: layernorm_bwd_clip_fused_triton + layernorm_dwdb_fused_triton
 *           (flashdp/core/layernorm_clip.py:63-160,241-315) with the per-sample
 *           math of layernorm_dw_clip / layernorm_db_clip
 *           (flashdp/core/layernorm_clip.py:163-198) and one noise draw each
 *           (flashdp/layers/layernorm.py:139-155).
 * dy, x, dx: [B, T, H] contiguous, dtype `dtype` (dx may alias nothing);
 *            1 <= H <= 2^30.
 * w        : [H] of `w_dtype` or NULL (weight 1).
 * mean,rstd: [B*T] fp32 from fdp_layernorm_fwd.
 * dw, db   : [H] of `w_dtype`; either may be NULL to skip it.
 * norms    : NULL or [2*B] fp32 (||P_b|| then ||Q_b||); factors likewise.
 * noise_key: as for fdp_wgrad_clip; dw draws stream k = 0, db k = 1.
 * ---------------------------------------------------------------------- */
int fdp_layernorm_bwd_clip_workspace_size(int64_t B, int64_t T, int64_t H,
                                          int dtype, size_t* bytes);

int fdp_layernorm_bwd_clip(const void* dy, const void* x, const void* w,
                           const float* mean, const float* rstd, int64_t B,
                           int64_t T, int64_t H, int dtype, int w_dtype, float C,
                           float clamp, const float* clip_args_dev,
                           float out_scale, const void* noise_w,
                           const void* noise_b, float noise_scale,
                           const fdp_noise_key* noise_key, void* dx, void* dw, void* db,
                           float* norms, float* factors, void* workspace,
                           size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHDP_HIP_H */
