"""CPU oracle for the FlashDP DP-SGD hot path, in float64 numpy.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline) -- never as a fallback of the product path,
which runs on the HIP library and raises when it is missing.

Each function restates the reference's math (paths relative to the reference
repository liangyuwang/FlashDP4Review) on float64 copies of its inputs:

  clip_factor           flashdp/core/clip_fn.py:6-8
  wgrad_clip            flashdp/core/linear_clip.py:94-104 (per-sample einsum,
                        norm, clamp, mul, sum), flashdp/core/bmtm_clip_loop.py:162-173
                        (layout "tn"), flashdp/core/bmm_clip_loop.py:150-162 ("nn")
  mm_clip               flashdp/core/mm_clip_loop.py:127-139
  linear_backward       flashdp/layers/linear.py:48-104 (+ linear_clip.py:107-123)
  conv1d_backward       flashdp/core/transformers_conv1d_clip.py:22-28 with the
                        bias of flashdp/layers/transformers_conv1d.py:59-66
  colsum_clip           flashdp/core/linear_clip.py:116-123 (FROB) and
                        flashdp/core/layernorm_clip.py:163-198 (SUM)
  layernorm_fwd         flashdp/core/layernorm_clip.py:26-60
  layernorm_bwd_clip    flashdp/core/layernorm_clip.py:98-107 (dx) with the
                        per-sample dgamma/dbeta of layernorm_clip.py:163-198 and
                        flashdp/layers/layernorm.py:128-155

Deliberate deviations from the reference (each pinned by a test):
  - grad_output is never modified in place (reference: linear_clip.py:118-121);
  - Conv1D uses the intended x^T g orientation (transformers_conv1d_clip.py:22-28;
    the reference layer routes through the Linear helper, layers/transformers_conv1d.py:80-95);
  - LayerNorm clips per sample with one noise draw each for dgamma and dbeta
    (reference fused path clamps lock-group partials elementwise,
    layernorm_clip.py:118-127; non-fused path adds both draws to dgamma,
    layers/layernorm.py:140-155);
  - noise is an explicit argument z (standard normal) scaled by
    noise_multiplier / sqrt(B), the reference's std (layers/linear.py:74-80).

How each function is pinned (tests/test_oracle.py): clip_factor by closed
forms; wgrad_clip by a brute-force loop over (b, m, n, k) on tiny inputs, the
Gram identity ||a^T b||_F^2 = sum_{t,s}(a_t.a_s)(b_t.b_s), the single-GEMM
identity sum_b c_b a_b^T b_b = A^T diag(c) B, torch autograd of nn.Linear at
C -> inf, and the exact norm C*clamp of every clipped term when ||G_b|| >> C;
mm_clip by ||a (x) b|| = ||a|| ||b||; colsum_clip and layernorm_bwd_clip by
torch autograd of F.layer_norm / sums at C -> inf and by brute-force loops;
layernorm_fwd by torch.nn.functional.layer_norm.  No function is left
"parity unpinned".
"""
from __future__ import annotations

import numpy as np

EPS_CLIP = 1e-10


def _f64(a):
    if a is None:
        return None
    if hasattr(a, "detach"):  # torch tensor
        a = a.detach().cpu().double().numpy() if a.dtype.is_floating_point else a.cpu().numpy()
    return np.asarray(a, dtype=np.float64)


def clip_factor(norm, C, clamp_value):
    """min(clamp, C / (norm + 1e-10)) -- flashdp/core/clip_fn.py:6-8."""
    norm = np.asarray(norm, dtype=np.float64)
    return np.minimum(C / (norm + EPS_CLIP), clamp_value)


def wgrad_clip(a, b, C=1.0, clamp_value=1.0, layout="tn", out_scale=1.0, noise=None,
               noise_scale=1.0, noclip=False):
    """Clipped per-sample product sum.

    layout "tn": a [B,K,M], b [B,K,N], G_b = a_b^T b_b  (bmtm_clip_loop.py:162-173)
    layout "nn": a [B,M,K], b [B,K,N], G_b = a_b b_b    (bmm_clip_loop.py:150-162)
    Returns (out [M,N], norms [B], factors [B]) with
    out = out_scale * sum_b c_b G_b + noise_scale * noise.
    """
    a, b = _f64(a), _f64(b)
    if layout == "tn":
        G = np.einsum("bkm,bkn->bmn", a, b)
    elif layout == "nn":
        G = np.einsum("bmk,bkn->bmn", a, b)
    else:
        raise ValueError(layout)
    norms = np.sqrt((G * G).sum(axis=(1, 2)))
    if noclip:
        fac = np.full_like(norms, clamp_value)
        norms = np.zeros_like(norms)
    else:
        fac = clip_factor(norms, C, clamp_value)
    out = out_scale * np.einsum("b,bmn->mn", fac, G)
    if noise is not None:
        out = out + noise_scale * _f64(noise)
    return out, norms, fac


def mm_clip(mat1, mat2, C=1.0, clamp_value=1.0):
    """sum_k clip(||a_k (x) b_k||) a_k (x) b_k, a_k = mat1[:,k], b_k = mat2[k,:]
    -- flashdp/core/mm_clip_loop.py:127-139 (one rank-1 term per k)."""
    m1, m2 = _f64(mat1), _f64(mat2)
    a = m1.T[:, None, :]  # [K,1,M]
    b = m2[:, None, :]    # [K,1,N]
    out, _, _ = wgrad_clip(a, b, C, clamp_value, layout="tn")
    return out


def colsum_clip(u, v=None, C=1.0, clamp_value=1.0, norm_kind="sum", out_scale=1.0,
                noise=None, noise_scale=1.0):
    """S_b = sum_t u_bt (* v_bt); n_b = ||S_b|| ("sum") or ||u_b||_F ("frob");
    out = out_scale * sum_b c_b S_b + noise_scale * noise.
    "frob": flashdp/core/linear_clip.py:116-123; "sum": layernorm_clip.py:163-198."""
    u = _f64(u)
    B, H = u.shape[0], u.shape[-1]
    u3 = u.reshape(B, -1, H)
    p = u3 if v is None else u3 * _f64(v).reshape(B, -1, H)
    S = p.sum(axis=1)
    if norm_kind == "sum":
        norms = np.sqrt((S * S).sum(axis=1))
    elif norm_kind == "frob":
        norms = np.sqrt((u3 * u3).sum(axis=(1, 2)))
    else:
        raise ValueError(norm_kind)
    fac = clip_factor(norms, C, clamp_value)
    out = out_scale * (fac[:, None] * S).sum(axis=0)
    if noise is not None:
        out = out + noise_scale * _f64(noise)
    return out, norms, fac


def _as_btf(t):
    """Reference reshape of layers/linear.py:51-58: 2-D -> [B,1,F]; >3-D -> [B,K,F]."""
    if t.ndim == 2:
        return t[:, None, :]
    if t.ndim > 3:
        return t.reshape(t.shape[0], -1, t.shape[-1])
    return t


def linear_backward(x, g, W, C=1.0, clamp_value=1.0, noise_multiplier=0.0, z_w=None, z_b=None,
                    bias=True):
    """_DPLinearFunc.backward, flashdp/layers/linear.py:48-104.

    x [..., I], g [..., O], W [O, I].  Returns dict with dx (shape of x), dw [O,I],
    db [O] (or None), norms_w, fac_w, norms_b, fac_b.  z_w / z_b are standard
    normal draws scaled here by noise_multiplier / sqrt(B)."""
    x, g, W = _f64(x), _f64(g), _f64(W)
    x3, g3 = _as_btf(x), _as_btf(g)
    B, T = x3.shape[0], x3.shape[1]
    std = noise_multiplier / np.sqrt(B)
    dx = (g3 @ W).reshape(x.shape)
    dw, nw, fw = wgrad_clip(g3, x3, C, clamp_value, "tn", out_scale=1.0 / B,
                            noise=z_w, noise_scale=std)
    out = {"dx": dx, "dw": dw, "norms_w": nw, "fac_w": fw, "db": None}
    if bias:
        db, nb, fb = colsum_clip(g3, None, C, clamp_value, "frob", out_scale=1.0 / (B * T),
                                 noise=z_b, noise_scale=std)
        out.update(db=db, norms_b=nb, fac_b=fb)
    return out


def conv1d_backward(x, g, W, C=1.0, clamp_value=1.0, noise_multiplier=0.0, z_w=None, z_b=None):
    """DPConv1D backward with the intended orientation (transformers_conv1d_clip.py:22-28):
    W [I, O], dW = (sum_b c_b x_b^T g_b)/B + noise, db as the Linear bias."""
    x, g, W = _f64(x), _f64(g), _f64(W)
    x3, g3 = _as_btf(x), _as_btf(g)
    B, T = x3.shape[0], x3.shape[1]
    std = noise_multiplier / np.sqrt(B)
    dx = (g3 @ W.T).reshape(x.shape)
    dw, nw, fw = wgrad_clip(x3, g3, C, clamp_value, "tn", out_scale=1.0 / B,
                            noise=z_w, noise_scale=std)
    db, nb, fb = colsum_clip(g3, None, C, clamp_value, "frob", out_scale=1.0 / (B * T),
                             noise=z_b, noise_scale=std)
    return {"dx": dx, "dw": dw, "norms_w": nw, "fac_w": fw, "db": db, "norms_b": nb,
            "fac_b": fb}


def layernorm_fwd(x, w=None, b=None, eps=1e-5):
    """flashdp/core/layernorm_clip.py:26-60: mean, biased var, rstd, y."""
    x = _f64(x)
    mean = x.mean(axis=-1)
    var = ((x - mean[..., None]) ** 2).mean(axis=-1)
    rstd = 1.0 / np.sqrt(var + eps)
    xhat = (x - mean[..., None]) * rstd[..., None]
    y = xhat * (1.0 if w is None else _f64(w)) + (0.0 if b is None else _f64(b))
    return y, mean, rstd


def layernorm_bwd_clip(dy, x, w=None, eps=1e-5, C=1.0, clamp_value=1.0, out_scale=None,
                       noise_multiplier=0.0, z_w=None, z_b=None, mean=None, rstd=None):
    """LayerNorm backward with per-sample clipped dgamma / dbeta.

    dx: flashdp/core/layernorm_clip.py:98-107.  P_b = sum_t dy*x_hat,
    Q_b = sum_t dy (layernorm_clip.py:163-198), dw = out_scale*sum_b c(P_b) P_b
    + std*z_w, db likewise, out_scale = 1/B, std = noise_multiplier/sqrt(B).
    mean/rstd: if given, used in place of recomputing them from x (as the
    kernels do with the forward's saved statistics)."""
    dy, x = _f64(dy), _f64(x)
    B, H = x.shape[0], x.shape[-1]
    if mean is None or rstd is None:
        _, mean, rstd = layernorm_fwd(x, None, None, eps)
    else:
        mean = _f64(mean).reshape(x.shape[:-1])
        rstd = _f64(rstd).reshape(x.shape[:-1])
    xhat = (x - mean[..., None]) * rstd[..., None]
    wv = np.ones(H) if w is None else _f64(w)
    wdy = dy * wv
    c1 = (xhat * wdy).sum(axis=-1, keepdims=True) / H
    c2 = wdy.sum(axis=-1, keepdims=True) / H
    dx = (wdy - (xhat * c1 + c2)) * rstd[..., None]
    if out_scale is None:
        out_scale = 1.0 / B
    std = noise_multiplier / np.sqrt(B)
    dw, nw, fw = colsum_clip(dy, xhat, C, clamp_value, "sum", out_scale, z_w, std)
    db, nb, fb = colsum_clip(dy, None, C, clamp_value, "sum", out_scale, z_b, std)
    return {"dx": dx, "dw": dw, "db": db, "norms_w": nw, "fac_w": fw, "norms_b": nb,
            "fac_b": fb}


def rel_err(y, y_ref):
    """max|y - y_ref| / max|y_ref| (0 when both are all-zero)."""
    y, y_ref = _f64(y), _f64(y_ref)
    den = np.abs(y_ref).max() if y_ref.size else 0.0
    num = np.abs(y - y_ref).max() if y_ref.size else 0.0
    if den == 0.0:
        return float(num)
    return float(num / den)
