"""Clipped per-sample column sums on the HIP kernels (fdp_colsum_clip).

Serves the bias gradients (flashdp/core/linear_clip.py:116-123,
flashdp/core/transformers_conv1d_clip.py:31-39) and the LayerNorm affine
gradients of the operator API (flashdp/core/layernorm_clip.py:163-198).
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from .clip_fn import clip_args_of


def _as_bth(t: torch.Tensor) -> torch.Tensor:
    """[B, ..., H] -> contiguous [B, T, H] (2-D inputs get T = 1)."""
    if t.dim() < 2:
        raise ValueError(f"expected at least 2 dimensions, got shape {tuple(t.shape)}")
    if t.dim() == 2:
        t = t.unsqueeze(1)
    elif t.dim() > 3:
        t = t.reshape(t.shape[0], -1, t.shape[-1])
    return t.contiguous()


def colsum_clip(u: torch.Tensor, v: torch.Tensor | None = None, C: float = 1.0,
                clamp_value: float = 1.0, *, norm: str = "sum", clip_args=None,
                out_scale: float = 1.0, noise: torch.Tensor | None = None,
                noise_scale: float = 1.0, noise_key: tuple[int, int] | None = None,
                out_dtype: torch.dtype | None = None, return_stats: bool = False):
    """out[h] = out_scale * sum_b c_b S_b[h] + noise_scale * z[h],
    S_b = sum_t u_bt (* v_bt), c_b from ||S_b|| (norm="sum") or ||u_b||_F (norm="frob");
    z is ``noise`` or the in-kernel draw of ``noise_key = (seed, offset)``."""
    dev = _lib.require_hip(u, v, noise)
    u3 = _as_bth(u)
    v3 = None
    if v is not None:
        if v.shape != u.shape:
            raise ValueError(f"u and v shapes differ: {tuple(u.shape)} vs {tuple(v.shape)}")
        v3 = _as_bth(v.to(u.dtype))
    B, T, H = u3.shape
    if B == 0:
        raise ValueError("batch size must be at least 1")
    dt = _lib.dtype_code(u.dtype)
    out_dtype = out_dtype or u.dtype
    odt = _lib.dtype_code(out_dtype)
    kind = {"sum": _lib.NORM_SUM, "frob": _lib.NORM_FROB}[norm]
    if noise is not None:
        if noise.numel() != H:
            raise ValueError(f"noise must have {H} elements")
        noise = noise.reshape(H).to(out_dtype).contiguous()
    C_, clamp_, cad = clip_args_of(clip_args, dev) if clip_args is not None else (
        float(C), float(clamp_value), None)
    out = torch.empty(H, dtype=out_dtype, device=dev)
    norms = factors = None
    if return_stats:
        norms = torch.empty(B, dtype=torch.float32, device=dev)
        factors = torch.empty(B, dtype=torch.float32, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.fdp_colsum_clip_workspace_size, B, T, H, dt), dev)
    st = L.fdp_colsum_clip(
        _lib.ptr(u3), _lib.ptr(v3), B, T, H, dt, kind, ctypes.c_float(C_),
        ctypes.c_float(clamp_), _lib.ptr(cad), ctypes.c_float(out_scale), _lib.ptr(noise),
        ctypes.c_float(noise_scale), _lib.noise_key(noise_key), out.data_ptr(), odt,
        _lib.ptr(norms), _lib.ptr(factors),
        ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    _lib.check(st, "fdp_colsum_clip")
    if return_stats:
        return out, norms, factors
    return out


def linear_bias_grad_clip(grad_output: torch.Tensor, C: float, clamp_value: float) -> torch.Tensor:
    """(1/(B*T)) sum_b clip(||g_b||_F) sum_t g_bt -> [O]  (flashdp/core/linear_clip.py:116-123).
    Unlike the reference, grad_output is left unmodified."""
    g3 = _as_bth(grad_output)
    B, T = g3.shape[0], g3.shape[1]
    return colsum_clip(g3, None, C, clamp_value, norm="frob", out_scale=1.0 / (B * T))


def conv1d_bias_grad_clip(grad_output: torch.Tensor, C: float, clamp_value: float) -> torch.Tensor:
    """flashdp/core/transformers_conv1d_clip.py:31-39 (same math as the Linear bias; the
    reference's unused helper uses eps 1e-6, the layer itself uses 1e-10 via
    linear_bias_grad_clip, transformers_conv1d.py:60)."""
    return linear_bias_grad_clip(grad_output, C, clamp_value)


def _keepdim_shape(grad_output: torch.Tensor, H: int):
    return (1,) * (grad_output.dim() - 1) + (H,)


def layernorm_dw_clip(input: torch.Tensor, grad_output: torch.Tensor, weight: torch.Tensor,
                      C, clamp_value) -> torch.Tensor:
    """(1/B) sum_b clip(||P_b||) P_b, P_b = sum_t g_bt * x_hat_bt, in the reference's
    keepdim shape (1, ..., H)  (flashdp/core/layernorm_clip.py:163-180).
    ``input`` is the normalised x_hat as in the reference."""
    C, clamp_value = float(torch.as_tensor(C).reshape(-1)[0]), float(
        torch.as_tensor(clamp_value).reshape(-1)[0])
    g3 = _as_bth(grad_output)
    out = colsum_clip(g3, _as_bth(input), C, clamp_value, norm="sum", out_scale=1.0 / g3.shape[0])
    return out.reshape(_keepdim_shape(grad_output, g3.shape[-1]))


def layernorm_db_clip(grad_output: torch.Tensor, bias: torch.Tensor, C, clamp_value) -> torch.Tensor:
    """(1/B) sum_b clip(||Q_b||) Q_b, Q_b = sum_t g_bt  (flashdp/core/layernorm_clip.py:183-198)."""
    C, clamp_value = float(torch.as_tensor(C).reshape(-1)[0]), float(
        torch.as_tensor(clamp_value).reshape(-1)[0])
    g3 = _as_bth(grad_output)
    out = colsum_clip(g3, None, C, clamp_value, norm="sum", out_scale=1.0 / g3.shape[0])
    return out.reshape(_keepdim_shape(grad_output, g3.shape[-1]))
