"""LayerNorm forward and per-sample-clipped backward on the HIP kernels.

Operator names follow flashdp/core/__init__.py:8-11: layernorm_fwd_fused
(layernorm_clip.py:201-239), layernorm_bwd_clip_fused (layernorm_clip.py:241-286)
and layernorm_dwdb_fused (layernorm_clip.py:289-315).  The reference's fused
backward clamps lock-group partial sums element-wise in scheduler order; here the
same operator pair computes the per-sample clipped mean of layernorm_dw_clip /
layernorm_db_clip (layernorm_clip.py:163-198): layernorm_bwd_clip_fused returns
the clipped, batch-averaged gradients as single fp32 rows and
layernorm_dwdb_fused reduces those rows to the parameter dtype.
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from .clip_fn import clip_args_of

# Rows of up to 4096 elements take one wavefront each, up to 16384 a
# 1024-thread workgroup each (16 elements per thread); longer rows are swept in
# segments, so the kernels take rows of any length.  The reference's fused
# kernels stop at rows of 64 KB (flashdp/core/layernorm_clip.py:217-221) and its
# non-fused layer has no limit (flashdp/layers/layernorm.py:77-96): the
# fused-mode entry points keep that limit and its error.
FUSED_MAX_ROW_BYTES = 65536


def check_fused_row(x: torch.Tensor) -> None:
    """The reference's fused-mode limit: RuntimeError for rows of more than
    64 KB (flashdp/core/layernorm_clip.py:217-221)."""
    if x.shape[-1] * x.element_size() > FUSED_MAX_ROW_BYTES:
        raise RuntimeError("This layer norm doesn't support feature dim >= 64KB.")


def _rows(x: torch.Tensor, H: int) -> int:
    return x.numel() // H if H else 0


def layernorm_fwd(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
                  eps: float):
    """y, mean [rows] fp32, rstd [rows] fp32 over the last axis."""
    dev = _lib.require_hip(x, weight, bias)
    H = x.shape[-1]
    x = x.contiguous()
    rows = _rows(x, H)
    dt = _lib.dtype_code(x.dtype)
    wdt = _lib.dtype_code(weight.dtype if weight is not None else
                          (bias.dtype if bias is not None else x.dtype))
    if weight is not None:
        weight = weight.contiguous()
    if bias is not None:
        bias = bias.to(weight.dtype if weight is not None else bias.dtype).contiguous()
    y = torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32, device=dev)
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    L = _lib.lib()
    st = L.fdp_layernorm_fwd(_lib.ptr(x), _lib.ptr(weight), _lib.ptr(bias), rows, H,
                             ctypes.c_float(eps), dt, wdt, y.data_ptr(), mean.data_ptr(),
                             rstd.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, "fdp_layernorm_fwd")
    return y, mean, rstd


def layernorm_bwd_clip(grad_output: torch.Tensor, x: torch.Tensor, weight: torch.Tensor | None,
                       mean: torch.Tensor, rstd: torch.Tensor, C: float = 1.0,
                       clamp_value: float = 1.0, *, clip_args=None, out_scale: float | None = None,
                       noise_w: torch.Tensor | None = None, noise_b: torch.Tensor | None = None,
                       noise_scale: float = 1.0, noise_key: tuple[int, int] | None = None,
                       need_dw: bool = True, need_db: bool = True,
                       param_dtype: torch.dtype | None = None, return_stats: bool = False):
    """dx, dw, db of LayerNorm over the last axis with per-sample clipped dw/db.

    x, grad_output [B, ..., H]; samples are the leading axis.  dw / db are
    out_scale * sum_b clip(||.||) (.) + noise_scale * z with out_scale = 1/B by
    default, z the noise_w / noise_b tensors or, for one without a tensor, the
    in-kernel draw of ``noise_key = (seed, offset)`` (dw stream 0, db stream 1).  With ``return_stats`` also returns norms [2B] and factors [2B]
    (dgamma's per-sample values first, then dbeta's)."""
    dev = _lib.require_hip(grad_output, x, weight, mean, rstd, noise_w, noise_b)
    H = x.shape[-1]
    if grad_output.shape != x.shape:
        raise ValueError("grad_output and input shapes differ")
    B = x.shape[0] if x.dim() > 1 else 1
    T = _rows(x, H) // B if B else 0
    x = x.contiguous()
    dy = grad_output.to(x.dtype).contiguous()
    dt = _lib.dtype_code(x.dtype)
    pdt = param_dtype or (weight.dtype if weight is not None else x.dtype)
    wdt = _lib.dtype_code(pdt)
    if weight is not None:
        weight = weight.to(pdt).contiguous()
    for n in (noise_w, noise_b):
        if n is not None and n.numel() != H:
            raise ValueError(f"noise must have {H} elements")
    noise_w = None if noise_w is None else noise_w.reshape(H).to(pdt).contiguous()
    noise_b = None if noise_b is None else noise_b.reshape(H).to(pdt).contiguous()
    C_, clamp_, cad = clip_args_of(clip_args, dev) if clip_args is not None else (
        float(C), float(clamp_value), None)
    if out_scale is None:
        out_scale = 1.0 / B
    dx = torch.empty_like(x)
    dw = torch.empty(H, dtype=pdt, device=dev) if need_dw else None
    db = torch.empty(H, dtype=pdt, device=dev) if need_db else None
    norms = factors = None
    if return_stats:
        norms = torch.empty(2 * B, dtype=torch.float32, device=dev)
        factors = torch.empty(2 * B, dtype=torch.float32, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(
        _lib.size_query(L.fdp_layernorm_bwd_clip_workspace_size, B, T, H, dt), dev)
    st = L.fdp_layernorm_bwd_clip(
        dy.data_ptr(), x.data_ptr(), _lib.ptr(weight), mean.data_ptr(), rstd.data_ptr(), B, T, H,
        dt, wdt, ctypes.c_float(C_), ctypes.c_float(clamp_), _lib.ptr(cad),
        ctypes.c_float(out_scale), _lib.ptr(noise_w), _lib.ptr(noise_b),
        ctypes.c_float(noise_scale), _lib.noise_key(noise_key), dx.data_ptr(), _lib.ptr(dw),
        _lib.ptr(db), _lib.ptr(norms),
        _lib.ptr(factors), ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    _lib.check(st, "fdp_layernorm_bwd_clip")
    if return_stats:
        return dx, dw, db, norms, factors
    return dx, dw, db


# ------------------------------------------------------------ reference names
def layernorm_fwd_fused(input: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float):
    """(y, {'mean','rstd'}, {'BLOCK_SIZE','num_warps','eps'})  (layernorm_clip.py:201-239)."""
    check_fused_row(input)
    H = input.shape[-1]
    y, mean, rstd = layernorm_fwd(input, weight, bias, eps)
    block = 1 << max(0, (H - 1).bit_length())
    return y, {"mean": mean, "rstd": rstd}, {
        "BLOCK_SIZE": block, "num_warps": min(max(block // 256, 1), 8), "eps": eps}


def layernorm_bwd_clip_fused(grad_output: torch.Tensor, input: torch.Tensor, weight: torch.Tensor,
                             bias: torch.Tensor, clip_args, buffer: dict, args: dict):
    """(dx, dw_, db_, {'GROUP_SIZE_M','M'})  (layernorm_clip.py:241-286).

    dw_ / db_ are [1, H] fp32 rows holding the per-sample clipped, batch-averaged
    gradients; layernorm_dwdb_fused reduces them to the parameter dtype."""
    dx, dw, db = layernorm_bwd_clip(grad_output, input, weight, buffer["mean"], buffer["rstd"],
                                    clip_args=clip_args if clip_args is not None else (1.0, 1.0),
                                    need_db=bias is not None, param_dtype=torch.float32)
    H = input.shape[-1]
    return dx, dw.reshape(1, H), (db.reshape(1, H) if db is not None else None), {
        "GROUP_SIZE_M": 1, "M": _rows(input, H)}


def layernorm_dwdb_fused(weight: torch.Tensor, bias: torch.Tensor, _dw: torch.Tensor,
                         _db: torch.Tensor, args: dict | None = None):
    """(dw, db) in the parameter dtype from the rows of layernorm_bwd_clip_fused
    (layernorm_clip.py:289-315)."""
    if _dw.shape[0] != 1 or (_db is not None and _db.shape[0] != 1):
        raise ValueError("expected the single-row outputs of layernorm_bwd_clip_fused")
    dw = _dw.reshape(-1).to(weight.dtype)
    db = _db.reshape(-1).to(bias.dtype) if _db is not None and bias is not None else None
    return dw, db
