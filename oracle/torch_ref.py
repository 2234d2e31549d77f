"""The reference's PyTorch op sequence for the hot path, restated for the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/dp_clip.py).  This module is the timed
"cpu_baseline" of bench.py: it issues the same torch ops, in the same order
and dtype, as the reference's CPU-runnable torch path, so its wall time is the
reference path's cost on the host cores.  tests/test_oracle.py checks it
against the float64 oracle.

  weight_grad_block_clip  flashdp/core/linear_clip.py:94-104
                          (einsum -> norm -> clamp -> mul_ -> sum -> +=)
  linear_weight_backward  flashdp/layers/linear.py:72-80 (.div_(B), normal, add_)
  linear_bias_grad_clip   flashdp/core/linear_clip.py:116-123 (norm, clamp, mul_,
                          mean); mutates its argument like the reference does
  layernorm_dw_clip / layernorm_db_clip
                          flashdp/core/layernorm_clip.py:163-198
"""
from __future__ import annotations

import math

import torch


def clip_factor(norm: torch.Tensor, clip_args: torch.Tensor) -> torch.Tensor:
    """flashdp/core/clip_fn.py:6-8."""
    return torch.clamp(clip_args[0] / (norm + 1e-10), max=clip_args[1])


def weight_grad_block_clip(grad_output: torch.Tensor, input: torch.Tensor,
                           clip_args: torch.Tensor) -> torch.Tensor:
    """sum_b clip(||g_b^T x_b||) g_b^T x_b, one sample per step
    (flashdp/core/linear_clip.py:94-104 with BK=1)."""
    M, K, N = grad_output.shape[-1], input.shape[0], input.shape[-1]
    out = torch.zeros([M, N], dtype=input.dtype)
    for k in range(K):
        g = torch.einsum("k...m,k...n->kmn", grad_output[k:k + 1], input[k:k + 1])
        n = torch.norm(g, p=2, dim=(-1, -2), keepdim=True)
        g.mul_(clip_factor(n, clip_args))
        out += g.sum(0)
    return out


def linear_weight_backward(input: torch.Tensor, grad_output: torch.Tensor, C: float,
                           clamp_value: float, noise_multiplier: float,
                           generator: torch.Generator | None = None) -> torch.Tensor:
    """dW of flashdp/layers/linear.py:72-80 on the torch path."""
    B = input.shape[0]
    clip_args = torch.tensor([C, clamp_value])
    dw = weight_grad_block_clip(grad_output, input.to(grad_output.dtype), clip_args).div_(B)
    dw.add_(torch.normal(0.0, noise_multiplier / math.sqrt(B), size=dw.shape,
                         generator=generator, dtype=dw.dtype))
    return dw


def linear_bias_grad_clip(grad_output: torch.Tensor, C: float, clamp_value: float) -> torch.Tensor:
    """flashdp/core/linear_clip.py:116-123; scales grad_output in place as the
    reference does (callers pass a scratch copy)."""
    clip_args = torch.tensor([C, clamp_value])
    flat = grad_output.view(grad_output.shape[0], -1)
    n = torch.norm(flat, p=2, dim=-1, keepdim=True)
    flat.mul_(clip_factor(n, clip_args))
    return flat.view(-1, grad_output.shape[-1]).mean(0)


def layernorm_dw_clip(input: torch.Tensor, grad_output: torch.Tensor, C: float,
                      clamp_value: float) -> torch.Tensor:
    """flashdp/core/layernorm_clip.py:163-180 for 3-D [B,T,H] inputs."""
    pre = (grad_output * input).sum(dim=1, keepdim=True)
    n = torch.norm(pre, p=2, dim=(1, 2), keepdim=True)
    pre.mul_(clip_factor(n, torch.tensor([C, clamp_value])))
    return pre.mean(0, keepdim=True)


def layernorm_db_clip(grad_output: torch.Tensor, C: float, clamp_value: float) -> torch.Tensor:
    """flashdp/core/layernorm_clip.py:183-198 for 3-D [B,T,H] inputs."""
    pre = grad_output.sum(dim=1, keepdim=True)
    n = torch.norm(pre, p=2, dim=(1, 2), keepdim=True)
    pre.mul_(clip_factor(n, torch.tensor([C, clamp_value])))
    return pre.mean(0, keepdim=True)


def layernorm_backward(x: torch.Tensor, weight: torch.Tensor, grad_output: torch.Tensor,
                       eps: float, C: float, clamp_value: float, noise_multiplier: float,
                       generator: torch.Generator | None = None):
    """The non-fused DPLayerNorm backward (flashdp/layers/layernorm.py:92-96,128-155):
    torch-autograd normalisation, per-sample clipped affine grads, one noise draw
    each for dgamma and dbeta."""
    B = x.shape[0]
    xr = x.detach().requires_grad_(True)
    mean = xr.mean(dim=-1, keepdim=True)
    var = xr.var(dim=-1, keepdim=True, unbiased=False)
    xhat = (xr - mean) / torch.sqrt(var + eps)
    dxhat = grad_output * weight
    (dx,) = torch.autograd.grad(xhat, xr, dxhat)
    xh = xhat.detach()
    dw = layernorm_dw_clip(xh, grad_output, C, clamp_value).reshape(-1)
    db = layernorm_db_clip(grad_output, C, clamp_value).reshape(-1)
    std = noise_multiplier / math.sqrt(B)
    dw = dw + torch.normal(0.0, std, size=dw.shape, generator=generator, dtype=dw.dtype)
    db = db + torch.normal(0.0, std, size=db.shape, generator=generator, dtype=db.dtype)
    return dx, dw, db
