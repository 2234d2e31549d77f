"""DPLayerNorm: nn.LayerNorm with per-sample clipped gamma/beta gradients.

Reference: flashdp/layers/layernorm.py:25-204.  Forward and backward run on the
HIP LayerNorm kernels (fdp_layernorm_fwd / fdp_layernorm_bwd_clip).  Backward:
  x_hat = (x - mean) * rstd, dx = standard LayerNorm backward of g * gamma
  P_b = sum_t g_bt * x_hat_bt,  Q_b = sum_t g_bt                 (per sample b)
  dgamma = (1/B) sum_b clip(||P_b||) P_b + (sigma/sqrt(B)) z_gamma
  dbeta  = (1/B) sum_b clip(||Q_b||) Q_b + (sigma/sqrt(B)) z_beta
(sigma/sqrt(B) is the reference's noise std; set_noise_convention("dpsgd")
selects sigma*C/B.)
The reference's default fused backward instead clamps lock-group partial sums
element-wise (flashdp/core/layernorm_clip.py:118-127) and its non-fused
backward adds both noise draws to dgamma (flashdp/layers/layernorm.py:140-155);
``use_fused`` is kept and both settings compute the per-sample math above.
As in the reference, fused mode rejects rows of more than 64 KB
(flashdp/core/layernorm_clip.py:217-221) and the non-fused mode takes rows of
any length.
"""
from __future__ import annotations

import math
import numbers

import torch
import torch.nn as nn
from torch.autograd.function import Function

from ..core import layernorm_bwd_clip, layernorm_fwd
from ..core.layernorm import check_fused_row
from .utils import DPParameter as Parameter
from .utils import NoiseStream, advance_noise, draw_noise, noise_counter, noise_std


class DPLayerNorm(nn.LayerNorm):
    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True,
                 bias: bool = True, device=None, dtype=None, use_fused: bool = True,
                 C: float = 1.0, clamp_value: float = 1.0, noise_multiplier: float = 1.0) -> None:
        if isinstance(normalized_shape, numbers.Integral):
            normalized_shape = (normalized_shape,)
        use_bias = not (bias is None or bias is False)
        if use_fused and not use_bias:
            raise NotImplementedError("In fused mode, bias must be enabled. Set use_fused=False "
                                      "to use the default implementation.")
        factory_kwargs = {"device": device, "dtype": dtype}
        super().__init__(normalized_shape, eps, elementwise_affine, use_bias, **factory_kwargs)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        self.use_fused = use_fused
        self.dp = True
        self.C = C
        self.clamp_value = clamp_value
        self.noise_multiplier = noise_multiplier
        if self.elementwise_affine:
            self.weight = Parameter(torch.empty(self.normalized_shape, **factory_kwargs))
            if use_bias:
                self.bias = Parameter(torch.empty(self.normalized_shape, **factory_kwargs))
            else:
                self.register_parameter("bias", None)
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)
        self.reset_parameters()
        self.noise_generator = None
        self.noise_stream = NoiseStream()
        self.register_buffer("noise_counter", noise_counter(device), persistent=False)
        self.record_stats = False
        self.last_stats = None

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        k = len(self.normalized_shape)
        if self.use_fused:
            if k != 1:
                raise NotImplementedError("Currently layernorm only support normalized_dim=-1.")
            if self.normalized_shape[0] != input.shape[-1]:
                raise NotImplementedError(
                    "In fused mode, currently layernorm only support normalized_dim=-1. "
                    "Set use_fused=False to use the default implementation.")
            check_fused_row(input)
        elif tuple(input.shape[input.dim() - k:]) != self.normalized_shape:
            raise NotImplementedError("normalized_shape must match the trailing input dims")
        return _DPLayerNormFunction.apply(input, self.weight, self.bias, self)


class _DPLayerNormFunction(Function):
    @staticmethod
    def forward(ctx, input, weight, bias, module):
        k = len(module.normalized_shape)
        H = math.prod(module.normalized_shape)
        x = input.reshape(input.shape[: input.dim() - k] + (H,))
        w = None if weight is None else weight.reshape(H)
        b = None if bias is None else bias.reshape(H)
        y, mean, rstd = layernorm_fwd(x, w, b, module.eps)
        ctx.save_for_backward(x, w, mean, rstd)
        ctx.in_shape = input.shape
        ctx.param_shape = None if weight is None else weight.shape
        ctx.param_dtype = None if weight is None else weight.dtype
        ctx.has_bias = bias is not None
        ctx.cfg = (float(module.C), float(module.clamp_value), float(module.noise_multiplier),
                   module.noise_generator, module.noise_stream, module.noise_counter)
        ctx.module = module if module.record_stats else None
        return y.reshape(input.shape)

    @staticmethod
    def backward(ctx, grad_output):
        x, w, mean, rstd = ctx.saved_tensors
        C, clamp_value, sigma, gen, nstream, counter = ctx.cfg
        H = x.shape[-1]
        B = x.shape[0] if x.dim() > 1 else 1
        std = noise_std(sigma, B, C)
        need_dw = w is not None and ctx.needs_input_grad[1]
        need_db = ctx.has_bias and ctx.needs_input_grad[2]
        zw = zb = key = None
        adv = 0
        if std > 0 and (need_dw or need_db):
            if gen is not None:
                zw = draw_noise((H,), ctx.param_dtype, x.device, gen) if need_dw else None
                zb = draw_noise((H,), ctx.param_dtype, x.device, gen) if need_db else None
            else:  # one key: dgamma draws counter stream 0, dbeta stream 1
                keys, adv = nstream.keys([H], counter)
                key = keys[0]
        r = layernorm_bwd_clip(grad_output.reshape(x.shape), x, w, mean, rstd, C, clamp_value,
                               out_scale=1.0 / B, noise_w=zw, noise_b=zb, noise_scale=std,
                               noise_key=key,
                               need_dw=need_dw, need_db=need_db,
                               param_dtype=ctx.param_dtype or x.dtype,
                               return_stats=ctx.module is not None)
        advance_noise(counter, adv)
        if ctx.module is not None:
            dx, dw, db, norms, factors = r
            ctx.module.last_stats = {"norms_w": norms[:B], "fac_w": factors[:B],
                                     "norms_b": norms[B:], "fac_b": factors[B:]}
        else:
            dx, dw, db = r
        dx = dx.reshape(ctx.in_shape)
        if dw is not None:
            dw = dw.reshape(ctx.param_shape)
        if db is not None:
            db = db.reshape(ctx.param_shape)
        return dx, dw, db, None
