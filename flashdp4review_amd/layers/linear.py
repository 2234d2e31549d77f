"""DPLinear: nn.Linear whose backward clips per-sample weight/bias gradients.

Reference: flashdp/layers/linear.py:11-106.  Backward math (per parameter tensor):
  dX = g W                                 (unclipped; fdp_dgrad or torch's matmul)
  dW = (1/B) sum_b clip(||g_b^T x_b||_F) g_b^T x_b + (sigma/sqrt(B)) z_W
  db = (1/(B*T)) sum_b clip(||g_b||_F) sum_t g_bt  + (sigma/sqrt(B)) z_b
(sigma/sqrt(B) is the reference's noise std; set_noise_convention("dpsgd")
selects sigma*C/B.)
with clip(n) = min(clamp_value, C/(n + 1e-10)).  dW and db run as one HIP call
(fdp_wgrad_bias_clip; fdp_wgrad_clip / fdp_colsum_clip when only one of them
is needed): norm, clip, 1/B and noise add happen on the device, and
grad_output is never modified.  For 16-bit operands the product kernels take
the bias from the grad_output fragments they already hold (no second pass).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.autograd.function import Function

from ..core import colsum_clip, input_grad, wgrad_clip
from ..core.utils import RuntimeAutoTuner
from .utils import DPParameter as Parameter
from .utils import (NoiseStream, advance_noise, as_btf, exact_fp32, noise_counter, noise_draws,
                    noise_std)


class DPLinear(nn.Linear):
    def __init__(self, in_features: int, out_features: int, bias: bool = True, device=None,
                 dtype=None, C: float = 1.0, clamp_value: float = 1.0,
                 noise_multiplier: float = 1.0, auto_tune: bool = True):
        # bias may be a bool or (as wrap_with_flashdp_layers passes it) a tensor/None;
        # False and None both mean "no bias" (the reference keeps a bias for False).
        use_bias = not (bias is None or bias is False)
        super().__init__(in_features, out_features, use_bias, device=device, dtype=dtype)
        factory_kwargs = {"device": device, "dtype": dtype}
        self.dp = True
        self.C = C
        self.clamp_value = clamp_value
        self.noise_multiplier = noise_multiplier
        self.runtime_tuner = RuntimeAutoTuner(enable=auto_tune)
        self.weight = Parameter(torch.empty((out_features, in_features), **factory_kwargs))
        if use_bias:
            self.bias = Parameter(torch.empty(out_features, **factory_kwargs))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()
        # Noise: drawn inside the kernels from noise_stream, or, when a
        # torch.Generator is set here, drawn with it (z_W first, then z_b).
        self.noise_generator = None
        self.noise_stream = NoiseStream()
        self.register_buffer("noise_counter", noise_counter(device), persistent=False)
        # When True, backward stores per-sample norms / clip factors in last_stats.
        self.record_stats = False
        self.last_stats = None

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        self.runtime_tuner.final_tune()
        return _DPLinearFunction.apply(input, self.weight, self.bias, self)


class _DPLinearFunction(Function):
    @staticmethod
    def forward(ctx, input, weight, bias, module):
        ctx.save_for_backward(input, weight)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = bias.dtype if bias is not None else None
        ctx.cfg = (float(module.C), float(module.clamp_value), float(module.noise_multiplier),
                   module.noise_generator, module.noise_stream, module.noise_counter)
        ctx.module = module if module.record_stats else None
        w = weight if weight.dtype == input.dtype else weight.to(input.dtype)
        b = None if bias is None else (bias if bias.dtype == input.dtype else bias.to(input.dtype))
        return F.linear(input, w, b)

    @staticmethod
    def backward(ctx, grad_output):
        input, weight = ctx.saved_tensors
        C, clamp_value, sigma, gen, nstream, counter = ctx.cfg
        x3, g3 = as_btf(input), as_btf(grad_output)
        B, T = x3.shape[0], x3.shape[1]
        std = noise_std(sigma, B, C)
        stats = {} if ctx.module is not None else None
        grad_input = grad_weight = grad_bias = None
        if ctx.needs_input_grad[0]:
            grad_input = input_grad(g3, weight, "nn").reshape(input.shape)
        want_bias = ctx.has_bias and ctx.needs_input_grad[2]
        O = g3.shape[-1]
        if ctx.needs_input_grad[1]:
            # both in one call when the bias is needed (noise in the order weight, bias)
            shapes, dts = [tuple(weight.shape)], [weight.dtype]
            if want_bias:
                shapes.append((O,))
                dts.append(ctx.bias_dtype)
            zs, keys, adv = noise_draws(std, gen, nstream, shapes, dts, g3.device, counter)
            extra = {}
            if want_bias:
                grad_bias = torch.empty(O, dtype=ctx.bias_dtype, device=g3.device)
                extra = dict(bias_out=grad_bias, bias_scale=1.0 / (B * T), bias_noise=zs[1],
                             bias_noise_scale=std, bias_noise_key=keys[1])
            r = wgrad_clip(g3.contiguous() if want_bias else g3, x3.to(g3.dtype), C, clamp_value,
                           layout="tn", out_scale=1.0 / B, noise=zs[0], noise_scale=std,
                           noise_key=keys[0], out_dtype=weight.dtype,
                           two_pass=exact_fp32(weight.dtype), return_stats=stats is not None,
                           **extra)
            advance_noise(counter, adv)
            if stats is not None:
                grad_weight, stats["norms_w"], stats["fac_w"] = r[:3]
                if want_bias:
                    stats["norms_b"], stats["fac_b"] = r[3], r[4]
            else:
                grad_weight = r
            want_bias = False
        if want_bias:
            zs, keys, adv = noise_draws(std, gen, nstream, [(O,)], [ctx.bias_dtype], g3.device,
                                        counter)
            r = colsum_clip(g3, None, C, clamp_value, norm="frob", out_scale=1.0 / (B * T),
                            noise=zs[0], noise_scale=std, noise_key=keys[0],
                            out_dtype=ctx.bias_dtype, return_stats=stats is not None)
            advance_noise(counter, adv)
            if stats is not None:
                grad_bias, stats["norms_b"], stats["fac_b"] = r
            else:
                grad_bias = r
        if stats is not None:
            ctx.module.last_stats = stats
        return grad_input, grad_weight, grad_bias, None
