"""DPConv1D: HuggingFace Conv1D (y = x W + b, W is [nx, nf]) with per-sample clipping.

Reference: flashdp/layers/transformers_conv1d.py:12-101 and the intended math of
flashdp/core/transformers_conv1d_clip.py:22-39.  The reference layer routes its
weight gradient through the Linear helper, which yields g^T x ([nf, nx]) for a
[nx, nf] weight and fails unless nx == nf, and clips the bias first, in place,
so that dX and dW see the scaled grad_output.  Here:
  dX = g W^T                               (unclipped; fdp_dgrad or torch's matmul)
  dW = (1/B) sum_b clip(||x_b^T g_b||_F) x_b^T g_b + (sigma/sqrt(B)) z_W
  db = (1/(B*T)) sum_b clip(||g_b||_F) sum_t g_bt  + (sigma/sqrt(B)) z_b
(sigma/sqrt(B) is the reference's noise std; set_noise_convention("dpsgd")
selects sigma*C/B.)
so DPConv1D(W) computes exactly DPLinear(W^T)'s gradients, transposed.  dW and
db run as one HIP call (fdp_wgrad_bias_clip with the bias of operand b = g):
the product kernels take the bias's column sums and squares from the
grad_output fragments they already hold, so grad_output is read once.
"""
from __future__ import annotations

import torch
import torch.nn as nn
from torch.autograd.function import Function

from ..core import colsum_clip, input_grad, wgrad_clip
from ..core.utils import RuntimeAutoTuner
from .utils import DPParameter as Parameter
from .utils import (NoiseStream, advance_noise, as_btf, exact_fp32, noise_counter, noise_draws,
                    noise_std)

try:  # the HF module type is what wrap_with_flashdp_layers replaces
    from transformers.pytorch_utils import Conv1D as _HFConv1D
except Exception:  # pragma: no cover - transformers is part of the image
    _HFConv1D = None


class _Conv1DBase(nn.Module):
    """Stand-in base with HF Conv1D's attributes when transformers is absent."""

    def __init__(self, nf, nx):
        super().__init__()
        self.nf = nf
        self.nx = nx
        self.weight = nn.Parameter(torch.empty(nx, nf))
        self.bias = nn.Parameter(torch.zeros(nf))
        nn.init.normal_(self.weight, std=0.02)


_Base = _HFConv1D if _HFConv1D is not None else _Conv1DBase


class DPConv1D(_Base):
    def __init__(self, nf, nx, C: float = 1.0, clamp_value: float = 1.0,
                 noise_multiplier: float = 1.0, auto_tune: bool = True):
        super().__init__(nf, nx)
        self.dp = True
        self.C = C
        self.clamp_value = clamp_value
        self.noise_multiplier = noise_multiplier
        self.nf = nf
        self.nx = nx
        self.runtime_tuner = RuntimeAutoTuner(enable=auto_tune)
        self.weight = Parameter(torch.empty(nx, nf))
        self.bias = Parameter(torch.zeros(nf))
        nn.init.normal_(self.weight, std=0.02)
        self.noise_generator = None
        self.noise_stream = NoiseStream()
        self.register_buffer("noise_counter", noise_counter(), persistent=False)
        self.record_stats = False
        self.last_stats = None

    def forward(self, x):
        self.runtime_tuner.final_tune()
        size_out = x.size()[:-1] + (self.nf,)
        y = _DPConv1DFunction.apply(x, self.weight, self.bias, self)
        return y.view(size_out)


class _DPConv1DFunction(Function):
    @staticmethod
    def forward(ctx, input, weight, bias, module):
        ctx.save_for_backward(input, weight)
        ctx.bias_dtype = bias.dtype
        ctx.cfg = (float(module.C), float(module.clamp_value), float(module.noise_multiplier),
                   module.noise_generator, module.noise_stream, module.noise_counter)
        ctx.module = module if module.record_stats else None
        w = weight if weight.dtype == input.dtype else weight.to(input.dtype)
        b = bias if bias.dtype == input.dtype else bias.to(input.dtype)
        x2 = input.reshape(-1, input.shape[-1])
        return torch.addmm(b, x2, w).view(input.shape[:-1] + (w.shape[1],))

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
            grad_input = input_grad(g3, weight, "nt").reshape(input.shape)
        want_bias = ctx.needs_input_grad[2]
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
                             bias_noise_scale=std, bias_noise_key=keys[1], bias_operand="b")
            r = wgrad_clip(x3.to(g3.dtype), g3.contiguous() if want_bias else g3, C, clamp_value,
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
