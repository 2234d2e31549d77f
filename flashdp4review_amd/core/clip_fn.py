"""Clip factor c = min(clamp_value, C / (norm + 1e-10)) -- flashdp/core/clip_fn.py:6-25.

The HIP kernels evaluate it in fp32 on the device.  ``get_clip_factor_torch``
keeps the reference helper's name and math for callers that use it on their
own tensors; ``clip_args_of`` turns the reference's ``clip_args`` argument
(a 2-element tensor [C, clamp] or a pair of floats) into what the C ABI takes.
"""
from __future__ import annotations

import torch


def get_clip_factor_torch(norm: torch.Tensor, clip_args: torch.Tensor) -> torch.Tensor:
    return torch.clamp(clip_args[0] / (norm + 1e-10), max=clip_args[1])


def clip_args_of(clip_args, device: torch.device):
    """Returns (C, clamp, device_tensor_or_None).

    A float32 tensor already on ``device`` is passed to the kernels by pointer,
    so reading it needs no host synchronisation (the reference's Triton kernels
    read it the same way, clip_fn.py:21-25).  Anything else is read on the host.
    """
    if clip_args is None:
        return 1.0, 1.0, None
    if isinstance(clip_args, torch.Tensor):
        if clip_args.numel() != 2:
            raise ValueError("clip_args must hold exactly [C, clamp_value]")
        if clip_args.device == device:
            t = clip_args.reshape(2)
            if t.dtype != torch.float32 or not t.is_contiguous():
                t = t.to(torch.float32).contiguous()
            return 1.0, 1.0, t
        vals = clip_args.detach().to("cpu", torch.float64).reshape(2).tolist()
        return float(vals[0]), float(vals[1]), None
    C, clamp = clip_args
    return float(C), float(clamp), None
