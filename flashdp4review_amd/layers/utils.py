"""DPParameter marker and helpers shared by the DP layers.

Reference: flashdp/layers/utils.py:6-11 (DPParameter), flashdp/layers/linear.py:51-58
(per-sample reshape).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn


class DPParameter(nn.Parameter):
    """nn.Parameter carrying ``requires_dp`` (flashdp/layers/utils.py:6-11)."""

    def __new__(cls, data=None, requires_grad=True, requires_dp=True):
        t = nn.Parameter.__new__(cls, data, requires_grad)
        t.requires_dp = requires_dp
        return t


def as_btf(t: torch.Tensor) -> torch.Tensor:
    """[B, F] -> [B, 1, F]; [B, ..., F] -> [B, T, F] with T the product of the middle axes.

    The reference reshapes this way (flashdp/layers/linear.py:51-58) but then
    returns the reshaped gradient; the layers here return it in the input's shape.
    """
    if t.dim() == 2:
        return t.unsqueeze(1)
    if t.dim() > 3:
        return t.reshape(t.shape[0], -1, t.shape[-1])
    if t.dim() < 2:
        raise ValueError(f"DP layers need a leading batch axis; got shape {tuple(t.shape)}")
    return t


# Standard deviation of the noise the DP layers add after the 1/B average:
#   "reference": noise_multiplier / sqrt(B), what the reference draws
#                (flashdp/layers/linear.py:74-80, layers/layernorm.py:140-155);
#                the default;
#   "dpsgd":     noise_multiplier * C / B, i.e. (sum_b clip(G_b) + N(0, (sigma C)^2)) / B,
#                the Gaussian mechanism of DP-SGD (Abadi et al., 2016).
NOISE_CONVENTIONS = ("reference", "dpsgd")
_noise_convention = "reference"


def set_noise_convention(name: str) -> None:
    """Select the noise standard deviation of every DP layer's backward (process-wide):
    "reference" (sigma / sqrt(B), the default) or "dpsgd" (sigma * C / B)."""
    global _noise_convention
    if name not in NOISE_CONVENTIONS:
        raise ValueError(f"noise convention must be one of {NOISE_CONVENTIONS}, got {name!r}")
    _noise_convention = name


def get_noise_convention() -> str:
    return _noise_convention


def noise_std(noise_multiplier: float, batch: int, C: float = 1.0) -> float:
    """Standard deviation of the Gaussian noise added after the 1/B average under
    the selected convention: noise_multiplier / sqrt(B) ("reference",
    flashdp/layers/linear.py:74-80) or noise_multiplier * C / B ("dpsgd")."""
    if _noise_convention == "dpsgd":
        return float(noise_multiplier) * float(C) / batch
    return float(noise_multiplier) / math.sqrt(batch)


def draw_noise(shape, dtype, device, generator) -> torch.Tensor:
    """Standard-normal draw on the device; scaled by noise_std inside the kernels."""
    return torch.randn(shape, dtype=dtype, device=device, generator=generator)


class NoiseStream:
    """Keys of one DP module's in-kernel Gaussian draws (fdp_noise_key): a 64-bit
    Philox seed taken from torch's default CPU generator at the first draw (so
    torch.manual_seed makes a run reproducible) and a counter offset advanced
    past every draw (an output of n elements uses ceil(n / 4) counter blocks).
    The reference draws the same N(0, 1) noise with torch.normal
    (flashdp/layers/linear.py:74-80); drawing it in the output epilogue saves
    writing and re-reading a noise tensor per parameter."""

    def __init__(self):
        self.seed = None
        self.offset = 0

    def next(self, numel: int) -> tuple[int, int]:
        if self.seed is None:
            self.seed = int(torch.randint(0, 2**62, (1,), dtype=torch.int64).item())
        key = (self.seed, self.offset)
        self.offset += (int(numel) + 3) // 4
        return key


def noise_args(std: float, generator, stream: NoiseStream, shape, dtype, device):
    """(z, key) for one noisy output: nothing at std == 0; an explicit torch draw
    when the module has a noise_generator; else the next in-kernel key."""
    if std <= 0:
        return None, None
    if generator is not None:
        return draw_noise(shape, dtype, device, generator), None
    return None, stream.next(math.prod(shape))
