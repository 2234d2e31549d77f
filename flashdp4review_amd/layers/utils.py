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


# Accumulation of the DP layers' fp32 weight gradients from 16-bit operands
# (an fp32 model under autocast, the reference's AMP training):
#   "fast": the single-pass kernels, which hold or exchange each per-sample
#           product once in bf16 before the fp32 sum (about 2e-3 relative error
#           at the config shapes; the reference's own autocast einsum forms the
#           per-sample products in bf16);
#   "fp32": the streamed two-pass schedule, which sums every sample's product
#           in fp32 in one accumulator (about 1e-6), at the cost of a norm pass.
WGRAD_PRECISIONS = ("fast", "fp32")
_wgrad_precision = "fast"


def set_wgrad_precision(mode: str) -> None:
    """Select how the DP layers form fp32 weight gradients from 16-bit operands
    (process-wide): "fast" (the default) or "fp32"."""
    global _wgrad_precision
    if mode not in WGRAD_PRECISIONS:
        raise ValueError(f"wgrad precision must be one of {WGRAD_PRECISIONS}, got {mode!r}")
    _wgrad_precision = mode


def get_wgrad_precision() -> str:
    return _wgrad_precision


def exact_fp32(out_dtype: torch.dtype) -> bool:
    """Whether a weight gradient of out_dtype takes the fp32-accumulating schedule."""
    return _wgrad_precision == "fp32" and out_dtype == torch.float32


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


def noise_blocks(numel: int) -> int:
    """Philox counter blocks of an output of numel elements (four normals each)."""
    return (int(numel) + 3) // 4


class NoiseStream:
    """Keys of one DP module's in-kernel Gaussian draws (fdp_noise_key).

    Eager calls: a 64-bit Philox seed taken from torch's default CPU generator
    at the first draw (so torch.manual_seed makes a run reproducible) and a
    counter offset advanced on the host past every draw (an output of n
    elements uses ceil(n / 4) counter blocks).
    Calls captured into a HIP graph: a second seed, the module's device counter
    (``counter``, an int64 [1] buffer) read by the kernels when they run, and a
    device-side advance of that counter after the call (fdp_noise_advance), so
    that every replay of the graph draws fresh noise.  The two seeds keep eager
    and replayed draws apart.
    The reference draws the same N(0, 1) noise with torch.normal on the device
    generator (flashdp/layers/linear.py:74-80), whose offset torch's graphs
    also advance per replay; drawing it in the output epilogue saves writing
    and re-reading a noise tensor per parameter."""

    def __init__(self):
        self.seed = None
        self.graph_seed = None
        self.offset = 0

    def _seeds(self):
        if self.seed is None:
            s = torch.randint(0, 2**62, (2,), dtype=torch.int64)
            self.seed, self.graph_seed = int(s[0]), int(s[1])

    def next(self, numel: int) -> tuple[int, int]:
        """The eager key of one output of numel elements."""
        self._seeds()
        key = (self.seed, self.offset)
        self.offset += noise_blocks(numel)
        return key

    def keys(self, sizes, counter: torch.Tensor | None = None):
        """Keys of one call's outputs (sizes in elements, in draw order) and the
        counter blocks to advance ``counter`` by after the call (0: none).
        Under graph capture (with a device counter) the keys read the counter;
        otherwise they are the next eager keys."""
        if counter is not None and counter.is_cuda and torch.cuda.is_current_stream_capturing():
            self._seeds()
            keys, off = [], 0
            for n in sizes:
                keys.append((self.graph_seed, off, counter.data_ptr()))
                off += noise_blocks(n)
            return keys, off
        return [self.next(n) for n in sizes], 0


def noise_counter(device=None) -> torch.Tensor:
    """A DP module's device noise counter (int64 [1], zero): registered as a
    non-persistent buffer so that it moves with the module."""
    return torch.zeros(1, dtype=torch.int64, device=device)


def noise_draws(std: float, generator, stream: NoiseStream, shapes, dtypes, device,
                counter: torch.Tensor | None = None):
    """(z list, key list, counter blocks to advance) for one call's noisy outputs:
    nothing at std == 0; explicit torch draws (in order) when the module has a
    noise_generator; else in-kernel keys (NoiseStream.keys)."""
    n = len(shapes)
    if std <= 0:
        return [None] * n, [None] * n, 0
    if generator is not None:
        return [draw_noise(s, dt, device, generator) for s, dt in zip(shapes, dtypes)], [None] * n, 0
    keys, adv = stream.keys([math.prod(s) for s in shapes], counter)
    return [None] * n, keys, adv


def advance_noise(counter: torch.Tensor | None, blocks: int) -> None:
    """The device-side advance after a call whose keys read ``counter``."""
    if blocks:
        from .. import _lib
        _lib.noise_advance(counter, blocks)
