"""Input gradient of the DP layers: torch's matmul, or the HIP kernel (fdp_dgrad).

The reference forms a DP layer's grad_input with torch's matmul
(flashdp/layers/linear.py:62-67: ``grad_output @ weight``;
flashdp/layers/transformers_conv1d.py:70-77: ``grad_output @ weight.t()``).
The library also has a dX kernel of its own for 16-bit operands (fdp_dgrad:
the clipped products' LDS-DMA / MFMA core with grad_output taken k-contiguous,
256x192 or 128x192 output tiles, no workspace), exact to the bf16 tolerance
and deterministic.  On MI355X it is faster than hipBLASLt at some layer shapes
(GPT-2 small's attention projection, 8192x768x768: 15.8 against 20.3 us) and
slower at others (d = 2048 layers, where 192-column tiles leave CUs idle), so
the path is chosen per shape (``set_dgrad``):
  "auto"  (default) the first call of each (device, M, N, K, layout, dtype)
          times both paths on the current stream (a few calls each, outside
          HIP-graph capture) and keeps the faster; the reference's layers
          choose between implementations by timing in the same way
          (flashdp/core/utils.py:15-47); under capture an untimed shape
          takes torch's matmul;
  "torch" torch's matmul (hipBLASLt) always;
  "hip"   the HIP kernel for every operand pair it takes.
Operands the kernel does not take (fp32, K not a multiple of 64, unaligned
rows, an operand of 2^30 elements or more) always use torch's matmul, as the
reference does.
"""
from __future__ import annotations

import os

import torch

from .. import _lib

_MODES = ("auto", "torch", "hip")
_mode = os.environ.get("FDP_DGRAD", "auto")
_choice: dict = {}  # (device, M, N, K, layout, dtype) -> "hip" | "torch" ("auto" mode)
if _mode not in _MODES:
    raise ValueError(f"FDP_DGRAD must be one of {_MODES}, got {_mode!r}")

LAYOUT_NN, LAYOUT_NT = 0, 1  # fdp_dgrad_layout


def set_dgrad(mode: str) -> str:
    """Input-gradient path of DPLinear / DPConv1D ("auto", "torch" or "hip");
    returns the previous mode."""
    global _mode
    if mode not in _MODES:
        raise ValueError(f"dgrad mode must be one of {_MODES}, got {mode!r}")
    prev, _mode = _mode, mode
    return prev


def dgrad_choices() -> dict:
    """The "auto" mode's choices so far: (device, M, N, K, layout, dtype) -> path."""
    return dict(_choice)


def _median_us(fn, reps: int = 5, warmup: int = 2) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        ts.append(start.elapsed_time(end))
    return sorted(ts)[len(ts) // 2] * 1e3


def _auto_choice(grad_output, weight, layout, M, N, K) -> str:
    key = (grad_output.device.index, M, N, K, layout, grad_output.dtype)
    c = _choice.get(key)
    if c is not None:
        return c
    if torch.cuda.is_current_stream_capturing():
        return "torch"
    w = weight if layout == "nn" else weight.t()
    t_torch = _median_us(lambda: grad_output @ w)
    t_hip = _median_us(lambda: dgrad(grad_output, weight, layout))
    c = "hip" if t_hip < t_torch else "torch"
    _choice[key] = c
    return c


def _fits_record(rows: int, ld: int) -> bool:
    """The operand fits one 32-bit buffer record: rows rounded up to 128, times
    the row stride, below 2^30 elements (fdp_dgrad's own check)."""
    return (rows + 127) // 128 * 128 * ld < (1 << 30)


def _takes(g2: torch.Tensor, w: torch.Tensor, K: int) -> bool:
    """Operands the kernel takes as they are: 16-bit, one device, K a multiple
    of 64, rows of 16-byte multiples on 16-byte aligned storage, each operand
    within one 32-bit buffer record."""
    return (g2.dtype in (torch.float16, torch.bfloat16) and w.dtype == g2.dtype
            and g2.is_cuda and w.is_cuda and g2.device == w.device
            and K >= 64 and K % 64 == 0 and g2.shape[0] > 0 and w.numel() > 0
            and g2.stride(1) == 1 and g2.stride(0) % 8 == 0 and g2.data_ptr() % 16 == 0
            and w.stride(1) == 1 and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0
            and _fits_record(g2.shape[0], g2.stride(0)) and _fits_record(w.shape[0], w.stride(0)))


def dgrad(grad_output: torch.Tensor, weight: torch.Tensor, layout: str = "nn") -> torch.Tensor:
    """dX = grad_output @ W on the HIP kernel: W = weight [K, N] ("nn", a Linear
    weight [out, in]) or weight.t() with weight [N, K] ("nt", a Conv1D weight
    [in, out]).  grad_output [..., K] -> dX [..., N] in grad_output's dtype."""
    dev = _lib.require_hip(grad_output, weight)
    if layout not in ("nn", "nt"):
        raise ValueError(f"layout must be 'nn' or 'nt', got {layout!r}")
    K = grad_output.shape[-1]
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D, got shape {tuple(weight.shape)}")
    Kw, N = (weight.shape[0], weight.shape[1]) if layout == "nn" else (weight.shape[1],
                                                                         weight.shape[0])
    if Kw != K:
        raise ValueError(f"grad_output's last dimension {K} does not match the weight "
                         f"{tuple(weight.shape)} ({layout})")
    dt = _lib.dtype_code(grad_output.dtype)
    if weight.dtype != grad_output.dtype:
        raise KeyError(f"weight dtype {weight.dtype} differs from grad_output's "
                       f"{grad_output.dtype}")
    g2 = grad_output.reshape(-1, K)
    M = g2.shape[0]
    out = torch.empty(M, N, dtype=grad_output.dtype, device=dev)
    if M == 0 or N == 0:
        return out.reshape(*grad_output.shape[:-1], N)
    if g2.stride(1) != 1 or g2.stride(0) % 8 != 0 or g2.data_ptr() % 16 != 0:
        g2 = g2.contiguous()
    w = weight
    if w.stride(1) != 1 or w.stride(0) % 8 != 0 or w.data_ptr() % 16 != 0:
        w = w.contiguous()
    lay = LAYOUT_NN if layout == "nn" else LAYOUT_NT
    st = _lib.lib().fdp_dgrad(g2.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K,
                              g2.stride(0), w.stride(0), N, lay, dt, _lib.stream_handle(dev))
    _lib.check(st, "fdp_dgrad")
    return out.reshape(*grad_output.shape[:-1], N)


def input_grad(grad_output: torch.Tensor, weight: torch.Tensor, layout: str = "nn") -> torch.Tensor:
    """A DP layer's grad_input: the HIP kernel or torch's matmul, by the mode
    (see the module docstring); torch's matmul for operands the kernel does
    not take."""
    if weight.dtype != grad_output.dtype:  # AMP: the weight in grad_output's dtype
        weight = weight.to(grad_output.dtype)
    K = grad_output.shape[-1]
    if _mode != "torch" and _takes(grad_output.reshape(-1, K), weight, K):
        N = weight.shape[1] if layout == "nn" else weight.shape[0]
        M = grad_output.numel() // K
        if _mode == "hip" or _auto_choice(grad_output, weight, layout, M, N, K) == "hip":
            return dgrad(grad_output, weight, layout)
    return grad_output @ (weight if layout == "nn" else weight.t())
