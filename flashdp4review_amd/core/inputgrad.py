"""Input gradient of the DP layers: torch's matmul, or the HIP kernel (fdp_dgrad).

The reference forms a DP layer's grad_input with torch's matmul
(flashdp/layers/linear.py:62-67: ``grad_output @ weight``;
flashdp/layers/transformers_conv1d.py:70-77: ``grad_output @ weight.t()``).
The library also has a dX kernel of its own for 16-bit operands (fdp_dgrad:
the clipped products' LDS-DMA / MFMA core with grad_output taken k-contiguous,
256x192 tiles, a split contraction where the tiles alone would leave CUs
idle).  It is exact to the bf16 tolerance and deterministic, and on MI355X
about as fast as hipBLASLt at GPT-2's 768-wide inputs (cfg3's dX 54.4 against
55.6 us, cfg2's 53.6 against 52.4 us) and slower elsewhere (GPT-2 small
30.8 against 20.2 us, a 2048x2048 Linear 118 against 61 us), so the layers
keep torch's matmul unless ``set_dgrad("hip")`` selects the kernel:
  "torch" (default) torch's matmul (hipBLASLt);
  "hip"   the HIP kernel for every operand pair it takes.
Operands the kernel does not take (fp32, K not a multiple of 64, unaligned
rows) always use torch's matmul, as the reference does.
"""
from __future__ import annotations

import os

import torch

from .. import _lib
from .wgrad import _persistent_workspace, _raise_expired

_MODES = ("torch", "hip")
_mode = os.environ.get("FDP_DGRAD", "torch")
if _mode not in _MODES:
    raise ValueError(f"FDP_DGRAD must be one of {_MODES}, got {_mode!r}")

LAYOUT_NN, LAYOUT_NT = 0, 1  # fdp_dgrad_layout


def set_dgrad(mode: str) -> str:
    """Input-gradient path of DPLinear / DPConv1D ("torch" or "hip"); returns
    the previous mode."""
    global _mode
    if mode not in _MODES:
        raise ValueError(f"dgrad mode must be one of {_MODES}, got {mode!r}")
    prev, _mode = _mode, mode
    return prev


def _takes(g2: torch.Tensor, w: torch.Tensor, K: int) -> bool:
    """Operands the kernel takes as they are: 16-bit, one device, K a multiple
    of 64, rows of 16-byte multiples on 16-byte aligned storage."""
    return (g2.dtype in (torch.float16, torch.bfloat16) and w.dtype == g2.dtype
            and g2.is_cuda and w.is_cuda and g2.device == w.device
            and K >= 64 and K % 64 == 0
            and g2.stride(1) == 1 and g2.stride(0) % 8 == 0 and g2.data_ptr() % 16 == 0
            and w.stride(1) == 1 and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0)


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
    if g2.stride(1) != 1 or g2.stride(0) % 8 != 0 or g2.data_ptr() % 16 != 0:
        g2 = g2.contiguous()
    w = weight if weight.stride(1) == 1 and weight.stride(0) % 8 == 0 else weight.contiguous()
    M = g2.shape[0]
    out = torch.empty(M, N, dtype=grad_output.dtype, device=dev)
    L = _lib.lib()
    lay = LAYOUT_NN if layout == "nn" else LAYOUT_NT
    nbytes = _lib.size_query(L.fdp_dgrad_workspace_size, M, N, K, lay, dt)
    stream = _lib.stream_handle(dev)
    ws = _persistent_workspace(nbytes, dev, stream, "dgrad")
    if ws.event is not None:
        probed = ws.take_probe()
        if probed != 0:
            _raise_expired(ws, "reported asynchronously for an earlier call on this stream",
                           probed)
    st = L.fdp_dgrad(g2.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K, g2.stride(0),
                     w.stride(0), N, lay, dt, ws.buf.data_ptr(), ws.buf.numel(), stream)
    _lib.check(st, "fdp_dgrad")
    ws.queue_probe()
    return out.reshape(*grad_output.shape[:-1], N)


def input_grad(grad_output: torch.Tensor, weight: torch.Tensor, layout: str = "nn") -> torch.Tensor:
    """A DP layer's grad_input: the HIP kernel in "hip" mode for the operands
    it takes, torch's matmul otherwise."""
    if weight.dtype != grad_output.dtype:  # AMP: the weight in grad_output's dtype
        weight = weight.to(grad_output.dtype)
    K = grad_output.shape[-1]
    if _mode == "hip" and _takes(grad_output.reshape(-1, K), weight, K):
        return dgrad(grad_output, weight, layout)
    return grad_output @ (weight if layout == "nn" else weight.t())
