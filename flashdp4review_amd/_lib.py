"""ctypes binding of libflashdp_hip.so (declared in include/flashdp_hip.h).

The library is built in-tree by ``flashdp4review_amd.build``.  There is no
fallback: if the library is missing, or a tensor is not on a HIP device, the
call raises.  Status codes map to the exception types the reference raises
for the same condition (flashdp/core/linear_clip.py:69-73,
flashdp/core/layernorm_clip.py:207,221): dtype -> KeyError, sizes/arguments ->
ValueError, everything else -> RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libflashdp_hip.so")

FDP_F32, FDP_F16, FDP_BF16 = 0, 1, 2
LAYOUT_TN, LAYOUT_NN = 0, 1
NORM_SUM, NORM_FROB = 0, 1
WGRAD_NOCLIP = 1
WGRAD_TWO_PASS = 2
WGRAD_PLAIN_LAUNCH = 4
WGRAD_CLEAN_WORKSPACE = 8
WGRAD_WIDE = 16
WGRAD_NARROW = 32
WGRAD_BIAS_OF_B = 64  # fdp_wgrad_bias_clip: the bias of operand b instead of a
WGRAD_UNPAIRED = 128  # the wide schedule with one sample per workgroup only
WGRAD_CONTROL_BYTES = 2048  # control words at the head of an fdp_wgrad_clip workspace

_DTYPE_CODES = {torch.float32: FDP_F32, torch.float16: FDP_F16, torch.bfloat16: FDP_BF16}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_f = ctypes.c_float
_c_p = ctypes.c_void_p
_c_sz_p = ctypes.POINTER(ctypes.c_size_t)


class NoiseKey(ctypes.Structure):
    """fdp_noise_key: the Philox4x32-10 key (seed), first counter block and
    optional device counter of an in-kernel Gaussian draw (include/flashdp_hip.h)."""
    _fields_ = [("seed", ctypes.c_uint64), ("offset", ctypes.c_uint64),
                ("counter", ctypes.c_void_p)]


_c_key = ctypes.POINTER(NoiseKey)


class BiasOut(ctypes.Structure):
    """fdp_bias_out: where and how fdp_wgrad_bias_clip writes the bias of
    operand a (include/flashdp_hip.h)."""
    _fields_ = [("out", ctypes.c_void_p), ("out_dtype", ctypes.c_int),
                ("out_scale", ctypes.c_float), ("noise", ctypes.c_void_p),
                ("noise_scale", ctypes.c_float), ("noise_key", _c_key),
                ("norms", ctypes.c_void_p), ("factors", ctypes.c_void_p)]


_c_bias = ctypes.POINTER(BiasOut)


def noise_key(key) -> "ctypes._Pointer | None":
    """(seed, offset) or (seed, offset, device counter address) -> a fdp_noise_key
    pointer for the call (None -> NULL)."""
    if key is None:
        return None
    seed, offset = key[0], key[1]
    counter = key[2] if len(key) > 2 else None
    return ctypes.pointer(NoiseKey(int(seed) & (2**64 - 1), int(offset) & (2**64 - 1), counter))


def noise_advance(counter: torch.Tensor, blocks: int) -> None:
    """Stream-ordered ``counter += blocks`` on the device (fdp_noise_advance): the
    advance of a graph-captured draw's counter (``counter`` an int64 [1] tensor)."""
    check(lib().fdp_noise_advance(counter.data_ptr(), int(blocks),
                                  stream_handle(counter.device)), "fdp_noise_advance")

# Every exported symbol with its (restype, argtypes); tests check this list
# against include/flashdp_hip.h.
SIGNATURES = {
    "fdp_strerror": (ctypes.c_char_p, [_c_int]),
    "fdp_version": (_c_int, []),
    "fdp_noise_advance": (_c_int, [_c_p, ctypes.c_uint64, _c_p]),
    "fdp_wgrad_clip_workspace_size": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                               _c_sz_p]),
    "fdp_wgrad_clip": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                _c_i64, _c_i64, _c_int, _c_int, _c_f, _c_f, _c_p, _c_f, _c_p,
                                _c_f, _c_key, _c_p, _c_i64, _c_int, _c_p, _c_p, _c_int, _c_p,
                                ctypes.c_size_t, _c_p]),
    "fdp_wgrad_bias_clip_workspace_size": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int,
                                                    _c_int, _c_sz_p]),
    "fdp_wgrad_bias_clip": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                     _c_i64, _c_i64, _c_int, _c_int, _c_f, _c_f, _c_p, _c_f, _c_p,
                                     _c_f, _c_key, _c_p, _c_i64, _c_int, _c_p, _c_p, _c_int,
                                     _c_bias, _c_p, ctypes.c_size_t, _c_p]),
    "fdp_wgrad_clip_noalloc": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                        _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f, _c_f, _c_p,
                                        _c_f, _c_p, _c_f, _c_key, _c_p, _c_i64, _c_int, _c_p, _c_p,
                                        _c_int, _c_p]),
    "fdp_dgrad": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                           _c_int, _c_int, _c_p]),
    "fdp_colsum_clip_workspace_size": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int, _c_sz_p]),
    "fdp_colsum_clip": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_f, _c_f,
                                 _c_p, _c_f, _c_p, _c_f, _c_key, _c_p, _c_int, _c_p, _c_p, _c_p,
                                 ctypes.c_size_t, _c_p]),
    "fdp_layernorm_fwd": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_f, _c_int, _c_int, _c_p,
                                   _c_p, _c_p, _c_p]),
    "fdp_layernorm_bwd_clip_workspace_size": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int, _c_sz_p]),
    "fdp_layernorm_bwd_clip": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                        _c_int, _c_int, _c_f, _c_f, _c_p, _c_f, _c_p, _c_p, _c_f,
                                        _c_key, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                        ctypes.c_size_t, _c_p]),
}

_lock = threading.Lock()
_lib = None


class FlashDPError(RuntimeError):
    """A HIP-side failure reported by libflashdp_hip.so."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it was not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `python -m flashdp4review_amd.build` "
                        "(flashdp4review_amd has no CPU fallback)")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


_fast = None


def fast_call():
    """The _fdp_call extension (the per-call path into the library without
    ctypes' argument conversion), or None if it was not built."""
    global _fast
    if _fast is None:
        lib()  # the library first: the extension links against it
        try:
            from . import _fdp_call
            _fast = _fdp_call
        except ImportError:
            _fast = False
    return _fast or None


def check(status: int, what: str) -> None:
    if status == 0:
        return
    msg = f"{what}: {lib().fdp_strerror(status).decode()} (status {status})"
    if status == 1:
        raise KeyError(msg)
    if status in (2, 3, 6, 7):
        raise ValueError(msg)
    raise FlashDPError(msg)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise KeyError(f"The type of input mat is not supported: {dtype}") from None


def require_hip(*tensors: torch.Tensor | None) -> torch.device:
    """All tensors must live on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "flashdp4review_amd kernels run on the GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor arguments")
    return dev


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The HIP stream torch currently uses on `device` (its raw handle)."""
    if _raw_stream is not None:
        idx = device.index
        return _raw_stream(idx if idx is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned workspace from the torch caching allocator (256-byte aligned)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def size_query(fn, *args) -> int:
    out = ctypes.c_size_t(0)
    check(fn(*args, ctypes.byref(out)), fn.__name__)
    return out.value
