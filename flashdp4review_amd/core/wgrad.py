"""Clipped per-sample product sums on the HIP kernels (fdp_wgrad_clip).

Operator names and argument meanings follow flashdp/core/__init__.py:1-13:
bmtm_clip (bmtm_clip_loop.py:162-173), bmm_clip (bmm_clip_loop.py:150-162),
mm_clip (mm_clip_loop.py:127-139), mm_fused (linear_clip.py:64-91) and
linear_weight_flashdp (linear_clip.py:107-113).  All of them call one entry
point, ``wgrad_clip``, which never materialises a per-sample gradient.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

from .. import _lib
from .clip_fn import clip_args_of
from .utils import RuntimeAutoTuner


_LAUNCH_MODES = ("cooperative", "plain")
_SINGLE_PASS = {"auto": 0, "wide": _lib.WGRAD_WIDE,
                "unpaired": _lib.WGRAD_WIDE | _lib.WGRAD_UNPAIRED, "narrow": _lib.WGRAD_NARROW}
_launch_mode = os.environ.get("FDP_WGRAD_LAUNCH", "plain")
if _launch_mode not in _LAUNCH_MODES:
    raise ValueError(f"FDP_WGRAD_LAUNCH must be one of {_LAUNCH_MODES}, got {_launch_mode!r}")
_ws_sizes: dict = {}
_ws_lock = threading.Lock()
_ws_cache: dict = {}
# Every STATUS_PERIOD calls on a workspace, a 4-byte copy of its status word to
# pinned host memory is queued behind the call; a later call reads it once the
# copy has completed, so an expired wait is reported without a host sync.
STATUS_PERIOD = 64


class _Workspace:
    """A zero-filled fdp_wgrad_clip workspace kept per (device, stream), with the
    asynchronous probe of its status word.  Calls on one stream run in order and
    each leaves the control words valid (a zero-filled head is valid), so the
    buffer is reused with FDP_WGRAD_CLEAN_WORKSPACE and no clearing kernel."""

    def __init__(self, nbytes: int, dev: torch.device):
        self.buf = torch.zeros(max(int(nbytes), 4096), dtype=torch.uint8, device=dev)
        self.status_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.event = None
        self.calls = 0
        self.unchecked = False  # calls since the last check before an optimizer step
        self.guard_event = None  # status copy behind a step guarded on the device

    def status_word(self) -> torch.Tensor:
        return self.buf[:4].view(torch.int32)

    def take_probe(self) -> int:
        """Status seen by a completed probe (0 if none has completed, or while
        the stream is being captured into a graph)."""
        if self.event is None or torch.cuda.is_current_stream_capturing() or not self.event.query():
            return 0
        self.event = None
        return int(self.status_host[0])

    def queue_probe(self) -> None:
        self.calls += 1
        self.unchecked = True
        if (self.event is None and self.calls % STATUS_PERIOD == 0
                and not torch.cuda.is_current_stream_capturing()):
            self.status_host.copy_(self.status_word(), non_blocking=True)
            self.event = torch.cuda.Event()
            self.event.record()


def _persistent_workspace(nbytes: int, dev: torch.device, stream: int) -> _Workspace:
    key = (dev.index, stream)
    ws = _ws_cache.get(key)  # (a dict read is atomic; the lock guards replacement)
    if ws is not None and ws.buf.numel() >= nbytes:
        return ws
    with _ws_lock:
        ws = _ws_cache.get(key)
        if ws is None or ws.buf.numel() < nbytes:
            if len(_ws_cache) >= 16:
                _ws_cache.clear()
            ws = _Workspace(nbytes, dev)
            _ws_cache[key] = ws
        _install_step_check()
        return ws


# Before every optimizer step (a global torch.optim pre-step hook, installed with
# the first workspace), the status words of the workspaces used since the last
# step are checked, so that no step consumes the NaN gradients of a call whose
# bounded wait expired:
#   - optimizers that can skip a step on the device (torch's fused ones, which
#     honour a `found_inf` tensor as GradScaler uses it) get found_inf = 1 when
#     a status word is set, without a host synchronisation; the expiry is then
#     raised at the next step (or the next call that reads a completed probe);
#   - every other optimizer: one device synchronisation, and the step raises
#     before it runs.
# "async" leaves only the periodic asynchronous probe (no check before steps).
_EXPIRY_CHECKS = ("optimizer_step", "async")
_expiry_check = os.environ.get("FDP_EXPIRY_CHECK", "optimizer_step")
if _expiry_check not in _EXPIRY_CHECKS:
    raise ValueError(f"FDP_EXPIRY_CHECK must be one of {_EXPIRY_CHECKS}, got {_expiry_check!r}")
_step_hook = None
_guarded: dict = {}  # id(optimizer) -> its found_inf before the guard (restored after the step)


def set_expiry_check(mode: str) -> str:
    """When an expired bounded wait is reported; returns the previous mode.

    "optimizer_step" (default): before every optimizer step the status words
    of the workspaces used since the last step are checked.  An optimizer that
    can skip a step on the device (torch's fused optimizers) skips it when a
    word is set, with no host synchronisation, and the next step raises
    FlashDPError; any other optimizer synchronises once per step and raises
    before the step runs.  "async": only the asynchronous probe every
    STATUS_PERIOD calls (a later call raises; no check before steps).
    """
    global _expiry_check
    if mode not in _EXPIRY_CHECKS:
        raise ValueError(f"expiry check must be one of {_EXPIRY_CHECKS}, got {mode!r}")
    prev, _expiry_check = _expiry_check, mode
    return prev


def _check_before_step(optimizer, args, kwargs):
    if _expiry_check != "optimizer_step":
        return
    wss = list(_ws_cache.values())
    for ws in wss:  # an expiry that an earlier guarded step skipped on the device
        if ws.guard_event is not None and ws.guard_event.query():
            ws.guard_event = None
            if int(ws.status_host[0]) != 0:
                _raise_expired(ws, "an earlier optimizer step was skipped on the device for it")
    dirty = [ws for ws in wss if ws.unchecked]
    if not dirty:
        return
    devs = {ws.buf.device for ws in dirty}
    if getattr(optimizer, "_step_supports_amp_scaling", False) and len(devs) == 1:
        dev = devs.pop()
        with torch.cuda.device(dev):
            if torch.cuda.is_current_stream_capturing():
                return
            flag = torch.zeros((), dtype=torch.float32, device=dev)  # (a scalar, as GradScaler's)
            for ws in dirty:
                ws.unchecked = False
                flag = torch.maximum(flag, ws.status_word().ne(0).float().reshape(()))
                if ws.guard_event is None:  # report it at the next step
                    ws.status_host.copy_(ws.status_word(), non_blocking=True)
                    ws.guard_event = torch.cuda.Event()
                    ws.guard_event.record()
        prev = getattr(optimizer, "found_inf", None)
        _guarded[id(optimizer)] = prev
        optimizer.found_inf = (flag if prev is None else
                               torch.maximum(flag, prev.to(dev).float().reshape(())))
        return
    for ws in dirty:
        dev = ws.buf.device
        with torch.cuda.device(dev):
            if torch.cuda.is_current_stream_capturing():
                return
            torch.cuda.synchronize(dev)
        ws.unchecked = False
        status = int(ws.status_word().item())
        if status != 0:
            _raise_expired(ws, "found before optimizer.step(); the step did not run", status)


def _restore_after_step(optimizer, args, kwargs):
    key = id(optimizer)
    if key not in _guarded:
        return
    prev = _guarded.pop(key)
    if prev is None:
        if hasattr(optimizer, "found_inf"):
            del optimizer.found_inf
    else:
        optimizer.found_inf = prev


def _install_step_check() -> None:
    global _step_hook
    if _step_hook is None:
        from torch.optim.optimizer import (register_optimizer_step_post_hook,
                                           register_optimizer_step_pre_hook)
        _step_hook = (register_optimizer_step_pre_hook(_check_before_step),
                      register_optimizer_step_post_hook(_restore_after_step))


def release_workspaces() -> None:
    """Drop the cached per-stream workspaces (they are re-made on the next call)."""
    with _ws_lock:
        _ws_cache.clear()


def _raise_expired(ws: _Workspace, when: str, status: int = 1) -> None:
    del status  # every nonzero status is an expired wait
    ws.status_word().zero_()  # stream-ordered: later calls see a clear status word
    raise _lib.FlashDPError(
        f"fdp_wgrad_clip: a bounded inter-workgroup wait of the single-pass kernel timed out "
        f"({when}); the results of that call are NaN")


def wgrad_status(device=None, clear: bool = True) -> int:
    """Synchronise and return the status word of the current stream's workspace
    (nonzero: a bounded wait of an earlier call timed out and its outputs are
    NaN); ``clear`` resets it."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    ws = _ws_cache.get((dev.index, _lib.stream_handle(dev)))
    if ws is None:
        return 0
    torch.cuda.synchronize(dev)
    v = int(ws.status_word().item())
    if v and clear:
        ws.status_word().zero_()
    return v


def set_wgrad_launch(mode: str) -> str:
    """Default launch of the single-pass kernel; returns the previous mode.

    "plain" (default): an ordinary dispatch.  The grid is sized to the
    kernel's occupancy, so on a device with nothing else resident every
    workgroup runs at once; work on other streams only delays workgroups
    until it finishes.  If a grid wait nevertheless expires (seconds), the
    affected outputs are NaN and the workspace status word is set
    (``check=True`` raises): results are never silently wrong.
    "cooperative": hipLaunchCooperativeKernel, which guarantees co-residency
    at the cost of the runtime's synchronisation around each launch (about
    15 us per call on MI355X); use it when another kernel running at the
    same time may wait on this one.
    """
    global _launch_mode
    if mode not in _LAUNCH_MODES:
        raise ValueError(f"launch mode must be one of {_LAUNCH_MODES}, got {mode!r}")
    prev, _launch_mode = _launch_mode, mode
    return prev


class _Prepared:
    """A checked call signature of wgrad_clip (contiguous operands, no injected
    noise, no stats): the per-call work left is the output allocation, the
    stream's workspace and the library call."""
    __slots__ = ("fn", "fast", "name", "bias", "dims", "out_shape", "out_dtype", "odt", "flags",
                 "nbytes", "dev")

    def __init__(self, bias, dims, out_shape, out_dtype, odt, flags, nbytes, dev):
        L = _lib.lib()
        fc = _lib.fast_call()
        self.fast = None if fc is None else (fc.wgrad_bias if bias else fc.wgrad)
        self.fn = L.fdp_wgrad_bias_clip if bias else L.fdp_wgrad_clip
        self.name = "fdp_wgrad_bias_clip" if bias else "fdp_wgrad_clip"
        self.bias = bias
        self.dims, self.out_shape, self.out_dtype, self.odt = dims, out_shape, out_dtype, odt
        self.flags, self.nbytes, self.dev = flags, nbytes, dev

    def call(self, a, b, C, clamp, out_scale, noise_scale, noise_key, bias_out, bias_scale,
             bias_noise_scale, bias_noise_key):
        dev = self.dev
        out = torch.empty(self.out_shape, dtype=self.out_dtype, device=dev)
        stream = _lib.stream_handle(dev)
        ws = _persistent_workspace(self.nbytes, dev, stream)
        if ws.event is not None:
            probed = ws.take_probe()
            if probed != 0:
                _raise_expired(ws, "reported asynchronously for an earlier call on this stream",
                               probed)
        if self.fast is not None:
            # (the extension masks keys to 64 bits and takes ints for floats)
            if noise_key is not None and type(noise_key) is not tuple:
                noise_key = tuple(noise_key)
            common = (a.data_ptr(), b.data_ptr(), *self.dims, C, clamp, out_scale, noise_scale,
                      noise_key, out.data_ptr(), self.out_shape[1], self.odt, self.flags)
            if self.bias:
                if bias_noise_key is not None and type(bias_noise_key) is not tuple:
                    bias_noise_key = tuple(bias_noise_key)
                st = self.fast(*common, bias_out.data_ptr(), _lib.dtype_code(bias_out.dtype),
                               bias_scale, bias_noise_scale, bias_noise_key, ws.buf.data_ptr(),
                               ws.buf.numel(), stream)
            else:
                st = self.fast(*common, ws.buf.data_ptr(), ws.buf.numel(), stream)
            if st != 0:
                _lib.check(st, self.name)
            ws.queue_probe()
            return out
        key = None if noise_key is None else _lib.noise_key(noise_key)
        args = (a.data_ptr(), b.data_ptr(), *self.dims, float(C), float(clamp), None,
                float(out_scale), None, float(noise_scale), key, out.data_ptr(),
                self.out_shape[1], self.odt, None, None, self.flags)
        if self.bias:
            bkey = _lib.noise_key(bias_noise_key)
            bias = _lib.BiasOut(bias_out.data_ptr(), _lib.dtype_code(bias_out.dtype),
                                float(bias_scale), None, float(bias_noise_scale), bkey, None, None)
            st = self.fn(*args, ctypes.byref(bias), ws.buf.data_ptr(), ws.buf.numel(), stream)
        else:
            st = self.fn(*args, ws.buf.data_ptr(), ws.buf.numel(), stream)
        if st != 0:
            _lib.check(st, self.name)
        ws.queue_probe()
        return out


_prepared: dict = {}


def _inner_contig(t: torch.Tensor) -> torch.Tensor:
    if t.dim() != 3:
        raise ValueError(f"expected a 3-D tensor, got shape {tuple(t.shape)}")
    if t.stride(2) != 1 or (t.shape[1] > 1 and t.stride(1) < t.shape[2]):
        t = t.contiguous()
    return t


def wgrad_clip(a: torch.Tensor, b: torch.Tensor, C: float = 1.0, clamp_value: float = 1.0, *,
               layout: str = "tn", clip_args=None, out_scale: float = 1.0,
               noise: torch.Tensor | None = None, noise_scale: float = 1.0,
               noise_key: tuple[int, int] | None = None,
               out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
               return_stats: bool = False, noclip: bool = False, two_pass: bool = False,
               launch: str | None = None, single_pass: str = "auto", check: bool = False,
               bias_out: torch.Tensor | None = None, bias_scale: float = 1.0,
               bias_noise: torch.Tensor | None = None, bias_noise_scale: float = 1.0,
               bias_noise_key: tuple[int, int] | None = None, bias_operand: str = "a"):
    """out = out_scale * sum_b c_b G_b + noise_scale * z, c_b = clip(||G_b||_F).

    layout "tn": a [B,K,M], b [B,K,N], G_b = a_b^T b_b;
    layout "nn": a [B,M,K], b [B,K,N], G_b = a_b b_b.
    ``clip_args`` (tensor [C, clamp] or pair) overrides C / clamp_value.
    z is the ``noise`` tensor, or, without one, the in-kernel Philox draw of
    ``noise_key = (seed, offset)`` (fdp_noise_key in include/flashdp_hip.h);
    neither: no noise.
    With ``return_stats`` also returns the fp32 per-sample norms and factors.
    ``two_pass`` forces the norm-pass + clipped-sum-pass schedule instead of the
    single-pass kernels; ``single_pass`` picks between those: "auto" (the wide
    schedule when the layer's products fill at least 70% of the CUs, else the
    grouped 128x128 kernel), "wide" (the wide schedule whenever the products
    fit the CUs), "unpaired" (as "wide", one sample per CU only) or "narrow"
    (grouped only).  The wide schedule holds two samples' 192x192 tiles per CU
    where the batch is even (6..72) and the contraction a multiple of 32 (a
    bias is formed in the same launch either way), else one sample's 384x192
    tile.  ``launch``
    ("cooperative" / "plain", default: the mode of ``set_wgrad_launch``) picks
    how that kernel is dispatched.
    ``check`` synchronises and raises if a bounded inter-workgroup wait of the
    single-pass kernel expired (in this call or an earlier one on the stream
    whose expiry was not reported yet).  Without it, expiries are reported by a
    later call: every STATUS_PERIOD calls the status word is copied to the host
    behind the call, and the first call after the copy completes raises.  An
    expiry poisons only the launch it happened in (its outputs are NaN).

    ``bias_out`` (layout "tn") also writes the bias of one operand
    (fdp_wgrad_bias_clip): of a (``bias_operand="a"``, an [M] tensor: the DP
    Linear bias, a = grad_output) or of b (``"b"``, an [N] tensor: the DP
    Conv1D bias, b = grad_output):
    bias_out[c] = bias_scale * sum_b c'_b sum_k op_b[k, c] + bias_noise_scale * zb[c],
    c'_b = clip(||op_b||_F) with the same C / clamp; zb is ``bias_noise`` or the
    draw of ``bias_noise_key``.  The 16-bit kernels form it from the operand
    fragments they hold, in the same call; fp32 operands run the column-sum
    kernel after the weight gradient.  With ``return_stats`` the bias's norms
    and factors follow the weight's.
    """
    simple = (clip_args is None and noise is None and out is None and not return_stats
              and not check and bias_noise is None)
    if simple:
        fkey = (a.shape, a.stride(), b.shape, b.stride(), a.dtype, b.dtype, a.device, b.device,
                layout, out_dtype, noclip, two_pass, launch or _launch_mode, single_pass,
                None if bias_out is None else (bias_out.shape, bias_out.dtype, bias_out.device,
                                               bias_out.is_contiguous(), bias_operand))
        prep = _prepared.get(fkey)
        if prep is not None:
            return prep.call(a, b, C, clamp_value, out_scale, noise_scale, noise_key, bias_out,
                             bias_scale, bias_noise_scale, bias_noise_key)
    dev = _lib.require_hip(a, b, noise, out, bias_out, bias_noise)
    if a.dtype != b.dtype:
        raise KeyError(f"operand dtypes differ: {a.dtype} vs {b.dtype}")
    dt = _lib.dtype_code(a.dtype)
    a0, b0 = a, b
    a, b = _inner_contig(a), _inner_contig(b)
    if bias_out is not None:
        if layout != "tn" or noclip:
            raise ValueError("the bias of an operand needs layout 'tn' and a clip")
        if bias_operand == "a":
            a = a.contiguous()
        elif bias_operand == "b":
            b = b.contiguous()
        else:
            raise ValueError(f"bias_operand must be 'a' or 'b', got {bias_operand!r}")
    if layout == "tn":
        Bn, K, M = a.shape
        lay = _lib.LAYOUT_TN
    elif layout == "nn":
        Bn, M, K = a.shape
        lay = _lib.LAYOUT_NN
    else:
        raise ValueError(f"unknown layout {layout!r}")
    if b.shape[0] != Bn or b.shape[1] != K:
        raise ValueError(f"operand shapes {tuple(a.shape)} and {tuple(b.shape)} do not match "
                         f"for layout {layout}")
    N = b.shape[2]
    if Bn == 0:
        raise ValueError("batch size must be at least 1")
    if out_dtype is None:
        out_dtype = out.dtype if out is not None else a.dtype
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    elif out.shape != (M, N) or out.stride(1) != 1 or out.dtype != out_dtype:
        raise ValueError("out must be an [M, N] row-major tensor of out_dtype")
    odt = _lib.dtype_code(out_dtype)
    if noise is not None:
        if noise.shape != (M, N):
            raise ValueError(f"noise must have shape {(M, N)}, got {tuple(noise.shape)}")
        noise = noise.to(out_dtype).contiguous()
    C_, clamp_, cad = clip_args_of(clip_args, dev) if clip_args is not None else (
        float(C), float(clamp_value), None)
    norms = factors = None
    if return_stats:
        factors = torch.empty(Bn, dtype=torch.float32, device=dev)
        norms = None if noclip else torch.empty(Bn, dtype=torch.float32, device=dev)
    bias_arg = bnorms = bfactors = None
    if bias_out is not None:
        blen = M if bias_operand == "a" else N
        if bias_out.shape != (blen,) or not bias_out.is_contiguous():
            raise ValueError(f"bias_out must be a contiguous [{blen}] tensor")
        if bias_noise is not None:
            if bias_noise.numel() != blen:
                raise ValueError(f"bias_noise must have {blen} elements")
            bias_noise = bias_noise.reshape(blen).to(bias_out.dtype).contiguous()
        if return_stats:
            bnorms = torch.empty(Bn, dtype=torch.float32, device=dev)
            bfactors = torch.empty(Bn, dtype=torch.float32, device=dev)
        bias_arg = _lib.BiasOut(bias_out.data_ptr(), _lib.dtype_code(bias_out.dtype),
                                float(bias_scale), _lib.ptr(bias_noise), float(bias_noise_scale),
                                _lib.noise_key(bias_noise_key), _lib.ptr(bnorms),
                                _lib.ptr(bfactors))
    mode = _launch_mode if launch is None else launch
    if mode not in _LAUNCH_MODES:
        raise ValueError(f"launch must be one of {_LAUNCH_MODES}, got {mode!r}")
    if single_pass not in _SINGLE_PASS:
        raise ValueError(f"single_pass must be one of {tuple(_SINGLE_PASS)}, got {single_pass!r}")
    flags = ((_lib.WGRAD_NOCLIP if noclip else 0) | (_lib.WGRAD_TWO_PASS if two_pass else 0)
             | (_lib.WGRAD_PLAIN_LAUNCH if mode == "plain" else 0) | _lib.WGRAD_CLEAN_WORKSPACE
             | _SINGLE_PASS[single_pass]
             | (_lib.WGRAD_BIAS_OF_B if bias_out is not None and bias_operand == "b" else 0))
    L = _lib.lib()
    key = (dev.index, Bn, K, M, N, dt, flags, bias_arg is not None)
    nbytes = _ws_sizes.get(key)
    if nbytes is None:
        query = (L.fdp_wgrad_clip_workspace_size if bias_arg is None
                 else L.fdp_wgrad_bias_clip_workspace_size)
        nbytes = _lib.size_query(query, Bn, K, M, N, dt, flags)
        _ws_sizes[key] = nbytes
    stream = _lib.stream_handle(dev)
    ws = _persistent_workspace(nbytes, dev, stream)
    probed = ws.take_probe()
    if probed != 0:
        _raise_expired(ws, "reported asynchronously for an earlier call on this stream", probed)
    args = (_lib.ptr(a), _lib.ptr(b), Bn, K, M, N, a.stride(0), a.stride(1), b.stride(0),
            b.stride(1), lay, dt, ctypes.c_float(C_), ctypes.c_float(clamp_), _lib.ptr(cad),
            ctypes.c_float(out_scale), _lib.ptr(noise), ctypes.c_float(noise_scale),
            _lib.noise_key(noise_key), out.data_ptr(), out.stride(0), odt, _lib.ptr(norms),
            _lib.ptr(factors), flags)
    if bias_arg is None:
        st = L.fdp_wgrad_clip(*args, ws.buf.data_ptr(), ws.buf.numel(), stream)
        _lib.check(st, "fdp_wgrad_clip")
    else:
        st = L.fdp_wgrad_bias_clip(*args, ctypes.byref(bias_arg), ws.buf.data_ptr(),
                                   ws.buf.numel(), stream)
        _lib.check(st, "fdp_wgrad_bias_clip")
    if check:
        status = int(ws.status_word().item())
        if status != 0:
            _raise_expired(ws, "this call or an earlier one on this stream", status)
    else:
        ws.queue_probe()
    if (simple and a is a0 and b is b0 and a.is_contiguous() and b.is_contiguous()
            and len(_prepared) < 256):
        # this call's arguments checked out and reached the kernel as given (no
        # copy was made): later calls of the same signature (shapes, strides,
        # dtypes, devices, options) go straight to the library.  A call that
        # needed a contiguous copy is never cached, since a later tensor with
        # the same strides would reach the kernel uncopied.
        _prepared[fkey] = _Prepared(bias_arg is not None, (Bn, K, M, N, a.stride(0), a.stride(1),
                                    b.stride(0), b.stride(1), lay, dt), (M, N), out_dtype, odt,
                                    flags, nbytes, dev)
    if return_stats:
        return (out, norms, factors) if bias_arg is None else (out, norms, factors, bnorms, bfactors)
    return out


def bmtm_clip(tensor1: torch.Tensor, tensor2: torch.Tensor, clip_args=None) -> torch.Tensor:
    """sum_b clip(||t1_b^T t2_b||) t1_b^T t2_b; t1 [B,K,M], t2 [B,K,N] -> [M,N] in t1's dtype."""
    return wgrad_clip(tensor1, tensor2.to(tensor1.dtype), layout="tn",
                      clip_args=clip_args if clip_args is not None else (1.0, 1.0))


def bmm_clip(tensor1: torch.Tensor, tensor2: torch.Tensor, clip_args=None) -> torch.Tensor:
    """sum_b clip(||t1_b t2_b||) t1_b t2_b; t1 [B,M,K], t2 [B,K,N] -> [M,N] fp32
    (the reference accumulates this operator in its fp32 acc dtype, bmm_clip_loop.py:138)."""
    return wgrad_clip(tensor1, tensor2.to(tensor1.dtype), layout="nn",
                      clip_args=clip_args if clip_args is not None else (1.0, 1.0),
                      out_dtype=torch.float32)


def mm_clip(mat1: torch.Tensor, mat2: torch.Tensor, clip_args=None) -> torch.Tensor:
    """sum_k clip(||a_k (x) b_k||) a_k (x) b_k with a_k = mat1[:,k], b_k = mat2[k,:] -> [M,N]:
    one rank-1 "sample" per k, i.e. the clipped product sum with B=K and K=1."""
    if mat1.dim() != 2 or mat2.dim() != 2 or mat1.shape[1] != mat2.shape[0]:
        raise ValueError("mm_clip expects mat1 [M,K] and mat2 [K,N]")
    a = mat1.t().contiguous().unsqueeze(1)             # [K,1,M]
    b = mat2.to(mat1.dtype).contiguous().unsqueeze(1)  # [K,1,N]
    return wgrad_clip(a, b, layout="tn",
                      clip_args=clip_args if clip_args is not None else (1.0, 1.0))


def mm_fused(tensor1: torch.Tensor, tensor2: torch.Tensor) -> torch.Tensor:
    """Plain product tensor1 @ tensor2 in the fp32 accumulation dtype
    (flashdp/core/linear_clip.py:64-91): the product sum with one sample and no clip."""
    if tensor1.dim() < 2 or tensor2.dim() < 2:
        raise KeyError("The dimensions of input tensors must be at least 2.")
    if tensor1.shape[-1] != tensor2.shape[0]:
        raise ValueError("tensor1 last dimension must match tensor2 first dimension")
    s1, s2 = tensor1.shape, tensor2.shape
    a = tensor1.reshape(1, -1, s1[-1])
    b = tensor2.to(tensor1.dtype).reshape(1, s2[0], -1)
    out = wgrad_clip(a, b, layout="nn", clip_args=(float("inf"), 1.0), noclip=True,
                     out_dtype=torch.float32)
    return out.reshape(tuple(s1[:-1]) + tuple(s2[1:]))


def linear_weight_flashdp(input: torch.Tensor, grad_output: torch.Tensor, C: float,
                          clamp_value: float, runtime_tuner: RuntimeAutoTuner | None = None):
    """sum_b clip(||g_b^T x_b||) g_b^T x_b -> [O, I] in grad_output's dtype
    (flashdp/core/linear_clip.py:107-113; the tuner argument is accepted only)."""
    if runtime_tuner is not None:
        runtime_tuner.choose_function([bmtm_clip])
    return wgrad_clip(grad_output, input.to(grad_output.dtype), C, clamp_value, layout="tn")


def conv1d_weight_flashdp(input: torch.Tensor, grad_output: torch.Tensor, C: float,
                          clamp_value: float, runtime_tuner: RuntimeAutoTuner | None = None):
    """sum_b clip(||x_b^T g_b||) x_b^T g_b -> [I, O]
    (flashdp/core/transformers_conv1d_clip.py:22-28)."""
    if runtime_tuner is not None:
        runtime_tuner.choose_function([bmtm_clip])
    return wgrad_clip(input.to(grad_output.dtype), grad_output, C, clamp_value, layout="tn")
