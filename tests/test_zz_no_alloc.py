"""fdp_wgrad_clip_noalloc (the entry point whose workspace is the library's own
file-scope device array) against fdp_wgrad_clip with a caller workspace, both
called through the C ABI.  Same kernels, same plan: the outputs, norms and
factors must be bit-identical, on consecutive calls that leave the shared
array dirty for the next one (the second call smaller than the first)."""
import ctypes

import pytest
import torch

from oracle import dp_clip as O
from tests._tol import assert_close, assert_elementwise

from flashdp4review_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, K, M, N, layout, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn((B, K, M) if layout == "tn" else (B, M, K), generator=g)
    b = torch.randn((B, K, N), generator=g) * 0.02
    return a.to(torch.bfloat16).to(DEV), b.to(torch.bfloat16).to(DEV)


def _call(noalloc, a, b, shape, layout, C, key, flags):
    """One clipped sum through the C ABI; returns (status, out, norms, factors)."""
    L = _lib.lib()
    B, K, M, N = shape
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device=DEV)
    norms = torch.full((B,), float("nan"), dtype=torch.float32, device=DEV)
    fac = torch.full((B,), float("nan"), dtype=torch.float32, device=DEV)
    lay = _lib.LAYOUT_TN if layout == "tn" else _lib.LAYOUT_NN
    common = (a.data_ptr(), b.data_ptr(), B, K, M, N, a.stride(0), a.stride(1), b.stride(0),
              b.stride(1), lay, _lib.FDP_BF16, ctypes.c_float(C), ctypes.c_float(1.0), None,
              ctypes.c_float(1.0 / B), None, ctypes.c_float(0.5 / B), _lib.noise_key(key),
              out.data_ptr(), N, _lib.FDP_F32, norms.data_ptr(), fac.data_ptr())
    stream = _lib.stream_handle(torch.device(DEV))
    if noalloc:
        st = L.fdp_wgrad_clip_noalloc(*common, flags | _lib.WGRAD_CLEAN_WORKSPACE, stream)
    else:
        nb = _lib.size_query(L.fdp_wgrad_clip_workspace_size, B, K, M, N, _lib.FDP_BF16,
                             flags | _lib.WGRAD_PLAIN_LAUNCH)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=DEV)
        st = L.fdp_wgrad_clip(*common, flags | _lib.WGRAD_PLAIN_LAUNCH, ws.data_ptr(), ws.numel(),
                              stream)
    torch.cuda.synchronize()
    return st, out, norms, fac


# (shape, layout, noise key): the cfg2 layer (single-pass wide kernel, in-kernel
# noise), then smaller problems on the grouped single-pass kernel.
CALLS = [
    ((8, 1024, 3072, 768), "tn", (1234, 0)),
    ((4, 128, 768, 768), "nn", None),
    ((16, 16, 256, 256), "tn", (99, 7)),
]


@pytest.mark.parametrize("flags", [0, _lib.WGRAD_NARROW], ids=["auto", "narrow"])
def test_noalloc_matches_workspace_entry(flags):
    print(f"no-alloc: flags={flags}", flush=True)
    for i, (shape, layout, key) in enumerate(CALLS):
        print(f"  call {i}: shape={shape} layout={layout} noise={key}", flush=True)
        a, b = _inputs(*shape, layout, seed=40 + i)
        # C at the median per-sample norm: some samples clip, some do not
        C = float(_call(False, a, b, shape, layout, 1.0, None, flags)[2].median())
        st, out, norms, fac = _call(True, a, b, shape, layout, C, key, flags)
        assert st == 0, _lib.lib().fdp_strerror(st)
        st0, out0, norms0, fac0 = _call(False, a, b, shape, layout, C, key, flags)
        assert st0 == 0
        assert torch.equal(out, out0), f"call {i}: clipped sum differs"
        assert torch.equal(norms, norms0) and torch.equal(fac, fac0), f"call {i}: stats differ"
        ref, nref, fref = O.wgrad_clip(a, b, C, 1.0, layout, out_scale=1.0 / shape[0])
        assert_elementwise(norms, nref, torch.bfloat16, "no-alloc norms")
        assert_elementwise(fac, fref, torch.bfloat16, "no-alloc factors")
        if key is None:
            assert_close(out, ref, torch.bfloat16, "no-alloc clipped sum")


def test_noalloc_repeat_after_smaller_call():
    """The large call again after the smaller ones: the array's leftover
    contents from the previous call do not change the result."""
    shape, layout, key = CALLS[0]
    a, b = _inputs(*shape, layout, seed=40)
    first = _call(True, a, b, shape, layout, 0.05, key, 0)
    small_shape, small_layout, _ = CALLS[1]
    a2, b2 = _inputs(*small_shape, small_layout, seed=41)
    assert _call(True, a2, b2, small_shape, small_layout, 0.05, None, 0)[0] == 0
    again = _call(True, a, b, shape, layout, 0.05, key, 0)
    assert first[0] == 0 and again[0] == 0
    for x, y in zip(first[1:], again[1:]):
        assert torch.equal(x, y)


def test_noalloc_rejects_oversize_without_launch():
    """A problem whose workspace exceeds FDP_NOALLOC_SCRATCH_BYTES returns
    FDP_ERR_TOO_LARGE (7) and writes nothing."""
    L = _lib.lib()
    limit = 64 << 20
    cands = [(128, 16, 2048, 2048), (512, 16, 2048, 2048), (1024, 8, 1024, 1024)]
    big = [s for s in cands
           if _lib.size_query(L.fdp_wgrad_clip_workspace_size, *s, _lib.FDP_BF16,
                              _lib.WGRAD_PLAIN_LAUNCH) > limit]
    assert big, "no candidate shape exceeds the scratch array on this device"
    shape = big[0]
    print(f"no-alloc oversize: shape={shape}", flush=True)
    a, b = _inputs(*shape, "tn", seed=50)
    st, out, norms, fac = _call(True, a, b, shape, "tn", 1.0, None, 0)
    assert st == 7
    assert torch.isnan(out).all() and torch.isnan(norms).all() and torch.isnan(fac).all()
    with pytest.raises(ValueError):
        _lib.check(st, "fdp_wgrad_clip_noalloc")


def _noalloc_into(a, b, shape, C, key, out, norms, fac, flags=0):
    """fdp_wgrad_clip_noalloc (layout TN) into caller-made outputs; returns the status."""
    B, K, M, N = shape
    return _lib.lib().fdp_wgrad_clip_noalloc(
        a.data_ptr(), b.data_ptr(), B, K, M, N, a.stride(0), a.stride(1), b.stride(0),
        b.stride(1), _lib.LAYOUT_TN, _lib.FDP_BF16, ctypes.c_float(C), ctypes.c_float(1.0), None,
        ctypes.c_float(1.0 / B), None, ctypes.c_float(0.5 / B), _lib.noise_key(key),
        out.data_ptr(), N, _lib.FDP_F32, norms.data_ptr(), fac.data_ptr(), flags,
        _lib.stream_handle(torch.device(DEV)))


def test_noalloc_allocates_nothing():
    """Two calls (the large one, then a smaller one) leave the device's free
    memory unchanged: the call makes no device allocation (its inputs and
    outputs are made before the first reading; a first call loads the
    library's code on the device)."""
    calls = []
    for i, shape in enumerate([(8, 1024, 3072, 768), (16, 16, 256, 256)]):
        a, b = _inputs(*shape, "tn", seed=60 + i)
        B, K, M, N = shape
        outs = (torch.empty(M, N, device=DEV), torch.empty(B, device=DEV),
                torch.empty(B, device=DEV))
        calls.append((a, b, shape, outs))
    a, b, shape, outs = calls[0]
    assert _noalloc_into(a, b, shape, 0.05, (5, 0), *outs) == 0  # warm-up
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for a, b, shape, outs in calls:
        assert _noalloc_into(a, b, shape, 0.05, (5, 0), *outs) == 0
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"


def test_noalloc_in_a_graph_with_a_noise_counter():
    """The no-allocation call and fdp_noise_advance captured into one HIP graph
    and replayed three times, with eager work and synchronisations between the
    replays: each replay equals the eager call with the key's offset moved to
    that replay's counter value, and the replays differ from one another."""
    shape = (8, 256, 1536, 384)
    B, K, M, N = shape
    a, b = _inputs(*shape, "tn", seed=70)
    counter = torch.zeros(1, dtype=torch.int64, device=DEV)
    blocks = (M * N + 3) // 4
    out, norms, fac = (torch.empty(M, N, device=DEV), torch.empty(B, device=DEV),
                       torch.empty(B, device=DEV))
    key = (4321, 10, counter.data_ptr())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # one eager call on the capture stream first
        assert _noalloc_into(a, b, shape, 0.05, key, out, norms, fac) == 0
        _lib.noise_advance(counter, blocks)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        assert _noalloc_into(a, b, shape, 0.05, key, out, norms, fac) == 0
        _lib.noise_advance(counter, blocks)
    prev = None
    for rep in range(3):
        ctr = int(counter.item())
        graph.replay()
        torch.cuda.synchronize()
        assert int(counter.item()) == ctr + blocks
        got = out.clone()
        st, ref, _, _ = _call(False, a, b, shape, "tn", 0.05, (4321, 10 + ctr), 0)
        assert st == 0
        assert torch.equal(got, ref), f"replay {rep} differs from the eager call"
        if prev is not None:
            assert not torch.equal(prev, got)
        prev = got
