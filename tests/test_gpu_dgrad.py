"""GPU parity of the DP layers' input gradient on the HIP kernel (fdp_dgrad):
dX = g W (a Linear weight [out, in], flashdp/layers/linear.py:62-67) and
dX = g W^T (a Conv1D weight [in, out], flashdp/layers/transformers_conv1d.py:70-77)
against the float64 product of the same dtype-rounded operands (the oracle's
dx, oracle/dp_clip.py linear_backward / conv1d_backward, pinned to torch
autograd in tests/test_oracle.py), with
ragged edges, both tile heights, strided rows, determinism and graph replay."""
import numpy as np
import pytest
import torch

from oracle import dp_clip as O
from tests._tol import assert_close

from flashdp4review_amd import DPConv1D, DPLinear, _lib, core

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(M, K, N, dtype, layout, seed=0):
    gen = torch.Generator().manual_seed(seed)
    g = (torch.randn(M, K, generator=gen) * 0.02).to(dtype)
    w = (torch.randn((K, N) if layout == "nn" else (N, K), generator=gen) * 0.02).to(dtype)
    return g.to(DEV), w.to(DEV)


def ref_dx(g, w, layout):
    gd = g.double().cpu().numpy()
    wd = w.double().cpu().numpy()
    return gd @ (wd if layout == "nn" else wd.T)


def call(g, w, layout, ldg=None):
    """fdp_dgrad through the C ABI."""
    L = _lib.lib()
    M, K = g.shape[0], g.shape[1]
    N = w.shape[1] if layout == "nn" else w.shape[0]
    lay = 0 if layout == "nn" else 1
    dt = _lib.dtype_code(g.dtype)
    out = torch.full((M, N), float("nan"), dtype=g.dtype, device=DEV)
    st = L.fdp_dgrad(g.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K,
                     ldg if ldg is not None else g.stride(0), w.stride(0), N, lay, dt,
                     _lib.stream_handle(torch.device(DEV)))
    _lib.check(st, "fdp_dgrad")
    return out


SHAPES = [
    (300, 128, 100),     # ragged rows and columns
    (256, 4096, 192),    # one tile, a long contraction
    (1000, 192, 200),    # several tiles
    (17, 64, 40),        # fewer rows than a tile, the shortest contraction (no split)
    (4096, 768, 768),    # GPT-2 small Linear
    (8192, 3072, 768),   # cfg2's dX (MLP-up, Linear): 256 tiles of 128 rows
    (16384, 2304, 768),  # cfg3's dX (c_attn, Conv1D): 256 tiles, one pass
    (2048, 2048, 2048),  # more tiles than CUs
]


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,N", SHAPES)
def test_dgrad_parity(M, K, N, dtype, layout):
    if layout == "nn" and N % 8 != 0:
        pytest.skip("a Linear weight's rows must be 16-byte multiples")
    g, w = make(M, K, N, dtype, layout)
    out = call(g, w, layout)
    assert torch.isfinite(out.float()).all()
    assert_close(out, ref_dx(g, w, layout), dtype, f"dgrad {layout} {(M, K, N)}",
                 margin=f"dX {layout} (M,K,N)={(M, K, N)} ({str(dtype)[6:]})")


@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_dgrad_deterministic(layout):
    """Repeated calls give the same bits, interleaved with calls of other
    shapes (both tile heights)."""
    g, w = make(8192, 3072, 768, torch.bfloat16, layout, seed=1)      # 128-row tiles
    g2, w2 = make(16384, 2304, 768, torch.bfloat16, layout, seed=2)   # 256-row tiles
    first, second = call(g, w, layout), call(g2, w2, layout)
    for _ in range(3):
        assert torch.equal(call(g, w, layout), first)
        assert torch.equal(call(g2, w2, layout), second)


def test_dgrad_strided_rows():
    """g rows with a stride beyond K (a column slice of a wider tensor)."""
    big = (torch.randn(1500, 640) * 0.02).to(torch.bfloat16).to(DEV)
    g = big[:, 64:64 + 512]  # row stride 640 elements
    w = (torch.randn(512, 264) * 0.02).to(torch.bfloat16).to(DEV)
    out = call(g, w, "nn", ldg=640)
    assert_close(out, ref_dx(g.contiguous(), w, "nn"), torch.bfloat16, "dgrad strided rows")
    # and the operator on the same view
    y = core.dgrad(g, w, "nn")
    assert torch.equal(y, out)


@pytest.mark.parametrize("cls", ["linear", "conv1d"])
def test_layer_input_grad_on_the_kernel(cls):
    """DPLinear / DPConv1D with the HIP input gradient selected: dx against the
    oracle's layer backward, and within the tolerance of torch's matmul path."""
    prev = core.set_dgrad("hip")
    try:
        torch.manual_seed(0)
        I, Ofeat = 768, 3072 if cls == "linear" else 2304
        if cls == "linear":
            m = DPLinear(I, Ofeat, C=1.0, noise_multiplier=0.0).to(DEV, torch.bfloat16)
        else:
            m = DPConv1D(Ofeat, I, C=1.0, noise_multiplier=0.0).to(DEV, torch.bfloat16)
        x = torch.randn(2, 512, I, device=DEV).to(torch.bfloat16).requires_grad_(True)
        gy = (torch.randn(2, 512, Ofeat, device=DEV) * 0.02).to(torch.bfloat16)
        m(x).backward(gy)
        W = m.weight.detach()
        r = (O.linear_backward if cls == "linear" else O.conv1d_backward)(
            x.detach(), gy, W, 1.0, 1.0)
        assert_close(x.grad, r["dx"], torch.bfloat16, f"{cls} dx (hip)",
                     margin=f"{cls} layer dx on fdp_dgrad")
        dx_hip = x.grad.clone()
        core.set_dgrad("torch")
        x.grad = None
        m(x).backward(gy)
        assert_close(x.grad, r["dx"], torch.bfloat16, f"{cls} dx (torch)")
        assert O.rel_err(dx_hip, x.grad.double().cpu().numpy()) < 1e-2
    finally:
        core.set_dgrad(prev)


def test_auto_mode_times_each_shape_once():
    """The default "auto" mode times both paths on the first call of a shape
    and keeps the faster: later calls of the shape take the same path (the same
    bits), the result is within the tolerance either way, and under graph
    capture an untimed shape takes torch's matmul without timing."""
    from flashdp4review_amd.core import inputgrad as D
    assert D._mode == "auto"
    with pytest.raises(ValueError):
        core.set_dgrad("fastest")
    g, w = make(8192, 768, 768, torch.bfloat16, "nn", seed=4)
    first = core.input_grad(g, w, "nn")
    key = (g.device.index, 8192, 768, 768, "nn", torch.bfloat16)
    assert core.dgrad_choices()[key] in ("hip", "torch")
    assert torch.equal(core.input_grad(g, w, "nn"), first)
    assert_close(first, ref_dx(g, w, "nn"), torch.bfloat16, "auto dX")
    g2, w2 = make(4096, 1024, 512, torch.bfloat16, "nt", seed=5)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g2 @ w2.t()  # warm-up of torch's matmul on the capture stream (untimed: no choice)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = core.input_grad(g2, w2, "nt")
    torch.cuda.current_stream().wait_stream(s)
    graph.replay()
    torch.cuda.synchronize()
    assert (g2.device.index, 4096, 512, 1024, "nt", torch.bfloat16) not in core.dgrad_choices()
    assert_close(out, ref_dx(g2, w2, "nt"), torch.bfloat16, "captured auto dX")


def test_dgrad_rejects_unsupported_operands():
    g, w = make(256, 96, 64, torch.bfloat16, "nn")
    with pytest.raises(ValueError):  # K % 64 != 0
        core.dgrad(g, w, "nn")
    g32 = torch.randn(256, 64, device=DEV)
    with pytest.raises(KeyError):
        core.dgrad(g32, torch.randn(64, 64, device=DEV), "nn")
    # the layer falls back to torch's matmul for such shapes
    out = core.input_grad(g, w, "nn")
    np.testing.assert_allclose(out.float().cpu().numpy(), ref_dx(g, w, "nn"), rtol=0, atol=2e-3)


def test_dgrad_empty_batch_and_misaligned_weight():
    """An empty batch gives an empty dX on either path (no launch); a weight
    view whose storage is not 16-byte aligned is copied, not refused."""
    g, w = make(512, 128, 264, torch.bfloat16, "nn", seed=7)
    empty = g[:0].reshape(0, 1, 128)
    assert core.dgrad(empty, w, "nn").shape == (0, 1, 264)
    prev = core.set_dgrad("hip")
    try:
        assert core.input_grad(empty, w, "nn").shape == (0, 1, 264)
    finally:
        core.set_dgrad(prev)
    wide = torch.zeros(128, 264 + 8, dtype=torch.bfloat16, device=DEV)
    wide[:, 1:265] = w
    wv = wide[:, 1:265]  # row stride 272, storage 2 bytes past a 16-byte boundary
    assert wv.data_ptr() % 16 != 0
    assert torch.equal(core.dgrad(g, wv, "nn"), call(g, w, "nn"))


def test_input_grad_past_a_buffer_record_takes_torch():
    """grad_output of 2^30 elements (2^24 rows of 64) is more than one of the
    kernel's 32-bit buffer records addresses: fdp_dgrad refuses it, and the
    layers' input gradient takes torch's matmul even in "hip" mode."""
    g = torch.empty(1 << 24, 64, dtype=torch.bfloat16, device=DEV).normal_(0.0, 0.02)
    w = (torch.randn(64, 64) * 0.02).to(torch.bfloat16).to(DEV)
    with pytest.raises(ValueError):
        core.dgrad(g, w, "nn")
    prev = core.set_dgrad("hip")
    try:
        out = core.input_grad(g, w, "nn")
    finally:
        core.set_dgrad(prev)
    assert torch.equal(out, g @ w)


def test_dgrad_graph_replays_match_eager():
    """fdp_dgrad records one kernel and no memset, so a captured call replays
    exactly: three replays, with eager calls and synchronisations between
    them, each equal to the eager result."""
    g, w = make(8192, 3072, 768, torch.bfloat16, "nn", seed=3)
    eager = core.dgrad(g, w, "nn")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        core.dgrad(g, w, "nn")  # warm-up on the capture stream
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = core.dgrad(g, w, "nn")
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(core.dgrad(g, w, "nn"), eager)
        torch.cuda.synchronize()
