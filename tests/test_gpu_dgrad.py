"""GPU parity of the DP layers' input gradient on the HIP kernel (fdp_dgrad):
dX = g W (a Linear weight [out, in], flashdp/layers/linear.py:62-67) and
dX = g W^T (a Conv1D weight [in, out], flashdp/layers/transformers_conv1d.py:70-77)
against the float64 product of the same dtype-rounded operands (the oracle's
dx, oracle/dp_clip.py linear_backward / conv1d_backward, pinned to torch
autograd in tests/test_oracle.py), with and without the split contraction,
ragged edges, strided rows, determinism and the self-clearing control words."""
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


def call(g, w, layout, ws=None, ldg=None):
    """fdp_dgrad through the C ABI with a zero-filled workspace of its own."""
    L = _lib.lib()
    M, K = g.shape[0], g.shape[1]
    N = w.shape[1] if layout == "nn" else w.shape[0]
    lay = 0 if layout == "nn" else 1
    dt = _lib.dtype_code(g.dtype)
    nb = _lib.size_query(L.fdp_dgrad_workspace_size, M, N, K, lay, dt)
    if ws is None:
        ws = torch.zeros(nb, dtype=torch.uint8, device=DEV)
    out = torch.full((M, N), float("nan"), dtype=g.dtype, device=DEV)
    st = L.fdp_dgrad(g.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K,
                     ldg if ldg is not None else g.stride(0), w.stride(0), N, lay, dt,
                     ws.data_ptr(), nb, _lib.stream_handle(torch.device(DEV)))
    _lib.check(st, "fdp_dgrad")
    return out, ws


SHAPES = [
    (300, 128, 100),     # ragged rows and columns, one tile, split over K
    (1000, 192, 200),    # several tiles
    (17, 64, 40),        # fewer rows than a tile, the shortest contraction (no split)
    (4096, 768, 768),    # GPT-2 small Linear
    (8192, 3072, 768),   # cfg2's dX (MLP-up, Linear): 128 tiles, split in two
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
    out, ws = call(g, w, layout)
    assert torch.isfinite(out.float()).all()
    assert_close(out, ref_dx(g, w, layout), dtype, f"dgrad {layout} {(M, K, N)}",
                 margin=f"dX {layout} (M,K,N)={(M, K, N)} ({str(dtype)[6:]})")
    # every control word (status, tickets, flags) is zero again after the call
    assert int(ws[:256].count_nonzero()) == 0
    tiles = -(-M // 256) * -(-N // 192)
    ctl = ws[256:256 + 2 * ((4 * tiles + 255) // 256 * 256)]
    assert int(ctl.count_nonzero()) == 0


@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_dgrad_deterministic_and_workspace_reuse(layout):
    """Repeated calls on one workspace (split and unsplit plans) give the same
    bits; a second shape on the same buffer is exact too."""
    g, w = make(8192, 3072, 768, torch.bfloat16, layout, seed=1)
    first, ws = call(g, w, layout)
    for _ in range(3):
        again, _ = call(g, w, layout, ws=ws)
        assert torch.equal(first, again)
    g2, w2 = make(1000, 192, 200, torch.bfloat16, layout, seed=2)
    out2, _ = call(g2, w2, layout, ws=ws)
    assert_close(out2, ref_dx(g2, w2, layout), torch.bfloat16, "dgrad after reuse")


def test_dgrad_strided_rows():
    """g rows with a stride beyond K (a column slice of a wider tensor)."""
    big = (torch.randn(1500, 640) * 0.02).to(torch.bfloat16).to(DEV)
    g = big[:, 64:64 + 512]  # row stride 640 elements
    w = (torch.randn(512, 264) * 0.02).to(torch.bfloat16).to(DEV)
    out, _ = call(g, w, "nn", ldg=640)
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


def test_layers_default_to_torch_matmul():
    """hipBLASLt is as fast or faster at every measured layer shape: the layers
    call the kernel only when set_dgrad("hip") selects it."""
    from flashdp4review_amd.core import inputgrad as D
    assert D._mode == "torch"
    with pytest.raises(ValueError):
        core.set_dgrad("auto")


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


def test_dgrad_graph_replays_match_eager():
    """fdp_dgrad records kernels only (no memset) and its control words clear
    themselves, so a captured call replays exactly: three replays, with eager
    calls and synchronisations between them, each equal to the eager result."""
    g, w = make(8192, 3072, 768, torch.bfloat16, "nn", seed=3)  # the split plan
    eager = core.dgrad(g, w, "nn")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        core.dgrad(g, w, "nn")  # warm-up on the capture stream (its workspace)
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
