"""GPU parity of the DP layers (DPLinear, DPConv1D, DPLayerNorm) end to end
through autograd, against the float64 oracle, with seeded injected noise."""
import math

import numpy as np
import pytest
import torch

from oracle import dp_clip as O
from tests._tol import assert_close, assert_elementwise

from flashdp4review_amd import DPConv1D, DPLayerNorm, DPLinear, wrap_with_flashdp_layers

pytestmark = pytest.mark.gpu
DEV = "cuda"


def draws(seed, shapes, dtype):
    """The layers draw z_W then z_b with torch.randn from their noise_generator."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    return [torch.randn(s, dtype=dtype, device=DEV, generator=gen) for s in shapes]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("sigma", [0.0, 1.0])
def test_dplinear_cfg1(dtype, sigma):
    """cfg1: Linear 768->768 with bias, x [4,128,768] ~ N(0,1), g ~ N(0, 0.01^2)."""
    torch.manual_seed(0)
    lin = DPLinear(768, 768, bias=True, C=1.0, noise_multiplier=sigma).to(DEV, dtype)
    lin.record_stats = True
    lin.noise_generator = torch.Generator(device=DEV).manual_seed(1234)
    x = torch.randn(4, 128, 768, device=DEV).to(dtype).requires_grad_(True)
    g = (torch.randn(4, 128, 768, device=DEV) * 0.01).to(dtype)
    g0 = g.clone()
    lin(x).backward(g)
    assert torch.equal(g, g0)
    zw, zb = draws(1234, [(768, 768), (768,)], dtype) if sigma > 0 else (None, None)
    ref = O.linear_backward(x.detach(), g, lin.weight.detach(), 1.0, 1.0, sigma, zw, zb)
    assert_close(x.grad, ref["dx"], dtype, "dx")
    assert_close(lin.weight.grad, ref["dw"], dtype, "dW")
    assert_close(lin.bias.grad, ref["db"], dtype, "db")
    st = lin.last_stats
    assert_elementwise(st["norms_w"], ref["norms_w"], dtype, "weight norms")
    assert_elementwise(st["fac_w"], ref["fac_w"], dtype, "weight factors")
    assert_elementwise(st["norms_b"], ref["norms_b"], dtype, "bias norms")
    assert_elementwise(st["fac_b"], ref["fac_b"], dtype, "bias factors")
    assert np.all(ref["norms_w"] > 1.0)  # all samples clipped at this config


def test_dplinear_cfg2_bias_in_one_launch():
    """cfg2: DPLinear 768 -> 3072 with bias, B=8, T=1024, bf16: the backward's
    weight and bias gradients come from one wide-kernel launch (the bias from
    the grad_output fragments the product already holds); parity with the
    float64 oracle of the reference's two separate ops."""
    torch.manual_seed(0)
    dtype = torch.bfloat16
    lin = DPLinear(768, 3072, bias=True, C=1.0, noise_multiplier=1.0).to(DEV, dtype)
    lin.record_stats = True
    lin.noise_generator = torch.Generator(device=DEV).manual_seed(4321)
    x = torch.randn(8, 1024, 768, device=DEV).to(dtype).requires_grad_(True)
    g = (torch.randn(8, 1024, 3072, device=DEV) * 0.01).to(dtype)
    lin(x).backward(g)
    zw, zb = draws(4321, [(3072, 768), (3072,)], dtype)
    ref = O.linear_backward(x.detach(), g, lin.weight.detach(), 1.0, 1.0, 1.0, zw, zb)
    assert_close(lin.weight.grad, ref["dw"], dtype, "dW", margin="cfg2 DPLinear: dW")
    assert_close(lin.bias.grad, ref["db"], dtype, "db", margin="cfg2 DPLinear: db (fused bias)")
    st = lin.last_stats
    assert_elementwise(st["norms_b"], ref["norms_b"], dtype, "bias norms")
    assert_elementwise(st["fac_b"], ref["fac_b"], dtype, "bias factors")
    assert_elementwise(st["norms_w"], ref["norms_w"], dtype, "weight norms")


@pytest.mark.parametrize("shape", [(6, 20), (3, 4, 5, 20)], ids=["2d", "4d"])
def test_dplinear_other_ranks(shape):
    """2-D inputs (T=1) and >3-D inputs (T = product of middle axes) return
    gradients in the input's shape."""
    lin = DPLinear(20, 12, C=0.05, noise_multiplier=0.0).to(DEV)
    x = torch.randn(*shape, device=DEV, requires_grad=True)
    g = torch.randn(*shape[:-1], 12, device=DEV)
    lin(x).backward(g)
    assert x.grad.shape == x.shape
    ref = O.linear_backward(x.detach(), g, lin.weight.detach(), 0.05, 1.0)
    assert_close(x.grad, ref["dx"], torch.float32, "dx")
    assert_close(lin.weight.grad, ref["dw"], torch.float32, "dW")
    assert_close(lin.bias.grad, ref["db"], torch.float32, "db")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_dpconv1d_matches_linear_transposed(dtype):
    """cfg3-style Conv1D (nx=768 -> nf=2304 scaled down in T) with log-uniform per-sample
    norms: DPConv1D(W) == DPLinear(W^T) transposed, and both match the oracle."""
    torch.manual_seed(4)
    B, T, nx, nf = 4, 64, 768, 2304
    conv = DPConv1D(nf, nx, C=1.0, noise_multiplier=0.0).to(DEV, dtype)
    conv.record_stats = True
    x = torch.randn(B, T, nx, device=DEV).to(dtype).requires_grad_(True)
    gh = torch.randn(B, T, nf, device=DEV) * 0.02
    # scale each sample so that ||x_b^T g_b|| = 10^u_b, u_b ~ U(-1, 1)
    G = torch.einsum("btm,btn->bmn", x.detach().float(), gh)
    u = torch.rand(B, generator=torch.Generator().manual_seed(4)) * 2 - 1
    r = (10 ** u).to(DEV)
    g = (gh * (r / G.flatten(1).norm(dim=1))[:, None, None]).to(dtype)
    conv(x).backward(g)
    ref = O.conv1d_backward(x.detach(), g, conv.weight.detach(), 1.0, 1.0)
    assert_close(x.grad, ref["dx"], dtype, "dx")
    assert_close(conv.weight.grad, ref["dw"], dtype, "dW")
    assert_close(conv.bias.grad, ref["db"], dtype, "db")
    f = conv.last_stats["fac_w"].cpu().numpy()
    assert np.any(f < 1.0) and np.any(f >= 1.0 - 1e-6)  # partially clipped
    lin = DPLinear(nx, nf, C=1.0, noise_multiplier=0.0).to(DEV, dtype)
    with torch.no_grad():
        lin.weight.copy_(conv.weight.t())
        lin.bias.copy_(conv.bias)
    x2 = x.detach().clone().requires_grad_(True)
    lin(x2).backward(g)
    assert_close(conv.weight.grad.t(), lin.weight.grad.double().cpu().numpy(), dtype, "W^T")
    assert_close(conv.bias.grad, lin.bias.grad.double().cpu().numpy(), dtype, "bias")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("use_fused,H", [(True, 1024), (False, 1024), (True, 8192),
                                         (False, 40000)])
def test_dplayernorm(dtype, use_fused, H):
    """cfg4-style LayerNorm (gamma=1, beta=0) with seeded noise; H=8192 takes
    the kernels that share a row among wavefronts, H=40000 (beyond the fused
    mode's 64 KB rows) the segment-swept ones."""
    B, T = 4, (128 if H <= 8192 else 16)
    ln = DPLayerNorm(H, use_fused=use_fused, C=1.0, noise_multiplier=1.0).to(DEV, dtype)
    ln.record_stats = True
    ln.noise_generator = torch.Generator(device=DEV).manual_seed(77)
    x = torch.randn(B, T, H, device=DEV).to(dtype).requires_grad_(True)
    g = (torch.randn(B, T, H, device=DEV) * 0.01).to(dtype)
    y = ln(x)
    yr, _, _ = O.layernorm_fwd(x.detach(), ln.weight.detach(), ln.bias.detach(), 1e-5)
    assert_close(y, yr, dtype, "y")
    y.backward(g)
    zw, zb = draws(77, [(H,), (H,)], dtype)
    ref = O.layernorm_bwd_clip(g, x.detach(), ln.weight.detach(), 1e-5, C=1.0,
                               noise_multiplier=1.0, z_w=zw, z_b=zb)
    assert_close(x.grad, ref["dx"], dtype, "dx")
    assert_close(ln.weight.grad, ref["dw"], dtype, "dgamma")
    assert_close(ln.bias.grad, ref["db"], dtype, "dbeta")
    assert_elementwise(ln.last_stats["norms_w"], ref["norms_w"], dtype, "gamma norms")
    assert_elementwise(ln.last_stats["norms_b"], ref["norms_b"], dtype, "beta norms")


def test_dpsgd_noise_convention():
    """set_noise_convention("dpsgd"): the layers add noise of std sigma*C/B (DP-SGD's
    (sum_b clip(G_b) + N(0, (sigma C)^2)) / B) instead of sigma/sqrt(B); checked against
    the oracle drawing sigma' / sqrt(B) with sigma' = sigma*C/sqrt(B)."""
    import flashdp4review_amd as fdp
    B, T, C, sigma = 4, 16, 0.5, 1.3
    torch.manual_seed(3)
    lin = DPLinear(256, 128, bias=True, C=C, noise_multiplier=sigma).to(DEV)
    lin.noise_generator = torch.Generator(device=DEV).manual_seed(99)
    ln = DPLayerNorm(256, C=C, noise_multiplier=sigma).to(DEV)
    ln.noise_generator = torch.Generator(device=DEV).manual_seed(98)
    x = torch.randn(B, T, 256, device=DEV, requires_grad=True)
    g = torch.randn(B, T, 128, device=DEV) * 0.01
    xl = torch.randn(B, T, 256, device=DEV, requires_grad=True)
    gl = torch.randn(B, T, 256, device=DEV) * 0.01
    fdp.set_noise_convention("dpsgd")
    try:
        lin(x).backward(g)
        ln(xl).backward(gl)
    finally:
        fdp.set_noise_convention("reference")
    s_eq = sigma * C / math.sqrt(B)
    zw, zb = draws(99, [(128, 256), (128,)], torch.float32)
    ref = O.linear_backward(x.detach(), g, lin.weight.detach(), C, 1.0, s_eq, zw, zb)
    assert_close(lin.weight.grad, ref["dw"], torch.float32, "dpsgd noise: dW")
    assert_close(lin.bias.grad, ref["db"], torch.float32, "dpsgd noise: db")
    zg, zbe = draws(98, [(256,), (256,)], torch.float32)
    refl = O.layernorm_bwd_clip(gl, xl.detach(), ln.weight.detach(), 1e-5, C=C,
                                noise_multiplier=s_eq, z_w=zg, z_b=zbe)
    assert_close(ln.weight.grad, refl["dw"], torch.float32, "dpsgd noise: dgamma")
    assert_close(ln.bias.grad, refl["db"], torch.float32, "dpsgd noise: dbeta")


def test_wrapped_mlp_trains():
    """A wrapped 2-layer MLP with LayerNorm steps under Adam and its loss decreases
    with sigma = 0 (sanity of the whole backward wiring)."""
    torch.manual_seed(0)
    m = torch.nn.Sequential(torch.nn.LayerNorm(64), torch.nn.Linear(64, 128), torch.nn.GELU(),
                            torch.nn.Linear(128, 64)).to(DEV)
    wrap_with_flashdp_layers(m, target_modules=[torch.nn.Linear, torch.nn.LayerNorm], C=10.0,
                             noise_multiplier=0.0, feedback=False)
    assert all(type(mod).__name__.startswith("DP") for mod in (m[0], m[1], m[3]))
    opt = torch.optim.Adam(m.parameters(), lr=1e-2)
    x = torch.randn(16, 8, 64, device=DEV)
    target = torch.randn(16, 8, 64, device=DEV)
    losses = []
    for _ in range(20):
        loss = ((m(x) - target) ** 2).mean()
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < 0.8 * losses[0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_layers_in_kernel_noise(dtype):
    """Without a noise_generator the layers draw their noise inside the kernels:
    dW gets counter blocks [0, O*I/4) of the module's Philox key, db the next
    ones; LayerNorm's dgamma / dbeta share one key (streams 0 and 1).  The
    oracle's Philox stream (oracle/philox.py) reproduces every draw."""
    from oracle import philox as PX
    torch.manual_seed(3)
    lin = DPLinear(96, 64, bias=True, C=1.0, noise_multiplier=1.0).to(DEV, dtype)
    x = torch.randn(4, 16, 96, device=DEV).to(dtype).requires_grad_(True)
    g = (torch.randn(4, 16, 64, device=DEV) * 0.01).to(dtype)
    lin(x).backward(g)
    seed = lin.noise_stream.seed
    assert seed is not None and lin.noise_stream.offset == (64 * 96) // 4 + 64 // 4
    zw = torch.tensor(PX.normals(64 * 96, seed, 0).reshape(64, 96))
    zb = torch.tensor(PX.normals(64, seed, (64 * 96) // 4))
    ref = O.linear_backward(x.detach(), g, lin.weight.detach(), 1.0, 1.0, 1.0, zw, zb)
    assert_close(lin.weight.grad, ref["dw"], dtype, "dW")
    assert_close(lin.bias.grad, ref["db"], dtype, "db")

    ln = DPLayerNorm(256, C=1.0, noise_multiplier=1.0).to(DEV, dtype)
    xl = torch.randn(4, 8, 256, device=DEV).to(dtype).requires_grad_(True)
    gl = (torch.randn(4, 8, 256, device=DEV) * 0.01).to(dtype)
    ln(xl).backward(gl)
    s2 = ln.noise_stream.seed
    zgw = torch.tensor(PX.normals(256, s2, 0, stream=0))
    zgb = torch.tensor(PX.normals(256, s2, 0, stream=1))
    refl = O.layernorm_bwd_clip(gl, xl.detach(), ln.weight.detach(), ln.eps, C=1.0,
                                noise_multiplier=1.0, z_w=zgw, z_b=zgb)
    assert_close(ln.weight.grad, refl["dw"], dtype, "dgamma")
    assert_close(ln.bias.grad, refl["db"], dtype, "dbeta")
    # a second step continues the stream instead of repeating it
    w1 = lin.weight.grad.clone()
    lin.weight.grad = None
    lin(x).backward(g)
    assert not torch.equal(w1, lin.weight.grad)


def test_graph_captured_backward_draws_fresh_noise():
    """A DPLinear backward (weight and bias, in-kernel noise) captured once into
    a HIP graph and replayed three times, with eager DP work and
    synchronisations between the replays: the kernels read the module's device
    noise counter when they run and fdp_noise_advance (captured with them)
    moves it on, so every replay draws the next range of the module's graph
    seed -- the replays differ, and each equals the oracle with the Philox
    stream at that replay's counter (the reference's torch.normal on the device
    generator, flashdp/layers/linear.py:74-80, also advances per replay)."""
    from oracle import philox as PX
    torch.manual_seed(11)
    B, T, I, Od = 4, 64, 256, 384
    dtype = torch.bfloat16
    lin = DPLinear(I, Od, bias=True, C=1.0, noise_multiplier=1.0).to(DEV, dtype)
    other = DPLinear(I, Od, bias=True, C=1.0, noise_multiplier=1.0).to(DEV, dtype)
    x = torch.randn(B, T, I, device=DEV).to(dtype).requires_grad_(True)
    g = (torch.randn(B, T, Od, device=DEV) * 0.01).to(dtype)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up on the capture stream (its workspace exists)
        for _ in range(2):
            lin.weight.grad = lin.bias.grad = x.grad = None
            lin(x).backward(g)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    lin.weight.grad = lin.bias.grad = x.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        lin(x).backward(g)
    torch.cuda.synchronize()
    seed = lin.noise_stream.graph_seed
    assert seed is not None and seed != lin.noise_stream.seed
    nw = Od * I
    bw, bb = (nw + 3) // 4, (Od + 3) // 4
    prev = None
    for rep in range(3):
        ctr = int(lin.noise_counter.item())
        graph.replay()
        torch.cuda.synchronize()
        dw, db = lin.weight.grad.clone(), lin.bias.grad.clone()
        assert int(lin.noise_counter.item()) == ctr + bw + bb
        zw = torch.tensor(PX.normals(nw, seed, ctr).reshape(Od, I))
        zb = torch.tensor(PX.normals(Od, seed, ctr + bw))
        ref = O.linear_backward(x.detach(), g, lin.weight.detach(), 1.0, 1.0, 1.0, zw, zb)
        assert_close(dw, ref["dw"], dtype, f"replay {rep}: dW")
        assert_close(db, ref["db"], dtype, f"replay {rep}: db")
        if prev is not None:
            assert not torch.equal(prev, dw)
        prev = dw
        other.weight.grad = None
        other(x.detach()).backward(g)  # eager DP work between the replays
        torch.cuda.synchronize()


def test_expired_wait_raises_before_optimizer_step(monkeypatch):
    """An expired bounded wait in a DP layer's backward (forced from the host:
    FDP_WGRAD_SPIN_LIMIT=0, every kernel still runs to completion) is reported
    by the optimizer pre-step check, before the step runs: the parameters stay
    as they were, and the next step (normal limit) goes through."""
    from flashdp4review_amd import _lib
    from flashdp4review_amd.core import wgrad as W
    assert W._expiry_check == "optimizer_step"
    torch.manual_seed(12)
    lin = DPLinear(384, 512, bias=False, C=0.5, noise_multiplier=0.0).to(DEV, torch.bfloat16)
    opt = torch.optim.SGD(lin.parameters(), lr=0.1)
    x = torch.randn(8, 1024, 384, device=DEV).to(torch.bfloat16)
    g = (torch.randn(8, 1024, 512, device=DEV) * 0.02).to(torch.bfloat16)
    core_status = __import__("flashdp4review_amd.core", fromlist=["wgrad_status"]).wgrad_status
    core_status()  # start from a clear status word
    w0 = lin.weight.detach().clone()
    monkeypatch.setenv("FDP_WGRAD_SPIN_LIMIT", "0")
    lin(x).backward(g)
    monkeypatch.delenv("FDP_WGRAD_SPIN_LIMIT")
    with pytest.raises(_lib.FlashDPError):
        opt.step()
    torch.cuda.synchronize()
    assert torch.isnan(lin.weight.grad.float()).any()
    assert torch.equal(lin.weight.detach(), w0), "the step ran on NaN gradients"
    opt.zero_grad(set_to_none=True)
    lin(x).backward(g)
    opt.step()
    assert torch.isfinite(lin.weight.float()).all() and not torch.equal(lin.weight.detach(), w0)


def test_expired_wait_skips_a_fused_optimizer_step_on_the_device(monkeypatch):
    """With an optimizer that can skip a step on the device (fused Adam), the
    pre-step check sets its found_inf from the status word instead of
    synchronising: the step on NaN gradients changes neither the parameters
    nor Adam's state, the next step raises, and training then continues."""
    from flashdp4review_amd import _lib
    from flashdp4review_amd.core import wgrad_status
    torch.manual_seed(13)
    lin = DPLinear(384, 512, bias=False, C=0.5, noise_multiplier=0.0).to(DEV, torch.bfloat16)
    opt = torch.optim.Adam(lin.parameters(), lr=1e-2, fused=True)
    x = torch.randn(8, 1024, 384, device=DEV).to(torch.bfloat16)
    g = (torch.randn(8, 1024, 512, device=DEV) * 0.02).to(torch.bfloat16)
    wgrad_status()  # start from a clear status word
    lin(x).backward(g)
    opt.step()  # a good step: Adam's state exists
    opt.zero_grad(set_to_none=True)
    w = lin.weight
    w0, st0 = w.detach().clone(), {k: v.clone() for k, v in opt.state[w].items()}
    monkeypatch.setenv("FDP_WGRAD_SPIN_LIMIT", "0")
    lin(x).backward(g)
    monkeypatch.delenv("FDP_WGRAD_SPIN_LIMIT")
    opt.step()  # skipped on the device
    torch.cuda.synchronize()
    assert torch.isnan(w.grad.float()).any()
    assert torch.equal(w.detach(), w0), "the step ran on NaN gradients"
    for k, v in opt.state[w].items():
        assert torch.equal(v, st0[k]), f"Adam state {k} changed"
    assert not hasattr(opt, "found_inf")
    opt.zero_grad(set_to_none=True)
    lin(x).backward(g)
    with pytest.raises(_lib.FlashDPError):
        opt.step()
    assert torch.equal(w.detach(), w0)
    opt.zero_grad(set_to_none=True)
    lin(x).backward(g)
    opt.step()
    torch.cuda.synchronize()
    assert torch.isfinite(w.float()).all() and not torch.equal(w.detach(), w0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_dplayernorm_two_axis_shape_and_no_affine(dtype):
    """The non-fused DPLayerNorm over a 2-D normalized_shape normalises the
    trailing axes together and clips the per-sample sums over the remaining
    axis, as the reference's non-fused layer does (flashdp/layers/
    layernorm.py:77-112): the oracle on the flattened [B, T, 4*64] tensors.
    elementwise_affine=False has no gamma/beta: only dx."""
    import torch.nn.functional as F
    torch.manual_seed(21)
    B, T = 4, 32
    ln = DPLayerNorm((4, 64), use_fused=False, C=0.05, noise_multiplier=1.0).to(DEV, dtype)
    with torch.no_grad():
        ln.weight.copy_(1 + 0.1 * torch.randn(4, 64, device=DEV))
        ln.bias.copy_(0.1 * torch.randn(4, 64, device=DEV))
    ln.record_stats = True
    ln.noise_generator = torch.Generator(device=DEV).manual_seed(78)
    x = torch.randn(B, T, 4, 64, device=DEV).to(dtype).requires_grad_(True)
    g = (torch.randn(B, T, 4, 64, device=DEV) * 0.01).to(dtype)
    y = ln(x)
    yt = F.layer_norm(x.detach().float(), (4, 64), ln.weight.detach().float(),
                      ln.bias.detach().float(), 1e-5)
    assert_close(y, yt.double().cpu().numpy(), dtype, "y vs F.layer_norm")
    y.backward(g)
    zw, zb = draws(78, [(4, 64), (4, 64)], dtype)
    ref = O.layernorm_bwd_clip(g.reshape(B, T, 256), x.detach().reshape(B, T, 256),
                               ln.weight.detach().reshape(256), 1e-5, C=0.05,
                               noise_multiplier=1.0, z_w=zw.reshape(256), z_b=zb.reshape(256))
    assert ln.weight.grad.shape == (4, 64) and x.grad.shape == x.shape
    assert_close(x.grad.reshape(B, T, 256), ref["dx"], dtype, "dx")
    assert_close(ln.weight.grad.reshape(256), ref["dw"], dtype, "dgamma")
    assert_close(ln.bias.grad.reshape(256), ref["db"], dtype, "dbeta")
    assert_elementwise(ln.last_stats["norms_w"], ref["norms_w"], dtype, "gamma norms")
    assert np.all(ref["fac_w"] < 1.0)  # clipped

    for fused in (False, True):
        ln2 = DPLayerNorm(256, elementwise_affine=False, use_fused=fused, C=0.05).to(DEV, dtype)
        assert ln2.weight is None and ln2.bias is None
        x2 = torch.randn(B, T, 256, device=DEV).to(dtype).requires_grad_(True)
        g2 = (torch.randn(B, T, 256, device=DEV) * 0.01).to(dtype)
        ln2(x2).backward(g2)
        ref2 = O.layernorm_bwd_clip(g2, x2.detach(), None, 1e-5, C=0.05)
        assert_close(x2.grad, ref2["dx"], dtype, f"dx without affine (fused={fused})")
