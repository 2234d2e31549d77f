"""GPU tests at the BASELINE configurations' full sizes, and the wrap API on
bf16 models and under autocast.

  cfg3  DP Conv1D c_attn 768 -> 2304, x [16,1024,768], per-sample norms
        log-uniform in 0.1C..10C, plus bmm_clip / bmtm_clip on the same tensors,
        against an fp32 torch reference of the per-sample products on the GPU
        (flashdp/layers/transformers_conv1d.py:40-66, flashdp/core/
        transformers_conv1d_clip.py:22-28, bmm_clip_loop.py:150-162,
        bmtm_clip_loop.py:162-173).
  cfg5  a full-width two-block slice of the GPT-2-style decoder (d=2048,
        16 heads, FFN 8192, V=50257, B=8, T=1024, bf16) wrapped by
        wrap_with_flashdp_layers except lm_head: with C -> inf and sigma = 0
        every wrapped gradient is the non-DP gradient / B (a property the
        per-sample clipping math fixes: clip factors are all 1, the sum over
        samples is the batch gradient, then 1/B; flashdp/layers/linear.py:72-92,
        flashdp/layers/layernorm.py:128-165); with C at half the smallest
        per-sample norm (every sample clipped) and sigma = 0, the per-sample
        norms, clip factors and the clipped dW of
        c_fc (2048 -> 8192) and mlp_proj (8192 -> 2048) -- the streamed
        Gram-norm + clipped-sum schedule at B=8, T=1024 -- match fp32
        per-sample products on the GPU (flashdp/core/linear_clip.py:94-104).
  AMP   an fp32 model wrapped and run under torch.autocast(bfloat16), as the
        reference's example trains (example/gpt2/train.py:77-79), and a bf16
        model: every DP layer's gradients match the oracle on the bf16 tensors
        its kernels saw; with set_wgrad_precision("fp32") the fp32 weight and
        bias gradients meet the fp32 tolerance.
"""
import copy

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import bench
from oracle import dp_clip as O
from tests._tol import assert_close, assert_elementwise

from flashdp4review_amd import DPConv1D, DPLayerNorm, DPLinear, wrap_with_flashdp_layers
from flashdp4review_amd import core

pytestmark = pytest.mark.gpu
DEV = "cuda"


def per_sample_products(a, b):
    """G_b = a_b^T b_b in fp32 for a [B,K,M], b [B,K,N] (bf16 or fp32), one sample at a time."""
    return torch.stack([a[i].float().t().contiguous() @ b[i].float() for i in range(a.shape[0])])


# ------------------------------------------------------------------------ cfg3
def test_cfg3_conv1d_full_size():
    torch.manual_seed(4)
    B, T, nx, nf = 16, 1024, 768, 2304
    dtype = torch.bfloat16
    x, g = bench.cfg3_inputs(torch.device(DEV))
    conv = DPConv1D(nf, nx, C=1.0, noise_multiplier=0.0).to(DEV, dtype)
    conv.record_stats = True
    xr = x.clone().requires_grad_(True)
    conv(xr).backward(g)
    G = per_sample_products(x, g)                       # [16, 768, 2304] = x_b^T g_b
    n_ref = G.flatten(1).norm(dim=1)
    c_ref = torch.clamp(1.0 / (n_ref + 1e-10), max=1.0)
    S = (c_ref[:, None, None] * G).sum(0)               # sum_b c_b x_b^T g_b
    clipped = int((n_ref > 1.0).sum())
    assert 3 <= clipped <= 13, f"norms should straddle C: {n_ref.tolist()}"
    st = conv.last_stats
    assert_elementwise(st["norms_w"], n_ref.double().cpu().numpy(), dtype, "weight norms",
                       margin="cfg3 Conv1D: weight per-sample norms")
    assert_elementwise(st["fac_w"], c_ref.double().cpu().numpy(), dtype, "weight factors",
                       margin="cfg3 Conv1D: weight clip factors")
    assert_close(conv.weight.grad, (S / B).double().cpu().numpy(), dtype, "dW",
                 margin="cfg3 Conv1D: dW (bf16 out)")
    # bias: ||g_b||_F over all T*O entries, mean over B*T
    gf = g.float()
    m_ref = gf.flatten(1).norm(dim=1)
    cb = torch.clamp(1.0 / (m_ref + 1e-10), max=1.0)
    db_ref = (cb[:, None] * gf.sum(1)).sum(0) / (B * T)
    assert_close(conv.bias.grad, db_ref.double().cpu().numpy(), dtype, "db",
                 margin="cfg3 Conv1D: db (bf16 out)")
    # dX = g W^T from the unmodified g
    dx_ref = g.float() @ conv.weight.detach().float().t()
    assert_close(xr.grad, dx_ref.double().cpu().numpy(), dtype, "dx")
    # the operator API on the same tensors (no 1/B): bmm_clip(x^T, g) in fp32 and
    # bmtm_clip(x, g) in the input dtype
    ca = torch.tensor([1.0, 1.0], device=DEV)
    r_bmm = core.bmm_clip(x.transpose(1, 2).contiguous(), g, ca)
    assert r_bmm.dtype == torch.float32
    assert_close(r_bmm, S.double().cpu().numpy(), dtype, "bmm_clip",
                 margin="cfg3 bmm_clip(x^T, g): fp32 out")
    r_bmtm = core.bmtm_clip(x, g, ca)
    assert r_bmtm.dtype == dtype
    assert_close(r_bmtm, S.double().cpu().numpy(), dtype, "bmtm_clip",
                 margin="cfg3 bmtm_clip(x, g): bf16 out")


# ------------------------------------------------------------------------ cfg5
def _wrapped(model, C, sigma):
    import contextlib
    import io
    with contextlib.redirect_stdout(io.StringIO()):
        wrap_with_flashdp_layers(model, target_modules=[nn.Linear, nn.LayerNorm],
                                 skip_layers=["lm_head"], C=C, noise_multiplier=sigma,
                                 feedback=False)
    return model


def _loss(model, idx):
    V = 50257
    x, y = idx[:, :-1], idx[:, 1:]
    return F.cross_entropy(model(x).view(-1, V).float(), y.reshape(-1))


def test_cfg5_decoder_dp_grads_equal_non_dp_over_batch():
    B = 8
    torch.manual_seed(0)
    base = bench.gpt_model(n_layer=2).to(DEV, torch.bfloat16)
    dp = _wrapped(copy.deepcopy(base), C=1e30, sigma=0.0)
    assert isinstance(dp.h[0].c_fc, DPLinear) and isinstance(dp.h[1].ln_2, DPLayerNorm)
    assert not isinstance(dp.lm_head, DPLinear)
    assert dp.h[0].c_fc.weight.dtype == torch.bfloat16          # the wrap keeps the dtype
    idx = torch.randint(0, 50257, (B, 1025), device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(0))
    checked = ("h.0.c_fc", "h.1.mlp_proj")
    for name in checked:
        dp.get_submodule(name).record_stats = True
    _loss(base, idx).backward()
    _loss(dp, idx).backward()
    # a C below every per-sample norm of the two checked layers: all samples clip
    C = 0.5 * min(float(dp.get_submodule(n).last_stats["norms_w"].min()) for n in checked)
    dp_params = {id(p) for m in dp.modules() if isinstance(m, (DPLinear, DPLayerNorm))
                 for p in m.parameters(recurse=False)}
    worst, worst_name = 0.0, ""
    for (name, p), (_, q) in zip(base.named_parameters(), dp.named_parameters()):
        expect = p.grad.float() / B if id(q) in dp_params else p.grad.float()
        e = assert_close(q.grad, expect.double().cpu().numpy(), torch.bfloat16, name)
        if e > worst:
            worst, worst_name = e, name
    from tests._tol import report
    report(f"cfg5 decoder (2 blocks, d=2048), C=inf: DP grad vs non-DP/B, worst ({worst_name})",
           worst, 2e-2)

    # every sample clipped, sigma = 0: norms, factors and the clipped dW of two
    # layers against fp32 per-sample products
    torch.manual_seed(0)
    dp1 = _wrapped(copy.deepcopy(base), C=C, sigma=0.0)
    seen = {}
    for name in checked:
        mod = dp1.get_submodule(name)
        mod.record_stats = True

        def fwd_hook(m, inp, out, name=name):
            seen[name] = [inp[0].detach()]
            out.register_hook(lambda gr: seen[name].append(gr.detach()))

        mod.register_forward_hook(fwd_hook)
    _loss(dp1, idx).backward()
    for name, (x, g) in seen.items():
        G = per_sample_products(g, x)  # g_b^T x_b, fp32
        n_ref = G.flatten(1).norm(dim=1)
        mod = dp1.get_submodule(name)
        st = mod.last_stats
        assert_elementwise(st["norms_w"], n_ref.double().cpu().numpy(), torch.bfloat16,
                           f"{name} norms", margin=f"cfg5 {name}: per-sample norms")
        c_ref = torch.clamp(C / (n_ref + 1e-10), max=1.0)
        assert bool((c_ref < 1.0).all()), f"{name}: every sample clips"
        assert_elementwise(st["fac_w"], c_ref.double().cpu().numpy(), torch.bfloat16,
                           f"{name} factors", margin=f"cfg5 {name}: clip factors (all clipped)")
        dw_ref = (c_ref[:, None, None] * G).sum(0) / B
        del G
        assert_close(mod.weight.grad, dw_ref.double().cpu().numpy(), torch.bfloat16,
                     f"{name} clipped dW",
                     margin=f"cfg5 {name}: clipped dW (all clipped, bf16 out)")


# ------------------------------------------------------------------- AMP, bf16
def _capture(model):
    """(module, [input, grad_output]) of every DP layer, as its kernels saw them."""
    seen = []
    for m in model.modules():
        if isinstance(m, (DPLinear, DPLayerNorm)):
            rec = [m]

            def fwd_hook(mod, inp, out, rec=rec):
                rec[1:] = [inp[0].detach()]
                out.register_hook(lambda gr: rec.append(gr.detach()))

            m.register_forward_hook(fwd_hook)
            seen.append(rec)
    return seen


def _check_layers(seen, C, tag):
    for m, x, g in seen:
        if isinstance(m, DPLinear):
            xk = x.to(g.dtype)  # the kernel contracts x in grad_output's dtype
            ref = O.linear_backward(xk, g, m.weight.detach(), C, 1.0)
            assert m.weight.grad.dtype == m.weight.dtype
            assert_close(m.weight.grad, ref["dw"], torch.bfloat16, f"{tag} dW",
                         margin=f"{tag}: Linear {tuple(m.weight.shape)} dW")
            if m.bias is not None:
                assert_close(m.bias.grad, ref["db"], torch.bfloat16, f"{tag} db")
        else:
            ref = O.layernorm_bwd_clip(g, x, m.weight.detach(), m.eps, C=C)
            assert_close(m.weight.grad, ref["dw"], torch.bfloat16, f"{tag} dgamma",
                         margin=f"{tag}: LayerNorm dgamma")
            assert_close(m.bias.grad, ref["db"], torch.bfloat16, f"{tag} dbeta")


def _mlp(dtype):
    torch.manual_seed(3)
    return nn.Sequential(nn.Linear(256, 512), nn.GELU(), nn.LayerNorm(512),
                         nn.Linear(512, 128)).to(DEV, dtype)


def test_autocast_bf16_wrapped_fp32_model():
    model = _wrapped(_mlp(torch.float32), C=0.05, sigma=0.0)
    assert model[0].weight.dtype == torch.float32
    seen = _capture(model)
    x = torch.randn(4, 64, 256, device=DEV)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        out = model(x)
        assert out.dtype == torch.bfloat16
        loss = (out.float() ** 2).mean()
    loss.backward()
    assert all(len(r) == 3 for r in seen)
    assert seen[0][2].dtype == torch.bfloat16
    _check_layers(seen, 0.05, "autocast(bf16) fp32 model")
    # the fp32 master weights take an optimizer step
    w0 = model[0].weight.detach().clone()
    torch.optim.Adam(model.parameters(), lr=1e-3).step()
    assert not torch.equal(w0, model[0].weight)


def test_autocast_fp32_precision_mode():
    """set_wgrad_precision("fp32"): fp32 weight gradients from bf16 operands
    are summed in fp32 (streamed schedule) and meet the fp32 tolerance against
    the float64 oracle on the same bf16 tensors."""
    import flashdp4review_amd as fdp
    model = _wrapped(_mlp(torch.float32), C=0.05, sigma=0.0)
    seen = _capture(model)
    x = torch.randn(4, 64, 256, device=DEV)
    fdp.set_wgrad_precision("fp32")
    try:
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss = (model(x).float() ** 2).mean()
        loss.backward()
    finally:
        fdp.set_wgrad_precision("fast")
    assert fdp.get_wgrad_precision() == "fast"
    with pytest.raises(ValueError):
        fdp.set_wgrad_precision("fp64")
    checked = 0
    for m, xin, g in seen:
        if not isinstance(m, DPLinear):
            continue
        assert g.dtype == torch.bfloat16 and m.weight.grad.dtype == torch.float32
        ref = O.linear_backward(xin.to(g.dtype), g, m.weight.detach(), 0.05, 1.0)
        assert float(ref["fac_w"].min()) < 1.0, "some samples clip"
        assert_close(m.weight.grad, ref["dw"], torch.float32, "fp32 mode dW",
                     margin=f"autocast fp32 mode: Linear {tuple(m.weight.shape)} dW")
        assert_close(m.bias.grad, ref["db"], torch.float32, "fp32 mode db",
                     margin=f"autocast fp32 mode: Linear {tuple(m.weight.shape)} db")
        checked += 1
    assert checked == 2


def test_wrapped_bf16_model():
    model = _wrapped(_mlp(torch.bfloat16), C=0.05, sigma=0.0)
    assert model[3].weight.dtype == torch.bfloat16
    seen = _capture(model)
    x = torch.randn(4, 64, 256, device=DEV).to(torch.bfloat16)
    (model(x).float() ** 2).mean().backward()
    _check_layers(seen, 0.05, "bf16 model")
