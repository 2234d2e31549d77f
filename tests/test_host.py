"""Host-side logic that runs without a GPU: the wrap API's selection rules
(flashdp/api/wrap_model.py:17-211), layer constructors and attributes, and the
absence of any CPU fallback."""
import pytest
import torch
import torch.nn as nn

import flashdp4review_amd as fdp
from flashdp4review_amd import DPConv1D, DPLayerNorm, DPLinear, wrap_with_flashdp_layers
from flashdp4review_amd.core import bmtm_clip, colsum_clip, wgrad_clip
from flashdp4review_amd.core.clip_fn import clip_args_of
from flashdp4review_amd.layers.utils import DPParameter, as_btf, noise_std

transformers = pytest.importorskip("transformers.pytorch_utils")
Conv1D = transformers.Conv1D


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.ln = nn.LayerNorm(8)
        self.fc = nn.Linear(8, 16)
        self.proj = nn.Linear(16, 8, bias=False)
        self.attn = Conv1D(24, 8)


class Net(nn.Module):
    def __init__(self):
        super().__init__()
        self.h = nn.ModuleList([Block(), Block()])
        self.ln_f = nn.LayerNorm(8)
        self.lm_head = nn.Linear(8, 10, bias=False)


def kinds(model):
    return {n: type(m).__name__ for n, m in model.named_modules() if n}


def test_public_surface():
    for name in ["DPLinear", "DPLayerNorm", "DPConv1D", "wrap_with_flashdp_layers",
                 "dp_supported_modules"]:
        assert hasattr(fdp, name)
    assert fdp.dp_supported_modules[nn.Linear] is DPLinear
    assert fdp.dp_supported_modules[nn.LayerNorm] is DPLayerNorm
    assert fdp.dp_supported_modules[Conv1D] is DPConv1D


def test_wrap_skip_lm_head_and_copy_weights():
    torch.manual_seed(0)
    m = Net()
    before = {k: v.clone() for k, v in m.state_dict().items()}
    wrap_with_flashdp_layers(m, target_modules=[nn.Linear, nn.LayerNorm, Conv1D],
                             skip_layers=["lm_head"], C=0.5, noise_multiplier=0.3)
    k = kinds(m)
    assert k["lm_head"] == "Linear"
    assert k["h.0.fc"] == "DPLinear" and k["h.1.proj"] == "DPLinear"
    assert k["h.0.ln"] == "DPLayerNorm" and k["ln_f"] == "DPLayerNorm"
    assert k["h.0.attn"] == "DPConv1D"
    assert m.h[0].proj.bias is None and m.h[0].fc.bias is not None
    assert m.h[0].fc.C == 0.5 and m.h[0].fc.noise_multiplier == 0.3
    assert m.h[0].attn.weight.shape == (8, 24)
    for key, val in m.state_dict().items():
        assert torch.equal(val, before[key]), key
    assert isinstance(m.h[0].fc.weight, DPParameter) and m.h[0].fc.weight.requires_dp


def test_wrap_only_selected_types():
    m = Net()
    wrap_with_flashdp_layers(m, target_modules=[nn.LayerNorm])
    k = kinds(m)
    assert k["h.0.ln"] == "DPLayerNorm" and k["h.0.fc"] == "Linear" and k["lm_head"] == "Linear"


def test_wrap_skip_parent_does_not_skip_children():
    """Selection matches names exactly (wrap_model.py:169-182): skipping 'h.0'
    still wraps 'h.0.fc'."""
    m = Net()
    wrap_with_flashdp_layers(m, target_modules=[nn.Linear], skip_layers=["h.0"])
    assert kinds(m)["h.0.fc"] == "DPLinear"


def test_wrap_target_layers_and_priority():
    m = Net()
    wrap_with_flashdp_layers(m, target_modules=[nn.Linear], target_layers=["h.0.fc", "lm_head"],
                             skip_layers=["lm_head"])
    k = kinds(m)
    assert k["h.0.fc"] == "DPLinear" and k["lm_head"] == "Linear" and k["h.1.fc"] == "Linear"
    m = Net()
    wrap_with_flashdp_layers(m, target_modules=[nn.Linear], target_layers=["lm_head"],
                             skip_layers=["lm_head"], priority_to_target=True)
    assert kinds(m)["lm_head"] == "Linear"  # set difference either way (wrap_model.py:177-180)


def test_wrap_errors():
    with pytest.raises(ValueError):
        wrap_with_flashdp_layers(Net())
    with pytest.raises(ValueError):
        wrap_with_flashdp_layers(Net(), target_modules=[])
    with pytest.raises(ValueError):
        wrap_with_flashdp_layers(Net(), target_modules=[nn.Conv2d])


def test_wrap_messages(capsys):
    """Skip names are validated after prefix expansion against the model's own
    names (wrap_model.py:83,91-92), so an unknown name expands to nothing and
    draws no warning; an unused module type does."""
    wrap_with_flashdp_layers(Net(), target_modules=[nn.Linear], skip_layers=["nope"])
    out = capsys.readouterr().out
    assert "Warning" not in out
    assert "Layers Skipped: nope" in out and "Model wrapped with FlashDP." in out

    class Tiny(nn.Module):
        def __init__(self):
            super().__init__()
            self.fc = nn.Linear(2, 2)

    wrap_with_flashdp_layers(Tiny(), target_modules=[nn.Linear, nn.LayerNorm])
    assert "Module type 'LayerNorm' specified in target_modules is not used" in capsys.readouterr().out


def test_wrap_preserves_dtype():
    m = Net().to(torch.bfloat16)
    wrap_with_flashdp_layers(m, target_modules=[nn.Linear, nn.LayerNorm, Conv1D])
    for p in m.parameters():
        assert p.dtype == torch.bfloat16


def test_layer_constructors():
    lin = DPLinear(4, 3, bias=False)
    assert lin.bias is None and lin.dp and lin.C == 1.0
    lin = DPLinear(4, 3, bias=None)
    assert lin.bias is None
    lin = DPLinear(4, 3, bias=torch.zeros(3), C=2.0, clamp_value=0.5, noise_multiplier=0.1)
    assert lin.bias is not None and lin.clamp_value == 0.5
    ln = DPLayerNorm(8)
    assert ln.use_fused and ln.normalized_shape == (8,)
    with pytest.raises(NotImplementedError):
        DPLayerNorm(8, bias=False)  # fused mode needs a bias (layers/layernorm.py:44-45)
    ln = DPLayerNorm(8, bias=False, use_fused=False)
    assert ln.bias is None
    conv = DPConv1D(6, 4)
    assert conv.weight.shape == (4, 6) and conv.bias.shape == (6,)


def test_no_cpu_fallback():
    a = torch.randn(2, 4, 3)
    b = torch.randn(2, 4, 5)
    with pytest.raises(RuntimeError, match="GPU only"):
        wgrad_clip(a, b)
    with pytest.raises(RuntimeError, match="GPU only"):
        bmtm_clip(a, b, torch.tensor([1.0, 1.0]))
    with pytest.raises(RuntimeError, match="GPU only"):
        colsum_clip(a)
    lin = DPLinear(3, 5)
    x = torch.randn(2, 4, 3, requires_grad=True)
    y = lin(x)  # forward is a plain GEMM
    with pytest.raises(RuntimeError, match="GPU only"):
        y.sum().backward()


def test_helpers():
    assert as_btf(torch.zeros(3, 5)).shape == (3, 1, 5)
    assert as_btf(torch.zeros(3, 2, 4, 5)).shape == (3, 8, 5)
    assert noise_std(1.0, 4) == 0.5
    assert noise_std(1.0, 4, C=3.0) == 0.5  # the reference's convention ignores C


def test_noise_convention():
    """sigma / sqrt(B) by default (flashdp/layers/linear.py:74-80); sigma * C / B opt-in."""
    assert fdp.get_noise_convention() == "reference"
    try:
        fdp.set_noise_convention("dpsgd")
        assert noise_std(2.0, 8, C=0.5) == 2.0 * 0.5 / 8
        with pytest.raises(ValueError):
            fdp.set_noise_convention("textbook")
        assert fdp.get_noise_convention() == "dpsgd"
    finally:
        fdp.set_noise_convention("reference")
    assert noise_std(2.0, 8, C=0.5) == 2.0 / 8 ** 0.5
    assert clip_args_of(torch.tensor([2.0, 0.5]), torch.device("cuda", 0))[:2] == (2.0, 0.5)
    assert clip_args_of((3, 1), torch.device("cpu")) == (3.0, 1.0, None)
    with pytest.raises(ValueError):
        clip_args_of(torch.tensor([1.0, 2.0, 3.0]), torch.device("cpu"))


def test_wgrad_precision_mode():
    """fp32 accumulation is opt-in and applies to fp32 weight gradients only."""
    from flashdp4review_amd.layers.utils import exact_fp32
    assert fdp.get_wgrad_precision() == "fast"
    assert not exact_fp32(torch.float32)
    try:
        fdp.set_wgrad_precision("fp32")
        assert exact_fp32(torch.float32)
        assert not exact_fp32(torch.bfloat16) and not exact_fp32(torch.float16)
        with pytest.raises(ValueError):
            fdp.set_wgrad_precision("exact")
        assert fdp.get_wgrad_precision() == "fp32"
    finally:
        fdp.set_wgrad_precision("fast")
    assert not exact_fp32(torch.float32)


def test_layernorm_fused_row_limit():
    """Fused mode keeps the reference's limit of 64 KB rows and its error
    (flashdp/core/layernorm_clip.py:217-221); rows at the limit pass the check
    (the CPU tensor is then refused for want of the HIP path)."""
    from flashdp4review_amd.core import layernorm_fwd_fused
    for H, dtype in [(32769, torch.bfloat16), (16385, torch.float32)]:
        ln = DPLayerNorm(H, use_fused=True, dtype=dtype)
        with pytest.raises(RuntimeError, match="64KB"):
            ln(torch.zeros(1, 2, H, dtype=dtype))
        with pytest.raises(RuntimeError, match="64KB"):
            layernorm_fwd_fused(torch.zeros(2, H, dtype=dtype), None, None, 1e-5)
    for H, dtype in [(32768, torch.bfloat16), (16384, torch.float32)]:
        with pytest.raises(RuntimeError) as e:
            DPLayerNorm(H, use_fused=True, dtype=dtype)(torch.zeros(1, 2, H, dtype=dtype))
        assert "64KB" not in str(e.value)
    # the non-fused mode has no row limit
    with pytest.raises(RuntimeError) as e:
        DPLayerNorm(40000, use_fused=False)(torch.zeros(1, 2, 40000))
    assert "64KB" not in str(e.value)


def test_optimizer_pre_step_check_installs_and_passes_without_workspaces():
    """The expiry check before optimizer steps installs as a global torch.optim
    pre-step hook; with no workspace in use it lets every step through."""
    import torch
    from flashdp4review_amd.core import wgrad as W
    W._install_step_check()
    assert W._step_hook is not None
    p = torch.nn.Parameter(torch.ones(3))
    p.grad = torch.ones(3)
    torch.optim.SGD([p], lr=0.5).step()
    assert torch.equal(p.detach(), torch.full((3,), 0.5))
    assert W.set_expiry_check("async") == "optimizer_step"
    assert W.set_expiry_check("optimizer_step") == "async"


def test_wrap_leaves_subclasses_and_wrapped_layers_alone(capsys):
    """Only exact types are replaced: wrapping twice changes nothing the second
    time (a DPLinear is a subclass of nn.Linear), and a LayerNorm without a
    bias or over two axes gets the non-fused DPLayerNorm; the feedback names
    the layers actually replaced."""
    m = Net()
    wrap_with_flashdp_layers(m, target_modules=[nn.Linear])
    first = {n: id(x) for n, x in m.named_modules()}
    wrap_with_flashdp_layers(m, target_modules=[nn.Linear])
    assert {n: id(x) for n, x in m.named_modules()} == first
    out = capsys.readouterr().out
    assert "No layers Wrapped." in out and "Layers Wrapped: h.0.fc, h.0.proj" in out

    class Norms(nn.Module):
        def __init__(self):
            super().__init__()
            self.a = nn.LayerNorm(8, bias=False)
            self.b = nn.LayerNorm((4, 8))
            self.c = nn.LayerNorm(8, elementwise_affine=False)

    n = Norms()
    wrap_with_flashdp_layers(n, target_modules=[nn.LayerNorm], feedback=False)
    assert isinstance(n.a, DPLayerNorm) and not n.a.use_fused and n.a.bias is None
    assert isinstance(n.b, DPLayerNorm) and not n.b.use_fused and n.b.weight.shape == (4, 8)
    assert isinstance(n.c, DPLayerNorm) and n.c.use_fused and n.c.weight is None
