"""GPU parity of the weight and bias gradients in one call (fdp_wgrad_bias_clip)
for the bias of either operand -- a DP Linear's (operand a = grad_output,
flashdp/core/linear_clip.py:116-123) and a DP Conv1D's (operand b =
grad_output, flashdp/core/transformers_conv1d_clip.py:31-39) -- on every
schedule: the wide and grouped single-pass kernels and the streamed two-pass
schedule form the bias from the fragments they hold (the column-sum region of
the workspace, filled with a canary, is never touched); fp32 operands take the
column-sum kernel after the generic schedule.  References: the float64 oracle
on the same dtype-rounded inputs (tests/_tol.py), and at cfg5's full size fp32
per-sample products on the GPU."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import dp_clip as O
from oracle import philox as PX
from tests._tol import assert_close, assert_elementwise

from flashdp4review_amd import _lib, core

pytestmark = pytest.mark.gpu
DEV = "cuda"

SCHEDULES = {"wide": _lib.WGRAD_WIDE, "unpaired": _lib.WGRAD_WIDE | _lib.WGRAD_UNPAIRED,
             "narrow": _lib.WGRAD_NARROW, "stream": _lib.WGRAD_TWO_PASS}


def make(B, K, M, N, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn((B, K, M), generator=g)
    b = torch.randn((B, K, N), generator=g) * 0.02
    return a.to(dtype).to(DEV), b.to(dtype).to(DEV)


def run_bias_call(a, b, C, flags, operand, zw, zb, canary):
    """fdp_wgrad_bias_clip through the C ABI: (out, norms, factors, bias,
    bias norms, bias factors, column-sum region untouched)."""
    B, K, M = a.shape
    N = b.shape[2]
    L = _lib.lib()
    dt = _lib.dtype_code(a.dtype)
    if operand == "b":
        flags |= _lib.WGRAD_BIAS_OF_B
    blen = M if operand == "a" else N
    out = torch.empty(M, N, dtype=torch.float32, device=DEV)
    norms = torch.empty(B, dtype=torch.float32, device=DEV)
    fac = torch.empty(B, dtype=torch.float32, device=DEV)
    bo = torch.empty(blen, dtype=a.dtype, device=DEV)
    bn = torch.empty(B, dtype=torch.float32, device=DEV)
    bf = torch.empty(B, dtype=torch.float32, device=DEV)
    wb = _lib.size_query(L.fdp_wgrad_clip_workspace_size, B, K, M, N, dt,
                         flags & ~_lib.WGRAD_BIAS_OF_B)
    cb = _lib.size_query(L.fdp_colsum_clip_workspace_size, B, K, blen, dt)
    nb = _lib.size_query(L.fdp_wgrad_bias_clip_workspace_size, B, K, M, N, dt, flags)
    span = (wb + 255) // 256 * 256
    ws = torch.zeros(nb, dtype=torch.uint8, device=DEV)
    if canary:
        ws[span:span + cb] = 0xA5
    bias = _lib.BiasOut(bo.data_ptr(), dt, 1.0 / (B * K), zb.data_ptr(), 0.5, None,
                        bn.data_ptr(), bf.data_ptr())
    st = L.fdp_wgrad_bias_clip(a.data_ptr(), b.data_ptr(), B, K, M, N, a.stride(0), a.stride(1),
                               b.stride(0), b.stride(1), _lib.LAYOUT_TN, dt, ctypes.c_float(C),
                               ctypes.c_float(1.0), None, ctypes.c_float(1.0 / B), zw.data_ptr(),
                               ctypes.c_float(0.25), None, out.data_ptr(), N, _lib.FDP_F32,
                               norms.data_ptr(), fac.data_ptr(), flags, ctypes.byref(bias),
                               ws.data_ptr(), nb, _lib.stream_handle(torch.device(DEV)))
    assert st == 0, L.fdp_strerror(st)
    torch.cuda.synchronize()
    untouched = bool(torch.all(ws[span:span + cb] == 0xA5)) if canary else None
    return out, norms, fac, bo, bn, bf, untouched


# (shape B, K, M, N; the schedules that take it)
CASES = [
    # cfg2 (paired wide kernel by default; the one-sample wide kernel unpaired)
    ((8, 1024, 3072, 768), ("wide", "unpaired", "narrow", "stream")),
    ((16, 1024, 768, 2304), ("narrow", "stream")),        # cfg3: Conv1D x^T g (grouped by default)
    ((12, 64, 1000, 704), ("wide", "unpaired", "narrow", "stream")),  # ragged tiles both ways
    ((6, 96, 392, 1160), ("wide",)),                      # paired, 3 x 7 tiles of 192
    ((5, 40, 520, 392), ("wide", "narrow", "stream")),    # one partial k-tile: idle partial slots
    ((4, 200, 1536, 384), ("wide", "narrow", "stream")),  # partial last k-tile
    ((20, 32, 3072, 1536), ("narrow", "stream")),         # grouped: five launches of 4 samples
    ((16, 64, 512, 512), ("narrow", "stream")),           # streamed: four sample groups
]
PARAMS = [(shape, sched) for shape, scheds in CASES for sched in scheds]


@pytest.mark.parametrize("operand", ["a", "b"])
@pytest.mark.parametrize("shape,sched", PARAMS,
                         ids=["x".join(map(str, s)) + "-" + k for s, k in PARAMS])
def test_wgrad_bias_fused(shape, sched, operand):
    B, K, M, N = shape
    dtype = torch.bfloat16
    print(f"bias fused: shape={shape} schedule={sched} operand={operand}", flush=True)
    a, b = make(B, K, M, N, dtype, seed=21)
    # C inside the norm range (fp32 products on the GPU), so that some samples clip
    wn = [float((a[i].float().t() @ b[i].float()).norm()) for i in range(B)]
    C = float(np.median(wn))
    op = a if operand == "a" else b
    blen = op.shape[2]
    zb = torch.randn(blen, generator=torch.Generator().manual_seed(5)).to(dtype).to(DEV)
    zw = torch.randn(M, N, generator=torch.Generator().manual_seed(6)).to(DEV)
    out, norms, fac, bo, bn, bf, untouched = run_bias_call(a, b, C, SCHEDULES[sched], operand, zw,
                                                           zb, canary=True)
    assert untouched, "the bias took the column-sum kernel instead of the product kernel"
    # the bias (norm of the whole op_b, mean over B*K)
    # (the fp64 column sums of a [16, 1024, 2304] operand take a few seconds)
    ref_b, ref_bn, ref_bf = O.colsum_clip(op, None, C, 1.0, "frob", 1.0 / (B * K), zb, 0.5)
    tag = (f"fused bias of {operand} {shape} ({sched})"
           if shape in ((8, 1024, 3072, 768), (16, 1024, 768, 2304)) else None)
    assert_close(bo, ref_b, dtype, "bias", margin=tag)
    assert_elementwise(bn, ref_bn, dtype, "bias norms")
    assert_elementwise(bf, ref_bf, dtype, "bias factors")
    # the weight gradient is the one fdp_wgrad_clip gives on the same schedule
    # and kernel: bit for bit, except on the grouped schedule, which splits no
    # products when it also forms a bias (a split product is handed over in bf16)
    w_only = core.wgrad_clip(a, b, C, 1.0, out_scale=1.0 / B, noise=zw, noise_scale=0.25,
                             out_dtype=torch.float32, two_pass=sched == "stream",
                             single_pass={"wide": "wide", "unpaired": "unpaired",
                                          "narrow": "narrow", "stream": "auto"}[sched],
                             check=True)
    if sched == "narrow":
        assert_close(out, w_only.double().cpu().numpy(), dtype, "weight vs weight-only call")
    else:
        assert torch.equal(out, w_only), "the weight gradient changed with the bias"
    if B * K * M * N <= 10**9:  # (larger: the weight's own tests cover its schedule)
        ref_w, ref_n, ref_f = O.wgrad_clip(a, b, C, 1.0, "tn", out_scale=1.0 / B, noise=zw,
                                           noise_scale=0.25)
        assert_close(out, ref_w, dtype, "weight")
        assert_elementwise(norms, ref_n, dtype, "weight norms")
        assert_elementwise(fac, ref_f, dtype, "weight factors")


@pytest.mark.parametrize("operand", ["a", "b"])
def test_wgrad_bias_fp32_takes_column_sums(operand):
    """fp32 operands run the generic schedule; the bias then comes from the
    column-sum kernel (its workspace region is used) and matches the oracle."""
    B, K, M, N = 3, 70, 96, 160
    a, b = make(B, K, M, N, torch.float32, seed=23)
    op = a if operand == "a" else b
    zb = torch.randn(op.shape[2], generator=torch.Generator().manual_seed(7)).to(DEV)
    zw = torch.randn(M, N, generator=torch.Generator().manual_seed(8)).to(DEV)
    out, _, _, bo, bn, bf, untouched = run_bias_call(a, b, 0.05, 0, operand, zw, zb, canary=True)
    assert not untouched
    ref_b, ref_bn, ref_bf = O.colsum_clip(op, None, 0.05, 1.0, "frob", 1.0 / (B * K), zb, 0.5)
    assert_close(bo, ref_b, torch.float32, "bias")
    assert_elementwise(bn, ref_bn, torch.float32, "bias norms")
    assert_elementwise(bf, ref_bf, torch.float32, "bias factors")
    ref_w, _, _ = O.wgrad_clip(a, b, 0.05, 1.0, "tn", out_scale=1.0 / B, noise=zw, noise_scale=0.25)
    assert_close(out, ref_w, torch.float32, "weight")


@pytest.mark.parametrize("sched", ["wide", "unpaired", "narrow", "stream"])
def test_wgrad_bias_of_b_in_kernel_noise(sched):
    """The bias noise drawn in the product kernels is the column-sum kernel's
    draw for the same key (Philox stream 0, element n)."""
    B, K, M, N = 8, 256, 768, 3072
    a, b = make(B, K, M, N, torch.bfloat16, seed=24)
    bo = torch.empty(N, dtype=torch.float32, device=DEV)
    core.wgrad_clip(a, b, 0.05, 1.0, out_dtype=torch.float32, bias_out=bo, bias_operand="b",
                    bias_scale=1.0 / (B * K), bias_noise_key=(777, 12), bias_noise_scale=0.5,
                    two_pass=sched == "stream",
                    single_pass="auto" if sched == "stream" else sched, check=True)
    z = torch.from_numpy(PX.normals(N, 777, 12, 0)).float()
    ref, _, _ = O.colsum_clip(b, None, 0.05, 1.0, "frob", 1.0 / (B * K), z, 0.5)
    assert_close(bo, ref, torch.bfloat16, f"bias of b with in-kernel noise ({sched})")


WIDE_BIAS_SHAPES = [
    (72, 32, 96, 96),     # paired: 36 pairs of one tile, one block per region
    (18, 32, 384, 384),   # paired: 9 pairs over 2 x 2 tiles
    (6, 256, 576, 768),   # paired: 3 pairs over 3 x 4 tiles, regions of 12 blocks
]


@pytest.mark.parametrize("operand", ["a", "b"])
@pytest.mark.parametrize("kernel", ["wide", "unpaired"])
@pytest.mark.parametrize("shape", WIDE_BIAS_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_wgrad_bias_wide_device_clip_args(shape, kernel, operand):
    """The wide kernels with a bias, C and clamp read from a device tensor
    (clamp 0.9), fp16 operands and bf16 outputs: weight, bias, both norms and
    both factors against the float64 oracle."""
    B, K, M, N = shape
    dtype = torch.float16
    print(f"wide bias, device clip args: shape={shape} kernel={kernel} operand={operand}",
          flush=True)
    a, b = make(B, K, M, N, dtype, seed=26)
    wn = [float((a[i].float().t() @ b[i].float()).norm()) for i in range(B)]
    C = float(np.median(wn))
    op = a if operand == "a" else b
    blen = op.shape[2]
    clip_args = torch.tensor([C, 0.9], device=DEV)
    bo = torch.empty(blen, dtype=torch.bfloat16, device=DEV)
    out, n, f, bn, bf = core.wgrad_clip(
        a, b, clip_args=clip_args, out_scale=1.0 / B, out_dtype=torch.bfloat16,
        return_stats=True, single_pass=kernel, check=True, bias_out=bo,
        bias_operand=operand, bias_scale=1.0 / (B * K))
    ref_w, ref_n, ref_f = O.wgrad_clip(a, b, C, 0.9, "tn", out_scale=1.0 / B)
    ref_b, ref_bn, ref_bf = O.colsum_clip(op, None, C, 0.9, "frob", 1.0 / (B * K), None, 0.0)
    assert_close(out, ref_w, dtype, "weight")
    assert_elementwise(n, ref_n, dtype, "weight norms")
    assert_elementwise(f, ref_f, dtype, "weight factors")
    assert_close(bo, ref_b, dtype, "bias")
    assert_elementwise(bn, ref_bn, dtype, "bias norms")
    assert_elementwise(bf, ref_bf, dtype, "bias factors")


@pytest.mark.parametrize("sched", ["wide", "unpaired", "narrow", "stream"])
def test_wgrad_bias_deterministic_and_zero_factors(sched):
    """Repeated calls are bitwise equal; with C = 0 every factor (weight and
    bias) is zero and so are both outputs, while the bias norms are still
    reported (the streamed pass reads a zero-factor sample's fragments for
    the bias only)."""
    B, K, M, N = 6, 96, 640, 896
    a, b = make(B, K, M, N, torch.bfloat16, seed=25)
    kw = dict(out_dtype=torch.float32, bias_operand="b", bias_scale=1.0 / (B * K),
              two_pass=sched == "stream", single_pass="auto" if sched == "stream" else sched,
              check=True, return_stats=True)
    outs = []
    for _ in range(2):
        bo = torch.empty(N, device=DEV)
        r = core.wgrad_clip(a, b, 0.1, 1.0, bias_out=bo, **kw)
        outs.append((r[0], bo))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    bo = torch.empty(N, device=DEV)
    out, n, f, bn, bf = core.wgrad_clip(a, b, 0.0, 1.0, bias_out=bo, **kw)
    assert torch.count_nonzero(out) == 0 and torch.count_nonzero(bo) == 0
    assert torch.count_nonzero(f) == 0 and torch.count_nonzero(bf) == 0
    _, ref_bn, _ = O.colsum_clip(b, None, 1.0, 1.0, "frob", 1.0, None, 0.0)
    assert_elementwise(bn, ref_bn, torch.bfloat16, "bias norms at C = 0")


def test_wgrad_bias_streamed_cfg5_shape():
    """The streamed schedule at cfg5's c_fc shape (d=2048 -> 8192, B=8, T=1024)
    with a bias and active clipping: dW against fp32 per-sample products on the
    GPU, the bias against float64 column sums on the GPU."""
    B, K, M, N = 8, 1024, 8192, 2048   # a = grad_output [B, T, 8192], b = x [B, T, 2048]
    dtype = torch.bfloat16
    g = torch.Generator(device=DEV).manual_seed(31)
    a = (torch.randn(B, K, M, device=DEV, generator=g) * 0.02).to(dtype)
    b = torch.randn(B, K, N, device=DEV, generator=g).to(dtype)
    bo = torch.empty(M, dtype=torch.float32, device=DEV)
    out, n, f, bn, bf = core.wgrad_clip(a, b, 1.0, 1.0, out_scale=1.0 / B, out_dtype=torch.float32,
                                        return_stats=True, bias_out=bo, bias_scale=1.0 / (B * K),
                                        check=True)
    # fp32 per-sample products, one sample at a time
    S = torch.zeros(M, N, device=DEV)
    n_ref = []
    for i in range(B):
        Gi = a[i].float().t().contiguous() @ b[i].float()
        ni = Gi.norm()
        n_ref.append(float(ni))
        S += Gi * min(1.0, 1.0 / (float(ni) + 1e-10))
        del Gi
    n_ref = np.array(n_ref)
    assert np.all(n_ref > 1.0), "every sample clips at C = 1"
    assert_elementwise(n, n_ref, dtype, "weight norms", margin="cfg5 c_fc streamed: norms")
    assert_close(out, (S / B).double().cpu().numpy(), dtype, "dW",
                 margin="cfg5 c_fc streamed, C = 1: clipped dW (fp32 out)")
    ad = a.double()
    m_ref = ad.flatten(1).norm(dim=1)
    cb = torch.clamp(1.0 / (m_ref + 1e-10), max=1.0)
    db_ref = (cb[:, None] * ad.sum(1)).sum(0) / (B * K)
    assert_elementwise(bn, m_ref.cpu().numpy(), dtype, "bias norms")
    assert_close(bo, db_ref.cpu().numpy(), dtype, "db",
                 margin="cfg5 c_fc streamed: fused bias (fp32 out)")
