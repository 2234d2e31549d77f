"""GPU parity of the clipped per-sample product sum (fdp_wgrad_clip) against the
float64 oracle on the same dtype-rounded inputs.  Tolerances: tests/_tol.py."""
import math

import numpy as np
import pytest
import torch

from oracle import dp_clip as O
from tests._tol import assert_close, assert_elementwise

from flashdp4review_amd import core

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def make(B, K, M, N, dtype, layout, seed=0, scale_b=0.02):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn((B, K, M) if layout == "tn" else (B, M, K), generator=g)
    b = torch.randn((B, K, N), generator=g) * scale_b
    return a.to(dtype).to(DEV), b.to(dtype).to(DEV)


SHAPES = [
    (4, 128, 768, 768),   # cfg1 per-layer shape; one unit per workgroup, 4-way tile hand-over
    (3, 37, 100, 70),     # ragged in every dimension, unaligned rows
    (3, 37, 104, 72),     # ragged tiles, aligned rows (single-pass kernel)
    (2, 64, 130, 257),    # odd N: unaligned rows, scalar loads
    (1, 1, 16, 16),       # B = 1, T = 1
    (5, 200, 64, 300),
    (16, 16, 256, 256),   # many samples, short contraction; 16-way tile hand-over
    (8, 64, 392, 520),    # several units per workgroup
]


@pytest.mark.parametrize("path", ["auto", "plain", "two_pass"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("layout", ["tn", "nn"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_wgrad_parity(shape, layout, dtype, path):
    B, K, M, N = shape
    a, b = make(B, K, M, N, dtype, layout)
    _, norms_ref, _ = O.wgrad_clip(a, b, 1.0, 1.0, layout)
    # choose C inside the norm range so that some samples clip and some do not
    C = float(np.median(norms_ref)) if B > 1 else float(norms_ref[0]) * 0.5
    ref, norms_ref, fac_ref = O.wgrad_clip(a, b, C, 1.0, layout)
    tp = path == "two_pass"
    launch = "plain" if path == "plain" else "cooperative"
    out, norms, fac = core.wgrad_clip(a, b, C, 1.0, layout=layout, out_dtype=torch.float32,
                                      return_stats=True, two_pass=tp, launch=launch, check=True)
    assert_close(out, ref, dtype, "out")
    assert_elementwise(norms, norms_ref, dtype, "norms")
    assert_elementwise(fac, fac_ref, dtype, "factors")
    # output in the input dtype (what the layers write)
    out2 = core.wgrad_clip(a, b, C, 1.0, layout=layout, two_pass=tp, launch=launch, check=True)
    assert out2.dtype == dtype
    assert_close(out2, ref, dtype, "out (input dtype)")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", [(8, 128, 3072, 768), (8, 200, 3000, 760)],
                         ids=lambda s: "x".join(map(str, s)))
def test_wgrad_split_products(shape, dtype):
    """144 tiles x 8 samples on 512 workgroups: the 128 workgroups holding three
    products each contract the last one over its first half of K only, and a
    workgroup of a CU holding two lighter ones contracts the rest and hands it
    over (2 and 4 k-tiles, a partial last k-tile, ragged tiles; the full cfg2
    shape, K = 1024, is test_wgrad_cfg2_full_size).  Parity, norms, factors and
    bitwise-equal repeats, in both launch modes."""
    B, K, M, N = shape
    a, b = make(B, K, M, N, dtype, "tn", seed=21)
    _, n0, _ = O.wgrad_clip(a, b, 1.0, 1.0, "tn")
    C = float(np.median(n0))
    ref, nref, fref = O.wgrad_clip(a, b, C, 1.0, "tn")
    for launch in ("plain", "cooperative"):
        out, n, f = core.wgrad_clip(a, b, C, 1.0, out_dtype=torch.float32, return_stats=True,
                                    launch=launch, single_pass="narrow", check=True)
        assert_close(out, ref, dtype, "out")
        assert_elementwise(n, nref, dtype, "norms")
        assert_elementwise(f, fref, dtype, "factors")
        again = core.wgrad_clip(a, b, C, 1.0, out_dtype=torch.float32, launch=launch,
                                single_pass="narrow", check=True)
        assert torch.equal(out, again)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_wgrad_scale_noise_and_device_clip_args(dtype):
    B, K, M, N = 4, 96, 192, 160
    a, b = make(B, K, M, N, dtype, "tn", seed=3)
    z = torch.randn(M, N, generator=torch.Generator().manual_seed(9)).to(dtype).to(DEV)
    clip_args = torch.tensor([0.05, 0.9], device=DEV)
    out = core.wgrad_clip(a, b, layout="tn", clip_args=clip_args, out_scale=1.0 / B, noise=z,
                          noise_scale=0.5, out_dtype=torch.float32)
    ref, _, _ = O.wgrad_clip(a, b, 0.05, 0.9, "tn", out_scale=1.0 / B, noise=z, noise_scale=0.5)
    assert_close(out, ref, dtype, "scaled+noise")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_wgrad_special_cases(dtype):
    B, K, M, N = 3, 50, 70, 90
    a, b = make(B, K, M, N, dtype, "tn", seed=5)
    # C = 0: every factor is 0
    out, _, fac = core.wgrad_clip(a, b, 0.0, 1.0, return_stats=True)
    assert torch.count_nonzero(out) == 0 and torch.count_nonzero(fac) == 0
    # C huge: plain product sum == torch fp32 batched product
    out = core.wgrad_clip(a, b, 1e30, 1.0, out_dtype=torch.float32)
    ref = torch.einsum("bkm,bkn->mn", a.double().cpu(), b.double().cpu()).numpy()
    assert_close(out, ref, dtype, "no clip")
    # huge norms: each clipped term has norm C, single sample -> ||out|| = C
    out = core.wgrad_clip(a[:1] * 8, b[:1] * 8, 0.25, 1.0, out_dtype=torch.float32)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert abs(out.double().norm().item() - 0.25) / 0.25 < tol
    # noclip flag = clamp everywhere
    out = core.wgrad_clip(a, b, 5.0, 0.5, noclip=True, out_dtype=torch.float32)
    ref, _, _ = O.wgrad_clip(a, b, 5.0, 0.5, "tn", noclip=True)
    assert_close(out, ref, dtype, "noclip")


@pytest.mark.parametrize("two_pass", [False, True])
def test_wgrad_deterministic(two_pass):
    a, b = make(8, 256, 512, 384, torch.bfloat16, "tn", seed=7)
    o1 = core.wgrad_clip(a, b, 0.5, 1.0, two_pass=two_pass, check=True)
    for launch in ("cooperative", "plain", "cooperative"):
        o2 = core.wgrad_clip(a, b, 0.5, 1.0, two_pass=two_pass, launch=launch, check=True)
        assert torch.equal(o1, o2)


@pytest.mark.parametrize("shape", [(8, 64, 392, 520), (16, 16, 256, 256), (20, 32, 3072, 1536)],
                         ids=lambda s: "x".join(map(str, s)))
def test_wgrad_reused_workspace_stays_clean(shape):
    """Calls that reuse one workspace without clearing it (FDP_WGRAD_CLEAN_WORKSPACE)
    match a call on a garbage-filled workspace that the library clears, and leave
    the status word and the grid-barrier counter (words 0 and 1) zero; the launch
    epoch (word 2) advances once per launch.  Tiles are shared by groups and a call
    makes several launches; the tile tickets after the head are cleared by the
    kernel itself, so the dirty workspace's tickets start as garbage."""
    import ctypes
    from flashdp4review_amd import _lib
    B, K, M, N = shape
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=12)
    L = _lib.lib()
    nb = _lib.size_query(L.fdp_wgrad_clip_workspace_size, B, K, M, N, _lib.FDP_BF16, 0)

    def call(ws, flags):
        out = torch.empty(M, N, dtype=torch.float32, device=DEV)
        st = L.fdp_wgrad_clip(a.data_ptr(), b.data_ptr(), B, K, M, N, a.stride(0), a.stride(1),
                              b.stride(0), b.stride(1), _lib.LAYOUT_TN, _lib.FDP_BF16,
                              ctypes.c_float(0.05), ctypes.c_float(1.0), None, ctypes.c_float(1.0),
                              None, ctypes.c_float(1.0), None, out.data_ptr(), N, _lib.FDP_F32, None,
                              None, flags, ws.data_ptr(), ws.numel(),
                              _lib.stream_handle(torch.device(DEV)))
        assert st == 0
        return out

    dirty = torch.full((nb,), 0xA5, dtype=torch.uint8, device=DEV)
    ref = call(dirty, 0)
    clean = torch.zeros(nb, dtype=torch.uint8, device=DEV)
    for _ in range(3):
        out = call(clean, _lib.WGRAD_CLEAN_WORKSPACE)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        words = clean[:16].view(torch.int32).cpu()
        assert int(words[0]) == 0 and int(words[1]) == 0
        assert int(words[2]) > 0
    exp, _, _ = O.wgrad_clip(a, b, 0.05, 1.0, "tn")
    assert_close(ref, exp, torch.bfloat16, "clipped sum")


def test_wgrad_expired_grid_wait_is_loud(monkeypatch):
    """Force the single-pass kernel's bounded waits to expire at their first poll
    (FDP_WGRAD_SPIN_LIMIT=0; every kernel still runs to completion): the outputs
    are NaN, the status word is set and check=True raises.  An expiry poisons only
    its own launch: the next call (normal spin limit, no check) is exact although
    the status word is still set, and wgrad_status() then reports and clears it.
    8 x 1024 x 512 x 384 has split products, so a stale hand-over flag left by the
    expired launch would also show up here."""
    from flashdp4review_amd import _lib
    a, b = make(8, 1024, 512, 384, torch.bfloat16, "tn", seed=13)
    ref, _, _ = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
    for launch in ("plain", "cooperative"):
        monkeypatch.setenv("FDP_WGRAD_SPIN_LIMIT", "0")
        with pytest.raises(_lib.FlashDPError):
            core.wgrad_clip(a, b, 0.5, 1.0, launch=launch, out_dtype=torch.float32, check=True)
        out = core.wgrad_clip(a, b, 0.5, 1.0, launch=launch, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.isnan(out).any()
        monkeypatch.delenv("FDP_WGRAD_SPIN_LIMIT")
        for _ in range(2):
            out = core.wgrad_clip(a, b, 0.5, 1.0, launch=launch, out_dtype=torch.float32)
            assert_close(out, ref, torch.bfloat16, f"after expiry ({launch})")
        assert core.wgrad_status() != 0
        assert core.wgrad_status() == 0
    out = core.wgrad_clip(a, b, 0.5, 1.0, out_dtype=torch.float32, check=True)
    assert_close(out, ref, torch.bfloat16, "after expiry, checked")


def test_wgrad_expiry_reported_asynchronously(monkeypatch):
    """Without check=True an expiry is reported by a later call on the stream: the
    status word is copied to pinned host memory behind every STATUS_PERIOD-th call,
    and the first call after that copy completes raises (once) and clears it."""
    from flashdp4review_amd import _lib
    from flashdp4review_amd.core import wgrad as W
    a, b = make(8, 256, 512, 384, torch.bfloat16, "tn", seed=15)
    core.wgrad_status()  # start from a clear status word
    monkeypatch.setattr(W, "STATUS_PERIOD", 1)
    monkeypatch.setenv("FDP_WGRAD_SPIN_LIMIT", "0")
    out = core.wgrad_clip(a, b, 0.5, 1.0, launch="plain")  # expires; the probe is queued
    monkeypatch.delenv("FDP_WGRAD_SPIN_LIMIT")
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).any()
    with pytest.raises(_lib.FlashDPError):
        core.wgrad_clip(a, b, 0.5, 1.0)
    torch.cuda.synchronize()
    assert core.wgrad_status(clear=False) == 0
    ref, _, _ = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
    for _ in range(3):  # later probes read a clear word: no further raise
        out = core.wgrad_clip(a, b, 0.5, 1.0, out_dtype=torch.float32)
        torch.cuda.synchronize()
    assert_close(out, ref, torch.bfloat16, "after the report")


@pytest.mark.parametrize("shape", [(5, 96, 4000, 2300), (2, 64, 8192, 2048), (3, 33, 6000, 3000)],
                         ids=lambda s: "x".join(map(str, s)))
def test_wgrad_more_tiles_than_workgroups(shape):
    """Layers with more 128x128 output tiles than resident workgroups take the
    streamed two-pass schedule by default (Gram-form norms for 2x64x8192x2048,
    direct norms where M or N is not a multiple of 64)."""
    B, K, M, N = shape
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=14)
    _, norms_ref, _ = O.wgrad_clip(a, b, 1.0, 1.0, "tn")
    C = float(np.median(norms_ref))
    ref, norms_ref, fac_ref = O.wgrad_clip(a, b, C, 1.0, "tn")
    out, norms, fac = core.wgrad_clip(a, b, C, 1.0, out_dtype=torch.float32, return_stats=True,
                                      check=True)
    assert_close(out, ref, torch.bfloat16, "out")
    assert_elementwise(norms, norms_ref, torch.bfloat16, "norms")
    assert_elementwise(fac, fac_ref, torch.bfloat16, "factors")
    out2 = core.wgrad_clip(a, b, C, 1.0, out_dtype=torch.float32, check=True)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("shape", [(3, 300, 2048, 1024), (2, 256, 4096, 1536), (16, 64, 512, 512),
                                   (4, 128, 640, 1088), (3, 130, 1024, 3000)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_wgrad_stream_two_pass(shape, dtype):
    """The streamed two-pass schedule: per-sample norms from the Gram matrices
    (sum over t, s of (g_t . g_s)(x_t . x_s)) where that is cheaper and M, N are
    multiples of 64, else from the per-tile products; then one clipped-sum
    contraction per 128x256 output tile, split over sample groups when there
    are few tiles (16x64x512x512)."""
    B, K, M, N = shape
    a, b = make(B, K, M, N, dtype, "tn", seed=31)
    _, norms_ref, _ = O.wgrad_clip(a, b, 1.0, 1.0, "tn")
    C = float(np.median(norms_ref))
    ref, norms_ref, fac_ref = O.wgrad_clip(a, b, C, 1.0, "tn")
    out, norms, fac = core.wgrad_clip(a, b, C, 1.0, out_dtype=torch.float32, return_stats=True,
                                      two_pass=True, check=True)
    assert_close(out, ref, dtype, "out")
    assert_elementwise(norms, norms_ref, dtype, "norms")
    assert_elementwise(fac, fac_ref, dtype, "factors")
    noise = torch.randn(M, N, generator=torch.Generator().manual_seed(5)).to(dtype).to(DEV)
    out2 = core.wgrad_clip(a, b, C, 1.0, out_scale=0.25, noise=noise, noise_scale=0.5,
                           two_pass=True, check=True)
    ref2 = 0.25 * ref + 0.5 * noise.double().cpu().numpy()
    assert_close(out2, ref2, dtype, "out (scale, noise)")


def test_wgrad_stream_zero_factors():
    """C = 0 makes every clip factor 0: the streamed clipped sum loads zeros for
    each sample and the output is exactly out_scale * 0 + noise_scale * z."""
    B, K, M, N = 3, 64, 4096, 1536
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=33)
    noise = torch.randn(M, N, generator=torch.Generator().manual_seed(6)).to(DEV)
    out, norms, fac = core.wgrad_clip(a, b, 0.0, 1.0, out_scale=0.5, noise=noise, noise_scale=0.25,
                                      out_dtype=torch.float32, return_stats=True, two_pass=True,
                                      check=True)
    assert torch.all(fac == 0)
    assert torch.equal(out, 0.25 * noise)
    _, norms_ref, _ = O.wgrad_clip(a, b, 1.0, 1.0, "tn")
    assert_elementwise(norms, norms_ref, torch.bfloat16, "norms")


def test_wgrad_operand_rows_past_a_buffer_record():
    """A sample operand whose rows span 4 GiB (the last 128 columns of
    [8192, 262144] bf16 rows, lda = 2^18) is more than a 32-bit buffer record
    addresses: the call takes the generic schedule (64-bit addressing) instead
    of the single-pass or streamed kernels, and matches the oracle.  Clipping
    is active (norm about 160 against C = 1)."""
    K, M, N, W = 8192, 128, 64, 1 << 18
    gen = torch.Generator().manual_seed(61)
    big = torch.zeros(K, W, dtype=torch.bfloat16, device=DEV)
    big[:, W - M:] = torch.randn(K, M, generator=gen).to(torch.bfloat16).to(DEV)
    a = big[:, W - M:].unsqueeze(0)  # [1, K, M], lda = W
    b = (torch.randn(1, K, N, generator=gen) * 0.02).to(torch.bfloat16).to(DEV)
    assert a.stride(1) == W
    ref, nref, fref = O.wgrad_clip(a.contiguous(), b, 1.0, 1.0, "tn")
    assert float(fref.max()) < 0.1
    for tp in (False, True):
        out, n, f = core.wgrad_clip(a, b, 1.0, 1.0, out_dtype=torch.float32, two_pass=tp,
                                    return_stats=True, check=True)
        assert_close(out, ref, torch.bfloat16, f"4 GiB operand rows, two_pass={tp}")
        assert_elementwise(n, nref, torch.bfloat16, "norms")
        assert_elementwise(f, fref, torch.bfloat16, "factors")
    del big


def test_wgrad_padding_rows_never_wrap_into_a_record():
    """K = 1 with a row stride of 2^29 elements: a 64-deep k-tile's padding rows
    k = 1..63 lie k * 2^30 bytes on, and 32-bit offsets would wrap every fourth
    one back to row 0 inside the operand's record.  Such a stride takes the
    generic schedule, and the sum counts row 0 once."""
    B, M, N, LD = 4, 256, 256, 1 << 29
    gen = torch.Generator().manual_seed(62)
    flat = torch.randn(B * M, generator=gen).to(torch.bfloat16).to(DEV)
    a = flat.as_strided((B, 1, M), (M, LD, 1))
    b = (torch.randn(B, 1, N, generator=gen) * 0.02).to(torch.bfloat16).to(DEV)
    assert a.stride(1) == LD
    ref, nref, fref = O.wgrad_clip(a.contiguous(), b, 0.05, 1.0, "tn")
    for tp in (False, True):
        out, n, f = core.wgrad_clip(a, b, 0.05, 1.0, out_dtype=torch.float32, two_pass=tp,
                                    return_stats=True, check=True)
        assert_close(out, ref, torch.bfloat16, f"K=1, lda=2^29, two_pass={tp}")
        assert_elementwise(n, nref, torch.bfloat16, "norms")
        assert_elementwise(f, fref, torch.bfloat16, "factors")


def test_wgrad_workspace_reused_across_shapes():
    """Consecutive calls of different shapes share the cached per-stream workspace;
    each shape lays it out differently (one call's partial norms sit where the
    next one's tile tickets go), and every result must still be exact."""
    for i, (B, K, M, N) in enumerate([(8, 64, 1536, 768), (2, 64, 3072, 768), (4, 64, 128, 128),
                                      (3, 64, 3072, 768), (2, 64, 3072, 768)]):
        a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=20 + i)
        ref, _, _ = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
        for tp in (True, False):
            out = core.wgrad_clip(a, b, 0.5, 1.0, out_dtype=torch.float32, two_pass=tp, check=True)
            assert_close(out, ref, torch.bfloat16, f"{(B, K, M, N)} two_pass={tp}")


def test_wgrad_does_not_modify_inputs():
    a, b = make(4, 64, 128, 128, torch.bfloat16, "tn", seed=8)
    a0, b0 = a.clone(), b.clone()
    core.wgrad_clip(a, b, 0.1, 1.0)
    assert torch.equal(a, a0) and torch.equal(b, b0)


def test_operator_api():
    dtype = torch.bfloat16
    B, K, M, N = 4, 64, 96, 80
    t1, t2 = make(B, K, M, N, dtype, "tn", seed=11)
    ca = torch.tensor([0.3, 1.0], device=DEV)
    ref, _, _ = O.wgrad_clip(t1, t2, 0.3, 1.0, "tn")
    assert_close(core.bmtm_clip(t1, t2, ca), ref, dtype, "bmtm_clip")
    t1n = t1.transpose(1, 2).contiguous()
    r = core.bmm_clip(t1n, t2, ca)
    assert r.dtype == torch.float32
    assert_close(r, ref, dtype, "bmm_clip")
    m1 = torch.randn(M, K, device=DEV, dtype=torch.float32)
    m2 = torch.randn(K, N, device=DEV, dtype=torch.float32) * 0.1
    assert_close(core.mm_clip(m1, m2, ca), O.mm_clip(m1, m2, 0.3, 1.0), torch.float32, "mm_clip")
    mf = core.mm_fused(m1, m2)
    assert_close(mf, m1.double().cpu().numpy() @ m2.double().cpu().numpy(), torch.float32,
                 "mm_fused")
    x = torch.randn(B, K, 48, device=DEV, dtype=dtype)
    g = torch.randn(B, K, 40, device=DEV, dtype=dtype) * 0.01
    ref, _, _ = O.wgrad_clip(g, x, 0.2, 1.0, "tn")
    assert_close(core.linear_weight_flashdp(x, g, 0.2, 1.0, core.RuntimeAutoTuner()), ref, dtype,
                 "linear_weight_flashdp")
    ref, _, _ = O.wgrad_clip(x, g, 0.2, 1.0, "tn")
    assert_close(core.conv1d_weight_flashdp(x, g, 0.2, 1.0), ref, dtype, "conv1d_weight_flashdp")


@pytest.mark.parametrize("single_pass", ["auto", "unpaired", "narrow"])
@pytest.mark.parametrize("dtype", [torch.bfloat16], ids=str)
def test_wgrad_cfg2_full_size(dtype, single_pass):
    """cfg2 (Linear 768->3072, B=8, T=1024): norms and the clipped sum against an fp32
    torch reference on the GPU (per-sample bmm in fp32), all samples clipped; the
    default kernel (the paired wide one at this shape), the one-sample wide
    kernel and the grouped one."""
    torch.manual_seed(0)
    x = torch.randn(8, 1024, 768, device=DEV).to(dtype)
    g = (torch.randn(8, 1024, 3072, device=DEV) * 0.02).to(dtype)
    out, norms, fac = core.wgrad_clip(g, x, 1.0, 1.0, out_dtype=torch.float32, return_stats=True,
                                      single_pass=single_pass, check=True)
    G = torch.bmm(g.float().transpose(1, 2).contiguous(), x.float())  # [8, 3072, 768]
    n_ref = G.flatten(1).norm(dim=1)
    c_ref = torch.clamp(1.0 / (n_ref + 1e-10), max=1.0)
    ref = (c_ref[:, None, None] * G).sum(0)
    assert torch.all(n_ref > 1.0)
    tag = f"cfg2 wgrad ({single_pass} kernel)"
    assert_elementwise(norms, n_ref.double().cpu().numpy(), dtype, "norms",
                       margin=f"{tag}: per-sample norms (bf16 in)")
    assert_elementwise(fac, c_ref.double().cpu().numpy(), dtype, "factors",
                       margin=f"{tag}: clip factors (bf16 in)")
    assert_close(out, ref.double().cpu().numpy(), dtype, "clipped sum",
                 margin=f"{tag}: clipped sum, fp32 out (bf16 in)")
    # with every sample clipped, the 1/B-free sum has norm <= B*C
    assert out.norm().item() <= 8.0 * (1 + 1e-3)


@pytest.mark.parametrize("single_pass", ["wide", "narrow"])
def test_wgrad_memory_no_per_sample_materialisation(single_pass):
    """Peak memory the call adds to its output (the workspace) stays below
    B*M*N*elt, what materialising one bf16 gradient per sample would take: the
    wide kernel exchanges (B-1)/B of each sample's tile in bf16, the grouped
    kernel sums of several samples."""
    from flashdp4review_amd.core import wgrad as W
    B, K, M, N = 8, 1024, 3072, 768
    x = torch.randn(B, K, N, device=DEV, dtype=torch.bfloat16)
    g = torch.randn(B, K, M, device=DEV, dtype=torch.bfloat16) * 0.02
    out = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    W.release_workspaces()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    core.wgrad_clip(g, x, 1.0, 1.0, out=out, single_pass=single_pass)
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated() - base
    assert extra < B * M * N * 2, extra


# ------------------------------------------------------------ in-kernel noise
from oracle import philox as PX  # noqa: E402

NOISE_KEY = (0x9E3779B97F4A7C15, 12345)


@pytest.mark.parametrize("shape,layout,dtype,two_pass", [
    ((8, 64, 392, 520), "tn", torch.bfloat16, False),    # single pass, ragged tiles
    ((4, 128, 768, 768), "tn", torch.bfloat16, False),   # single pass, 4 groups
    ((3, 37, 104, 72), "tn", torch.float16, False),
    ((3, 300, 2048, 1024), "tn", torch.bfloat16, True),  # streamed two-pass (Gram norms)
    ((2, 64, 130, 257), "tn", torch.bfloat16, False),    # unaligned rows: generic two-pass
    ((3, 37, 100, 70), "nn", torch.float32, False),      # generic two-pass, odd N
    ((16, 16, 256, 256), "tn", torch.float32, True),     # generic, several groups (finalize)
], ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_wgrad_in_kernel_noise(shape, layout, dtype, two_pass):
    """z drawn inside the output epilogue equals the oracle's Philox4x32-10 /
    Box-Muller stream element for element (row-major over [M, N])."""
    B, K, M, N = shape
    a, b = make(B, K, M, N, dtype, layout, seed=40)
    ref, _, _ = O.wgrad_clip(a, b, 0.5, 1.0, layout)
    kw = dict(layout=layout, out_scale=0.5, out_dtype=torch.float32, two_pass=two_pass, check=True)
    out0 = core.wgrad_clip(a, b, 0.5, 1.0, noise_scale=0.25, **kw)  # no z: no noise
    out = core.wgrad_clip(a, b, 0.5, 1.0, noise_scale=0.25, noise_key=NOISE_KEY, **kw)
    z = PX.normals(M * N, *NOISE_KEY).reshape(M, N)
    assert_close(out0, 0.5 * ref, dtype, "no noise")
    got = (out.double() - out0.double()).cpu().numpy() / 0.25
    assert np.max(np.abs(got - z)) < 1e-4, np.max(np.abs(got - z))
    # bf16 output: the same draw, rounded once with the clipped sum
    out16 = core.wgrad_clip(a, b, 0.5, 1.0, noise_scale=0.25, noise_key=NOISE_KEY,
                            **{**kw, "out_dtype": torch.bfloat16})
    assert_close(out16, 0.5 * ref + 0.25 * z, torch.bfloat16, "bf16 out with noise")


def test_wgrad_noise_key_advances():
    """Disjoint offsets give independent draws; the same key repeats exactly."""
    a, b = make(2, 32, 256, 128, torch.bfloat16, "tn", seed=41)
    f = lambda key: core.wgrad_clip(a, b, 1.0, 1.0, noise_scale=1.0, noise_key=key,
                                    out_dtype=torch.float32)
    base = core.wgrad_clip(a, b, 1.0, 1.0, noise_scale=1.0, out_dtype=torch.float32)
    z1 = (f((7, 0)) - base).cpu().numpy()
    z2 = (f((7, 256 * 128 // 4)) - base).cpu().numpy()
    assert torch.equal(f((7, 0)), f((7, 0)))
    assert abs(np.corrcoef(z1.ravel(), z2.ravel())[0, 1]) < 0.05
    assert abs(z1.std() - 1) < 0.05


# ------------------------------------------------------------ wide single pass
WIDE_SHAPES = [
    (8, 1024, 3072, 768),   # cfg2: 32 tiles of 384x192 x 8 samples = 256 products
    (4, 100, 1000, 704),    # ragged tiles in both directions, K not a multiple of 32
    (16, 64, 512, 384),     # 16 samples per tile: regions of 4-5 blocks
    (2, 32, 384, 192),      # one tile, two samples: regions of 36 blocks
    (72, 16, 96, 96),       # 72 samples of one (mostly empty) tile: one block per region
    (3, 1, 200, 400),       # K = 1
    (6, 256, 576, 768),     # 192x384 tiles (6 against 8 of 384x192); paired: regions of 12
    (10, 64, 1000, 704),    # paired: ragged tiles, 5 pairs (regions of 7-8 blocks)
    (18, 32, 384, 384),     # paired: 9 pairs, chunks loaded in two batches
    (72, 32, 96, 96),       # paired: 36 pairs, one block per region
]


@pytest.mark.parametrize("kernel", ["wide", "unpaired"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", WIDE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_wgrad_wide_parity(shape, dtype, kernel):
    """The wide schedule, forced on shapes it fits ("wide": two samples per CU
    where the batch is even, 6..72, and K % 32 == 0, else one; "unpaired": one
    tile of one sample per CU): clipped sum, norms and factors against the fp64
    oracle, in fp32 and the input dtype, both launch modes, bitwise-equal
    repeats, and the grouped kernel within the same tolerance."""
    B, K, M, N = shape
    a, b = make(B, K, M, N, dtype, "tn", seed=50)
    _, n0, _ = O.wgrad_clip(a, b, 1.0, 1.0, "tn")
    C = float(np.median(n0))
    ref, nref, fref = O.wgrad_clip(a, b, C, 1.0, "tn")
    outs = []
    for launch in ("plain", "cooperative"):
        out, n, f = core.wgrad_clip(a, b, C, 1.0, out_dtype=torch.float32, return_stats=True,
                                    launch=launch, single_pass=kernel, check=True)
        assert_close(out, ref, dtype, "out", margin=None if shape != WIDE_SHAPES[0] else
                     f"{kernel} kernel cfg2 shape: clipped sum, fp32 out ({dtype})")
        assert_elementwise(n, nref, dtype, "norms")
        assert_elementwise(f, fref, dtype, "factors")
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    out16 = core.wgrad_clip(a, b, C, 1.0, single_pass=kernel, check=True)
    assert out16.dtype == dtype
    assert_close(out16, ref, dtype, "out (input dtype)")
    narrow = core.wgrad_clip(a, b, C, 1.0, out_dtype=torch.float32, single_pass="narrow",
                             check=True)
    assert_close(narrow, ref, dtype, "grouped kernel")


@pytest.mark.parametrize("kernel", ["wide", "unpaired"])
@pytest.mark.parametrize("shape", [(8, 64, 392, 520), (8, 1024, 3072, 768), (5, 40, 200, 96)],
                         ids=lambda s: "x".join(map(str, s)))
def test_wgrad_wide_noise(shape, kernel):
    """Noise in the wide kernel's finish: the in-kernel Philox draw (each quad of
    lanes draws four rows' blocks and transposes them) equals the oracle's
    stream element for element; an injected tensor is added as given."""
    B, K, M, N = shape
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=51)
    ref, _, _ = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
    kw = dict(out_scale=0.5, out_dtype=torch.float32, single_pass=kernel, check=True)
    out0 = core.wgrad_clip(a, b, 0.5, 1.0, noise_scale=0.25, **kw)
    out = core.wgrad_clip(a, b, 0.5, 1.0, noise_scale=0.25, noise_key=NOISE_KEY, **kw)
    z = PX.normals(M * N, *NOISE_KEY).reshape(M, N)
    assert_close(out0, 0.5 * ref, torch.bfloat16, "no noise")
    got = (out.double() - out0.double()).cpu().numpy() / 0.25
    assert np.max(np.abs(got - z)) < 1e-4, np.max(np.abs(got - z))
    zt = torch.randn(M, N, generator=torch.Generator().manual_seed(9)).to(DEV)
    out2 = core.wgrad_clip(a, b, 0.5, 1.0, noise=zt, noise_scale=0.25, **kw)
    assert_close(out2, 0.5 * ref + 0.25 * zt.double().cpu().numpy(), torch.bfloat16, "injected")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_wgrad_paired_strided_operands(dtype):
    """The paired wide kernel reads both samples of a pair through one buffer
    record (sample stride sab apart): samples taken every other one from a
    larger batch (sab = 2 * K * lda), rows padded past N (ldb > N) with
    N % 4 != 0 (the noise is then drawn element by element and the outputs
    stored one by one), against the fp64 oracle and the oracle's Philox stream."""
    B, K, M, N = 8, 64, 576, 390
    ga, gb = make(2 * B, K, M, 400, dtype, "tn", seed=53)
    a = ga[::2]                   # [8, 64, 576], sample stride 2 * K * M
    b = gb[::2, :, :N]            # [8, 64, 390], sample stride 2 * K * 400, ldb = 400
    assert a.stride(0) == 2 * K * M and b.stride(1) == 400
    ref, nref, fref = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
    kw = dict(out_scale=0.5, out_dtype=torch.float32, single_pass="wide", check=True)
    out, n, f = core.wgrad_clip(a, b, 0.5, 1.0, return_stats=True, **kw)
    assert_close(out, 0.5 * ref, dtype, "paired, strided operands")
    assert_elementwise(n, nref, dtype, "norms")
    assert_elementwise(f, fref, dtype, "factors")
    unpaired = core.wgrad_clip(a, b, 0.5, 1.0, **{**kw, "single_pass": "unpaired"})
    assert_close(unpaired, 0.5 * ref, dtype, "one sample per CU, same operands")
    noisy = core.wgrad_clip(a, b, 0.5, 1.0, noise_scale=0.25, noise_key=NOISE_KEY, **kw)
    z = PX.normals(M * N, *NOISE_KEY).reshape(M, N)
    got = (noisy.double() - out.double()).cpu().numpy() / 0.25
    assert np.max(np.abs(got - z)) < 1e-4, np.max(np.abs(got - z))


@pytest.mark.parametrize("kernel", ["wide", "unpaired"])
def test_wgrad_wide_expired_wait(monkeypatch, kernel):
    """A forced expiry of the wide kernels' waits (the grid barrier, and the
    paired kernel's per-tile wait): NaN outputs and a raised check; the next
    call on the same workspace is exact."""
    from flashdp4review_amd import _lib
    a, b = make(8, 256, 3072, 768, torch.bfloat16, "tn", seed=52)
    ref, _, _ = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
    core.wgrad_status()
    monkeypatch.setenv("FDP_WGRAD_SPIN_LIMIT", "0")
    with pytest.raises(_lib.FlashDPError):
        core.wgrad_clip(a, b, 0.5, 1.0, out_dtype=torch.float32, single_pass=kernel, check=True)
    out = core.wgrad_clip(a, b, 0.5, 1.0, out_dtype=torch.float32, single_pass=kernel)
    torch.cuda.synchronize()
    assert torch.isnan(out).any()
    monkeypatch.delenv("FDP_WGRAD_SPIN_LIMIT")
    out = core.wgrad_clip(a, b, 0.5, 1.0, out_dtype=torch.float32, single_pass=kernel)
    assert_close(out, ref, torch.bfloat16, "after expiry")
    assert core.wgrad_status() != 0


@pytest.mark.parametrize("kernel", ["wide", "unpaired"])
def test_wgrad_wide_bias_expired_wait(monkeypatch, kernel):
    """A forced expiry with a bias in the same launch (the paired kernel's
    bias polls expire too): a raised check and NaN in both outputs; the next
    call on the same workspace gives both exactly again."""
    from flashdp4review_amd import _lib
    B, K, M, N = 8, 256, 3072, 768
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=53)
    kw = dict(out_dtype=torch.float32, bias_scale=1.0 / (B * K), single_pass=kernel)
    ref_w, _, _ = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
    ref_b, _, _ = O.colsum_clip(a, None, 0.5, 1.0, "frob", 1.0 / (B * K), None, 0.0)
    core.wgrad_status()
    monkeypatch.setenv("FDP_WGRAD_SPIN_LIMIT", "0")
    bo = torch.empty(M, dtype=torch.float32, device=DEV)
    with pytest.raises(_lib.FlashDPError):
        core.wgrad_clip(a, b, 0.5, 1.0, bias_out=bo, check=True, **kw)
    bo = torch.empty(M, dtype=torch.float32, device=DEV)
    out = core.wgrad_clip(a, b, 0.5, 1.0, bias_out=bo, **kw)
    torch.cuda.synchronize()
    assert torch.isnan(out).any() and torch.isnan(bo).any()
    monkeypatch.delenv("FDP_WGRAD_SPIN_LIMIT")
    bo = torch.empty(M, dtype=torch.float32, device=DEV)
    out = core.wgrad_clip(a, b, 0.5, 1.0, bias_out=bo, **kw)
    assert_close(out, ref_w, torch.bfloat16, "weight after expiry")
    assert_close(bo, ref_b, torch.bfloat16, "bias after expiry")
    assert core.wgrad_status() != 0


# ------------------------------------------------- weight and bias in one call
BIAS_SHAPES = [
    (8, 1024, 3072, 768),  # cfg2: the DP Linear 768 -> 3072 layer, B=8, T=1024
    (12, 64, 1000, 704),   # ragged tiles in both directions (rows of 16-byte multiples)
    (4, 96, 1536, 384),    # 192x384 or 384x192 tiles, contraction of 3 k-tiles
]


@pytest.mark.parametrize("kernel", ["wide", "unpaired"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", BIAS_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_wgrad_bias_fused_in_wide_kernel(shape, dtype, kernel):
    """fdp_wgrad_bias_clip through the C ABI: with the wide kernels (paired
    where B allows, or the one-sample kernel) the bias of a comes from the same
    launch -- the column-sum half of the workspace (filled with a canary) is
    never touched -- and matches the float64 oracle
    (flashdp/core/linear_clip.py:116-123: norm of the whole a_b, mean over
    B*K) and the column-sum kernel's result (FDP_WGRAD_NARROW: the fallback);
    the weight gradient is the one fdp_wgrad_clip gives with the same kernel,
    bit for bit."""
    import ctypes
    from flashdp4review_amd import _lib
    B, K, M, N = shape
    flags = _lib.WGRAD_WIDE | (_lib.WGRAD_UNPAIRED if kernel == "unpaired" else 0)
    print(f"bias fused: shape={shape} dtype={dtype} kernel={kernel}", flush=True)
    a, b = make(B, K, M, N, dtype, "tn", seed=21)
    L = _lib.lib()
    dt = _lib.dtype_code(dtype)
    _, wn, _ = O.wgrad_clip(a, b, 1.0, 1.0, "tn")
    C = float(np.median(wn))
    zb = (torch.randn(M, generator=torch.Generator().manual_seed(5)) * 1.0).to(dtype).to(DEV)
    zw = torch.randn(M, N, generator=torch.Generator().manual_seed(6)).to(DEV)  # fp32, as out
    stream = _lib.stream_handle(torch.device(DEV))

    def run(flags, with_bias=True, canary=False):
        out = torch.empty(M, N, dtype=torch.float32, device=DEV)
        norms = torch.empty(B, dtype=torch.float32, device=DEV)
        fac = torch.empty(B, dtype=torch.float32, device=DEV)
        bo = torch.empty(M, dtype=dtype, device=DEV)
        bn = torch.empty(B, dtype=torch.float32, device=DEV)
        bf = torch.empty(B, dtype=torch.float32, device=DEV)
        common = (a.data_ptr(), b.data_ptr(), B, K, M, N, a.stride(0), a.stride(1), b.stride(0),
                  b.stride(1), _lib.LAYOUT_TN, dt, ctypes.c_float(C), ctypes.c_float(1.0), None,
                  ctypes.c_float(1.0 / B), zw.data_ptr(), ctypes.c_float(0.25), None,
                  out.data_ptr(), N, _lib.FDP_F32, norms.data_ptr(), fac.data_ptr(), flags)
        if not with_bias:
            nb = _lib.size_query(L.fdp_wgrad_clip_workspace_size, B, K, M, N, dt, flags)
            ws = torch.zeros(nb, dtype=torch.uint8, device=DEV)
            assert L.fdp_wgrad_clip(*common, ws.data_ptr(), nb, stream) == 0
            torch.cuda.synchronize()
            return out, norms, fac
        wb = _lib.size_query(L.fdp_wgrad_clip_workspace_size, B, K, M, N, dt, flags)
        nb = _lib.size_query(L.fdp_wgrad_bias_clip_workspace_size, B, K, M, N, dt, flags)
        span = (wb + 255) // 256 * 256
        ws = torch.zeros(nb, dtype=torch.uint8, device=DEV)
        if canary:
            ws[span:] = 0xA5
        bias = _lib.BiasOut(bo.data_ptr(), dt, 1.0 / (B * K), zb.data_ptr(), 0.5, None,
                            bn.data_ptr(), bf.data_ptr())
        st = L.fdp_wgrad_bias_clip(*common, ctypes.byref(bias), ws.data_ptr(), nb, stream)
        assert st == 0, L.fdp_strerror(st)
        torch.cuda.synchronize()
        untouched = bool(torch.all(ws[span:] == 0xA5)) if canary else None
        return out, norms, fac, bo, bn, bf, untouched

    out, norms, fac, bo, bn, bf, untouched = run(flags, canary=True)
    assert untouched, "the bias took the column-sum fallback instead of the wide kernel"
    # the weight as the same kernel forms it without a bias
    w_only = run(flags, with_bias=False)
    assert torch.equal(out, w_only[0]) and torch.equal(norms, w_only[1])
    ref_b, ref_bn, ref_bf = O.colsum_clip(a, None, C, 1.0, "frob", 1.0 / (B * K), zb, 0.5)
    tag = (f"bias fused in the {kernel} wide kernel {shape} ({dtype})"
           if shape == BIAS_SHAPES[0] else None)
    assert_close(bo, ref_b, dtype, "bias", margin=tag)
    assert_elementwise(bn, ref_bn, dtype, "bias norms")
    assert_elementwise(bf, ref_bf, dtype, "bias factors")
    ref_w, _, _ = O.wgrad_clip(a, b, C, 1.0, "tn", out_scale=1.0 / B, noise=zw, noise_scale=0.25)
    assert_close(out, ref_w, dtype, "weight")
    # the fallback (narrow schedule + column-sum kernel) agrees
    out2, _, _, bo2, bn2, _, untouched2 = run(_lib.WGRAD_NARROW, canary=True)
    assert not untouched2
    assert_close(bo2, ref_b, dtype, "bias (column-sum fallback)")
    assert_elementwise(bn2, bn.double().cpu().numpy(), dtype, "bias norms fused vs fallback")


def test_wgrad_bias_in_kernel_noise_matches_fallback():
    """The bias noise drawn in the wide kernel is the column-sum kernel's draw
    for the same key (Philox stream 0, element m), so the two paths agree."""
    import ctypes
    from flashdp4review_amd import _lib
    B, K, M, N = 8, 256, 3072, 768
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=22)
    outs = []
    for sp in ("wide", "unpaired", "narrow"):
        bo = torch.empty(M, dtype=torch.float32, device=DEV)
        core.wgrad_clip(a, b, 0.05, 1.0, out_dtype=torch.float32, bias_out=bo,
                        bias_scale=1.0 / (B * K), bias_noise_key=(777, 12), bias_noise_scale=0.5,
                        single_pass=sp, check=True)
        outs.append(bo)
    z = torch.from_numpy(PX.normals(M, 777, 12, 0)).float()
    ref, _, _ = O.colsum_clip(a, None, 0.05, 1.0, "frob", 1.0 / (B * K), z, 0.5)
    assert_close(outs[0], ref, torch.bfloat16, "bias with in-kernel noise (paired wide)")
    assert_close(outs[1], ref, torch.bfloat16, "bias with in-kernel noise (one-sample wide)")
    assert_close(outs[2], ref, torch.bfloat16, "bias with in-kernel noise (column sums)")


def test_wgrad_bias_argument_checks():
    import ctypes
    from flashdp4review_amd import _lib
    L = _lib.lib()
    a, b = make(2, 8, 16, 16, torch.bfloat16, "nn")
    out = torch.empty(16, 16, device=DEV)
    bo = torch.empty(16, device=DEV)
    bias = _lib.BiasOut(bo.data_ptr(), _lib.FDP_F32, 1.0, None, 0.0, None, None, None)

    def call(layout, flags=0, bias_p=ctypes.byref(bias)):
        return L.fdp_wgrad_bias_clip(a.data_ptr(), b.data_ptr(), 2, 8, 16, 16, 128, 16, 128, 16,
                                     layout, _lib.FDP_BF16, ctypes.c_float(1.0),
                                     ctypes.c_float(1.0), None, ctypes.c_float(1.0), None,
                                     ctypes.c_float(0.0), None, out.data_ptr(), 16, _lib.FDP_F32,
                                     None, None, flags, bias_p, None, 0, None)
    assert call(_lib.LAYOUT_NN) == 3          # the bias of a needs layout TN
    assert call(_lib.LAYOUT_TN, _lib.WGRAD_NOCLIP) == 3
    assert call(_lib.LAYOUT_TN, 0, None) == 3  # no bias description
    assert call(_lib.LAYOUT_TN) == 4           # workspace missing


def test_wgrad_prepared_call_matches_checked_call():
    """The first call of a signature (no stats, no injected noise, contiguous
    operands) is checked in full and recorded; later calls of the same
    signature go straight to the library.  Both give the same result, and a
    later call with another shape or bias length is checked again."""
    from flashdp4review_amd.core import wgrad as W
    B, K, M, N = 8, 256, 3072, 768
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=31)
    bo1 = torch.empty(M, dtype=torch.bfloat16, device=DEV)
    bo2 = torch.empty(M, dtype=torch.bfloat16, device=DEV)
    W._prepared.clear()
    kw = dict(out_scale=1.0 / B, noise_scale=0.3, noise_key=(9, 0), bias_scale=1.0 / (B * K),
              bias_noise_scale=0.3, bias_noise_key=(9, 10**6))
    first = W.wgrad_clip(a, b, 0.1, 1.0, bias_out=bo1, **kw)
    assert len(W._prepared) == 1
    second = W.wgrad_clip(a, b, 0.1, 1.0, bias_out=bo2, **kw)
    torch.cuda.synchronize()
    assert torch.equal(first, second) and torch.equal(bo1, bo2)
    # without noise the prepared call matches the oracle
    W.wgrad_clip(a, b, 0.1, 1.0, out_scale=1.0 / B, noise_scale=0.0)
    plain = W.wgrad_clip(a, b, 0.1, 1.0, out_scale=1.0 / B, noise_scale=0.0)
    ref, _, _ = O.wgrad_clip(a, b, 0.1, 1.0, "tn", out_scale=1.0 / B)
    assert_close(plain, ref, torch.bfloat16, "prepared call")
    with pytest.raises(ValueError):
        W.wgrad_clip(a, b, 0.1, 1.0, bias_out=torch.empty(M - 1, dtype=torch.bfloat16,
                                                          device=DEV), **kw)
    W._prepared.clear()


@pytest.mark.parametrize("which", ["a", "b"])
def test_wgrad_prepared_call_never_caches_a_copied_operand(which):
    """A call whose operand is a strided view (last axis not unit-stride) runs on a
    contiguous copy.  Such a call is not recorded for the prepared path, so a
    second call with an operand of the same shape and strides is checked and
    copied again instead of reaching the kernel as a raw pointer with the
    copy's strides.  Both calls match the oracle."""
    from flashdp4review_amd.core import wgrad as W
    B, K, M, N = 4, 96, 256, 192
    a, b = make(B, K, M, N, torch.bfloat16, "tn", seed=41)
    W._prepared.clear()
    for rep in range(2):
        if which == "a":
            base = a.transpose(1, 2).contiguous()   # [B, M, K]
            aa, bb = base.transpose(1, 2), b        # a view [B, K, M] with stride(2) = K
            assert aa.stride(2) != 1
        else:
            base = b.transpose(1, 2).contiguous()
            aa, bb = a, base.transpose(1, 2)
            assert bb.stride(2) != 1
        out = W.wgrad_clip(aa, bb, 0.05, 1.0, out_scale=1.0 / B)
        ref, _, _ = O.wgrad_clip(a, b, 0.05, 1.0, "tn", out_scale=1.0 / B)
        assert_close(out, ref, torch.bfloat16, f"strided view, call {rep}")
        assert len(W._prepared) == 0
    W._prepared.clear()


def test_dplinear_strided_input_twice():
    """DPLinear's backward with an input that is a transposed view, run twice:
    the second backward matches the oracle like the first."""
    from flashdp4review_amd import DPLinear
    from flashdp4review_amd.core import wgrad as W
    torch.manual_seed(7)
    W._prepared.clear()
    lin = DPLinear(192, 256, bias=True, C=0.05, noise_multiplier=0.0).to(DEV, torch.bfloat16)
    for rep in range(2):
        base = torch.randn(4, 192, 96, device=DEV).to(torch.bfloat16)
        x = base.transpose(1, 2).requires_grad_(True)    # [4, 96, 192], stride(2) = 96
        g = (torch.randn(4, 96, 256, device=DEV) * 0.02).to(torch.bfloat16)
        lin.weight.grad = lin.bias.grad = None
        lin(x).backward(g)
        ref = O.linear_backward(x.detach(), g, lin.weight.detach(), 0.05, 1.0)
        assert_close(lin.weight.grad, ref["dw"], torch.bfloat16, f"dW, backward {rep}")
        assert_close(lin.bias.grad, ref["db"], torch.bfloat16, f"db, backward {rep}")
    W._prepared.clear()
