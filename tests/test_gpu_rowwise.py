"""GPU parity of the bandwidth-bound kernels (fdp_colsum_clip, fdp_layernorm_fwd,
fdp_layernorm_bwd_clip) against the float64 oracle."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dp_clip as O
from tests._tol import assert_close, assert_elementwise

from flashdp4review_amd import core

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def randn(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(DEV)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", [(8, 1024, 768), (3, 7, 100), (2, 33, 2304), (5, 1, 9),
                                   (16, 64, 3072), (24, 16, 3000), (40, 8, 2050)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("norm", ["frob", "sum"])
def test_colsum_parity(shape, norm, dtype):
    """B*H up to 65536 takes the one-launch reduction, larger the two-launch one
    (the last two shapes; 2050 columns are not a multiple of 4)."""
    B, T, H = shape
    u = randn(shape, dtype, 1, 0.02)
    v = randn(shape, dtype, 2) if norm == "sum" else None
    _, n0, _ = O.colsum_clip(u, v, 1.0, 1.0, norm)
    C = float(np.median(n0))
    ref, nref, fref = O.colsum_clip(u, v, C, 1.0, norm, out_scale=1.0 / B)
    out, n, f = core.colsum_clip(u, v, C, 1.0, norm=norm, out_scale=1.0 / B,
                                 out_dtype=torch.float32, return_stats=True)
    assert_close(out, ref, dtype, "colsum")
    assert_elementwise(n, nref, dtype, "norms")
    assert_elementwise(f, fref, dtype, "factors")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_bias_ops(dtype):
    g = randn((4, 50, 96), dtype, 3, 0.05)
    g0 = g.clone()
    ref, _, _ = O.colsum_clip(g, None, 0.5, 1.0, "frob", out_scale=1.0 / 200)
    assert_close(core.linear_bias_grad_clip(g, 0.5, 1.0), ref, dtype, "linear_bias_grad_clip")
    assert torch.equal(g, g0), "grad_output must not be modified"
    assert_close(core.conv1d_bias_grad_clip(g, 0.5, 1.0), ref, dtype, "conv1d_bias_grad_clip")
    z = randn((96,), dtype, 4)
    out = core.colsum_clip(g, None, 0.5, 1.0, norm="frob", out_scale=1.0 / 200, noise=z,
                           noise_scale=0.25, out_dtype=torch.float32)
    ref, _, _ = O.colsum_clip(g, None, 0.5, 1.0, "frob", 1.0 / 200, z, 0.25)
    assert_close(out, ref, dtype, "bias + noise")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("H", [1024, 768, 2048, 100, 4096, 8, 4097, 8192, 12000, 16384,
                               16385, 20480, 32768])
def test_layernorm_fwd_parity(H, dtype):
    """Rows above 16384 elements are swept in segments (16385 is unaligned in
    every dtype and ends in a one-element segment)."""
    x = randn((3, 37, H), dtype, 5)
    w = randn((H,), dtype, 6)
    b = randn((H,), dtype, 7)
    y, mean, rstd = core.layernorm_fwd(x, w, b, 1e-5)
    yr, mr, rr = O.layernorm_fwd(x, w, b, 1e-5)
    assert_close(y, yr, dtype, "y")
    assert_close(mean.reshape(mr.shape), mr, dtype, "mean")
    assert_elementwise(rstd.reshape(rr.shape), rr, dtype, "rstd")
    # torch's own layer_norm on the same inputs (fp32 math)
    yt = F.layer_norm(x.float(), (H,), w.float(), b.float(), 1e-5)
    assert_close(y, yt.double().cpu().numpy(), dtype, "y vs torch")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", [(16, 1024, 1024), (4, 33, 768), (2, 5, 100), (3, 64, 4096),
                                   (1, 1, 64), (20, 8, 4096), (70, 3, 1000), (3, 9, 1001),
                                   (4, 128, 8192), (2, 40, 16384), (3, 17, 5000), (1, 3, 4100),
                                   (4, 1024, 512), (2, 9, 32768), (3, 17, 16385), (5, 8, 20000),
                                   (2, 70, 40000), (8, 1024, 2048), (270, 2, 64), (300, 2, 256)],
                         ids=lambda s: "x".join(map(str, s)))
def test_layernorm_bwd_parity(shape, dtype):
    """Paths: B*H <= 65536 with at most 16 row chunks per sample runs in one
    launch (cfg4, the small shapes, 270x2x64 with more workgroups than CUs);
    4x1024x512 and 8x1024x2048 (cfg5's LayerNorm; 32 chunks per sample) run
    the rows, then the one-workgroup-per-stream reduction; 20x8x4096,
    70x3x1000 and 300x2x256 (B*H > 65536) the rows, then the two reduction
    kernels.  Rows of
    1025..4096 elements share a row among 2 or 4 wavefronts; above 4096 among
    16 (8192, 16384, 5000, 4100; 5000 and 4100 leave threads without columns,
    4100 is also unaligned in 16-bit).  Longer rows take the per-row statistics
    launch, then 2048-column blocks, then the reduction: one launch for
    2x9x32768 and 3x17x16385 (unaligned), two for 5x8x20000 and 2x70x40000
    (three chunks of rows per sample)."""
    B, T, H = shape
    x = randn(shape, dtype, 8)
    w = randn((H,), dtype, 9)
    g = randn(shape, dtype, 10, 0.01)
    _, mean, rstd = core.layernorm_fwd(x, w, None, 1e-5)
    r0 = O.layernorm_bwd_clip(g, x, w, 1e-5, C=1.0, mean=mean, rstd=rstd)
    C = float(np.median(r0["norms_w"]))
    zw = randn((H,), dtype, 11)
    zb = randn((H,), dtype, 12)
    std = 0.7 / np.sqrt(B)
    dx, dw, db, norms, fac = core.layernorm_bwd_clip(
        g, x, w, mean, rstd, C, 1.0, noise_w=zw, noise_b=zb, noise_scale=std,
        param_dtype=torch.float32, return_stats=True)
    ref = O.layernorm_bwd_clip(g, x, w, 1e-5, C=C, noise_multiplier=0.7, z_w=zw, z_b=zb,
                               mean=mean, rstd=rstd)
    tag = f"cfg4 LN bwd ({dtype})" if shape == (16, 1024, 1024) else None
    assert_close(dx, ref["dx"], dtype, "dx", margin=tag and tag + ": dx")
    assert_close(dw, ref["dw"], dtype, "dgamma", margin=tag and tag + ": dgamma")
    assert_close(db, ref["db"], dtype, "dbeta", margin=tag and tag + ": dbeta")
    assert_elementwise(norms[:B], ref["norms_w"], dtype, "norms gamma")
    assert_elementwise(norms[B:], ref["norms_b"], dtype, "norms beta")
    assert_elementwise(fac[:B], ref["fac_w"], dtype, "factors gamma")
    assert_elementwise(fac[B:], ref["fac_b"], dtype, "factors beta")


@pytest.mark.parametrize("H", [20480, 40000])
@pytest.mark.parametrize("params", ["fp32", "misaligned"])
def test_layernorm_long_rows_parameter_layouts(H, params):
    """Long bf16 rows with fp32 gamma/beta (the autocast layout: 16-byte loads of
    two 4-element halves) or with gamma/beta starting 2 bytes past an aligned
    address (element loads); forward and backward against the oracle."""
    B, T, dtype = 2, 12, torch.bfloat16
    x = randn((B, T, H), dtype, 31)
    g = randn((B, T, H), dtype, 32, 0.01)
    if params == "fp32":
        w, b = randn((H,), torch.float32, 33), randn((H,), torch.float32, 34)
    else:
        w = randn((H + 1,), dtype, 33)[1:]
        b = randn((H + 1,), dtype, 34)[1:]
        assert w.data_ptr() % 16 != 0 and b.data_ptr() % 16 != 0
    y, mean, rstd = core.layernorm_fwd(x, w, b, 1e-5)
    yr, mr, rr = O.layernorm_fwd(x, w, b, 1e-5)
    assert_close(y, yr, dtype, "y")
    assert_elementwise(rstd.reshape(rr.shape), rr, dtype, "rstd")
    r0 = O.layernorm_bwd_clip(g, x, w, 1e-5, C=1.0, mean=mean, rstd=rstd)
    C = float(np.median(r0["norms_w"]))
    dx, dw, db, norms, fac = core.layernorm_bwd_clip(g, x, w, mean, rstd, C, 1.0,
                                                     noise_scale=0.0, return_stats=True)
    ref = O.layernorm_bwd_clip(g, x, w, 1e-5, C=C, mean=mean, rstd=rstd)
    assert_close(dx, ref["dx"], dtype, "dx")
    assert_close(dw, ref["dw"], dtype, "dgamma")
    assert_close(db, ref["db"], dtype, "dbeta")
    assert_elementwise(norms[:B], ref["norms_w"], dtype, "norms gamma")
    assert_elementwise(fac[B:], ref["fac_b"], dtype, "factors beta")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("shape", [(1, 7, 16391), (3, 5, 24577), (2, 6, 32776), (2, 3, 49157),
                                   (1, 4, 65536), (1, 3, 81921)],
                         ids=lambda s: "x".join(map(str, s)))
def test_layernorm_long_row_lengths(shape, dtype):
    """Row lengths around the long-row paths' boundaries: last segments of 1, 7 or
    8192 elements, rows held in registers (up to 32768) and swept three times
    (longer), odd lengths that leave 16-bit rows unaligned, and 2048-column
    blocks ending mid-block; forward and backward against the oracle."""
    B, T, H = shape
    x = randn(shape, dtype, 41)
    g = randn(shape, dtype, 42, 0.01)
    w, b = randn((H,), dtype, 43), randn((H,), dtype, 44)
    y, mean, rstd = core.layernorm_fwd(x, w, b, 1e-5)
    yr, _, rr = O.layernorm_fwd(x, w, b, 1e-5)
    assert_close(y, yr, dtype, "y")
    assert_elementwise(rstd.reshape(rr.shape), rr, dtype, "rstd")
    r0 = O.layernorm_bwd_clip(g, x, w, 1e-5, C=1.0, mean=mean, rstd=rstd)
    C = float(np.median(r0["norms_w"]))
    zw = randn((H,), dtype, 45)
    dx, dw, db, norms, fac = core.layernorm_bwd_clip(g, x, w, mean, rstd, C, 1.0, noise_w=zw,
                                                     noise_scale=0.3, param_dtype=torch.float32,
                                                     return_stats=True)
    ref = O.layernorm_bwd_clip(g, x, w, 1e-5, C=C, noise_multiplier=0.3 * np.sqrt(B), z_w=zw,
                               z_b=torch.zeros(H), mean=mean, rstd=rstd)
    assert_close(dx, ref["dx"], dtype, "dx")
    assert_close(dw, ref["dw"], dtype, "dgamma")
    assert_close(db, ref["db"], dtype, "dbeta")
    assert_elementwise(norms[:B], ref["norms_w"], dtype, "norms gamma")
    assert_elementwise(norms[B:], ref["norms_b"], dtype, "norms beta")
    assert_elementwise(fac[:B], ref["fac_w"], dtype, "factors gamma")


@pytest.mark.parametrize("shape", [(2, 1, 1 << 20), (1, 2, 1000003)],
                         ids=lambda s: "x".join(map(str, s)))
def test_layernorm_million_element_rows_fp32(shape):
    """Rows of about 10^6 elements in fp32 (each thread adds about H/1024 values
    in order before the fixed-order block sum): statistics, forward and
    backward within the fp32 bar, with the measured margins reported."""
    B, T, H = shape
    dtype = torch.float32
    x = randn(shape, dtype, 51)
    g = randn(shape, dtype, 52, 0.01)
    w, b = randn((H,), dtype, 53), randn((H,), dtype, 54)
    y, mean, rstd = core.layernorm_fwd(x, w, b, 1e-5)
    yr, _, rr = O.layernorm_fwd(x, w, b, 1e-5)  # (the mean, near 0, is checked through y)
    assert_elementwise(rstd.reshape(rr.shape), rr, dtype, "rstd",
                       margin=f"LN fp32 rows of {H}: rstd")
    assert_close(y, yr, dtype, "y", margin=f"LN fp32 rows of {H}: y")
    dx, dw, db = core.layernorm_bwd_clip(g, x, w, mean, rstd, 1e30, 1.0,
                                         param_dtype=torch.float32)
    ref = O.layernorm_bwd_clip(g, x, w, 1e-5, C=1e30)  # the oracle's own statistics
    assert_close(dx, ref["dx"], dtype, "dx", margin=f"LN fp32 rows of {H}: dx")
    assert_close(dw, ref["dw"], dtype, "dgamma", margin=f"LN fp32 rows of {H}: dgamma")
    assert_close(db, ref["db"], dtype, "dbeta")


@pytest.mark.parametrize("shape", [(2, 0, 64), (16, 0, 1024), (2, 0, 20000)],
                         ids=lambda s: "x".join(map(str, s)))
def test_layernorm_bwd_empty_rows(shape):
    """T = 0: no row is read, the per-sample sums are zero, so the clip factors
    are min(clamp, C / 1e-10) = clamp and dgamma / dbeta are the noise alone."""
    B, T, H = shape
    dtype = torch.bfloat16
    x = torch.zeros(shape, dtype=dtype, device=DEV)
    g = torch.zeros(shape, dtype=dtype, device=DEV)
    w = randn((H,), dtype, 13)
    mean = torch.zeros((B, T), dtype=torch.float32, device=DEV)
    rstd = torch.ones((B, T), dtype=torch.float32, device=DEV)
    zw, zb = randn((H,), dtype, 14), randn((H,), dtype, 15)
    dx, dw, db, norms, fac = core.layernorm_bwd_clip(
        g, x, w, mean, rstd, 1.0, 1.0, noise_w=zw, noise_b=zb, noise_scale=0.5,
        param_dtype=torch.float32, return_stats=True)
    ref = O.layernorm_bwd_clip(g, x, w, 1e-5, C=1.0, noise_multiplier=0.5 * np.sqrt(B),
                               z_w=zw, z_b=zb, mean=mean, rstd=rstd)
    assert dx.numel() == 0
    assert_close(dw, ref["dw"], dtype, "dgamma")
    assert_close(db, ref["db"], dtype, "dbeta")
    assert torch.all(norms == 0) and torch.all(fac == 1.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_layernorm_no_clip_matches_torch_autograd(dtype):
    """C -> inf: dgamma/dbeta are torch autograd's divided by B, dx is autograd's."""
    B, T, H = 4, 40, 512
    x = randn((B, T, H), dtype, 13)
    w = randn((H,), dtype, 14)
    b = randn((H,), dtype, 15)
    g = randn((B, T, H), dtype, 16, 0.1)
    y, mean, rstd = core.layernorm_fwd(x, w, b, 1e-5)
    dx, dw, db = core.layernorm_bwd_clip(g, x, w, mean, rstd, 1e30, 1.0, param_dtype=torch.float32)
    xr = x.float().cpu().double().requires_grad_(True)
    wr = w.float().cpu().double().requires_grad_(True)
    br = b.float().cpu().double().requires_grad_(True)
    gx, gw, gb = torch.autograd.grad(F.layer_norm(xr, (H,), wr, br, 1e-5), (xr, wr, br),
                                     g.cpu().double())
    assert_close(dx, gx.numpy(), dtype, "dx")
    assert_close(dw, gw.numpy() / B, dtype, "dgamma")
    assert_close(db, gb.numpy() / B, dtype, "dbeta")


def test_layernorm_operator_api():
    dtype = torch.bfloat16
    B, T, H = 4, 32, 256
    x = randn((B, T, H), dtype, 17)
    w = randn((H,), dtype, 18)
    b = randn((H,), dtype, 19)
    g = randn((B, T, H), dtype, 20, 0.05)
    y, buf, args = core.layernorm_fwd_fused(x, w, b, 1e-5)
    assert args["BLOCK_SIZE"] == 256 and set(buf) == {"mean", "rstd"}
    ca = torch.tensor([0.5, 1.0], device=DEV)
    dx, dw_, db_, a2 = core.layernorm_bwd_clip_fused(g, x, w, b, ca, buf, args)
    dw, db = core.layernorm_dwdb_fused(w, b, dw_, db_, a2)
    ref = O.layernorm_bwd_clip(g, x, w, 1e-5, C=0.5, mean=buf["mean"], rstd=buf["rstd"])
    assert dw.dtype == dtype and dw.shape == (H,)
    assert_close(dx, ref["dx"], dtype, "dx")
    assert_close(dw, ref["dw"], dtype, "dw")
    assert_close(db, ref["db"], dtype, "db")
    # per-sample clip ops on x_hat (layernorm_clip.py:163-198)
    xhat, _, _ = O.layernorm_fwd(x, None, None, 1e-5)
    xh = torch.tensor(xhat, dtype=dtype, device=DEV)
    r = core.layernorm_dw_clip(xh, g, w, torch.tensor([0.5]), torch.tensor([1.0]))
    assert r.shape == (1, 1, H)
    ref_dw, _, _ = O.colsum_clip(g, xh, 0.5, 1.0, "sum", out_scale=1.0 / B)
    assert_close(r.reshape(-1), ref_dw, dtype, "layernorm_dw_clip")
    r = core.layernorm_db_clip(g, b, 0.5, 1.0)
    ref_db, _, _ = O.colsum_clip(g, None, 0.5, 1.0, "sum", out_scale=1.0 / B)
    assert_close(r.reshape(-1), ref_db, dtype, "layernorm_db_clip")


def test_layernorm_bwd_deterministic():
    x = randn((16, 256, 1024), torch.bfloat16, 21)
    g = randn((16, 256, 1024), torch.bfloat16, 22, 0.01)
    _, mean, rstd = core.layernorm_fwd(x, None, None, 1e-5)
    a = core.layernorm_bwd_clip(g, x, None, mean, rstd, 1.0, 1.0)
    b = core.layernorm_bwd_clip(g, x, None, mean, rstd, 1.0, 1.0)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_colsum_and_layernorm_in_kernel_noise():
    """Bias / LayerNorm grads with the in-kernel draw: colsum output stream 0,
    LayerNorm dgamma stream 0 and dbeta stream 1 of the same key."""
    from oracle import philox as PX
    key = (0x0123456789ABCDEF, 99)
    g = randn((4, 33, 770), torch.bfloat16, 30, 0.01)
    o0 = core.colsum_clip(g, None, 0.5, 1.0, norm="frob", out_scale=0.1, noise_scale=0.5,
                          out_dtype=torch.float32)
    o1 = core.colsum_clip(g, None, 0.5, 1.0, norm="frob", out_scale=0.1, noise_scale=0.5,
                          noise_key=key, out_dtype=torch.float32)
    z = PX.normals(770, *key)
    assert np.max(np.abs((o1 - o0).double().cpu().numpy() / 0.5 - z)) < 1e-4
    x = randn((3, 40, 1024), torch.bfloat16, 31)
    dy = randn((3, 40, 1024), torch.bfloat16, 32, 0.01)
    _, mean, rstd = core.layernorm_fwd(x, None, None, 1e-5)
    _, w0, b0 = core.layernorm_bwd_clip(dy, x, None, mean, rstd, 1.0, 1.0, noise_scale=0.3,
                                        param_dtype=torch.float32)
    _, w1, b1 = core.layernorm_bwd_clip(dy, x, None, mean, rstd, 1.0, 1.0, noise_scale=0.3,
                                        noise_key=key, param_dtype=torch.float32)
    zw = PX.normals(1024, *key, stream=0)
    zb = PX.normals(1024, *key, stream=1)
    assert np.max(np.abs((w1 - w0).double().cpu().numpy() / 0.3 - zw)) < 1e-4
    assert np.max(np.abs((b1 - b0).double().cpu().numpy() / 0.3 - zb)) < 1e-4
