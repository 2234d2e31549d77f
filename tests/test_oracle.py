"""Pins the float64 oracle (oracle/dp_clip.py) with independent formulations:
closed forms, brute-force loops, algebraic identities and torch autograd.
None of these re-types the oracle's own einsum formula."""
import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dp_clip as O
from oracle import torch_ref as R

rng = np.random.default_rng(0)


def brute_G(a, b, layout):
    """Per-sample product by explicit loops over (b, m, n, k)."""
    if layout == "tn":
        B, K, M = a.shape
        N = b.shape[2]
        G = np.zeros((B, M, N))
        for s, m, n in itertools.product(range(B), range(M), range(N)):
            acc = 0.0
            for k in range(K):
                acc += a[s, k, m] * b[s, k, n]
            G[s, m, n] = acc
    else:
        B, M, K = a.shape
        N = b.shape[2]
        G = np.zeros((B, M, N))
        for s, m, n in itertools.product(range(B), range(M), range(N)):
            acc = 0.0
            for k in range(K):
                acc += a[s, m, k] * b[s, k, n]
            G[s, m, n] = acc
    return G


def test_clip_factor_closed_forms():
    assert O.clip_factor(0.0, 1.0, 1.0) == 1.0            # tiny norm -> clamp
    assert O.clip_factor(4.0, 2.0, 1.0) == pytest.approx(0.5)
    assert O.clip_factor(1e30, 1.0, 1.0) == pytest.approx(1e-30)
    assert O.clip_factor(2.0, 1.0, 0.25) == 0.25           # clamp wins
    assert O.clip_factor(3.0, 0.0, 1.0) == 0.0             # C = 0
    assert O.clip_factor(1.0, 1.0, 1.0) == pytest.approx(1.0 / (1.0 + 1e-10))


@pytest.mark.parametrize("layout", ["tn", "nn"])
def test_wgrad_brute_force(layout):
    B, K, M, N = 3, 5, 4, 6
    a = rng.standard_normal((B, K, M) if layout == "tn" else (B, M, K))
    b = rng.standard_normal((B, K, N))
    G = brute_G(a, b, layout)
    C = 2.0
    out, norms, fac = O.wgrad_clip(a, b, C, 1.0, layout)
    ref_norms = np.array([math.sqrt(sum(v * v for v in G[s].ravel())) for s in range(B)])
    ref_fac = np.array([min(1.0, C / (n + 1e-10)) for n in ref_norms])
    ref = sum(ref_fac[s] * G[s] for s in range(B))
    np.testing.assert_allclose(norms, ref_norms, rtol=1e-12)
    np.testing.assert_allclose(fac, ref_fac, rtol=1e-12)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_wgrad_gram_identity():
    """||a^T b||_F^2 = sum_{t,s} (a_t . a_s)(b_t . b_s) (ghost-norm identity)."""
    B, T, M, N = 4, 7, 9, 5
    a = rng.standard_normal((B, T, M))
    b = rng.standard_normal((B, T, N))
    _, norms, _ = O.wgrad_clip(a, b, 1.0, 1.0, "tn")
    for s in range(B):
        ga = a[s] @ a[s].T
        gb = b[s] @ b[s].T
        assert norms[s] ** 2 == pytest.approx(float((ga * gb).sum()), rel=1e-10)


def test_wgrad_single_gemm_identity():
    """sum_b c_b a_b^T b_b = A^T diag(c) B with A, B the batch-stacked operands."""
    B, T, M, N = 5, 6, 7, 3
    a = rng.standard_normal((B, T, M))
    b = rng.standard_normal((B, T, N))
    out, _, fac = O.wgrad_clip(a, b, 0.5, 1.0, "tn")
    A = a.reshape(B * T, M)
    Bm = b.reshape(B * T, N)
    c = np.repeat(fac, T)
    np.testing.assert_allclose(out, A.T @ (c[:, None] * Bm), rtol=1e-10, atol=1e-12)


def test_linear_no_clip_matches_autograd():
    """C -> inf: every c_b = clamp = 1 and dW is nn.Linear's weight grad / B."""
    torch.manual_seed(0)
    B, T, I, Oo = 3, 5, 6, 4
    x = torch.randn(B, T, I, dtype=torch.float64)
    lin = torch.nn.Linear(I, Oo).double()
    g = torch.randn(B, T, Oo, dtype=torch.float64)
    y = lin(x)
    y.backward(g)
    r = O.linear_backward(x, g, lin.weight.detach(), C=1e30)
    np.testing.assert_allclose(r["dw"], lin.weight.grad.numpy() / B, rtol=1e-12)
    np.testing.assert_allclose(r["db"], lin.bias.grad.numpy() / (B * T), rtol=1e-12)
    xr = x.clone().requires_grad_(True)
    torch.autograd.grad(lin(xr), xr, g)
    (dx,) = torch.autograd.grad(lin(xr), xr, g)
    np.testing.assert_allclose(r["dx"], dx.numpy(), rtol=1e-12)


def test_clipped_terms_have_norm_C():
    """||G_b|| >> C: every clipped term c_b G_b has Frobenius norm exactly C*clamp."""
    B, T, M, N = 4, 8, 5, 6
    a = 50 * rng.standard_normal((B, T, M))
    b = 50 * rng.standard_normal((B, T, N))
    C = 0.3
    _, norms, fac = O.wgrad_clip(a, b, C, 1.0, "tn")
    assert np.all(norms > 100 * C)
    np.testing.assert_allclose(fac * norms, C, rtol=1e-9)
    # and with a single sample, the output norm is C
    out, _, _ = O.wgrad_clip(a[:1], b[:1], C, 1.0, "tn")
    assert np.linalg.norm(out) == pytest.approx(C, rel=1e-9)


def test_special_cases():
    B, T, M, N = 3, 4, 5, 6
    a = rng.standard_normal((B, T, M))
    b = rng.standard_normal((B, T, N))
    out0, _, fac0 = O.wgrad_clip(a, b, 0.0, 1.0, "tn")
    assert np.all(fac0 == 0) and np.all(out0 == 0)
    # B = 1 with ||G|| <= C -> unclipped
    out1, norms1, _ = O.wgrad_clip(a[:1], b[:1], 1e6, 1.0, "tn")
    np.testing.assert_allclose(out1, a[0].T @ b[0], rtol=1e-12)
    # T = 1 -> rank-1 outer products, ||a (x) b|| = ||a|| ||b||
    _, n, _ = O.wgrad_clip(a[:, :1], b[:, :1], 1.0, 1.0, "tn")
    np.testing.assert_allclose(n, np.linalg.norm(a[:, 0], axis=1) * np.linalg.norm(b[:, 0], axis=1),
                               rtol=1e-12)


def test_invariants():
    B, T, I, Oo = 4, 6, 5, 7
    x = rng.standard_normal((B, T, I))
    g = rng.standard_normal((B, T, Oo))
    W = rng.standard_normal((Oo, I))
    perm = rng.permutation(B)
    o1, _, _ = O.wgrad_clip(g, x, 1.0, 1.0, "tn")
    o2, _, _ = O.wgrad_clip(g[perm], x[perm], 1.0, 1.0, "tn")
    np.testing.assert_allclose(o1, o2, rtol=1e-12)
    lin = O.linear_backward(x, g, W, 0.7, 1.0)
    conv = O.conv1d_backward(x, g, W.T, 0.7, 1.0)
    np.testing.assert_allclose(conv["dw"], lin["dw"].T, rtol=1e-12)
    np.testing.assert_allclose(conv["db"], lin["db"], rtol=1e-12)
    np.testing.assert_allclose(conv["dx"], lin["dx"], rtol=1e-12)
    # bmm_clip(x^T, g) == bmtm_clip(x, g)
    bm, _, _ = O.wgrad_clip(np.transpose(x, (0, 2, 1)), g, 0.7, 1.0, "nn")
    bt, _, _ = O.wgrad_clip(x, g, 0.7, 1.0, "tn")
    np.testing.assert_allclose(bm, bt, rtol=1e-12)


def test_mm_clip_rank_one():
    M, K, N = 4, 6, 3
    m1 = rng.standard_normal((M, K))
    m2 = rng.standard_normal((K, N))
    C = 1.5
    ref = np.zeros((M, N))
    for k in range(K):
        outer = np.outer(m1[:, k], m2[k, :])
        n = np.linalg.norm(m1[:, k]) * np.linalg.norm(m2[k, :])
        ref += min(1.0, C / (n + 1e-10)) * outer
    np.testing.assert_allclose(O.mm_clip(m1, m2, C, 1.0), ref, rtol=1e-12)


def test_colsum_brute_force():
    B, T, H = 3, 5, 4
    u = rng.standard_normal((B, T, H))
    v = rng.standard_normal((B, T, H))
    C = 1.1
    out, norms, fac = O.colsum_clip(u, v, C, 1.0, "sum", out_scale=0.25)
    ref = np.zeros(H)
    for s in range(B):
        S = np.array([sum(u[s, t, h] * v[s, t, h] for t in range(T)) for h in range(H)])
        n = math.sqrt(sum(x * x for x in S))
        ref += min(1.0, C / (n + 1e-10)) * S
    np.testing.assert_allclose(out, 0.25 * ref, rtol=1e-12)
    out, norms, _ = O.colsum_clip(u, None, C, 1.0, "frob")
    for s in range(B):
        assert norms[s] == pytest.approx(math.sqrt(sum(x * x for x in u[s].ravel())), rel=1e-12)


def test_layernorm_fwd_matches_torch():
    torch.manual_seed(1)
    x = torch.randn(3, 5, 16, dtype=torch.float64)
    w = torch.randn(16, dtype=torch.float64)
    b = torch.randn(16, dtype=torch.float64)
    y, mean, rstd = O.layernorm_fwd(x, w, b, 1e-5)
    np.testing.assert_allclose(y, F.layer_norm(x, (16,), w, b, 1e-5).numpy(), rtol=1e-10,
                               atol=1e-12)


def test_layernorm_bwd_no_clip_matches_autograd():
    """C -> inf: dgamma/dbeta are torch autograd's / B and dx is autograd's dx."""
    torch.manual_seed(2)
    B, T, H = 3, 6, 16
    x = torch.randn(B, T, H, dtype=torch.float64, requires_grad=True)
    w = torch.randn(H, dtype=torch.float64, requires_grad=True)
    b = torch.randn(H, dtype=torch.float64, requires_grad=True)
    g = torch.randn(B, T, H, dtype=torch.float64)
    dx, dw, db = torch.autograd.grad(F.layer_norm(x, (H,), w, b, 1e-5), (x, w, b), g)
    r = O.layernorm_bwd_clip(g, x.detach(), w.detach(), 1e-5, C=1e30)
    np.testing.assert_allclose(r["dx"], dx.numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(r["dw"], dw.numpy() / B, rtol=1e-10)
    np.testing.assert_allclose(r["db"], db.numpy() / B, rtol=1e-10)


def test_layernorm_bwd_clipped_norms():
    B, T, H = 4, 5, 8
    x = rng.standard_normal((B, T, H))
    g = 3 * rng.standard_normal((B, T, H))
    r = O.layernorm_bwd_clip(g, x, None, 1e-5, C=0.5)
    _, mean, rstd = O.layernorm_fwd(x)
    xhat = (x - mean[..., None]) * rstd[..., None]
    for s in range(B):
        P = (g[s] * xhat[s]).sum(0)
        Q = g[s].sum(0)
        assert r["norms_w"][s] == pytest.approx(np.linalg.norm(P), rel=1e-12)
        assert r["norms_b"][s] == pytest.approx(np.linalg.norm(Q), rel=1e-12)


def test_noise_placement():
    """Noise is added after the 1/B average with std sigma/sqrt(B)."""
    B, T, I, Oo = 4, 3, 5, 2
    x = rng.standard_normal((B, T, I))
    g = rng.standard_normal((B, T, Oo))
    W = rng.standard_normal((Oo, I))
    z = rng.standard_normal((Oo, I))
    r0 = O.linear_backward(x, g, W, 1.0, 1.0, 0.0)
    r1 = O.linear_backward(x, g, W, 1.0, 1.0, 2.0, z_w=z)
    np.testing.assert_allclose(r1["dw"] - r0["dw"], 2.0 / math.sqrt(B) * z, rtol=1e-12)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_torch_reference_sequence_matches_oracle(dtype):
    """oracle/torch_ref.py (the reference's torch op sequence, the CPU baseline)
    agrees with the float64 oracle."""
    torch.manual_seed(3)
    B, T, I, Oo = 3, 7, 6, 5
    x = torch.randn(B, T, I, dtype=dtype)
    g = torch.randn(B, T, Oo, dtype=dtype) * 0.5
    W = torch.randn(Oo, I, dtype=dtype)
    # clip_args is a float32 tensor in the reference (torch.Tensor([C, clamp])), so
    # even the float64 sequence carries float32 rounding of C.
    tol = 1e-7 if dtype == torch.float64 else 1e-5
    dw = R.linear_weight_backward(x, g, 0.8, 1.0, 0.0)
    db = R.linear_bias_grad_clip(g.clone(), 0.8, 1.0)
    r = O.linear_backward(x, g, W, 0.8, 1.0)
    assert O.rel_err(dw, r["dw"]) < tol
    assert O.rel_err(db, r["db"]) < tol
    xl = torch.randn(B, T, 8, dtype=dtype)
    gl = torch.randn(B, T, 8, dtype=dtype)
    wl = torch.randn(8, dtype=dtype)
    dx, dwl, dbl = R.layernorm_backward(xl, wl, gl, 1e-5, 0.6, 1.0, 0.0)
    rl = O.layernorm_bwd_clip(gl, xl, wl, 1e-5, C=0.6)
    assert O.rel_err(dx, rl["dx"]) < tol * 10
    assert O.rel_err(dwl, rl["dw"]) < tol * 10
    assert O.rel_err(dbl, rl["db"]) < tol * 10


def test_reference_bias_clip_mutates_input():
    """The reference's bias clip scales grad_output in place (linear_clip.py:118-121);
    the restated sequence reproduces that, the product path must not (tests/test_gpu_*)."""
    g = torch.randn(2, 3, 4) * 10
    g0 = g.clone()
    R.linear_bias_grad_clip(g, 1.0, 1.0)
    assert not torch.equal(g, g0)


# ---------------------------------------------------------------- noise stream
from oracle import philox as PX  # noqa: E402


@pytest.mark.parametrize("ctr,key,expect", [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox_known_answers(ctr, key, expect):
    """Philox4x32-10 against the Random123 known-answer vectors."""
    got = PX.philox4x32_10(np.array([ctr], dtype=np.uint32), np.array(key, dtype=np.uint32))
    assert tuple(int(v) for v in got[0]) == expect


def test_noise_stream_statistics():
    """Moments and tails of N(0,1), no correlation between neighbours or streams,
    and a different seed / offset / stream gives a different draw."""
    n = 1 << 18
    z = PX.normals(n, seed=0x123456789ABCDEF, offset=7)
    se = 1 / np.sqrt(n)
    assert abs(z.mean()) < 5 * se
    assert abs(z.std() - 1) < 5 * se
    assert abs(np.mean(z ** 3)) < 5 * np.sqrt(15 / n)      # skew 0
    assert abs(np.mean(z ** 4) - 3) < 5 * np.sqrt(96 / n)  # kurtosis 3
    assert abs(np.mean(np.abs(z) > 3) - 0.0026998) < 5 * np.sqrt(0.0027 / n)
    for lag in (1, 2, 3, 4):
        assert abs(np.corrcoef(z[:-lag], z[lag:])[0, 1]) < 5 * se
    z1 = PX.normals(n, seed=0x123456789ABCDEF, offset=7, stream=1)
    assert abs(np.corrcoef(z, z1)[0, 1]) < 5 * se
    # the same key reproduces; offsets address the stream block-wise
    assert np.array_equal(z, PX.normals(n, seed=0x123456789ABCDEF, offset=7))
    assert np.array_equal(z[8:16], PX.normals(8, seed=0x123456789ABCDEF, offset=9))
    assert not np.allclose(z[:64], PX.normals(64, seed=0x123456789ABCDEE, offset=7))


def test_noise_radius_uses_the_whole_word():
    """The Box-Muller radius comes from the 32-bit uniform (w + 0.5) / 2^32: the
    largest radius (w = 0) is sqrt(-2 ln 2^-33) = sqrt(66 ln 2) = 6.7636, so the
    sampler covers the normal's tail up to 6.76 sigma (a 24-bit uniform would
    stop at 5.89).  Checked on the counter block whose radius word is smallest
    among 2^16 blocks, against the closed form of its own word."""
    nblk = 1 << 16
    ctr = np.zeros((nblk, 4), dtype=np.uint32)
    ctr[:, 0] = np.arange(nblk, dtype=np.uint32)
    w = PX.philox4x32_10(ctr, np.array([5, 6], dtype=np.uint32))
    i = int(np.argmin(w[:, 0]))
    z = PX.normals(4 * nblk, seed=5 | (6 << 32))[4 * i:4 * i + 2]
    r_expect = np.sqrt(-2.0 * np.log((float(w[i, 0]) + 0.5) / 2.0**32))
    assert np.isclose(np.hypot(z[0], z[1]), r_expect, rtol=1e-12, atol=0)
    # (the 24-bit radius of the same word differs at about 1e-3 relative)
    r24 = np.sqrt(-2.0 * np.log((float(w[i, 0] >> 8) + 0.5) / 2.0**24))
    assert abs(r24 - r_expect) / r_expect > 1e-5
    r_max = np.sqrt(-2.0 * np.log(0.5 / 2.0**32))
    assert np.isclose(r_max, np.sqrt(66 * np.log(2.0))) and r_max > 6.76
    assert np.sqrt(-2.0 * np.log(0.5 / 2.0**24)) < 5.89
