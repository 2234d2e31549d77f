"""Parity tolerances of the hot path: max|y - y_ref| / max|y_ref| per tensor,
1e-5 for fp32 and 2e-2 for bf16/fp16, y_ref = float64 oracle on the same
dtype-rounded inputs."""
import numpy as np
import torch

from oracle.dp_clip import rel_err

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}

# (name, measured rel err, tolerance) of the checks that report their margin;
# tests/conftest.py prints them at the end of the run.
MARGINS = []


def report(name, err, tol):
    MARGINS.append((str(name), float(err), float(tol)))


def assert_close(y, y_ref, dtype, what="", margin=None):
    """max|y - y_ref| / max|y_ref| <= TOL[dtype]; ``margin`` names the check in the
    end-of-run margin report."""
    e = rel_err(y, y_ref)
    tol = TOL[dtype]
    if margin is not None:
        report(margin, e, tol)
    assert e <= tol, f"{what}: rel err {e:.3e} > {tol:.0e} ({dtype})"
    return e


def assert_elementwise(y, y_ref, dtype, what="", margin=None):
    """Element-wise relative error (norms, clip factors)."""
    y = np.asarray(y.detach().double().cpu().numpy() if hasattr(y, "detach") else y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    den = np.maximum(np.abs(y_ref), 1e-30)
    e = float(np.max(np.abs(y - y_ref) / den)) if y_ref.size else 0.0
    if margin is not None:
        report(margin, e, TOL[dtype])
    assert e <= TOL[dtype], f"{what}: elementwise rel err {e:.3e} > {TOL[dtype]:.0e}"
    return e
