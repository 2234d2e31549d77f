"""C ABI of libflashdp_hip.so: the library loads, exports exactly what
include/flashdp_hip.h declares with the argument counts the ctypes binding uses,
and argument validation returns the documented status codes.  No kernel is
launched here (validation happens before any launch)."""
import ctypes
import os
import re

import pytest

from flashdp4review_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "flashdp_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"(?:const\s+char\s*\*|int)\s+(fdp_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_library_loads():
    L = _lib.lib()
    assert L.fdp_version() == 200
    assert L.fdp_strerror(0) == b"ok"
    assert L.fdp_strerror(4).startswith(b"workspace")


def test_header_matches_exports_and_binding():
    decl = header_functions()
    assert decl, "no declarations parsed"
    assert set(decl) == set(_lib.SIGNATURES), (set(decl) ^ set(_lib.SIGNATURES))
    L = _lib.lib()
    for name, nargs in decl.items():
        fn = getattr(L, name)  # raises AttributeError if not exported
        assert fn is not None
        assert len(_lib.SIGNATURES[name][1]) == nargs, name


def _wgrad(**kw):
    args = dict(a=1, b=1, B=2, K=4, M=8, N=8, sab=32, lda=8, sbb=32, ldb=8, layout=0, dtype=2,
                C=1.0, clamp=1.0, cad=None, out_scale=1.0, noise=None, noise_scale=0.0, key=None,
                out=1,
                ldo=8, odt=2, norms=None, factors=None, flags=0, ws=None, wsb=0, stream=None)
    args.update(kw)
    return _lib.lib().fdp_wgrad_clip(*args.values())


def test_call_module_loads_and_validates():
    """_fdp_call (the per-call path without ctypes) loads next to the library,
    and its calls reach the library's checks (no device needed for these)."""
    F = _lib.fast_call()
    assert F is not None
    common = (1, 1, 2, 4, 8, 8, 32, 8, 32, 8, 0, 7, 1.0, 1.0, 1.0, 0.0, None, 1, 8, 2, 0)
    assert F.wgrad(*common, None, 0, None) == 1          # bad dtype
    assert F.wgrad_bias(*common, 1, 2, 1.0, 0.0, None, None, 0, None) == 1
    ok = common[:11] + (2,) + common[12:]
    assert F.wgrad(*ok, None, 0, None) == 4               # workspace missing
    assert F.wgrad_bias(*ok, None, 2, 1.0, 0.0, None, None, 0, None) == 3  # no bias output
    with pytest.raises(TypeError):
        F.wgrad(*ok, None, 0)                              # wrong argument count
    with pytest.raises(TypeError):
        F.wgrad(*ok[:16], [1, 2], *ok[17:], None, 0, None)  # key must be a tuple


def test_wgrad_validation_codes():
    assert _wgrad(dtype=7) == 1
    assert _wgrad(odt=-1) == 1
    assert _wgrad(layout=5) == 3
    assert _wgrad(B=0) == 2
    assert _wgrad(lda=4) == 2          # row stride shorter than M
    assert _wgrad(out=None) == 3
    assert _wgrad(flags=64) == 3       # no such flag
    assert _wgrad(flags=16 | 32) == 3  # FDP_WGRAD_WIDE and FDP_WGRAD_NARROW together
    assert _wgrad(flags=1, norms=16) == 3  # norms undefined without the norm pass
    assert _wgrad() == 4               # workspace missing


def test_noalloc_validation_codes():
    """fdp_wgrad_clip_noalloc validates like fdp_wgrad_clip and rejects problems
    whose workspace exceeds its scratch array (FDP_ERR_TOO_LARGE) before it
    touches a device, so these run without one."""
    L = _lib.lib()

    def call(B=2, K=4, M=8, N=8, dtype=2, flags=0):
        return L.fdp_wgrad_clip_noalloc(1, 1, B, K, M, N, K * M, M, K * N, N, 0, dtype, 1.0, 1.0,
                                        None, 1.0, None, 0.0, None, 1, N, 2, None, None, flags,
                                        None)
    assert call(dtype=7) == 1
    assert call(B=0) == 2
    assert call(flags=64) == 3
    limit = 64 << 20
    big = [s for s in [(128, 16, 2048, 2048), (512, 16, 2048, 2048), (1024, 8, 1024, 1024)]
           if _lib.size_query(L.fdp_wgrad_clip_workspace_size, *s, 2, 4) > limit]
    assert big
    assert call(*big[0]) == 7
    with pytest.raises(ValueError):
        _lib.check(7, "fdp_wgrad_clip_noalloc")


def test_workspace_queries():
    L = _lib.lib()
    n = _lib.size_query(L.fdp_wgrad_clip_workspace_size, 8, 1024, 3072, 768, 2, 0)
    assert n >= 8 * 4
    # cfg2 takes the wide kernel by default: 256 exchange slots of 63 bf16 32x32 blocks,
    # less than one bf16 gradient per sample (8 * 3072 * 768 * 2 bytes)
    assert 256 * 63 * 2048 <= n < 8 * 3072 * 768 * 2
    narrow = _lib.size_query(L.fdp_wgrad_clip_workspace_size, 8, 1024, 3072, 768, 2,
                             _lib.WGRAD_NARROW)
    assert narrow < n
    with pytest.raises(KeyError):
        _lib.size_query(L.fdp_wgrad_clip_workspace_size, 8, 1024, 3072, 768, 9, 0)
    with pytest.raises(ValueError):
        _lib.size_query(L.fdp_colsum_clip_workspace_size, 0, 4, 4, 2)
    with pytest.raises(ValueError):  # rows beyond 2^30 elements
        _lib.size_query(L.fdp_layernorm_bwd_clip_workspace_size, 2, 4, (1 << 30) + 1, 2)
    assert _lib.size_query(L.fdp_layernorm_bwd_clip_workspace_size, 2, 4, 16384, 2) > 0
    # longer rows also hold the per-row statistics: 8 bytes per row beyond the partials
    assert _lib.size_query(L.fdp_layernorm_bwd_clip_workspace_size, 2, 4, 40000, 2) >= 2 * 4 * 8
    assert _lib.size_query(L.fdp_layernorm_bwd_clip_workspace_size, 16, 1024, 1024, 2) > 0


def test_other_validation_codes():
    L = _lib.lib()
    st = L.fdp_colsum_clip(1, None, 2, 3, 4, 2, 9, 1.0, 1.0, None, 1.0, None, 0.0, None, 1, 2,
                           None, None, None, 0, None)
    assert st == 3  # bad norm kind
    # rows beyond 2^30 elements (every shorter row is launched, so no fake pointer below
    # may carry a valid shape)
    st = L.fdp_layernorm_fwd(1, None, None, 4, (1 << 30) + 1, 1e-5, 2, 2, 1, None, None, None)
    assert st == 2
    st = L.fdp_layernorm_fwd(1, None, None, 4, 64, 1e-5, 5, 2, 1, None, None, None)
    assert st == 1
    st = L.fdp_layernorm_bwd_clip(1, 1, None, 1, 1, 2, 4, 64, 2, 2, 1.0, 1.0, None, 0.5, None,
                                  None, 0.0, None, 1, None, None, None, None, None, 0, None)
    assert st == 4


def test_status_to_exception_mapping():
    with pytest.raises(KeyError):
        _lib.check(1, "x")
    with pytest.raises(ValueError):
        _lib.check(2, "x")
    with pytest.raises(RuntimeError):
        _lib.check(5, "x")


def test_noise_advance_rejects_null_counter():
    assert _lib.lib().fdp_noise_advance(None, 4, None) == 3


def test_bias_of_b_flag_only_with_the_bias_entry_point():
    """FDP_WGRAD_BIAS_OF_B selects the bias operand of fdp_wgrad_bias_clip;
    fdp_wgrad_clip rejects it as an unknown flag."""
    assert _wgrad(flags=_lib.WGRAD_BIAS_OF_B) == 3
    L = _lib.lib()
    n_a = _lib.size_query(L.fdp_wgrad_bias_clip_workspace_size, 4, 64, 512, 2048, 2, 0)
    n_b = _lib.size_query(L.fdp_wgrad_bias_clip_workspace_size, 4, 64, 512, 2048, 2,
                          _lib.WGRAD_BIAS_OF_B)
    assert n_a > 0 and n_b > n_a  # the bias partials scale with the bias length (512 vs 2048)


def test_dgrad_validation_codes():
    """fdp_dgrad checks sizes, layout, dtype, strides and alignment on the host
    and launches nothing on a bad call."""
    L = _lib.lib()
    args = dict(g=16, w=16, dx=16, M=64, N=64, K=64, ldg=64, ldw=64, ldo=64, layout=0, dtype=2,
                stream=None)

    def call(**kw):
        a = {**args, **kw}
        return L.fdp_dgrad(a["g"], a["w"], a["dx"], a["M"], a["N"], a["K"], a["ldg"], a["ldw"],
                           a["ldo"], a["layout"], a["dtype"], a["stream"])
    assert call(K=96) == 2            # K % 64 != 0
    assert call(dtype=0) == 1         # fp32 is torch's matmul
    assert call(layout=2) == 3        # no such layout
    assert call(ldg=32) == 2          # row stride below K
    assert call(ldw=32) == 2          # NN weight rows hold N values
    assert call(ldg=68) == 6          # 16-byte rows
    assert call(g=24) == 6            # 16-byte aligned operands
    assert call(g=None) == 3
    assert call(M=1 << 22, ldg=1 << 9) == 2  # g spans 2^32 bytes (32-bit buffer records)
    # strides whose byte spans overflow 64-bit arithmetic are refused, not wrapped
    assert call(M=2, ldg=1 << 62) == 2
    assert call(ldw=1 << 62) == 2
    # 2^23 rows x 2^23 columns: g and w each 1 GiB, but about 2^31 output tiles
    assert call(M=1 << 23, N=1 << 23, K=64, ldw=1 << 23, ldo=1 << 23) == 2
