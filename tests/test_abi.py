"""C ABI of libtension_hip.so, checked on the CPU (no kernel launches).

* the library loads and exports every function include/tension_hip.h declares;
* the ctypes signatures in bozo_amd/_lib.py have the header's arity;
* argument validation rejects bad calls with TENSION_ERR_ARG and a message,
  before any HIP call is made;
* the product path has no CPU fallback.
"""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tension_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = re.findall(r"^(?:const char\*|int64_t|int)\s+(tension_\w+)\s*\(([^;]*?)\)\s*;", text,
                       flags=re.M | re.S)
    out = {}
    for name, params in decls:
        params = params.strip()
        out[name] = 0 if params in ("", "void") else len(params.split(","))
    return out


@pytest.fixture(scope="module")
def lib():
    from bozo_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        from bozo_amd.build import build
        build(verbose=False)
    return L


def test_header_parses():
    fns = header_functions()
    assert "tension_window_fwd" in fns and "tension_decode_step" in fns
    assert len(fns) >= 12


def test_library_exports_every_declared_symbol(lib):
    h = ctypes.CDLL(lib.LIB_PATH)
    for name in header_functions():
        assert hasattr(h, name), f"{name} declared in tension_hip.h but not exported"


def test_ctypes_signatures_match_header(lib):
    fns = header_functions()
    assert set(fns) == set(lib.SIGNATURES), set(fns) ^ set(lib.SIGNATURES)
    for name, n in fns.items():
        assert len(lib.SIGNATURES[name][1]) == n, name


def test_version_and_empty_error(lib):
    assert b"gfx950" in lib.lib().tension_version()
    assert isinstance(lib.lib().tension_last_error(), bytes)


def _buf(ptr=0x1000, dtype=0, strides=(4096, 64, 16, 1)):
    from bozo_amd._lib import TensionBuf
    return ctypes.pointer(TensionBuf(ctypes.c_void_p(ptr), dtype, 0, (ctypes.c_int64 * 4)(*strides)))


def _fwd(lib, q=None, k=None, v=None, out=None, tau=None, bias=None, mass=None, B=1, T=16, H=1, D=16,
         W=4, scale=4.0, flags=0):
    q = q if q is not None else _buf()
    return lib.lib().tension_window_fwd(q, k if k is not None else _buf(), v if v is not None else _buf(),
                                        out if out is not None else _buf(), tau, bias, mass,
                                        B, T, H, D, W, scale, flags, None)


def test_validation_rejects_bad_arguments(lib):
    L = lib
    cases = [
        dict(W=0),                                       # window < 1
        dict(scale=0.0),                                 # zero scale
        dict(scale=float("nan")),
        dict(D=0),
        dict(q=_buf(ptr=0)),                             # null data pointer
        dict(k=_buf(dtype=7)),                           # bad dtype code
        dict(v=_buf(strides=(4096, 64, 16, 2))),         # innermost stride != 1
        dict(flags=L.NORM_MASS | L.NORM_COUNT),          # exclusive flags
        dict(flags=L.GLOBAL),                            # global through the local entry
    ]
    for kw in cases:
        assert _fwd(lib, **kw) == L.ERR_ARG, kw
        assert lib.lib().tension_last_error(), kw


def test_workspace_query(lib):
    f = lib.lib().tension_window_bwd_workspace
    assert f(2, 8, 3, lib.F32, 0) == 0
    assert f(2, 8, 3, lib.F32, lib.NORM_MASS) == 2 * 2 * 8 * 3 * 4
    assert f(2, 8, 3, lib.F64, lib.NORM_MASS) == 2 * 2 * 8 * 3 * 8
    assert lib.lib().tension_global_bwd_workspace(1, 4, 2, lib.F32, 0) == 2 * 4 * 2 * 4


def test_backward_needs_workspace_with_mass(lib):
    b = _buf()
    r = lib.lib().tension_window_bwd(b, b, b, b, None, None, b, b, b,
                                     None, 1, 16, 1, 16, 4, 4.0, lib.NORM_MASS, None)
    assert r == lib.ERR_ARG
    assert b"workspace" in lib.lib().tension_last_error()


def test_decode_validation(lib):
    q = _buf(strides=(64, 16, 1, 0))
    c = _buf()
    pos = ctypes.c_void_p(0x2000)
    f = lib.lib().tension_decode_step
    assert f(q, q, q, c, c, q, None, None, None, 1, 1, 16, 8, 4.0, 0, None) == lib.ERR_ARG  # no pos
    assert f(q, q, q, c, c, q, None, pos, pos, 1, 1, 16, 8, 4.0, 0, None) == lib.ERR_ARG    # aliasing
    assert f(q, q, q, c, c, q, None, pos, None, 1, 1, 16, 0, 4.0, 0, None) == lib.ERR_ARG   # W = 0


def test_decode_flag_validation(lib):
    q = _buf(strides=(64, 16, 1, 0))
    c = _buf()
    pos = ctypes.c_void_p(0x2000)
    f = lib.lib().tension_decode_step
    assert f(q, q, q, c, c, q, None, pos, None, 1, 1, 16, 8, 4.0, lib.NORM_MASS | lib.NORM_COUNT,
             None) == lib.ERR_ARG
    assert b"exclusive" in lib.lib().tension_last_error()
    tau = _buf(strides=(128, 8, 1, 0))
    assert f(q, q, q, c, c, q, tau, pos, None, 1, 1, 16, 8, 4.0, lib.NORM_MASS | lib.DECODE_SELF,
             None) == lib.ERR_ARG
    assert b"not supported" in lib.lib().tension_last_error()


def test_tau_export_validation(lib):
    arr = (lib.TensionBuf * 1)(_buf().contents)
    stats = ctypes.c_void_p(0x3000)
    f = lib.lib().tension_tau_head_stats
    assert f(arr, 0, 1, 16, 2, 8, stats, 0, None) == lib.ERR_ARG          # no layers
    assert f(arr, 33, 1, 16, 2, 8, stats, 0, None) == lib.ERR_ARG         # more than 32
    assert f(arr, 1, 1, 0, 2, 8, stats, 0, None) == lib.ERR_ARG           # T = 0
    assert f(arr, 1, 1, 16, 2, 8, None, 0, None) == lib.ERR_ARG           # no output
    bad = (lib.TensionBuf * 1)(_buf(strides=(4096, 64, 16, 2)).contents)
    assert f(bad, 1, 1, 16, 2, 8, stats, 0, None) == lib.ERR_ARG          # innermost stride
    g = lib.lib().tension_tau_aggregate
    assert g(arr, 1, 1, 16, 65, 8, stats, stats, None) == lib.ERR_UNSUPPORTED  # H > 64
    assert g(arr, 1, 1, 16, 2, 8, None, stats, None) == lib.ERR_ARG      # no mask


def test_bias_builder_validation(lib):
    p = ctypes.c_void_p(0x4000)
    ins = lib.lib().tension_bias_table_insert
    assert ins(p, p, 5, p, p, 3, None) == lib.ERR_ARG       # 5 keys need capacity >= 10 > 8
    assert ins(p, p, 4, p, p, 0, None) == lib.ERR_ARG       # log2cap < 1
    assert ins(None, None, 0, p, p, 3, None) == lib.OK       # nothing to insert, no launch
    build = lib.lib().tension_bias_build
    b = _buf(strides=(64, 8, 1, 0))
    assert build(p, 0, 8, 8, p, p, 4, 0.5, b, None, None) == lib.ERR_ARG              # B = 0
    assert build(p, 1, 8, 8, p, p, 4, float("inf"), b, None, None) == lib.ERR_ARG     # alpha
    assert build(p, 1, 8, 8, p, p, 4, 0.5, _buf(strides=(64, 8, 2, 0)), None, None) == lib.ERR_ARG
    assert build(p, 1, 0, 8, p, p, 4, 0.5, b, None, None) == lib.OK                   # empty context


def test_size_products_do_not_wrap(lib):
    """Sizes whose products overflow int64 (or whose casts to int would
    truncate) are rejected as too large: never taken for an empty call
    (OK without a launch) or for a small shape that passes the range checks."""
    big, huge = 1 << 31, 1 << 40
    # window: B * H * T = 2^90 wraps to 0 in int64
    assert _fwd(lib, B=(1 << 30) - 1, T=(1 << 30) - 1, H=(1 << 30) - 1) == lib.ERR_ARG
    assert _fwd(lib, B=1 << 29, T=1 << 29, H=1 << 30, D=64) == lib.ERR_ARG
    # head dim past int range: (int)(2^32 + 64) == 64
    assert _fwd(lib, D=(1 << 32) + 64) == lib.ERR_ARG
    # decode: N * H = 2^71 wraps to 0 (was reported as an empty call)
    q = _buf(strides=(64, 16, 1, 0))
    c = _buf()
    pos = ctypes.c_void_p(0x2000)
    f = lib.lib().tension_decode_step
    assert f(q, q, q, c, c, q, None, pos, None, big, huge, 64, 12, 8.0, 0, None) == lib.ERR_ARG
    assert f(q, q, q, c, c, q, None, pos, None, 1 << 62, 4, 64, 12, 8.0, 0, None) == lib.ERR_ARG
    # rope: pos_offset + T overflows past the table check
    x = _buf(strides=(4096, 64, 16, 1))
    tab = ctypes.c_void_p(0x5000)
    rope = lib.lib().tension_rope
    assert rope(x, x, tab, tab, 1024, 1, 16, 1, 16, (1 << 63) - 8, 0, None) == lib.ERR_ARG
    assert rope(x, x, tab, tab, 8, 1, 16, 1, 16, 0, 0, None) == lib.ERR_ARG          # T > rows
    # tau export: T * W and B * T * H * W wrap
    arr = (lib.TensionBuf * 1)(_buf().contents)
    stats = ctypes.c_void_p(0x3000)
    hs = lib.lib().tension_tau_head_stats
    assert hs(arr, 1, 1, 1 << 33, 2, 1 << 31, stats, 0, None) == lib.ERR_ARG
    assert hs(arr, 1, 1 << 40, 1 << 20, 1 << 20, 1, stats, 0, None) == lib.ERR_ARG
    # bias builder: B and W past int range; T * W past the launch range
    p = ctypes.c_void_p(0x4000)
    build = lib.lib().tension_bias_build
    b = _buf(strides=(64, 8, 1, 0))
    assert build(p, (1 << 32) + 1, 8, 8, p, p, 4, 0.5, b, None, None) == lib.ERR_ARG
    assert build(p, 1, 8, (1 << 32) + 8, p, p, 4, 0.5, b, None, None) == lib.ERR_ARG
    assert build(p, 1, 1 << 30, 1 << 30, p, p, 4, 0.5, b, None, None) == lib.ERR_ARG
    # bias table: 2 * n wraps negative below any capacity
    ins = lib.lib().tension_bias_table_insert
    assert ins(p, p, (1 << 63) - 1, p, p, 40, None) == lib.ERR_ARG
    # size queries: -1 / 0 instead of a wrapped byte count
    assert lib.lib().tension_window_bwd_workspace(big, big, big, lib.F32, lib.NORM_MASS) == -1
    assert lib.lib().tension_global_bwd_workspace(-1, 8, 2, lib.F32, 0) == -1
    assert lib.lib().tension_aux_loss_partials(big, big, big) == 0


def test_noalloc_refuses_requests_beyond_the_scratch(lib):
    """tension_global_bwd_noalloc checks the coefficient scratch it needs
    (2 * B*T*H floats) against its fixed size before it looks up the scratch
    or launches anything: one query past the limit is an argument error,
    with fake host pointers that are never read."""
    n = lib.NOALLOC_SCRATCH_BYTES // 8 + 1
    fake = _buf(strides=(n * 64, 64, 64, 1))
    r = lib.lib().tension_global_bwd_noalloc(*([fake] * 11), 1, n, 1, 64, 0, ctypes.c_double(8.0), 0, None)
    assert r == lib.ERR_ARG
    assert b"fixed scratch" in lib.lib().tension_last_error()


def test_window_bwd_saved_requires_rows(lib):
    """tension_window_bwd_saved takes the forward's rows: a call without out or
    mass is an argument error before any HIP call."""
    b = _buf()
    f = lib.lib().tension_window_bwd_saved
    args = lambda out, mass: (b, b, b, b, None, None, out, mass, b, b, b, None,  # noqa: E731
                              1, 16, 1, 16, 4, ctypes.c_double(4.0), 0, None)
    assert f(*args(None, b)) == lib.ERR_ARG
    assert f(*args(b, None)) == lib.ERR_ARG
    assert b"out and mass are required" in lib.lib().tension_last_error()


def test_no_cpu_fallback():
    from bozo_amd import causal_tension, global_tension
    x = torch.zeros(1, 8, 1, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        causal_tension(x, x, x, 4, 4.0)
    with pytest.raises(RuntimeError, match="GPU"):
        global_tension(x, x, x, 4.0)
