"""Seeded fuzz of the C ABI's argument validation, on a machine WITHOUT a GPU.

Every entry point of include/tension_hip.h is called a few thousand times
with random and hostile arguments: null or dangling descriptors, bad dtype
codes, negative / zero / 2^31 / 2^40 / int64-max sizes and strides, NaN and
infinite scales, random flag words.  Without a GPU, a call that passes
validation fails at its first HIP call, so each call must return a non-zero
status with a message -- or OK with nothing to do, which is allowed only when
one of its sizes is 0.  A size product that wraps (B * H * T = 2^90 read as
0) shows up here as an OK on a non-empty shape.  The size queries must return
-1 / 0 or a non-negative byte count, never a wrapped negative one.

The premise needs the absence of a GPU: on a machine with one, calls that pass
validation would launch kernels on the fake pointers used here, so its tests
skip themselves there.  Against a library built with host sanitizers
(`-Xarch_host -fsanitize=address`, or `=undefined`, on every hipcc line) the
same calls also check the validation code for out-of-bounds accesses and for
signed overflow in its size arithmetic.
"""
import ctypes as C
import os
import random

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def lib():
    if os.path.exists("/dev/kfd") or torch.cuda.is_available():
        pytest.skip("the fuzz relies on HIP calls failing: it never runs where a GPU is visible")
    from bozo_amd import _lib as L
    if not os.path.exists(L.LIB_PATH):
        from bozo_amd.build import build
        build(verbose=False)
    return L


_HOST = [np.zeros(64, np.uint8) for _ in range(16)]  # pointer targets; never launched on
_BIG = np.zeros(4096, np.uint8)  # 256-byte aligned pointer target of the valid descriptors


class _Gen:
    def __init__(self, L, seed):
        self.L, self.r = L, random.Random(seed)

    def dim(self):
        return self.r.choice([0, 1, 2, 3, 4, 12, 31, 32, 63, 64, 65, 128, 256, 1024, 2048, -1, -64,
                              1 << 31, (1 << 31) - 1, 1 << 40, -(1 << 62), (1 << 63) - 1])

    def buf(self):
        if self.r.random() < 0.15:
            return None
        b = self.L.TensionBuf()
        b.ptr = None if self.r.random() < 0.1 else _HOST[self.r.randrange(len(_HOST))].ctypes.data
        b.dtype = self.r.choice([-1, 0, 1, 2, 3, 4, 5, 99, 1 << 30])
        b.reserved = 0
        for i in range(4):
            b.s[i] = self.r.choice([0, 1, 1, 64, 768, 49152, -1, -64, 1 << 40, (1 << 63) - 1, self.dim()])
        return C.pointer(b)

    def ptr(self):
        return None if self.r.random() < 0.3 else _HOST[self.r.randrange(len(_HOST))].ctypes.data

    def scale(self):
        return self.r.choice([8.0, 1.0, 0.0, -1.0, float("nan"), float("inf"), 1e-300, 1e300])

    def flags(self):
        return self.r.choice([0, 1, 2, 3, 4, 8, 16, 32, 64, 128, 255, -1, 1 << 30, self.r.getrandbits(31)])

    def layers(self):
        return self.r.choice([0, 1, 9, 12, -1, 1 << 20])


def _calls(g):
    b, d, p, s, f, n = g.buf, g.dim, g.ptr, g.scale, g.flags, g.layers
    return {
        "tension_window_fwd": lambda: (b(), b(), b(), b(), b(), b(), b(), d(), d(), d(), d(), d(), s(), f(), None),
        "tension_window_bwd": lambda: (b(), b(), b(), b(), b(), b(), b(), b(), b(), p(), d(), d(), d(), d(), d(),
                                       s(), f(), None),
        "tension_window_bwd_dq": lambda: (b(), b(), b(), b(), b(), b(), b(), p(), d(), d(), d(), d(), d(), s(), f(),
                                          None),
        "tension_window_bwd_dkv": lambda: (b(), b(), b(), b(), b(), b(), b(), b(), p(), d(), d(), d(), d(), d(), s(),
                                           f(), None),
        "tension_global_fwd": lambda: (b(), b(), b(), b(), b(), b(), b(), d(), d(), d(), d(), d(), s(), f(), None),
        "tension_global_bwd": lambda: (b(), b(), b(), b(), b(), b(), b(), b(), b(), b(), b(), p(), d(), d(), d(), d(),
                                       d(), s(), f(), None),
        "tension_global_bwd_noalloc": lambda: (b(), b(), b(), b(), b(), b(), b(), b(), b(), b(), b(), d(), d(), d(),
                                               d(), d(), s(), f(), None),
        "tension_decode_step": lambda: (b(), b(), b(), b(), b(), b(), b(), p(), p(), d(), d(), d(), d(), s(), f(),
                                        None),
        "tension_rope": lambda: (b(), b(), p(), p(), d(), d(), d(), d(), d(), d(), g.r.choice([0, 1, 2]), None),
        "tension_tau_head_stats": lambda: (b(), n(), d(), d(), d(), d(), p(), f(), None),
        "tension_tau_aggregate": lambda: (b(), n(), d(), d(), d(), d(), p(), p(), None),
        "tension_aux_loss_fwd": lambda: (b(), n(), d(), d(), d(), d(), p(), None),
        "tension_aux_loss_bwd": lambda: (b(), b(), n(), d(), d(), d(), d(), p(), None),
        "tension_bias_table_insert": lambda: (p(), p(), d(), p(), p(), g.r.choice([0, 1, 10, 31, 62, 64, -1]), None),
        "tension_bias_build": lambda: (p(), d(), d(), d(), p(), p(), g.r.choice([0, 1, 10, 31, 62, 64, -1]),
                                       g.r.choice([0.5, -1.0, float("nan")]), b(), p(), None),
    }


# (name, index of the first size argument, number of size arguments): the
# int64 sizes that make a call empty when one of them is 0
_SIZES = {
    "tension_window_fwd": (7, 4), "tension_window_bwd": (10, 4), "tension_window_bwd_dq": (8, 4),
    "tension_window_bwd_dkv": (9, 4), "tension_global_fwd": (7, 4), "tension_global_bwd": (12, 4),
    "tension_global_bwd_noalloc": (11, 4), "tension_decode_step": (9, 2), "tension_rope": (5, 4),
    "tension_bias_table_insert": (2, 1), "tension_bias_build": (1, 3),
}


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_arguments_fail_cleanly(lib, seed):
    g = _Gen(lib, seed)
    h = lib.lib()
    for name, make in _calls(g).items():
        fn = getattr(h, name)
        for i in range(1500):
            args = make()
            r = fn(*args)
            if r == lib.OK:
                lo, cnt = _SIZES.get(name, (0, 0))
                sizes = list(args[lo:lo + cnt])
                assert 0 in sizes, f"{name} call {i}: OK without a GPU on sizes {sizes}"
            else:
                assert r in (lib.ERR_ARG, lib.ERR_UNSUPPORTED, lib.ERR_LAUNCH), (name, i, r)
                assert h.tension_last_error(), (name, i)


def test_size_queries_never_wrap(lib):
    g = _Gen(lib, 3)
    h = lib.lib()
    for _ in range(3000):
        B, T, H = g.dim(), g.dim(), g.dim()
        for q in (h.tension_window_bwd_workspace, h.tension_global_bwd_workspace):
            v = q(B, T, H, g.r.choice([lib.F32, lib.F64, 99]), g.flags())
            assert v >= -1
            if min(B, T, H) < 0:
                assert v <= 0
        assert h.tension_aux_loss_partials(B, T, H) >= 0


def _valid_calls(L, r):
    """Descriptors that pass validation (float dtypes, unit innermost stride,
    one 256-byte aligned host buffer) with extreme sizes and strides, so the
    host code behind it -- kernel selection, 32-bit view checks, launch
    geometry -- runs on them; without a GPU each such call ends in
    TENSION_ERR_LAUNCH."""
    base = (_BIG.ctypes.data + 255) // 256 * 256
    sizes = [1, 2, 3, 17, 63, 64, 65, 128, 1000, 1024, 4096, 65536, (1 << 20) + 3, (1 << 30) - 1]
    strides = [1, 8, 64, 768, 1536, 1 << 20, 1 << 31, (1 << 40) + 8, 1 << 62]

    def b(unit=3, dt=None):
        if r.random() < 0.1:
            return None
        x = L.TensionBuf()
        x.ptr = base
        x.dtype = dt if dt is not None else r.choice([L.F32, L.BF16, L.F16, L.F64])
        for i in range(4):
            x.s[i] = 1 if i == unit else r.choice(strides)
        return C.pointer(x)

    def taus():
        x = L.TensionBuf(C.c_void_p(base), L.F32, 0, (C.c_int64 * 4)(r.choice(strides), r.choice(strides),
                                                                        r.choice(strides), 1))
        return (L.TensionBuf * 1)(x)

    d = lambda: r.choice(sizes)  # noqa: E731
    f = lambda: r.choice([0, 1, 2, 4, 8, 16, 32, 64, 65, 66, 96])  # noqa: E731
    p = base

    def decode():
        dk = r.choice([L.F32, L.BF16, L.F64])
        dv = r.choice([dk, L.BF16])
        return (b(2, dk), b(2, dk), b(2, dv), b(3, dk), b(3, dv), b(2, dk), None if r.random() < 0.5 else b(2, dk),
                p, p + 64, r.choice([1, 3, 64, 1 << 14]), r.choice([1, 16, 1 << 10]), r.choice([32, 64, 128]),
                r.choice([1, 64, 256, 1024, 4096, 1 << 20]), 8.0, r.choice([0, 1, 2, 16, 17]), None)

    return {
        "tension_window_fwd": lambda: (b(), b(), b(), b(), b(), b(2), b(), d(), d(), d(), r.choice([16, 32, 64, 128]),
                                       d(), 8.0, f(), None),
        "tension_window_bwd": lambda: (b(), b(), b(), b(), b(), b(2), b(), b(), b(), p, d(), d(), d(), r.choice([32, 64]),
                                       d(), 8.0, f(), None),
        "tension_global_fwd": lambda: (b(), b(), b(), b(), b(), b(2), b(2), d(), d(), d(), 64, d(), 8.0, f(), None),
        "tension_global_bwd": lambda: (b(), b(), b(), b(), b(), b(2), b(), b(2), b(), b(), b(), p, d(), d(), d(), 64,
                                       d(), 8.0, f(), None),
        "tension_decode_step": decode,
        "tension_rope": lambda: (b(), b(), p, p, r.choice([d(), 1 << 40]), d(), d(), d(), r.choice([16, 64, 128]),
                                 r.choice([0, 5, 1 << 40]), 0, None),
        "tension_tau_head_stats": lambda: (taus(), 1, d(), d(), d(), r.choice([1, 8, 64, 100]), p, f(), None),
        "tension_aux_loss_fwd": lambda: (taus(), 1, d(), d(), d(), r.choice([1, 8, 64]), p, None),
        "tension_bias_build": lambda: (p, d(), d(), r.choice([0, 8, 64, d()]), p, p, r.choice([4, 20, 40]), 0.5, b(1),
                                       p, None),
    }


def test_valid_descriptors_reach_launch_cleanly(lib):
    """Non-empty calls with valid descriptors never return OK without a GPU
    (every one must end in an argument error or the failed launch), and a
    share of each entry point's calls gets through validation to the
    launch code."""
    r = random.Random(11)
    h = lib.lib()
    for name, make in _valid_calls(lib, r).items():
        fn = getattr(h, name)
        launched = 0
        for i in range(800):
            res = fn(*make())
            assert res in (lib.ERR_ARG, lib.ERR_UNSUPPORTED, lib.ERR_LAUNCH), (name, i, res)
            assert h.tension_last_error(), (name, i)
            launched += res == lib.ERR_LAUNCH
        assert launched >= 40, f"{name}: only {launched} of 800 calls passed validation"
