"""Host-side operand checks of bozo_amd.ops, on the CPU.

The C ABI sees strides, not sizes, so the Python host must refuse operands
whose shapes disagree before a launch would read past the end of one of
them: the decode step's caches, new rows, position counters and tau output
against q's [N, H, D], and the device of every operand against the first
one's.  These checks are pure shape / device logic; CPU tensors stand in for
device tensors, and meta tensors for tensors on another device.
"""
import pytest
import torch

from bozo_amd import ops


def _decode(N=3, H=2, D=64, W=16, **over):
    t = dict(q=torch.zeros(N, H, D), k_new=torch.zeros(N, H, D), v_new=torch.zeros(N, H, D, dtype=torch.bfloat16),
             k_cache=torch.zeros(N, H, W, D), v_cache=torch.zeros(N, H, W, D, dtype=torch.bfloat16),
             pos_in=torch.zeros(N, dtype=torch.int32), pos_out=torch.zeros(N, dtype=torch.int32),
             tau=torch.zeros(N, H, W))
    t.update(over)
    return t


def test_decode_operands_accepted():
    ops._check_decode_operands(**_decode())
    ops._check_decode_operands(**_decode(pos_out=None, tau=None))
    # the autocast flow: float32 q / K, bf16 V, same shapes
    ops._check_decode_operands(**_decode(v_cache=torch.zeros(3, 2, 16, 64, dtype=torch.bfloat16)))


@pytest.mark.parametrize("over, what", [
    (dict(q=torch.zeros(3, 2, 64, 1)), "q must be"),
    (dict(k_new=torch.zeros(3, 2, 32)), "k_new, v_new"),
    (dict(v_new=torch.zeros(2, 2, 64)), "k_new, v_new"),
    (dict(k_cache=torch.zeros(2, 2, 16, 64)), "k_cache, v_cache"),          # fewer sequences than q
    (dict(k_cache=torch.zeros(3, 1, 16, 64)), "k_cache, v_cache"),          # fewer heads
    (dict(k_cache=torch.zeros(3, 2, 16, 32)), "k_cache, v_cache"),          # narrower rows
    (dict(v_cache=torch.zeros(3, 2, 8, 64)), "k_cache, v_cache"),           # shorter V ring
    (dict(k_cache=torch.zeros(3, 2, 16)), "k_cache, v_cache"),
    (dict(pos_in=torch.zeros(2, dtype=torch.int32)), "pos_in"),             # counters for fewer sequences
    (dict(pos_out=torch.zeros(6, dtype=torch.int32)[::2]), "pos_out"),      # strided view
    (dict(pos_in=torch.zeros(3, dtype=torch.int64)), "int32"),
    (dict(tau=torch.zeros(3, 2, 8)), "tau must be"),
    (dict(v_new=torch.zeros(3, 2, 64, device="meta")), "all tensors must be on"),
    (dict(pos_in=torch.zeros(3, dtype=torch.int32, device="meta")), "all tensors must be on"),
])
def test_decode_operands_rejected(over, what):
    with pytest.raises((ValueError, TypeError), match=what):
        ops._check_decode_operands(**_decode(**over))


def test_same_device():
    a = torch.zeros(2)
    ops._same_device(a, a, None, torch.ones(3))
    with pytest.raises(ValueError, match="all tensors must be on"):
        ops._same_device(a, a, torch.zeros(2, device="meta"))


def test_buf_refuses_more_than_four_dimensions():
    from bozo_amd import _lib as L
    assert L.buf(torch.zeros(2, 2, 2, 2)) is not None
    with pytest.raises(ValueError, match="at most 4"):
        L.buf(torch.zeros(2, 2, 2, 2, 2))
    with pytest.raises(TypeError, match="unsupported dtype"):
        L.buf(torch.zeros(3, dtype=torch.int32))
