"""CPU-side checks of the QK-norm + RoPE + cache entry point: the C ABI rejects bad modes and
shapes before any launch, and the wrapper keeps the reference's assertions
(engine/kernels/qk_rope.py:103-121). No kernel runs here."""

import ctypes

import pytest
import torch

from kernels import _native
from kernels import qk_rope as R


class Norm:
    def __init__(self, d):
        self.weight, self.variance_epsilon = torch.ones(d, dtype=torch.bfloat16), 1e-6


def test_c_abi_rejects_before_launch():
    lib = _native.lib()
    f = ctypes.c_void_p(64)
    pos = ctypes.c_void_p(128)
    call = lib.ftk_qk_rope_cache_bf16

    def status(mode=0, dim=128, splits=1, stride=0, ptr=f, phases=None, tokens=1, cap=16):
        return call(ptr, splits, stride, f, f, 1e-6, 1e-6, f, f, 16, pos, phases, f, f, f, 1, tokens, 32, 8, cap,
                    dim, mode, None)

    assert status(ptr=None) == _native.FTK_ERR_INVALID
    assert status(mode=8) == _native.FTK_ERR_INVALID
    assert status(mode=_native.ROPE_PREFILL | _native.ROPE_ROWS) == _native.FTK_ERR_INVALID
    assert status(mode=_native.ROPE_TABLE) == _native.FTK_ERR_INVALID  # a table needs per-row positions
    assert status(mode=_native.ROPE_TABLE | _native.ROPE_ROWS) == _native.FTK_ERR_INVALID  # ... and phases
    assert status(tokens=17, cap=16) == _native.FTK_ERR_INVALID
    assert status(splits=2, stride=10) == _native.FTK_ERR_INVALID
    assert status(tokens=17, cap=32) == _native.FTK_ERR_INVALID  # 16 table rows for 17 tokens
    assert status(dim=96) == _native.FTK_ERR_UNSUPPORTED
    assert status(ptr=ctypes.c_void_p(66)) == _native.FTK_ERR_UNSUPPORTED  # 4-byte alignment


def _args(b=1, t=1, hq=4, hkv=2, d=64, cap=8):
    packed = torch.zeros(b, t, (hq + 2 * hkv) * d, dtype=torch.bfloat16)
    keys = torch.zeros(b, hkv, cap, d, dtype=torch.bfloat16)
    cos = torch.zeros(1, t, d, dtype=torch.bfloat16)
    return [packed, Norm(d), Norm(d), cos, cos.clone(), torch.zeros(1, dtype=torch.int64), keys, keys.clone(), hq]


def test_wrapper_keeps_the_reference_assertions():
    a = _args()
    with pytest.raises(AssertionError):
        R.qk_rope_cache(a[0].float(), *a[1:])  # BF16 packed unless a Split
    bad = list(a)
    bad[5] = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(AssertionError):
        R.qk_rope_cache(*bad)  # position [1] for a shared decode step
    with pytest.raises(AssertionError):
        R.qk_rope_cache(*a[:8], 5)  # packed width must match the heads
    with pytest.raises(AssertionError):
        R.qk_rope_cache(*a, prefill=True, rows=True)
    with pytest.raises(ValueError, match="GPU"):
        R.qk_rope_cache(*a)  # CPU tensors: no fallback
