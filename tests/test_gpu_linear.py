"""GPU parity of the skinny projection (kernels.linear) against the CPU oracle.

Bars: <= 0.75 BF16 ulp of the fp64 product at the reference's own test shapes
(agent/local_cpu/interp/run_numeric.py:46-62), and |y - ref| <= 2e-2 + 1e-2|ref|
(rel 1e-2 / abs 2e-2) against the oracle and torch's
F.linear at the model shapes. Launch shapes that only reorder the same FP32
sums must agree bit for bit.
"""

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from conftest import GOLDEN, from_bits, seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import linear as L

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2

MODEL_SHAPES = {
    "0.6B qkv": (4096, 1024), "0.6B o": (1024, 2048), "0.6B gate_up": (6144, 1024), "0.6B down": (1024, 3072),
    "8B qkv": (6144, 4096), "8B o": (4096, 4096), "8B gate_up": (24576, 4096), "8B down": (4096, 12288),
}


def within(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return bool(np.all(np.abs(got - ref) <= ATOL + RTOL * np.abs(ref)))


@pytest.mark.parametrize("m,n,k", [(1, 200, 300), (5, 200, 300), (16, 130, 517), (20, 70, 260), (1, 173, 259),
                                   (4, 257, 513), (16, 127, 256), (3, 64, 1024)])
def test_reference_shapes_three_quarter_ulp(cuda, m, n, k):
    data = np.load(GOLDEN / "linear.npz")
    key = f"{m}_{n}_{k}"
    x, w = from_bits(data[f"x_{key}"], cuda), from_bits(data[f"w_{key}"], cuda)
    got = L.linear(x, w)
    torch.cuda.synchronize()
    got = bf16.to_f32(to_bits(got)).astype(np.float64)
    exact = data[f"exact_{key}"]
    err = np.abs(got - exact) / bf16.ulp(exact)
    assert err.max() <= 0.75, f"max err {err.max():.3f} ulp"
    assert within(got, bf16.to_f32(data[f"torch_{key}"]))


@pytest.mark.parametrize("name", list(MODEL_SHAPES))
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_model_shapes_match_oracle(cuda, name, m):
    n, k = MODEL_SHAPES[name]
    x = seeded((m, k), seed=m, device=cuda)
    w = seeded((n, k), seed=100 + m, scale=0.02, device=cuda)
    got = L.linear(x, w)
    want = path.project(to_bits(x), to_bits(w))
    got_bits = to_bits(got)
    assert within(bf16.to_f32(got_bits), bf16.to_f32(want))
    assert np.mean(got_bits == want) >= 0.99
    ref = F.linear(x.float(), w.float())
    assert within(bf16.to_f32(got_bits), ref.cpu().numpy())


GEMV_SHAPES = {1: ((2, 4), (4, 2), (4, 4), (8, 1), (8, 2)), 2: ((1, 2), (2, 2), (2, 4)), 4: ((1, 1), (2, 1), (2, 2))}


@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("kw", [1, 2, 4])
def test_launch_shapes_agree_bit_for_bit(cuda, m, kw):
    """For a given K split (waves per row group), rows per group, unroll and grid cap only
    regroup the same per-lane FP32 sums: bit-equal. Across K splits: tolerance vs the oracle."""
    n, k = 1000, 2048
    x = seeded((m, k), seed=7, device=cuda)
    w = seeded((n, k), seed=8, scale=0.02, device=cuda)
    want = path.project(to_bits(x), to_bits(w))
    base = None
    for rpw, unroll in GEMV_SHAPES[kw]:
        for gpc in (1, 2, 8):
            got = L.project(x, w, _native.Config(_native.KIND_GEMV, rpw, unroll, gpc, kw))
            if base is None:
                base = got
                assert within(bf16.to_f32(to_bits(got)), bf16.to_f32(want))
            assert torch.equal(got, base), (rpw, unroll, gpc, kw)


@pytest.mark.parametrize("kw", [2, 4])
def test_split_k_gemv_fused_epilogues(cuda, kw):
    """K split across the waves of a row group, with the norm prologue, SwiGLU and argmax epilogues."""
    from kernels import argmax as A
    from kernels import swiglu as S

    k, i = 1024, 1536
    x = seeded((1, k), seed=30, device=cuda)
    g = seeded((k,), seed=31, scale=0.1, shift=1.0, device=cuda)
    w = seeded((2 * i, k), seed=32, scale=0.02, device=cuda)
    cfg = _native.Config(_native.KIND_GEMV, 2, 1 if kw == 4 else 2, 8, kw)
    got = S.gate_up_swiglu(x, w, g, 1e-6, config=cfg)
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), to_bits(g), 1e-6)
    assert within(bf16.to_f32(to_bits(got)), bf16.to_f32(want))
    got = L.rms_norm_linear(x, g, 1e-6, w, config=cfg)
    assert within(bf16.to_f32(to_bits(got)), bf16.to_f32(path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w))))
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=cfg)
    assert int(ids[0]) == int(path.argmax_first(to_bits(logits))[0])


def test_generic_kind_for_unaligned_input(cuda):
    k, n = 1024, 333
    buf = seeded((1, k + 1), seed=9, device=cuda)
    x = buf[:, 1:]  # 2-byte offset: not 16-byte aligned
    w = seeded((n, k), seed=10, scale=0.02, device=cuda)
    got = L.project(x, w)
    want = path.project(to_bits(x), to_bits(w))
    assert within(bf16.to_f32(to_bits(got)), bf16.to_f32(want))


@pytest.mark.parametrize("m", [5, 8, 16, 32])
def test_more_rows_match_oracle(cuda, m):
    n, k = 1536, 1024
    x = seeded((m, k), seed=11, device=cuda)
    w = seeded((n, k), seed=12, scale=0.02, device=cuda)
    got = L.linear(x, w)
    want = path.project(to_bits(x), to_bits(w))
    assert within(bf16.to_f32(to_bits(got)), bf16.to_f32(want))


@pytest.mark.parametrize("m", [17, 24, 32])
def test_rows_past_sixteen_default_to_the_native_gemm(cuda, m):
    """From 17 rows the default is torch's GEMM (measured faster there), as the reference keeps cuBLAS
    unless a timed kind beats it; the fused forms run their norm / epilogue kernels around it."""
    from kernels import swiglu as S
    from kernels.rmsnorm import rms_norm
    k, n = 1024, 1536
    x = seeded((m, k), seed=40 + m, device=cuda)
    w = seeded((n, k), seed=41, scale=0.02, device=cuda)
    g = seeded((k,), seed=42, scale=0.1, shift=1.0, device=cuda)
    assert torch.equal(L.linear(x, w), F.linear(x, w))
    normed = L.rms_norm_linear(x, g, 1e-6, w)
    assert torch.equal(normed, F.linear(rms_norm(x, g, 1e-6), w))
    assert within(bf16.to_f32(to_bits(normed)), bf16.to_f32(path.norm_project(to_bits(x), to_bits(g), 1e-6,
                                                                               to_bits(w))))
    act = S.gate_up_swiglu(x, w, g, 1e-6)
    assert torch.equal(act, S.swiglu(F.linear(rms_norm(x, g, 1e-6), w)))
    # an explicit launch choice still runs this library's kernel
    assert within(bf16.to_f32(to_bits(L.project(x, w, _native.Config(_native.KIND_MFMA, 0, 0, 0, 0)))),
                  bf16.to_f32(path.project(to_bits(x), to_bits(w))))


def test_linear_keeps_reference_signature_and_fallbacks(cuda):
    x = seeded((2, 3, 256), seed=13, device=cuda)
    w = seeded((512, 256), seed=14, scale=0.02, device=cuda)
    y = L.linear(x, w, split_ok=True)
    assert y.shape == (2, 3, 512) and y.dtype == torch.bfloat16 and y.is_contiguous()
    # rows > MAX_ROWS: native GEMM, as linear.py:492-493
    big = seeded((40, 256), seed=15, device=cuda)
    assert torch.equal(L.linear(big, w), F.linear(big, w))
    # inputs are not modified
    x0 = x.clone()
    L.linear(x, w)
    assert torch.equal(x, x0)


def test_deterministic(cuda):
    x = seeded((1, 4096), seed=16, device=cuda)
    w = seeded((6144, 4096), seed=17, scale=0.02, device=cuda)
    a, b = L.linear(x, w), L.linear(x, w)
    assert torch.equal(a, b)
