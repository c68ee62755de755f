"""GPU parity of the standalone norm, SwiGLU and argmax operators in both of their launch forms.

Rows of a multiple of 8 elements, at most 8192, on 16-byte aligned buffers run the
row-resident kernels (the whole row in registers, one round trip); other rows run the
element loop. Both are checked against the oracle (engine/kernels/rmsnorm.py:21-162,
engine/kernels/swiglu.py:13-40, engine/kernels/merged.py:37-45), the Split forms against
the merged BF16 tensor bit for bit, and rms_norm followed by an M = 1 projection against
the fused prologue bit for bit (both sum the squares in the same chunk order).
"""

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import path

from kernels import _native
from kernels import argmax as A
from kernels import linear as L
from kernels import merged as M
from kernels import rmsnorm as R
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

# 1000: 125 chunks (a partial first round); 2560 / 5120: partial later rounds;
# 8200: past the register form's 8192, so the element loop.
COLS = [128, 1000, 1024, 2048, 2560, 4096, 5120, 8192, 8200]
ROWS = [1, 5, 16]
EPS = 1e-6


def misaligned(t):
    """The same values 2 bytes past a 16-byte boundary: the launch takes the element loop."""
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    view = buf[1:1 + t.numel()].view(t.shape)
    view.copy_(t)
    assert view.data_ptr() % 16 != 0
    return view


def close(got, want, max_ulps=2):
    """At least 99.9 % of the BF16 outputs bit-equal and none more than ``max_ulps`` apart
    (the two forms and the oracle may sum the squares in different orders)."""
    d = np.abs(got.astype(np.int32) - want.astype(np.int32))
    return np.mean(d == 0) >= 0.999 and d.max() <= max_ulps


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("cols", COLS)
def test_rms_norm_both_forms(cuda, rows, cols):
    x = seeded((rows, cols), seed=cols + rows, device=cuda)
    g = seeded((cols,), seed=7, scale=0.1, shift=1.0, device=cuda)
    want = path.rms_norm(to_bits(x), to_bits(g), EPS)
    assert close(to_bits(R.rms_norm(x, g, EPS)), want)
    assert close(to_bits(R.rms_norm(misaligned(x), g, EPS)), want)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("cols", [1000, 4096, 8200])
def test_add_rms_norm_both_forms(cuda, rows, cols):
    x = seeded((rows, cols), seed=1, device=cuda)
    r = seeded((rows, cols), seed=2, device=cuda)
    g = seeded((cols,), seed=3, scale=0.1, shift=1.0, device=cuda)
    want_y, want_s = path.add_rms_norm(to_bits(x), to_bits(r), to_bits(g), EPS)
    for xi in (x, misaligned(x)):
        y, s = R.add_rms_norm(xi, r, g, EPS)
        assert np.array_equal(to_bits(s), want_s)
        assert close(to_bits(y), want_y)


@pytest.mark.parametrize("splits", [2, 3, 4, 5])
@pytest.mark.parametrize("rows,cols", [(1, 4096), (5, 4096), (16, 4096), (3, 1000), (2, 8200)])
def test_add_rms_norm_split_equals_merged(cuda, splits, rows, cols):
    """A Split of 2..4 planes runs the register form, 5 the element loop; either way the
    partials sum in split order and round once, so the outputs equal those of the merged
    BF16 tensor bit for bit, and the merge equals the oracle's."""
    gen = torch.Generator(device=cuda).manual_seed(splits * 100 + rows)
    partial = torch.randn((splits, rows, cols), generator=gen, device=cuda) * 3
    split = M.Split(partial, (rows, cols))
    r = seeded((rows, cols), seed=4, device=cuda)
    g = seeded((cols,), seed=5, scale=0.1, shift=1.0, device=cuda)
    merged = M.materialize(split)
    assert np.array_equal(to_bits(merged), path.merge_splits(partial.cpu().numpy()))
    y1, s1 = R.add_rms_norm(split, r, g, EPS)
    y2, s2 = R.add_rms_norm(merged, r, g, EPS)
    assert torch.equal(s1, s2) and torch.equal(y1, y2)


@pytest.mark.parametrize("cols", [1000, 4096])
def test_add_rms_norm_one_fp32_plane_through_the_c_abi(cuda, cols):
    """x_splits = 1 (one FP32 plane, which the Python protocol reads as a plain tensor)
    rounds the plane once and adds the residual: the BF16 path's bits."""
    rows = 5
    plane = torch.randn((rows, cols), device=cuda) * 3
    r = seeded((rows, cols), seed=6, device=cuda)
    g = seeded((cols,), seed=8, scale=0.1, shift=1.0, device=cuda)
    y, s = torch.empty_like(r), torch.empty_like(r)
    _native.call("ftk_add_rms_norm_bf16", _native.ptr(plane), 1, rows * cols, _native.ptr(r), _native.ptr(g),
                 _native.ptr(y), _native.ptr(s), rows, cols, EPS, _native.stream_of(r))
    want_y, want_s = R.add_rms_norm(plane.to(torch.bfloat16), r, g, EPS)
    assert torch.equal(s, want_s) and torch.equal(y, want_y)


@pytest.mark.parametrize("rows", [1, 7])
@pytest.mark.parametrize("cols", [1024, 4096, 8192, 8200])
def test_embed_rms_norm_both_forms(cuda, rows, cols):
    table = seeded((64, cols), seed=9, device=cuda)
    g = seeded((cols,), seed=10, scale=0.1, shift=1.0, device=cuda)
    ids = torch.randint(0, 64, (rows,), generator=torch.Generator().manual_seed(rows)).to(cuda)
    want_y, want_h = path.embed_rms_norm(ids.cpu().numpy(), to_bits(table), to_bits(g), EPS)
    y, h = R.embed_rms_norm(ids, table, g, EPS)
    assert np.array_equal(to_bits(h), want_h)
    assert close(to_bits(y), want_y)


@pytest.mark.parametrize("k", [1024, 2048, 4096])
def test_rms_norm_then_projection_equals_the_fused_prologue(cuda, k):
    """M = 1: the register form sums the squares in the STREAM prologue's order, so the
    decomposed norm + projection and the fused call produce the same bits."""
    x = seeded((1, k), seed=11, device=cuda)
    g = seeded((k,), seed=12, scale=0.1, shift=1.0, device=cuda)
    w = seeded((512, k), seed=13, scale=0.02, device=cuda)
    fused = L.rms_norm_linear(x, g, EPS, w)
    decomposed = L.project(R.rms_norm(x, g, EPS), w)
    assert torch.equal(fused, decomposed)


@pytest.mark.parametrize("splits", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("rows,width", [(1, 12288), (5, 3072), (16, 1000), (3, 100)])
def test_swiglu_forms(cuda, splits, rows, width):
    """BF16 or a Split of 1..5 planes, widths that take the 8-per-thread form (multiples of
    8) and one that takes the element loop (100): the oracle's bits, and a Split equals its
    merged tensor bit for bit."""
    if splits == 0:
        packed = seeded((rows, 2 * width), seed=rows, device=cuda)
        got = S.swiglu(packed)
        # Both forms run the same per-element arithmetic: equal bits.
        assert torch.equal(got, S.swiglu(misaligned(packed)))
        inputs = to_bits(packed)
    else:
        gen = torch.Generator(device=cuda).manual_seed(splits + rows)
        partial = torch.randn((splits, rows, 2 * width), generator=gen, device=cuda) * 2
        split = M.Split(partial, (rows, 2 * width))
        merged = M.materialize(split)
        got = S.swiglu(split)
        assert torch.equal(got, S.swiglu(merged))
        inputs = to_bits(merged)
    # SiLU's exp on the GPU is not correctly rounded: the oracle's bits on >= 99.9 %, 1 ulp at most.
    assert close(to_bits(got), path.swiglu(inputs), max_ulps=1)


@pytest.mark.parametrize("rows,vocab", [(1, 151936), (5, 151936), (3, 8200), (2, 1000)])
def test_argmax_both_forms(cuda, rows, vocab):
    """The 16-byte-load block stage (vocab % 8 == 0, aligned logits) and the element loop give the
    same ids and top logits, ties to the lowest index and NaN as the maximum included
    (engine/kernels/argmax.py:19-48)."""
    logits = seeded((rows, vocab), seed=vocab + rows, scale=3, device=cuda)
    logits[0, vocab // 3] = logits[0, vocab // 2] = 40.0  # a tie: the lower index wins
    if rows > 1:
        logits[1, vocab - 1] = float("nan")
    top_a, top_b = (torch.empty(rows, dtype=torch.float32, device=cuda) for _ in range(2))
    fast = A.argmax(logits, top=top_a)
    slow = A.argmax(misaligned(logits), top=top_b)
    assert torch.equal(fast, slow)
    assert torch.equal(top_a, top_b) or (torch.isnan(top_a) == torch.isnan(top_b)).all()
    assert fast[0].item() == vocab // 3
    if rows > 1:
        assert fast[1].item() == vocab - 1
    want = logits.float().argmax(-1)
    for r in range(2 if rows > 1 else 1, rows):
        assert fast[r].item() == want[r].item()


@pytest.mark.parametrize("splits", [1, 2, 3, 8, 9, 17])
@pytest.mark.parametrize("shape", [(1, 4096), (16, 24576), (3, 1000), (2, 999)])
def test_merge_splits_any_planes(cuda, splits, shape):
    """bf16(sum of the planes in split order), as the oracle sums them, for 1..17 planes, ragged
    counts and partials that start off a 16-byte boundary."""
    gen = torch.Generator(device=cuda).manual_seed(splits * 7 + shape[1])
    partial = torch.randn((splits, *shape), generator=gen, device=cuda) * 50
    want = path.merge_splits(partial.cpu().numpy())
    assert np.array_equal(to_bits(M.materialize(M.Split(partial, shape))), want)
    buf = torch.empty(partial.numel() + 1, device=cuda)
    odd = buf[1:].view(partial.shape)
    odd.copy_(partial)
    assert np.array_equal(to_bits(M.materialize(M.Split(odd, shape))), want)
