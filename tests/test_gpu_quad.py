"""GPU parity of the QUAD kind (M <= 16 on 16-block 4x4x4 MFMAs, STREAM schedule).

Against the CPU oracle: |y - ref| <= 2e-2 + 1e-2|ref| for every epilogue, with
and without the RMSNorm prologue (and its residual / gathered rows), and
bit-exact greedy ids. Within the kind: the grid (how many tiles each workgroup
walks) and the rows per tile only regroup the same sums, so they never change a
bit; and an x row's outputs come from its own MFMA column and its own row
scale, so a call with fewer rows reproduces those rows of a 16-row call bit for
bit, whatever group of 4 x rows the kernel is built for.
"""

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import argmax as A
from kernels import linear as L
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2

#: (rows per group, K, KW) launch shapes, each built for the row counts whose registers fit.
SHAPES = ((8, 4096, 4), (16, 4096, 4), (8, 4096, 8), (16, 4096, 8), (24, 4096, 8), (8, 12288, 8),
          (8, 12288, 16), (8, 1024, 4), (8, 2048, 4), (8, 3072, 4), (4, 4096, 4), (4, 4096, 8), (4, 12288, 8))


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def cfg(rows, kw, gpc=0):
    return _native.Config(_native.KIND_QUAD, rows, 0, gpc, kw)


def built(m, n, k, c, epilogue=_native.EPI_STORE, prologue=False):
    p = _native.Plan()
    flags = epilogue | (_native.PLAN_PROLOGUE if prologue else 0)
    return _native.lib().ftk_plan_project(m, n, k, flags, 256, c, p) == _native.FTK_OK


def _inputs(m, n, k, seed, device):
    x = seeded((m, k), seed=seed, device=device)
    w = seeded((n, k), seed=seed + 1, scale=0.02, device=device)
    g = seeded((k,), seed=seed + 2, scale=0.1, shift=1.0, device=device)
    return x, w, g


@pytest.mark.parametrize("rows,k,kw", SHAPES)
@pytest.mark.parametrize("m", [1, 3, 5, 8, 9, 16])
def test_store_matches_oracle(cuda, rows, k, kw, m):
    n = 1000 + rows + 5  # ragged last tile
    c = cfg(rows, kw)
    plain, normed = built(m, n, k, c), built(m, n, k, c, prologue=True)
    if not (plain or normed):
        pytest.skip("shape not built for this row count (registers)")
    x, w, g = _inputs(m, n, k, seed=2000 + rows + k // 64 + kw + m, device=cuda)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    if plain:
        assert L.plan(m, n, k, config=c).kind == _native.KIND_QUAD
        assert within(to_bits(L.project(x, w, c)), path.project(xb, wb))
    if normed:
        got = L.rms_norm_linear(x, g, 1e-6, w, config=c)
        assert within(to_bits(got), path.norm_project(xb, gb, 1e-6, wb))


@pytest.mark.parametrize("rows,k,kw", [s for s in SHAPES if s[0] % 8 == 0])
@pytest.mark.parametrize("m", [2, 5, 16])
@pytest.mark.parametrize("with_norm", [False, True])
def test_swiglu_matches_oracle(cuda, rows, k, kw, m, with_norm):
    i = 700 + rows // 2 + 3
    c = cfg(rows, kw)
    if not built(m, 2 * i, k, c, _native.EPI_SWIGLU, with_norm):
        pytest.skip("shape not built for this row count (registers)")
    x, w, g = _inputs(m, 2 * i, k, seed=2100 + rows + k // 64 + kw + m, device=cuda)
    g = g if with_norm else None
    got = S.gate_up_swiglu(x, w, g, 1e-6, config=c)
    assert got.shape == (m, i)
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), None if g is None else to_bits(g), 1e-6)
    assert within(to_bits(got), want)


@pytest.mark.parametrize("rows,kw", [(8, 4), (8, 8), (4, 8), (16, 8)])
@pytest.mark.parametrize("m", [1, 5, 16])
def test_argmax_matches_oracle(cuda, rows, kw, m):
    k, v = 4096, 20000 + rows + 7
    c = cfg(rows, kw)
    if not built(m, v, k, c, _native.EPI_ARGMAX, True):
        pytest.skip("shape not built for this row count (registers)")
    x, w, g = _inputs(m, v, k, seed=2200 + rows + kw + m, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=c)
    assert within(to_bits(logits), path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w)))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))
    ids_only, none = A.lm_head_argmax(x, w, g, 1e-6, logits=False, config=c)
    assert none is None and torch.equal(ids_only, ids)


def test_argmax_forced_ties_take_the_lowest_index(cuda):
    """Duplicated weight rows give exactly equal logits: the lowest index must win."""
    k, v, m = 4096, 9000, 6
    x, w, g = _inputs(m, v, k, seed=2300, device=cuda)
    w[5000] = w[17] * 4  # a clear winner, duplicated at a higher index
    w[7000] = w[5000]
    w[123] = w[5000]
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=cfg(8, 8))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


@pytest.mark.parametrize("gpc", [1, 2, 4, 16])
def test_grid_and_rows_per_tile_do_not_change_bits(cuda, gpc):
    x, w, g = _inputs(7, 6000, 4096, seed=2400, device=cuda)
    base = L.rms_norm_linear(x, g, 1e-6, w, config=cfg(8, 8, 64))
    p = L.plan(7, 6000, 4096, config=cfg(8, 8, gpc), prologue=True)
    assert 1 <= -(-p.tiles // p.grid) <= 8
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=cfg(8, 8, gpc)), base)
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=cfg(16, 8, gpc)), base)
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=cfg(4, 8, gpc)), base)


@pytest.mark.parametrize("with_norm", [False, True])
def test_rows_are_independent(cuda, with_norm):
    """Each x row's outputs come from its own MFMA column and its own row scale."""
    x, w, g = _inputs(16, 3000, 4096, seed=2500, device=cuda)
    c = cfg(4, 8) if with_norm else cfg(8, 8)  # the shapes built for every row count
    full = L.rms_norm_linear(x, g, 1e-6, w, config=c) if with_norm else L.project(x, w, c)
    for lo, hi in ((0, 1), (5, 6), (15, 16), (0, 3), (4, 12), (3, 11)):
        part = L.rms_norm_linear(x[lo:hi], g, 1e-6, w, config=c) if with_norm else L.project(x[lo:hi], w, c)
        assert torch.equal(part, full[lo:hi]), (lo, hi)


@pytest.mark.parametrize("m", [3, 8, 13])
def test_residual_and_gathered_rows(cuda, m):
    """The prologue's residual add and embedding gather, with the stored sum bit-exact."""
    k, n = 4096, 1500
    x, w, g = _inputs(m, n, k, seed=2600 + m, device=cuda)
    r = seeded((m, k), seed=2610 + m, device=cuda)
    c = cfg(4, 8)
    y, summed = L.add_rms_norm_linear(x, r, g, 1e-6, w, config=c)
    want_y, want_sum = path.add_norm_project(to_bits(x), to_bits(r), to_bits(g), 1e-6, to_bits(w))
    np.testing.assert_array_equal(to_bits(summed), want_sum)
    assert within(to_bits(y), want_y)
    table = seeded((64, k), seed=2620 + m, device=cuda)
    ids = torch.tensor([(7 * i + 3) % 64 for i in range(m)], device=cuda, dtype=torch.int64)
    y2, hidden = L.embed_rms_norm_linear(ids, table, g, 1e-6, w, config=c)
    rows = to_bits(table)[ids.cpu().numpy()]
    np.testing.assert_array_equal(to_bits(hidden), rows)
    assert within(to_bits(y2), path.norm_project(rows, to_bits(g), 1e-6, to_bits(w)))


def test_matches_mfma_stream_within_tolerance(cuda):
    x, w, g = _inputs(12, 4096, 4096, seed=2700, device=cuda)
    a = L.rms_norm_linear(x, g, 1e-6, w, config=cfg(4, 8))
    b = L.rms_norm_linear(x, g, 1e-6, w, config=_native.Config(_native.KIND_MFMA_STREAM, 16, 4, 0, 16))
    assert within(to_bits(a), to_bits(b))
