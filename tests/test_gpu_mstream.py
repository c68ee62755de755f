"""GPU parity of the MFMA_STREAM kind (M <= 16 on 16x16x32 MFMA tiles, STREAM schedule).

Against the CPU oracle: |y - ref| <= 2e-2 + 1e-2|ref| for every epilogue, with
and without the RMSNorm prologue, and bit-exact greedy ids. Within the kind:
the grid (how many tiles each workgroup walks) and the weight window never
change a bit, and an x row's outputs do not depend on the other rows (an MFMA
column and its row scale see only that row), so a one-row call reproduces any
row of a 16-row call bit for bit.
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

#: (T subtiles, K, KW, U) instantiated for every epilogue and both prologue settings ...
SHAPES_EVEN = ((2, 4096, 16, 4), (2, 4096, 8, 4), (2, 4096, 8, 8))
#: ... for store / argmax only ...
SHAPES_ONE = ((1, 4096, 16, 4), (1, 4096, 16, 8), (1, 4096, 8, 4), (1, 4096, 8, 8), (1, 4096, 8, 16))
#: ... and without the prologue only (x streamed beside the weights).
SHAPES_NO_PROLOGUE = ((2, 4096, 16, 8), (2, 4096, 8, 16), (1, 12288, 16, 2), (1, 12288, 16, 6), (1, 12288, 8, 16))


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def cfg(t, kw, u, gpc=0):
    return _native.Config(_native.KIND_MFMA_STREAM, 16 * t, u, gpc, kw)


def _inputs(m, n, k, seed, device):
    x = seeded((m, k), seed=seed, device=device)
    w = seeded((n, k), seed=seed + 1, scale=0.02, device=device)
    g = seeded((k,), seed=seed + 2, scale=0.1, shift=1.0, device=device)
    return x, w, g


@pytest.mark.parametrize("t,k,kw,u", SHAPES_EVEN + SHAPES_ONE + SHAPES_NO_PROLOGUE)
@pytest.mark.parametrize("m", [1, 5, 9, 16])
def test_store_matches_oracle(cuda, t, k, kw, u, m):
    n = 1000 + 16 * t + 5  # ragged last tile
    x, w, g = _inputs(m, n, k, seed=800 + 10 * t + kw + u + m, device=cuda)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    c = cfg(t, kw, u)
    assert L.plan(m, n, k, config=c).kind == _native.KIND_MFMA_STREAM
    got = L.project(x, w, c)
    assert within(to_bits(got), path.project(xb, wb))
    if (t, k, kw, u) not in SHAPES_NO_PROLOGUE:
        normed = L.rms_norm_linear(x, g, 1e-6, w, config=c)
        assert within(to_bits(normed), path.norm_project(xb, gb, 1e-6, wb))


@pytest.mark.parametrize("t,k,kw,u", SHAPES_EVEN)
@pytest.mark.parametrize("m", [5, 16])
@pytest.mark.parametrize("with_norm", [False, True])
def test_swiglu_matches_oracle(cuda, t, k, kw, u, m, with_norm):
    i = 700 + 8 * t + 3
    x, w, g = _inputs(m, 2 * i, k, seed=900 + 10 * t + kw + u + m, device=cuda)
    g = g if with_norm else None
    got = S.gate_up_swiglu(x, w, g, 1e-6, config=cfg(t, kw, u))
    assert got.shape == (m, i)
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), None if g is None else to_bits(g), 1e-6)
    assert within(to_bits(got), want)


@pytest.mark.parametrize("t,k,kw,u", [(2, 4096, 16, 4), (1, 4096, 16, 4), (1, 4096, 8, 8)])
@pytest.mark.parametrize("m", [5, 16])
def test_argmax_matches_oracle(cuda, t, k, kw, u, m):
    v = 20000 + 16 * t + 7
    x, w, g = _inputs(m, v, k, seed=1000 + 10 * t + kw + u + m, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=cfg(t, kw, u))
    want = path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w))
    assert within(to_bits(logits), want)
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))
    ids_only, none = A.lm_head_argmax(x, w, g, 1e-6, logits=False, config=cfg(t, kw, u))
    assert none is None and torch.equal(ids_only, ids)


@pytest.mark.parametrize("gpc", [1, 2, 4])
def test_grid_depth_does_not_change_bits(cuda, gpc):
    x, w, g = _inputs(11, 12000, 4096, seed=1100, device=cuda)
    base = L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 16, 4, 8))
    p = L.plan(11, 12000, 4096, config=cfg(1, 16, 4, gpc), prologue=True)
    assert 1 <= -(-p.tiles // p.grid) <= 4
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 16, 4, gpc)), base)
    # the weight window (U) only changes when loads are issued
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 16, 8, gpc)), base)


@pytest.mark.parametrize("with_norm", [False, True])
def test_rows_are_independent(cuda, with_norm):
    """Each x row's outputs come from its own MFMA column and its own row scale."""
    x, w, g = _inputs(16, 3000, 4096, seed=1200, device=cuda)
    c = cfg(1, 16, 4)
    full = L.rms_norm_linear(x, g, 1e-6, w, config=c) if with_norm else L.project(x, w, c)
    for r in (0, 7, 15):
        one = L.rms_norm_linear(x[r:r + 1], g, 1e-6, w, config=c) if with_norm else L.project(x[r:r + 1], w, c)
        assert torch.equal(one, full[r:r + 1]), r


def test_matches_mfma_kind_within_tolerance(cuda):
    x, w, g = _inputs(8, 4096, 4096, seed=1300, device=cuda)
    a = L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 16, 4))
    b = L.rms_norm_linear(x, g, 1e-6, w, config=_native.Config(_native.KIND_MFMA, 16, 4, 0, 16))
    assert within(to_bits(a), to_bits(b))


@pytest.mark.parametrize("m", [5, 16])
def test_residual_and_gathered_rows(cuda, m):
    """The prologue's residual add and embedding gather on this kind, the stored sum bit-exact."""
    k, n = 4096, 1500
    x, w, g = _inputs(m, n, k, seed=1400 + m, device=cuda)
    r = seeded((m, k), seed=1410 + m, device=cuda)
    c = cfg(1, 16, 4)
    y, summed = L.add_rms_norm_linear(x, r, g, 1e-6, w, config=c)
    want_y, want_sum = path.add_norm_project(to_bits(x), to_bits(r), to_bits(g), 1e-6, to_bits(w))
    np.testing.assert_array_equal(to_bits(summed), want_sum)
    assert within(to_bits(y), want_y)
    table = seeded((64, k), seed=1420 + m, device=cuda)
    ids = torch.tensor([(5 * i + 1) % 64 for i in range(m)], device=cuda, dtype=torch.int32)
    y2, hidden = L.embed_rms_norm_linear(ids, table, g, 1e-6, w, config=c)
    rows = to_bits(table)[ids.cpu().numpy()]
    np.testing.assert_array_equal(to_bits(hidden), rows)
    assert within(to_bits(y2), path.norm_project(rows, to_bits(g), 1e-6, to_bits(w)))


@pytest.mark.parametrize("u", [4, 8, 16])
def test_streamed_x_window_does_not_change_bits(cuda, u):
    """Without the prologue x streams beside the weights with the window's lookahead: the window
    depth only moves loads, so every depth gives the same bits (and the oracle's values)."""
    x, w, _ = _inputs(13, 3000, 4096, seed=1500 + u, device=cuda)
    streamed = L.project(x, w, cfg(1, 8, u))
    assert within(to_bits(streamed), path.project(to_bits(x), to_bits(w)))
    assert torch.equal(streamed, L.project(x, w, cfg(1, 8, 4)))
    k = 12288  # the long-K shapes exist only with x streamed
    x2, w2, _ = _inputs(16, 1000, k, seed=1510 + u, device=cuda)
    a = L.project(x2, w2, cfg(1, 8, 16))
    assert within(to_bits(a), path.project(to_bits(x2), to_bits(w2)))
    assert within(to_bits(L.project(x2, w2, cfg(1, 16, 6))), to_bits(a))
