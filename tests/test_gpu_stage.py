"""GPU parity of the STAGE kind (M <= 16: QUAD's weight loads staged through LDS into 16x16x32 MFMAs).

Against the CPU oracle: |y - ref| <= 2e-2 + 1e-2|ref| for every epilogue, with
and without the RMSNorm prologue (and its residual / gathered rows), and
bit-exact greedy ids. Within the kind: the grid (how many tiles each workgroup
walks) and the window depth only move work and loads, so they never change a
bit; an x row's outputs come from its own MFMA column and its own row scale,
so a call with fewer rows reproduces those rows of a 16-row call bit for bit.
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

#: (T subtiles, K, KW, U): every epilogue and both prologue settings ...
SHAPES_EVEN = ((2, 4096, 8, 2), (2, 4096, 8, 4))
#: ... store / argmax ...
SHAPES_ONE = ((1, 4096, 8, 2), (1, 4096, 8, 4))
#: ... and the long K without the prologue (x streamed beside the weights).
SHAPES_LONG = ((1, 12288, 8, 3), (1, 12288, 8, 4))


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def cfg(t, kw, u, gpc=0):
    return _native.Config(_native.KIND_STAGE, 16 * t, u, gpc, kw)


def _inputs(m, n, k, seed, device):
    x = seeded((m, k), seed=seed, device=device)
    w = seeded((n, k), seed=seed + 1, scale=0.02, device=device)
    g = seeded((k,), seed=seed + 2, scale=0.1, shift=1.0, device=device)
    return x, w, g


@pytest.mark.parametrize("t,k,kw,u", SHAPES_EVEN + SHAPES_ONE + SHAPES_LONG)
@pytest.mark.parametrize("m", [1, 5, 9, 16])
def test_store_matches_oracle(cuda, t, k, kw, u, m):
    n = 1000 + 16 * t + 5  # ragged last tile
    x, w, g = _inputs(m, n, k, seed=3000 + 10 * t + kw + u + m, device=cuda)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    c = cfg(t, kw, u)
    assert L.plan(m, n, k, config=c).kind == _native.KIND_STAGE
    assert within(to_bits(L.project(x, w, c)), path.project(xb, wb))
    if (t, k, kw, u) not in SHAPES_LONG:
        normed = L.rms_norm_linear(x, g, 1e-6, w, config=c)
        assert within(to_bits(normed), path.norm_project(xb, gb, 1e-6, wb))


@pytest.mark.parametrize("t,k,kw,u", SHAPES_EVEN)
@pytest.mark.parametrize("m", [5, 16])
@pytest.mark.parametrize("with_norm", [False, True])
def test_swiglu_matches_oracle(cuda, t, k, kw, u, m, with_norm):
    i = 700 + 8 * t + 3
    x, w, g = _inputs(m, 2 * i, k, seed=3100 + 10 * t + kw + u + m, device=cuda)
    g = g if with_norm else None
    got = S.gate_up_swiglu(x, w, g, 1e-6, config=cfg(t, kw, u))
    assert got.shape == (m, i)
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), None if g is None else to_bits(g), 1e-6)
    assert within(to_bits(got), want)


@pytest.mark.parametrize("t,k,kw,u", SHAPES_EVEN + SHAPES_ONE)
@pytest.mark.parametrize("m", [5, 16])
def test_argmax_matches_oracle(cuda, t, k, kw, u, m):
    v = 20000 + 16 * t + 7
    x, w, g = _inputs(m, v, k, seed=3200 + 10 * t + kw + u + m, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=cfg(t, kw, u))
    assert within(to_bits(logits), path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w)))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))
    ids_only, none = A.lm_head_argmax(x, w, g, 1e-6, logits=False, config=cfg(t, kw, u))
    assert none is None and torch.equal(ids_only, ids)


def test_argmax_forced_ties_take_the_lowest_index(cuda):
    """Duplicated weight rows give exactly equal logits: the lowest index must win."""
    k, v, m = 4096, 9000, 11
    x, w, g = _inputs(m, v, k, seed=3300, device=cuda)
    w[5000] = w[17] * 4  # a clear winner, duplicated at higher and lower indices
    w[7000] = w[5000]
    w[123] = w[5000]
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=cfg(1, 8, 2))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


@pytest.mark.parametrize("gpc", [1, 2, 4])
def test_grid_and_window_do_not_change_bits(cuda, gpc):
    x, w, g = _inputs(13, 12000, 4096, seed=3400, device=cuda)
    base = L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 8, 2, 8))
    p = L.plan(13, 12000, 4096, config=cfg(1, 8, 2, gpc), prologue=True)
    assert 1 <= p.grid <= p.tiles
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 8, 2, gpc)), base)
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 8, 4, gpc)), base)
    x2, w2, _ = _inputs(16, 3000, 12288, seed=3410, device=cuda)  # x streamed
    assert torch.equal(L.project(x2, w2, cfg(1, 8, 3, gpc)), L.project(x2, w2, cfg(1, 8, 4, 8)))


@pytest.mark.parametrize("epi", ["store", "swiglu", "argmax"])
def test_walks_longer_than_the_lds_depth(cuda, epi):
    """One workgroup per CU walks more tiles than its LDS parks (8 with one subtile, 4 with two): the
    epilogue runs every depth tiles inside the walk. The bits equal those of a grid whose walks fit,
    and the oracle's bar holds."""
    m, n, k = 5, 41000, 4096
    t = 2 if epi == "swiglu" else 1
    x, w, g = _inputs(m, n, k, seed=3600 + t, device=cuda)
    epilogue = {"store": _native.EPI_STORE, "swiglu": _native.EPI_SWIGLU, "argmax": _native.EPI_ARGMAX}[epi]
    long_walks, short_walks = cfg(t, 8, 2, 1), cfg(t, 8, 2, 16)
    p = L.plan(m, n, k, epilogue, config=long_walks, prologue=True)
    assert p.kind == _native.KIND_STAGE and -(-p.tiles // p.grid) > 64 // (8 * t)
    q = L.plan(m, n, k, epilogue, config=short_walks, prologue=True)
    assert -(-q.tiles // q.grid) <= 64 // (8 * t)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    if epi == "store":
        got = L.rms_norm_linear(x, g, 1e-6, w, config=long_walks)
        assert torch.equal(got, L.rms_norm_linear(x, g, 1e-6, w, config=short_walks))
        assert within(to_bits(got), path.norm_project(xb, gb, 1e-6, wb))
    elif epi == "swiglu":
        got = S.gate_up_swiglu(x, w, g, 1e-6, config=long_walks)
        assert torch.equal(got, S.gate_up_swiglu(x, w, g, 1e-6, config=short_walks))
        assert within(to_bits(got), path.gate_up_swiglu(xb, wb, gb, 1e-6))
    else:
        ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=long_walks)
        ids2, logits2 = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=short_walks)
        assert torch.equal(ids, ids2) and torch.equal(logits, logits2)
        assert within(to_bits(logits), path.lm_head_argmax(xb, wb, gb, 1e-6)[0])
        np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


@pytest.mark.parametrize("with_norm", [False, True])
def test_rows_are_independent(cuda, with_norm):
    """Each x row's outputs come from its own MFMA column and its own row scale."""
    x, w, g = _inputs(16, 3000, 4096, seed=3500, device=cuda)
    c = cfg(1, 8, 2)
    full = L.rms_norm_linear(x, g, 1e-6, w, config=c) if with_norm else L.project(x, w, c)
    for lo, hi in ((0, 1), (7, 8), (15, 16), (3, 12)):
        part = L.rms_norm_linear(x[lo:hi], g, 1e-6, w, config=c) if with_norm else L.project(x[lo:hi], w, c)
        assert torch.equal(part, full[lo:hi]), (lo, hi)


@pytest.mark.parametrize("m", [5, 16])
def test_residual_and_gathered_rows(cuda, m):
    """The prologue's residual add and embedding gather, the stored sum bit-exact."""
    k, n = 4096, 1500
    x, w, g = _inputs(m, n, k, seed=3600 + m, device=cuda)
    r = seeded((m, k), seed=3610 + m, device=cuda)
    c = cfg(1, 8, 2)
    y, summed = L.add_rms_norm_linear(x, r, g, 1e-6, w, config=c)
    want_y, want_sum = path.add_norm_project(to_bits(x), to_bits(r), to_bits(g), 1e-6, to_bits(w))
    np.testing.assert_array_equal(to_bits(summed), want_sum)
    assert within(to_bits(y), want_y)
    table = seeded((64, k), seed=3620 + m, device=cuda)
    ids = torch.tensor([(3 * i + 2) % 64 for i in range(m)], device=cuda, dtype=torch.int64)
    y2, hidden = L.embed_rms_norm_linear(ids, table, g, 1e-6, w, config=c)
    rows = to_bits(table)[ids.cpu().numpy()]
    np.testing.assert_array_equal(to_bits(hidden), rows)
    assert within(to_bits(y2), path.norm_project(rows, to_bits(g), 1e-6, to_bits(w)))


def test_matches_mfma_stream_within_tolerance(cuda):
    x, w, g = _inputs(16, 4096, 4096, seed=3700, device=cuda)
    a = L.rms_norm_linear(x, g, 1e-6, w, config=cfg(1, 8, 2))
    b = L.rms_norm_linear(x, g, 1e-6, w, config=_native.Config(_native.KIND_MFMA_STREAM, 16, 4, 0, 16))
    assert within(to_bits(a), to_bits(b))
