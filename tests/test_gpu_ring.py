"""GPU parity of the RING kind (M = 1..16: weight and x segments loaded straight into a per-wave LDS
ring, 16x16x32 MFMAs).

Against the CPU oracle: |y - ref| <= 2e-2 + 1e-2|ref| for every epilogue, with and without the
RMSNorm prologue (and its gathered rows), the residual add in the STORE epilogue, and bit-exact
greedy ids. Within the kind: the grid (how many tiles each workgroup walks, and so how often the
epilogue runs inside the walk) only moves work, so it never changes a bit; an x row's outputs come
from its own MFMA column and its own row scale, so a call with fewer rows reproduces those rows of
a 16-row call bit for bit. A captured graph replays bit for bit as the eager call.
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
EPS = 1e-6


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def cfg(depth=2, gpc=0, rows=16):
    return _native.Config(_native.KIND_RING, rows, depth, gpc, 8)


def _inputs(m, n, k, seed, device):
    x = seeded((m, k), seed=seed, device=device)
    w = seeded((n, k), seed=seed + 1, scale=0.02, device=device)
    g = seeded((k,), seed=seed + 2, scale=0.1, shift=1.0, device=device)
    return x, w, g


@pytest.mark.parametrize("m", [1, 2, 5, 8, 9, 16])
def test_store_matches_oracle(cuda, m):
    n, k = 1000 + 5, 4096  # ragged last tile
    x, w, g = _inputs(m, n, k, seed=5000 + m, device=cuda)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    assert L.plan(m, n, k, config=cfg()).kind == _native.KIND_RING
    assert within(to_bits(L.project(x, w, cfg())), path.project(xb, wb))
    assert within(to_bits(L.rms_norm_linear(x, g, EPS, w, config=cfg())), path.norm_project(xb, gb, EPS, wb))


@pytest.mark.parametrize("m", [2, 5, 8])
@pytest.mark.parametrize("n", [6144, 1000 + 5, 24 * 300 + 17])
def test_24_row_tiles_match_oracle(cuda, m, n):
    """24-row tiles (two MFMA subtiles, the second half used), with and without the prologue; the
    ragged last tile clamps its rows. Bit for bit the 16-row tiles' sums of the same rows."""
    k = 4096
    x, w, g = _inputs(m, n, k, seed=5050 + m + n, device=cuda)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    wide = cfg(rows=24)
    p = L.plan(m, n, k, config=wide)
    assert p.kind == _native.KIND_RING and p.rows_per_wave == 24 and p.tiles == -(-n // 24)
    y = L.project(x, w, wide)
    assert within(to_bits(y), path.project(xb, wb))
    assert torch.equal(y, L.project(x, w, cfg()))
    normed = L.rms_norm_linear(x, g, EPS, w, config=wide)
    assert within(to_bits(normed), path.norm_project(xb, gb, EPS, wb))
    assert torch.equal(normed, L.rms_norm_linear(x, g, EPS, w, config=cfg()))


@pytest.mark.parametrize("m", [2, 5, 8, 9, 16])
@pytest.mark.parametrize("n", [6144, 1000 + 5, 12 * 300 + 7])
def test_12_row_tiles_match_oracle(cuda, m, n):
    """12-row tiles (one MFMA subtile, its last four rows unused; the second tile runs from
    registers), with and without the prologue; the ragged last tile clamps its rows. Bit for bit
    the 16-row tiles' sums of the same rows."""
    k = 4096
    x, w, g = _inputs(m, n, k, seed=5070 + m + n, device=cuda)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    narrow = cfg(rows=12)
    p = L.plan(m, n, k, config=narrow)
    assert p.kind == _native.KIND_RING and p.rows_per_wave == 12 and p.tiles == -(-n // 12)
    y = L.project(x, w, narrow)
    assert within(to_bits(y), path.project(xb, wb))
    assert torch.equal(y, L.project(x, w, cfg()))
    normed = L.rms_norm_linear(x, g, EPS, w, config=narrow)
    assert within(to_bits(normed), path.norm_project(xb, gb, EPS, wb))
    assert torch.equal(normed, L.rms_norm_linear(x, g, EPS, w, config=cfg()))
    r = seeded((m, n), seed=5080 + m, device=cuda)
    assert torch.equal(L.linear_residual(x, w, r, config=narrow), L.linear_residual(x, w, r, config=cfg()))


def test_12_row_walks_and_graph_replays(cuda):
    """12-row tiles walked far past the LDS depth by one workgroup (the epilogue inside the walk),
    equal to short walks, and replayed from a captured graph bit for bit."""
    m, n, k = 8, 12 * 2600 + 5, 4096
    x, w, g = _inputs(m, n, k, seed=5090, device=cuda)
    long_walks, short_walks = cfg(2, 1, rows=12), cfg(2, 16, rows=12)
    p = L.plan(m, n, k, config=long_walks, prologue=True)
    assert p.kind == _native.KIND_RING and -(-p.tiles // p.grid) > 8
    got = L.rms_norm_linear(x, g, EPS, w, config=long_walks)
    assert torch.equal(got, L.rms_norm_linear(x, g, EPS, w, config=short_walks))
    assert within(to_bits(got), path.norm_project(to_bits(x), to_bits(g), EPS, to_bits(w)))
    eager = to_bits(got).copy()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        L.rms_norm_linear(x, g, EPS, w, config=long_walks)
        with torch.cuda.graph(graph, stream=stream):
            out = L.rms_norm_linear(x, g, EPS, w, config=long_walks)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_bits(out), eager)


@pytest.mark.parametrize("m,depth", [(5, 2), (5, 3), (8, 3), (16, 2)])
def test_long_k_matches_oracle(cuda, m, depth):
    """K = 12288 (the down projection): x travels with every unit."""
    n, k = 700 + 9, 12288
    x, w, _ = _inputs(m, n, k, seed=5100 + m + depth, device=cuda)
    assert within(to_bits(L.project(x, w, cfg(depth))), path.project(to_bits(x), to_bits(w)))


def test_shapes_the_ring_does_not_take_are_refused(cuda):
    for m, k, depth, epilogue, pro in ((16, 12288, 3, _native.EPI_STORE, False),  # 16 x rows x 3 units: no LDS
                                       (5, 12288, 2, _native.EPI_STORE, True),    # no prologue at K = 12288
                                       (5, 4096, 3, _native.EPI_STORE, False),    # 3 does not divide C = 4
                                       (17, 4096, 2, _native.EPI_STORE, False)):  # past 16 rows
        status = _native.lib().ftk_plan_project(m, 4096, k, epilogue | (_native.PLAN_PROLOGUE if pro else 0),
                                                256, cfg(depth), _native.Plan())
        assert status != _native.FTK_OK, (m, k, depth, pro)
    for m, epilogue in ((9, _native.EPI_STORE), (5, _native.EPI_SWIGLU), (5, _native.EPI_ARGMAX)):
        status = _native.lib().ftk_plan_project(m, 6144, 4096, epilogue, 256, cfg(rows=24), _native.Plan())
        assert status != _native.FTK_OK, (m, epilogue)  # 24-row tiles: STORE at up to 8 x rows
    for m, epilogue, k in ((5, _native.EPI_SWIGLU, 4096), (5, _native.EPI_ARGMAX, 4096), (5, _native.EPI_STORE, 12288)):
        status = _native.lib().ftk_plan_project(m, 6144, k, epilogue, 256, cfg(rows=12), _native.Plan())
        assert status != _native.FTK_OK, (m, epilogue, k)  # 12-row tiles: STORE at K = 4096


@pytest.mark.parametrize("m", [5, 16])
@pytest.mark.parametrize("with_norm", [False, True])
def test_swiglu_matches_oracle(cuda, m, with_norm):
    i = 700 + 3  # ragged: the last tile's gate / up rows clamp
    x, w, g = _inputs(m, 2 * i, 4096, seed=5200 + m, device=cuda)
    g = g if with_norm else None
    got = S.gate_up_swiglu(x, w, g, EPS, config=cfg())
    assert got.shape == (m, i)
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), None if g is None else to_bits(g), EPS)
    assert within(to_bits(got), want)


@pytest.mark.parametrize("m", [5, 16])
def test_argmax_matches_oracle(cuda, m):
    v = 20000 + 7
    x, w, g = _inputs(m, v, 4096, seed=5300 + m, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, EPS, logits=True, config=cfg())
    assert within(to_bits(logits), path.norm_project(to_bits(x), to_bits(g), EPS, to_bits(w)))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))
    ids_only, none = A.lm_head_argmax(x, w, g, EPS, logits=False, config=cfg(), ids_dtype=torch.int32)
    assert none is None and ids_only.dtype == torch.int32
    np.testing.assert_array_equal(ids_only.cpu().numpy(), ids.cpu().numpy())


def test_argmax_forced_ties_take_the_lowest_index(cuda):
    """Duplicated weight rows give exactly equal logits: the lowest index must win."""
    k, v, m = 4096, 9000, 11
    x, w, g = _inputs(m, v, k, seed=5400, device=cuda)
    w[5000] = w[17] * 4
    w[7000] = w[5000]
    w[123] = w[5000]
    ids, logits = A.lm_head_argmax(x, w, g, EPS, logits=True, config=cfg())
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


@pytest.mark.parametrize("epi", ["store", "swiglu", "argmax"])
def test_walks_longer_than_the_lds_depth(cuda, epi):
    """One workgroup per CU walks far more tiles than its LDS parks: the epilogue runs inside the
    walk with the ring in flight. The bits equal those of a grid whose walks are short."""
    m, n, k = 5, 41000, 4096
    x, w, g = _inputs(m, n, k, seed=5500, device=cuda)
    epilogue = {"store": _native.EPI_STORE, "swiglu": _native.EPI_SWIGLU, "argmax": _native.EPI_ARGMAX}[epi]
    long_walks, short_walks = cfg(2, 1), cfg(2, 16)
    p = L.plan(m, n, k, epilogue, config=long_walks, prologue=True)
    assert p.kind == _native.KIND_RING and -(-p.tiles // p.grid) > 8
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    if epi == "store":
        got = L.rms_norm_linear(x, g, EPS, w, config=long_walks)
        assert torch.equal(got, L.rms_norm_linear(x, g, EPS, w, config=short_walks))
        assert within(to_bits(got), path.norm_project(xb, gb, EPS, wb))
    elif epi == "swiglu":
        got = S.gate_up_swiglu(x, w, g, EPS, config=long_walks)
        assert torch.equal(got, S.gate_up_swiglu(x, w, g, EPS, config=short_walks))
        assert within(to_bits(got), path.gate_up_swiglu(xb, wb, gb, EPS))
    else:
        ids, logits = A.lm_head_argmax(x, w, g, EPS, logits=True, config=long_walks)
        ids2, logits2 = A.lm_head_argmax(x, w, g, EPS, logits=True, config=short_walks)
        assert torch.equal(ids, ids2) and torch.equal(logits, logits2)
        assert within(to_bits(logits), path.lm_head_argmax(xb, wb, gb, EPS)[0])
        np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


@pytest.mark.parametrize("with_norm", [False, True])
def test_rows_are_independent(cuda, with_norm):
    """Each x row's outputs come from its own MFMA column and its own row scale, whether 8 or 16 x
    rows travel with the weights."""
    x, w, g = _inputs(16, 3000, 4096, seed=5600, device=cuda)
    c = cfg()
    full = L.rms_norm_linear(x, g, EPS, w, config=c) if with_norm else L.project(x, w, c)
    for lo, hi in ((0, 2), (6, 8), (14, 16), (3, 12), (0, 9)):
        part = L.rms_norm_linear(x[lo:hi], g, EPS, w, config=c) if with_norm else L.project(x[lo:hi], w, c)
        assert torch.equal(part, full[lo:hi]), (lo, hi)


@pytest.mark.parametrize("m", [5, 16])
def test_gathered_rows_and_the_residual_epilogue(cuda, m):
    """The embedding-gather prologue; the residual add in the STORE epilogue (linear_residual)."""
    k, n = 4096, 1500
    x, w, g = _inputs(m, n, k, seed=5700 + m, device=cuda)
    table = seeded((64, k), seed=5710 + m, device=cuda)
    ids = torch.tensor([(3 * i + 2) % 64 for i in range(m)], device=cuda, dtype=torch.int64)
    y, hidden = L.embed_rms_norm_linear(ids, table, g, EPS, w, config=cfg())
    rows = to_bits(table)[ids.cpu().numpy()]
    np.testing.assert_array_equal(to_bits(hidden), rows)
    assert within(to_bits(y), path.norm_project(rows, to_bits(g), EPS, to_bits(w)))
    r = seeded((m, n), seed=5720 + m, device=cuda)
    got = L.linear_residual(x, w, r, config=cfg())
    # bit for bit the same kind's projection plus r (one BF16 add); the projection is the oracle's
    # within tolerance
    plain = to_bits(L.project(x, w, cfg()))
    np.testing.assert_array_equal(to_bits(got), bf16.round_bits(bf16.to_f32(plain) + bf16.to_f32(to_bits(r))))
    assert within(plain, path.project(to_bits(x), to_bits(w)))


def test_residual_prologue_is_refused(cuda):
    """The prologue's residual add is not a RING form: the C ABI refuses it (nothing launched) and
    add_rms_norm_linear takes its unfused path, still the oracle's result."""
    x, w, g = _inputs(5, 1500, 4096, seed=5800, device=cuda)
    r = seeded((5, 4096), seed=5810, device=cuda)
    out = torch.empty((5, 1500), device=cuda, dtype=torch.bfloat16)
    summed = torch.empty_like(r)
    status = L.fused_project(x, w, _native.EPI_STORE, out, g, EPS, residual=r, summed=summed, config=cfg())
    assert status == _native.FTK_ERR_UNSUPPORTED
    y, s = L.add_rms_norm_linear(x, r, g, EPS, w, config=cfg())
    want_y, want_sum = path.add_norm_project(to_bits(x), to_bits(r), to_bits(g), EPS, to_bits(w))
    np.testing.assert_array_equal(to_bits(s), want_sum)
    assert within(to_bits(y), want_y)


def test_graph_replays_match_eager(cuda):
    x, w, g = _inputs(8, 6144, 4096, seed=5900, device=cuda)
    wu = seeded((2 * 3072, 4096), seed=5903, scale=0.02, device=cuda)

    def step():
        return (L.rms_norm_linear(x, g, EPS, w, config=cfg()), S.gate_up_swiglu(x, wu, g, EPS, config=cfg()))

    eager = [to_bits(t).copy() for t in step()]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        step()
        with torch.cuda.graph(graph, stream=stream):
            outs = step()
    torch.cuda.synchronize()
    for _ in range(3):
        for t in outs:
            t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, eager):
            np.testing.assert_array_equal(to_bits(got), want)


def test_matches_stage_within_tolerance(cuda):
    x, w, g = _inputs(16, 4096, 4096, seed=6000, device=cuda)
    a = L.rms_norm_linear(x, g, EPS, w, config=cfg())
    b = L.rms_norm_linear(x, g, EPS, w, config=_native.Config(_native.KIND_STAGE, 16, 2, 0, 8))
    assert within(to_bits(a), to_bits(b))
