"""GPU parity of the STREAM kind (x slice in registers, rolling weight prefetch).

For the same K split (KW waves per row group) the STREAM kind adds the same FP32
products in the same order as the GEMV kind: per lane in chunk order, the DPP
tree over lanes, the KW wave totals in wave order; its RMSNorm prologue sums
squares in the other kinds' thread order. So STREAM output must equal the GEMV
kind's bit for bit, for every epilogue, with and without the prologue, for every
grid depth (1..8 tiles per workgroup). Against the CPU oracle the bar is
|y - ref| <= 2e-2 + 1e-2|ref| and bit-exact argmax ids.
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

#: (rows per group, chunks per lane C, KW): the instantiated STREAM shapes (K = 512 C KW).
STREAM_SHAPES = ((2, 1, 2), (4, 1, 2), (8, 1, 2), (2, 1, 4), (4, 1, 4), (2, 3, 2), (4, 3, 2), (2, 2, 4), (4, 2, 4),
                 (8, 2, 4), (2, 6, 4), (4, 6, 4), (2, 3, 8))
#: The 8-row kernel (M = 5..8; rows past M are zero and never stored).
STREAM_SHAPES_8 = ((2, 2, 4), (4, 2, 4), (2, 3, 8), (4, 3, 8))


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def stream(rpw, kw, gpc=0):
    return _native.Config(_native.KIND_STREAM, rpw, 0, gpc, kw)


def gemv(kw):
    # Any GEMV launch shape with the same KW adds in the same order; (2, 1, KW) exists for KW 2 and 4.
    return _native.Config(_native.KIND_GEMV, 2, 1 if kw > 1 else 4, 0, kw)


def _same_as_gemv(kw):
    # KW = 8 (an 8-wave workgroup) has no GEMV-kind twin.
    return kw <= 4


def _inputs(m, n, k, seed, device):
    x = seeded((m, k), seed=seed, device=device)
    w = seeded((n, k), seed=seed + 1, scale=0.02, device=device)
    g = seeded((k,), seed=seed + 2, scale=0.1, shift=1.0, device=device)
    return x, w, g


@pytest.mark.parametrize("rpw,c,kw", STREAM_SHAPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_store_equals_gemv_kind_and_oracle(cuda, rpw, c, kw, m):
    k = 512 * c * kw
    n = 1000 + 8 * rpw + 3  # ragged last tile
    x, w, g = _inputs(m, n, k, seed=200 + rpw + 10 * c + m, device=cuda)
    got = L.project(x, w, stream(rpw, kw))
    assert not _same_as_gemv(kw) or torch.equal(got, L.project(x, w, gemv(kw)))
    assert within(to_bits(got), path.project(to_bits(x), to_bits(w)))
    normed = L.rms_norm_linear(x, g, 1e-6, w, config=stream(rpw, kw))
    assert not _same_as_gemv(kw) or torch.equal(normed, L.rms_norm_linear(x, g, 1e-6, w, config=gemv(kw)))
    assert within(to_bits(normed), path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w)))


@pytest.mark.parametrize("rpw,c,kw", [s for s in STREAM_SHAPES if s[0] % 2 == 0])
@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("with_norm", [False, True])
def test_swiglu_equals_gemv_kind_and_oracle(cuda, rpw, c, kw, m, with_norm):
    k = 512 * c * kw
    i = 700 + rpw // 2 + 1
    x, w, g = _inputs(m, 2 * i, k, seed=300 + rpw + 10 * c + m, device=cuda)
    g = g if with_norm else None
    got = S.gate_up_swiglu(x, w, g, 1e-6, config=stream(rpw, kw))
    assert not _same_as_gemv(kw) or torch.equal(got, S.gate_up_swiglu(x, w, g, 1e-6, config=gemv(kw)))
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), None if g is None else to_bits(g), 1e-6)
    assert within(to_bits(got), want)


@pytest.mark.parametrize("rpw,c,kw", [(8, 1, 2), (4, 2, 4), (8, 2, 4), (2, 6, 4)])
@pytest.mark.parametrize("m", [1, 3])
def test_argmax_equals_gemv_kind_and_oracle(cuda, rpw, c, kw, m):
    k = 512 * c * kw
    v = 20000 + rpw
    x, w, g = _inputs(m, v, k, seed=400 + rpw + 10 * c + m, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=stream(rpw, kw))
    ids_g, logits_g = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=gemv(kw))
    assert torch.equal(logits, logits_g) and torch.equal(ids, ids_g)
    want = path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w))
    assert within(to_bits(logits), want)
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))
    # without the logits buffer: same ids
    ids_only, none = A.lm_head_argmax(x, w, g, 1e-6, logits=False, config=stream(rpw, kw))
    assert none is None and torch.equal(ids_only, ids)


@pytest.mark.parametrize("rpw,c,kw", STREAM_SHAPES_8)
@pytest.mark.parametrize("m", [5, 6, 7, 8])
def test_eight_row_kernel_matches_oracle(cuda, rpw, c, kw, m):
    """M = 5..8 on the 8-row kernel: every epilogue, with and without the norm prologue."""
    k = 512 * c * kw
    n = 2 * (600 + rpw) + 2
    x, w, g = _inputs(m, n, k, seed=700 + rpw + 10 * c + m, device=cuda)
    xb, wb, gb = to_bits(x), to_bits(w), to_bits(g)
    cfg = stream(rpw, kw)
    assert L.plan(m, n, k, _native.EPI_STORE, config=cfg).kind == _native.KIND_STREAM
    assert within(to_bits(L.project(x, w, cfg)), path.project(xb, wb))
    assert within(to_bits(L.rms_norm_linear(x, g, 1e-6, w, config=cfg)), path.norm_project(xb, gb, 1e-6, wb))
    for gain in (None, g):
        got = S.gate_up_swiglu(x, w, gain, 1e-6, config=cfg)
        assert got.shape == (m, n // 2)
        assert within(to_bits(got), path.gate_up_swiglu(xb, wb, None if gain is None else gb, 1e-6))
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=cfg)
    assert within(to_bits(logits), path.norm_project(xb, gb, 1e-6, wb))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))
    # the padded rows change nothing: row 0 alone gives the same bits as row 0 of the batch
    # (same K split, same per-lane order: bit for bit)
    one = L.rms_norm_linear(x[:1], g, 1e-6, w, config=stream(2, kw))
    assert torch.equal(one, L.rms_norm_linear(x, g, 1e-6, w, config=cfg)[:1])


def test_eight_row_kernel_is_the_default_for_long_k_with_the_norm(cuda):
    # (without the prologue, M = 5..8 at K = 12288 runs the QUAD kind)
    for m in (5, 8):
        assert L.plan(m, 4096, 12288, prologue=True).kind == _native.KIND_STREAM


@pytest.mark.parametrize("gpc", [1, 2, 3, 8, 64])
def test_grid_depth_does_not_change_bits(cuda, gpc):
    """Workgroups walking 1..8 tiles: the per-tile sums do not depend on the walk."""
    x, w, g = _inputs(2, 24000, 4096, seed=500, device=cuda)
    base = L.rms_norm_linear(x, g, 1e-6, w, config=stream(4, 4, 64))
    p = L.plan(2, 24000, 4096, _native.EPI_STORE, config=stream(4, 4, gpc))
    assert 1 <= -(-p.tiles // p.grid) <= 8
    assert torch.equal(L.rms_norm_linear(x, g, 1e-6, w, config=stream(4, 4, gpc)), base)


def test_argmax_ties_take_lowest_index(cuda):
    """Duplicate weight rows give exactly tied logits; the lowest index must win across workgroups."""
    k, v = 4096, 30000
    x, w, g = _inputs(1, v, k, seed=600, device=cuda)
    w[29999] = (x[0].float() * 0.05).to(torch.bfloat16)  # aligned with x: a clear winner ...
    w[15000] = w[29999]  # ... tied with an earlier row in another workgroup
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=stream(4, 4, 1))
    assert int(ids[0]) == int(path.argmax_first(to_bits(logits))[0])
    assert logits[0, 15000] == logits[0, 29999] and int(ids[0]) <= 15000


def test_default_plan_is_stream_for_model_shapes(cuda):
    for n, k in ((6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288), (4096, 1024), (1024, 2048), (1024, 3072)):
        assert L.plan(1, n, k).kind == _native.KIND_STREAM, (n, k)


#: One wave per row group (KW = 1) at one x row: whole rows per wave, no LDS round or barrier in the
#: STORE / SwiGLU epilogue (rows per wave, chunks per lane C; K = 512 C).
STREAM_SHAPES_KW1 = ((1, 1), (2, 1), (1, 2), (2, 2), (1, 3), (2, 3), (1, 4), (2, 4), (1, 6), (2, 6), (1, 8), (2, 8))


@pytest.mark.parametrize("rpw,c", STREAM_SHAPES_KW1)
@pytest.mark.parametrize("gpc", [0, 1])
def test_one_wave_per_row_group_equals_gemv_kind_and_oracle(cuda, rpw, c, gpc):
    """KW = 1: every epilogue, with and without the prologue (whose sum of squares each wave forms in
    the other kinds' thread order), bit for bit as the GEMV kind with KW = 1, within the bar of the
    oracle; the planner's grid (gpc 0) or one workgroup per CU walking 4..8 tiles (gpc 1)."""
    k = 512 * c
    n = 8000 + 4 * rpw + 3  # ragged last tile
    x, w, g = _inputs(1, n, k, seed=800 + rpw + 10 * c, device=cuda)
    cfg = stream(rpw, 1, gpc)
    assert L.plan(1, n, k, _native.EPI_STORE, config=cfg).kind == _native.KIND_STREAM
    got = L.project(x, w, cfg)
    assert torch.equal(got, L.project(x, w, gemv(1)))
    assert within(to_bits(got), path.project(to_bits(x), to_bits(w)))
    normed = L.rms_norm_linear(x, g, 1e-6, w, config=cfg)
    assert torch.equal(normed, L.rms_norm_linear(x, g, 1e-6, w, config=gemv(1)))
    assert within(to_bits(normed), path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w)))
    # the norm's scale is the other kinds' bit for bit: the standalone norm, then the plain call
    from kernels.rmsnorm import rms_norm
    assert torch.equal(normed, L.project(rms_norm(x, g, 1e-6), w, cfg))
    # residual prologue: the stored sum and the projection
    r = seeded((1, k), seed=801, device=cuda)
    y_r, s_r = L.add_rms_norm_linear(x, r, g, 1e-6, w, config=cfg)
    y_g, s_g = L.add_rms_norm_linear(x, r, g, 1e-6, w, config=gemv(1))
    assert torch.equal(y_r, y_g) and torch.equal(s_r, s_g)
    if rpw % 2 == 0:
        for gain in (None, g):
            sw = S.gate_up_swiglu(x, w[: 2 * (n // 2)], gain, 1e-6, config=cfg)
            assert torch.equal(sw, S.gate_up_swiglu(x, w[: 2 * (n // 2)], gain, 1e-6, config=gemv(1)))
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=cfg)
    ids_g, logits_g = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=gemv(1))
    assert torch.equal(logits, logits_g) and torch.equal(ids, ids_g)
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


@pytest.mark.parametrize("n,k,epi,pro", [(4096, 1024, 0, False), (4096, 1024, 0, True), (6144, 1024, 1, True),
                                         (1024, 2048, 0, False), (1024, 3072, 0, False), (6144, 4096, 0, True),
                                         (4096, 4096, 0, False), (24576, 4096, 1, True)])
def test_one_wave_per_row_group_at_model_shapes(cuda, n, k, epi, pro):
    """The Qwen3 0.6B / 8B M = 1 shapes on KW = 1 against the oracle (and against the planner's
    default launch within one BF16 ulp, two after SwiGLU's second rounding: the K split differs, so
    the FP32 sums are ordered differently)."""
    x, w, g = _inputs(1, n, k, seed=900 + n % 97 + k % 89, device=cuda)
    cfg = stream(2, 1)
    if epi == _native.EPI_SWIGLU:
        got = S.gate_up_swiglu(x, w, g if pro else None, 1e-6, config=cfg)
        want = path.gate_up_swiglu(to_bits(x), to_bits(w), to_bits(g) if pro else None, 1e-6)
        base = S.gate_up_swiglu(x, w, g if pro else None, 1e-6)
    elif pro:
        got = L.rms_norm_linear(x, g, 1e-6, w, config=cfg)
        want = path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w))
        base = L.rms_norm_linear(x, g, 1e-6, w)
    else:
        got = L.project(x, w, cfg)
        want = path.project(to_bits(x), to_bits(w))
        base = L.project(x, w)
    assert within(to_bits(got), want)
    diff = np.abs(to_bits(got).astype(np.int32) - to_bits(base).astype(np.int32))
    assert diff.max() <= (2 if epi == _native.EPI_SWIGLU else 1)
