"""GPU parity of the MFMA kind (M = 4..32) against the CPU oracle, for every epilogue,
with and without the RMSNorm prologue, split-K on and off."""

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


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    bad = np.abs(g - w) > ATOL + RTOL * np.abs(w)
    if bad.any():
        where = np.argwhere(bad)
        print(f"{bad.sum()} of {bad.size} outside tolerance; first at {where[:8].tolist()}; "
              f"got {g[bad][:8].tolist()} want {w[bad][:8].tolist()}; "
              f"rows with errors {sorted(set(where[:, 0].tolist()))[:16]}; "
              f"cols mod 64 {sorted(set((where[:, -1] % 64).tolist()))[:16]}", flush=True)
    return not bad.any()


def cfg(rows=16, unroll=8, waves=8):
    return _native.Config(_native.KIND_MFMA, rows, unroll, 0, waves)


SHAPES = {"8B qkv": (6144, 4096), "8B o": (4096, 4096), "8B down": (4096, 12288), "0.6B o": (1024, 2048),
          "ragged": (1000, 520)}


@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("m", [4, 5, 8, 16, 17, 32])
def test_mfma_projection(cuda, name, m):
    n, k = SHAPES[name]
    x = seeded((m, k), seed=200 + m, device=cuda)
    w = seeded((n, k), seed=201, scale=0.02, device=cuda)
    first = L.project(x, w, cfg())
    again = L.project(x, w, cfg())
    got = to_bits(first)
    want = path.project(to_bits(x), to_bits(w))
    ok = within(got, want)
    assert torch.equal(first, again), "two identical calls differ"
    assert ok
    assert np.mean(got == want) >= 0.99


@pytest.mark.parametrize("m", [5, 16, 32])
def test_mfma_launch_shapes_agree_bit_for_bit(cuda, m):
    """Rows per workgroup and unroll only regroup work: for a given wave count every output is
    the same FP32 sum in the same order, bit for bit."""
    n, k = 4096, 4096
    x = seeded((m, k), seed=210, device=cuda)
    w = seeded((n, k), seed=211, scale=0.02, device=cuda)
    for waves in (4, 8):
        base = L.project(x, w, cfg(16, 8, waves))
        for rows, unroll in ((16, 4), (32, 4), (32, 8)):
            assert torch.equal(L.project(x, w, cfg(rows, unroll, waves)), base), (rows, unroll, waves)
    # the wave count changes the interleaving of K, hence the FP32 summation order: tolerance only
    assert within(to_bits(L.project(x, w, cfg(16, 4, 16))), to_bits(base))
    assert within(to_bits(L.project(x, w)), to_bits(base))  # planner default


@pytest.mark.parametrize("m", [5, 8, 16])
def test_mfma_rms_norm_prologue(cuda, m):
    n, k = 6144, 4096
    x = seeded((m, k), seed=220 + m, device=cuda)
    g = seeded((k,), seed=221, scale=0.1, shift=1.0, device=cuda)
    w = seeded((n, k), seed=222, scale=0.02, device=cuda)
    got = to_bits(L.rms_norm_linear(x, g, 1e-6, w))
    want = path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w))
    assert within(got, want)
    assert np.mean(got == want) >= 0.99


@pytest.mark.parametrize("m", [5, 8, 16])
@pytest.mark.parametrize("with_norm", [False, True])
def test_mfma_gate_up_swiglu(cuda, m, with_norm):
    i, k = 3072, 1024
    x = seeded((m, k), seed=230 + m, device=cuda)
    w = seeded((2 * i, k), seed=231, scale=0.02, device=cuda)
    g = seeded((k,), seed=232, scale=0.1, shift=1.0, device=cuda) if with_norm else None
    got = to_bits(S.gate_up_swiglu(x, w, g, 1e-6))
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), None if g is None else to_bits(g), 1e-6)
    assert within(got, want)
    assert np.mean(got == want) >= 0.99


@pytest.mark.parametrize("m", [5, 16])
@pytest.mark.parametrize("v,k", [(151936, 4096), (5000, 1024)])
def test_mfma_lm_head_argmax(cuda, m, v, k):
    x = seeded((m, k), seed=240 + m, device=cuda)
    w = seeded((v, k), seed=241, scale=0.02, device=cuda)
    g = seeded((k,), seed=242, scale=0.1, shift=1.0, device=cuda)
    top = torch.empty(m, dtype=torch.float32, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, top=top)
    want_logits, want_ids, _ = path.lm_head_argmax(to_bits(x), to_bits(w), to_bits(g), 1e-6)
    got_logits = to_bits(logits)
    assert within(got_logits, want_logits)
    ids = ids.cpu().numpy()
    v_sorted = np.sort(bf16.to_f32(want_logits).astype(np.float64), axis=-1)
    clear = (v_sorted[:, -1] - v_sorted[:, -2]) > 1e-2
    assert np.array_equal(ids[clear], want_ids[clear])
    assert np.array_equal(ids, path.argmax_first(got_logits))
    assert np.array_equal(top.cpu().numpy(), bf16.to_f32(got_logits)[np.arange(m), ids])


def test_mfma_argmax_ties_lowest_index(cuda):
    m, v, k = 5, 8192, 512
    x = seeded((1, k), seed=250, device=cuda).expand(m, k).contiguous()
    w = seeded((v, k), seed=251, scale=0.02, device=cuda)
    best = (x[0].float() * 10).to(torch.bfloat16) / 10
    for row in (7000, 64, 65):
        w[row] = best
    ids, _ = A.lm_head_argmax(x, w, logits=False)
    assert ids.tolist() == [64] * m


def test_calls_of_other_shapes_do_not_interfere(cuda):
    """Regression: a call with few tiles, then one with many, repeatedly (a shared-workspace
    layout once let the first corrupt the second)."""
    m = 5
    small_x = seeded((m, 520), seed=260, device=cuda)
    small_w = seeded((1000, 520), seed=261, scale=0.02, device=cuda)
    big_x = seeded((m, 4096), seed=262, device=cuda)
    big_w = seeded((6144, 4096), seed=263, scale=0.02, device=cuda)
    want = path.project(to_bits(big_x), to_bits(big_w))
    for _ in range(3):
        L.project(small_x, small_w)
        got = to_bits(L.project(big_x, big_w))
        assert within(got, want)
