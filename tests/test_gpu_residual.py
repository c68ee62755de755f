"""GPU parity of the residual side of the prologue (add_rms_norm / embed_rms_norm folded in).

The fused calls must give what the reference's separate launches give
(engine/decode.py:229-261: add_rms_norm or embed_rms_norm, then the layer's
projection): projections within |y - ref| <= 2e-2 + 1e-2|ref| of the CPU
oracle, greedy ids bit-exact, and the stored residual stream (x + residual,
or the gathered embedding rows) bit for bit: it is a BF16 add or a copy.
Every kind that has the fused form is covered: STREAM (M <= 8), QUAD and STAGE
(M <= 16; MFMA_STREAM in its own file), the LDS-staged GEMV (K not 512 C KW), the
MFMA kind (its row-scale pre-pass stores the rows), and shapes with no fused
form fall back to the separate kernels with the same results.
"""

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import argmax as A
from kernels import linear as L
from kernels import rmsnorm as R
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def _inputs(m, n, k, seed, device):
    x = seeded((m, k), seed=seed, device=device)
    r = seeded((m, k), seed=seed + 1, device=device)
    w = seeded((n, k), seed=seed + 2, scale=0.02, device=device)
    g = seeded((k,), seed=seed + 3, scale=0.1, shift=1.0, device=device)
    return x, r, w, g


# (M, N, K, the kind the planner picks)
CASES = [
    (1, 1536, 4096, _native.KIND_STREAM), (3, 1000, 4096, _native.KIND_STREAM),
    (4, 777, 1024, _native.KIND_QUAD), (2, 500, 12288, _native.KIND_STREAM),
    (5, 1500, 4096, _native.KIND_QUAD), (16, 2000, 4096, _native.KIND_STAGE),
    (7, 900, 12288, _native.KIND_STREAM), (12, 1200, 4096, _native.KIND_STAGE),
    (2, 700, 1000, _native.KIND_GEMV), (6, 700, 1000, _native.KIND_MFMA), (20, 640, 4096, _native.KIND_MFMA),
]


@pytest.mark.parametrize("m,n,k,kind", CASES)
def test_add_rms_norm_linear(cuda, m, n, k, kind):
    x, r, w, g = _inputs(m, n, k, seed=1500 + m + k, device=cuda)
    assert L.plan(m, n, k, prologue=True, residual=True).kind == kind
    x0, r0 = x.clone(), r.clone()
    y, summed = L.add_rms_norm_linear(x, r, g, 1e-6, w)
    want_y, want_sum = path.add_norm_project(to_bits(x), to_bits(r), to_bits(g), 1e-6, to_bits(w))
    np.testing.assert_array_equal(to_bits(summed), want_sum)
    assert within(to_bits(y), want_y)
    assert torch.equal(x, x0) and torch.equal(r, r0)  # inputs untouched


@pytest.mark.parametrize("m,n,k,kind", [c for c in CASES if c[1] % 2 == 0])
def test_gate_up_swiglu_with_residual(cuda, m, n, k, kind):
    x, r, w, g = _inputs(m, n, k, seed=1600 + m + k, device=cuda)
    act, summed = S.gate_up_swiglu(x, w, g, 1e-6, residual=r)
    normed, want_sum = path.add_rms_norm(to_bits(x), to_bits(r), to_bits(g), 1e-6)
    np.testing.assert_array_equal(to_bits(summed), want_sum)
    assert act.shape == (m, n // 2)
    assert within(to_bits(act), path.gate_up_swiglu(normed, to_bits(w)))


@pytest.mark.parametrize("m", [1, 4, 5, 16])
def test_lm_head_argmax_with_residual(cuda, m):
    k, v = 4096, 30000 + 3
    x, r, w, g = _inputs(m, v, k, seed=1700 + m, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, residual=r)
    normed, _ = path.add_rms_norm(to_bits(x), to_bits(r), to_bits(g), 1e-6)
    assert within(to_bits(logits), path.project(normed, to_bits(w)))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


@pytest.mark.parametrize("m,k", [(1, 4096), (4, 1024), (5, 4096), (3, 1000)])
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_embed_rms_norm_linear(cuda, m, k, ids_dtype):
    vocab, n = 5000, 1200
    table = seeded((vocab, k), seed=1800 + m, device=cuda)
    g = seeded((k,), seed=1801, scale=0.1, shift=1.0, device=cuda)
    w = seeded((n, k), seed=1802, scale=0.02, device=cuda)
    token_ids = torch.tensor([4999, 0, 17, 17, 2500][:m], dtype=ids_dtype, device=cuda)
    y, hidden = L.embed_rms_norm_linear(token_ids, table, g, 1e-6, w)
    normed, want_hidden = path.embed_rms_norm(token_ids.cpu().numpy(), to_bits(table), to_bits(g), 1e-6)
    np.testing.assert_array_equal(to_bits(hidden), want_hidden)
    assert within(to_bits(y), path.project(normed, to_bits(w)))


@pytest.mark.parametrize("m", [1, 3, 5])
def test_embed_gather_clamps_ids_outside_the_table(cuda, m):
    """Device-side ids outside [0, rows) read the nearest table row: no read leaves the table."""
    vocab, k, n = 300, 1024, 512
    table = seeded((vocab, k), seed=1850, device=cuda)
    g = seeded((k,), seed=1851, scale=0.1, shift=1.0, device=cuda)
    w = seeded((n, k), seed=1852, scale=0.02, device=cuda)
    token_ids = torch.tensor([vocab, -1, 10 ** 9, 7, -(10 ** 9)][:m], dtype=torch.int64, device=cuda)
    y, hidden = L.embed_rms_norm_linear(token_ids, table, g, 1e-6, w)
    clamped = token_ids.clamp(0, vocab - 1).cpu().numpy()
    normed, want_hidden = path.embed_rms_norm(clamped, to_bits(table), to_bits(g), 1e-6)
    np.testing.assert_array_equal(to_bits(hidden), want_hidden)
    assert within(to_bits(y), path.project(normed, to_bits(w)))


def test_embed_rms_norm_standalone(cuda):
    table = seeded((1000, 1024), seed=1900, device=cuda)
    g = seeded((1024,), seed=1901, scale=0.1, shift=1.0, device=cuda)
    token_ids = torch.tensor([[5, 999, 0]], dtype=torch.int64, device=cuda)
    y, hidden = R.embed_rms_norm(token_ids, table, g, 1e-6)
    want_y, want_hidden = path.embed_rms_norm(token_ids.cpu().numpy(), to_bits(table), to_bits(g), 1e-6)
    assert y.shape == hidden.shape == (1, 3, 1024)
    np.testing.assert_array_equal(to_bits(hidden), want_hidden)
    assert np.mean(to_bits(y) == want_y) >= 0.999 and within(to_bits(y), want_y)


def test_fused_matches_separate_launches(cuda):
    """The fused residual prologue and the reference's two launches agree (tolerance: the norm's sum order)."""
    x, r, w, g = _inputs(1, 6144, 4096, seed=2000, device=cuda)
    y, summed = L.add_rms_norm_linear(x, r, g, 1e-6, w)
    normed, summed2 = R.add_rms_norm(x, r, g, 1e-6)
    assert torch.equal(summed, summed2)
    assert within(to_bits(y), to_bits(L.linear(normed, w)))


def test_decode_layer_chain(cuda):
    """Two layers of the decode data flow of engine/decode.py:229-261 with every norm fused."""
    k, n_qkv, n_gu = 1024, 2048, 3072
    vocab = 4000
    table = seeded((vocab, k), seed=2100, device=cuda)
    token = torch.tensor([1234], dtype=torch.int64, device=cuda)
    layers = []
    for i in range(2):
        layers.append(dict(
            ln1=seeded((k,), seed=2200 + i, scale=0.1, shift=1.0, device=cuda),
            ln2=seeded((k,), seed=2210 + i, scale=0.1, shift=1.0, device=cuda),
            qkv=seeded((n_qkv, k), seed=2220 + i, scale=0.02, device=cuda),
            gate_up=seeded((n_gu, k), seed=2230 + i, scale=0.02, device=cuda),
            down=seeded((k, n_gu // 2), seed=2240 + i, scale=0.02, device=cuda)))
    attn = seeded((1, k), seed=2300, device=cuda)  # stand-in attention output (outside the path)
    # fused
    qkv, resid = L.embed_rms_norm_linear(token, table, layers[0]["ln1"], 1e-6, layers[0]["qkv"])
    hidden = None
    for i, lw in enumerate(layers):
        if i:
            qkv, resid = L.add_rms_norm_linear(hidden, resid, lw["ln1"], 1e-6, lw["qkv"])
        act, resid = S.gate_up_swiglu(attn, lw["gate_up"], lw["ln2"], 1e-6, residual=resid)
        hidden = L.linear(act, lw["down"])
    # oracle
    _, o_resid = path.embed_rms_norm(token.cpu().numpy(), to_bits(table), to_bits(layers[0]["ln1"]), 1e-6)
    o_hidden = None
    for i, lw in enumerate(layers):
        if i:
            _, o_resid = path.add_norm_project(o_hidden, o_resid, to_bits(lw["ln1"]), 1e-6, to_bits(lw["qkv"]))
        normed, o_resid = path.add_rms_norm(to_bits(attn), o_resid, to_bits(lw["ln2"]), 1e-6)
        o_hidden = path.project(path.gate_up_swiglu(normed, to_bits(lw["gate_up"])), to_bits(lw["down"]))
    assert within(to_bits(hidden), o_hidden)
    assert within(to_bits(resid), o_resid)


def test_overlapping_sum_is_rejected(cuda):
    x, r, w, g = _inputs(1, 512, 1024, seed=2400, device=cuda)
    out = torch.empty((1, 512), dtype=torch.bfloat16, device=cuda)
    # sum aliasing the residual it is computed from: workgroup 0 would overwrite rows others still read
    with pytest.raises(_native.FtkError, match="invalid argument"):
        L.fused_project(x, w, _native.EPI_STORE, out, g, 1e-6, residual=r, summed=r)
    with pytest.raises(_native.FtkError, match="invalid argument"):  # a residual without the norm it feeds
        L.fused_project(x, w, _native.EPI_STORE, out, None, 1e-6, residual=r, summed=torch.empty_like(r))
