"""GPU parity of the fused prologue/epilogue forms against the CPU oracle.

  rms_norm_linear   RMSNorm prologue + projection  (oracle.path.norm_project)
  gate_up_swiglu    gate/up projection + SwiGLU    (oracle.path.gate_up_swiglu)
  lm_head_argmax    final norm + lm_head + argmax  (oracle.path.lm_head_argmax)

Tolerance |y - ref| <= 2e-2 + 1e-2|ref|; argmax ids bit-exact wherever the
oracle's top-2 logit gap exceeds 1e-2, and always bit-exact on exact ties.
"""

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import argmax as A
from kernels import linear as L
from kernels import rmsnorm as R
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def gamma(k, seed, device):
    return seeded((k,), seed=seed, scale=0.1, shift=1.0, device=device)


@pytest.mark.parametrize("n,k", [(4096, 1024), (6144, 4096), (1000, 512), (24, 2048)])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_rms_norm_linear(cuda, m, n, k):
    x = seeded((m, k), seed=20 + m, device=cuda)
    g = gamma(k, 30 + m, cuda)
    w = seeded((n, k), seed=40 + m, scale=0.02, device=cuda)
    got = to_bits(L.rms_norm_linear(x, g, 1e-6, w))
    want = path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w))
    assert within(got, want)
    assert np.mean(got == want) >= 0.99


def test_rms_norm_linear_ragged_k_decomposes(cuda):
    x = seeded((1, 300), seed=50, device=cuda)
    g = gamma(300, 51, cuda)
    w = seeded((200, 300), seed=52, scale=0.02, device=cuda)
    got = to_bits(L.rms_norm_linear(x, g, 1e-6, w))
    assert within(got, path.norm_project(to_bits(x), to_bits(g), 1e-6, to_bits(w)))


@pytest.mark.parametrize("i,k", [(3072, 1024), (12288, 4096), (500, 512)])
@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("with_norm", [False, True])
def test_gate_up_swiglu(cuda, m, i, k, with_norm):
    x = seeded((m, k), seed=60 + m, device=cuda)
    w = seeded((2 * i, k), seed=70 + m, scale=0.02, device=cuda)
    g = gamma(k, 80 + m, cuda) if with_norm else None
    got = to_bits(S.gate_up_swiglu(x, w, g, 1e-6))
    want = path.gate_up_swiglu(to_bits(x), to_bits(w), None if g is None else to_bits(g), 1e-6)
    assert got.shape == (m, i)
    assert within(got, want)
    assert np.mean(got == want) >= 0.99
    # same as the two-step reference composition on our own kernels
    xn = x if g is None else R.rms_norm(x, g, 1e-6)
    two_step = to_bits(S.swiglu(L.linear(xn, w)))
    assert within(got, two_step)


def _top2_gap(logits_bits):
    v = np.sort(bf16.to_f32(logits_bits).astype(np.float64), axis=-1)
    return v[..., -1] - v[..., -2]


@pytest.mark.parametrize("v,k", [(151936, 4096), (32000, 1024), (1001, 512)])
@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("with_norm", [False, True])
def test_lm_head_argmax(cuda, m, v, k, with_norm):
    x = seeded((m, k), seed=90 + m, device=cuda)
    w = seeded((v, k), seed=91 + m, scale=0.02, device=cuda)
    g = gamma(k, 92 + m, cuda) if with_norm else None
    top = torch.empty(m, dtype=torch.float32, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, top=top)
    want_logits, want_ids, _ = path.lm_head_argmax(to_bits(x), to_bits(w), None if g is None else to_bits(g), 1e-6)
    got_logits = to_bits(logits)
    assert within(got_logits, want_logits)
    ids = ids.cpu().numpy()
    clear = _top2_gap(want_logits) > 1e-2
    assert np.array_equal(ids[clear], want_ids[clear])
    # ids are exactly the argmax of the kernel's own BF16 logits, and top is that logit
    assert np.array_equal(ids, path.argmax_first(got_logits))
    assert np.array_equal(top.cpu().numpy(), bf16.to_f32(got_logits)[np.arange(m), ids])


@pytest.mark.parametrize("m", [1, 3])
def test_lm_head_argmax_exact_ties_lowest_index(cuda, m):
    """Rows 17, 4000 and 30001 of W are identical and win: the id must be 17 (argmax.py:1-9)."""
    v, k = 32768, 512
    x = seeded((m, k), seed=95, device=cuda)
    w = seeded((v, k), seed=96, scale=0.02, device=cuda)
    best = (x[0].float() * 10).to(torch.bfloat16) / 10
    for row in (30001, 4000, 17):
        w[row] = best
    ids, logits = A.lm_head_argmax(x[:1].expand(m, k).contiguous(), w, logits=True)
    assert ids.tolist() == [17] * m
    # int32 ids, no logits
    ids32, none = A.lm_head_argmax(x[:1], w, logits=False, ids_dtype=torch.int32)
    assert none is None and ids32.dtype == torch.int32 and ids32.tolist() == [17]


def test_fused_argmax_and_greedy_tokens_api(cuda):
    m, v, k = 2, 4096, 256
    x = seeded((m, k), seed=97, device=cuda)
    w = seeded((v, k), seed=98, scale=0.02, device=cuda)
    ids = A.fused_argmax(x, w)
    assert ids.dtype == torch.int64 and ids.shape == (m,)
    assert torch.equal(A.greedy_tokens(x, w, L.linear), ids)
    top = torch.empty(m, dtype=torch.float32, device=cuda)
    ids2, logits = A.greedy_tokens(x, w, L.linear, top=top)
    assert torch.equal(ids2, ids)
    assert torch.equal(A.argmax(logits), ids)
    # another linear is honoured
    ids3 = A.greedy_tokens(x, w, lambda a, b: torch.nn.functional.linear(a, b))
    assert ids3.shape == (m,)


def test_lm_head_deterministic(cuda):
    x = seeded((1, 4096), seed=99, device=cuda)
    w = seeded((151936, 4096), seed=100, scale=0.02, device=cuda)
    a = A.lm_head_argmax(x, w, logits=True)
    b = A.lm_head_argmax(x, w, logits=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
