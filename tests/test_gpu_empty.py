"""Empty inputs: every projection, norm, SwiGLU and argmax entry point returns outputs of the
right shape (zero rows) and launches nothing, as torch's own F.linear does on empty input."""

import pytest
import torch

from conftest import seeded

from kernels import argmax as A
from kernels import linear as L
from kernels import rmsnorm as R
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

K, N, I = 256, 64, 96
EPS = 1e-6


@pytest.mark.parametrize("lead", [(0,), (0, 1), (2, 0)])
def test_empty_rows(cuda, lead):
    x = torch.empty((*lead, K), device=cuda, dtype=torch.bfloat16)
    w = seeded((N, K), seed=1, scale=0.02, device=cuda)
    g = seeded((K,), seed=2, scale=0.1, shift=1.0, device=cuda)
    wgu = seeded((2 * I, K), seed=3, scale=0.02, device=cuda)
    out_shape = (*lead, N)

    assert L.linear(x, w).shape == out_shape
    assert L.project(x.reshape(0, K), w).shape == (0, N)
    assert L.rms_norm_linear(x, g, EPS, w).shape == out_shape
    y, s = L.add_rms_norm_linear(x, torch.empty_like(x), g, EPS, w)
    assert y.shape == out_shape and s.shape == x.shape
    assert L.linear_residual(x, w, torch.empty(out_shape, device=cuda, dtype=torch.bfloat16)).shape == out_shape
    assert S.gate_up_swiglu(x, wgu, g, EPS).shape == (*lead, I)
    act, s = S.gate_up_swiglu(x, wgu, g, EPS, residual=torch.empty_like(x))
    assert act.shape == (*lead, I) and s.shape == x.shape
    assert S.swiglu(torch.empty((*lead, 2 * I), device=cuda, dtype=torch.bfloat16)).shape == (*lead, I)
    assert R.rms_norm(x, g, EPS).shape == x.shape
    y, s = R.add_rms_norm(x, torch.empty_like(x), g, EPS)
    assert y.shape == s.shape == x.shape
    ids, logits = A.lm_head_argmax(x, w, g, EPS)
    assert ids.shape == lead and logits.shape == out_shape
    assert A.argmax(torch.empty(out_shape, device=cuda, dtype=torch.bfloat16)).shape == lead


def test_empty_token_ids(cuda):
    table = seeded((16, K), seed=4, device=cuda)
    g = seeded((K,), seed=5, scale=0.1, shift=1.0, device=cuda)
    w = seeded((N, K), seed=6, scale=0.02, device=cuda)
    ids = torch.empty((1, 0), device=cuda, dtype=torch.int64)
    y, h = R.embed_rms_norm(ids, table, g, EPS)
    assert y.shape == h.shape == (1, 0, K)
    y, h = L.embed_rms_norm_linear(ids, table, g, EPS, w)
    assert y.shape == (1, 0, N) and h.shape == (1, 0, K)
