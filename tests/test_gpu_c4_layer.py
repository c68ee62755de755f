"""GPU parity of a whole Qwen3-8B decode layer's projections at 5, 8 and 16 rows (speculative
verify), at full size, through the public calls and the planner's default launches.

The four calls of engine/layers.py:30-60 at those rows: RMSNorm-prologue QKV (4096 -> 6144), O
(4096 -> 4096), RMSNorm-prologue gate/up + SwiGLU (4096 -> 2 x 12288) and down (12288 -> 4096),
each against the CPU oracle with |y - ref| <= 2e-2 + 1e-2|ref| and >= 99 % of outputs bit-equal.
Each call's input is the oracle's output of the call before, so every call sees the value range
it sees in a real layer. The launches are the ones a decode step takes with no tuning.
"""

import numpy as np
import pytest
import torch

from conftest import from_bits, seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import linear as L
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
EPS = 1e-6
H, QKV, I = 4096, 6144, 12288


def check(got, want):
    got_bits = to_bits(got)
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want).astype(np.float64)
    bad = np.abs(g - w) > ATOL + RTOL * np.abs(w)
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tolerance, first at {np.argwhere(bad)[:4].tolist()}"
    assert np.mean(got_bits == want) >= 0.99


@pytest.fixture(scope="module")
def weights(cuda):
    return {
        "g1": seeded((H,), seed=7101, scale=0.1, shift=1.0, device=cuda),
        "qkv": seeded((QKV, H), seed=7102, scale=0.02, device=cuda),
        "o": seeded((H, H), seed=7103, scale=0.02, device=cuda),
        "g2": seeded((H,), seed=7104, scale=0.1, shift=1.0, device=cuda),
        "gate_up": seeded((2 * I, H), seed=7105, scale=0.02, device=cuda),
        "down": seeded((H, I), seed=7106, scale=0.02, device=cuda),
    }


@pytest.mark.parametrize("m", [5, 8, 16])
def test_layer_projections_at_default_launches(cuda, weights, m):
    w = weights
    bits = {name: to_bits(t) for name, t in w.items()}
    x = seeded((m, H), seed=7200 + m, device=cuda)

    assert L.plan(m, QKV, H, prologue=True).kind == _native.KIND_RING
    want = path.norm_project(to_bits(x), bits["g1"], EPS, bits["qkv"])
    check(L.rms_norm_linear(x, w["g1"], EPS, w["qkv"]), want)

    attn = from_bits(want[:, :H], cuda)  # stands in for the attention output
    assert L.plan(m, H, H).kind == _native.KIND_RING
    want = path.project(to_bits(attn), bits["o"])
    check(L.linear(attn, w["o"]), want)

    h = from_bits(want, cuda)
    assert L.plan(m, 2 * I, H, epilogue=_native.EPI_SWIGLU, prologue=True).kind == _native.KIND_RING
    want = path.gate_up_swiglu(to_bits(h), bits["gate_up"], bits["g2"], EPS)
    got = S.gate_up_swiglu(h, w["gate_up"], w["g2"], EPS)
    assert got.shape == (m, I)
    check(got, want)

    act = from_bits(want, cuda)
    assert L.plan(m, H, I).kind == _native.KIND_RING
    check(L.linear(act, w["down"]), path.project(to_bits(act), bits["down"]))
    torch.cuda.synchronize()
