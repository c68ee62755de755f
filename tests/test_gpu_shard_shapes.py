"""GPU parity at one GPU's share of a Qwen3-8B eight-way tensor-parallel layer (the shapes the path
would run sharded: QKV by heads, 768 x 4096; O by its input, 4096 x 512; gate/up by the intermediate
rows, 2 x 1536 x 4096; down by its input, 4096 x 1536; lm_head by vocabulary, 18992 x 4096), on the
planner's default launches, at 1..16 rows, against the oracle: |y - ref| <= 2e-2 + 1e-2|ref|, argmax
ids equal to the first maximum of the kernel's own BF16 logits. These shapes take launches the
full-size model does not: one wave per row group at K = 512 and 1536, and QUAD's 4-row tiles where
RING's would leave most CUs idle."""

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

H, Q, I, V = 4096, 768, 1536, 18992
EPS = 1e-6


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= 2e-2 + 1e-2 * np.abs(w)))


@pytest.fixture(scope="module")
def shard(cuda):
    return {"qkv": seeded((Q, H), seed=1100, scale=0.02, device=cuda),
            "o": seeded((H, H // 8), seed=1101, scale=0.02, device=cuda),
            "gate_up": seeded((2 * I, H), seed=1102, scale=0.02, device=cuda),
            "down": seeded((H, I), seed=1103, scale=0.02, device=cuda),
            "head": seeded((V, H), seed=1104, scale=0.02, device=cuda),
            "gain": seeded((H,), seed=1105, scale=0.1, shift=1.0, device=cuda)}


@pytest.mark.parametrize("m", [1, 2, 4, 5, 8, 16])
def test_shard_projections_match_oracle(cuda, shard, m):
    x = seeded((m, H), seed=1110 + m, device=cuda)
    g = shard["gain"]
    xb, gb = to_bits(x), to_bits(g)
    qkv = L.rms_norm_linear(x, g, EPS, shard["qkv"])
    assert within(to_bits(qkv), path.norm_project(xb, gb, EPS, to_bits(shard["qkv"])))
    attn = seeded((m, H // 8), seed=1120 + m, device=cuda)
    o = L.linear(attn, shard["o"])
    assert within(to_bits(o), path.project(to_bits(attn), to_bits(shard["o"])))
    act = S.gate_up_swiglu(x, shard["gate_up"], g, EPS)
    assert within(to_bits(act), path.gate_up_swiglu(xb, to_bits(shard["gate_up"]), gb, EPS))
    h = seeded((m, I), seed=1130 + m, device=cuda)
    down = L.linear(h, shard["down"])
    assert within(to_bits(down), path.project(to_bits(h), to_bits(shard["down"])))
    ids, logits = A.lm_head_argmax(x, shard["head"], g, EPS, logits=True)
    assert within(to_bits(logits), path.norm_project(xb, gb, EPS, to_bits(shard["head"])))
    np.testing.assert_array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))


def test_shard_launch_choices(cuda):
    """The launches these shapes get: one wave per row group at M = 1 for the short rows (K = 512,
    1536), and QUAD with 4-row tiles for the shard's QKV at 4..8 rows (192 tiles where RING has 64)."""
    for n, k in ((H, H // 8), (H, I)):
        p = L.plan(1, n, k)
        assert p.kind == _native.KIND_STREAM and p.waves == 1, (n, k)
    for m in (4, 5, 8):
        p = L.plan(m, Q, H, prologue=True)
        assert p.kind == _native.KIND_QUAD and p.rows_per_wave == 4 and p.tiles == Q // 4, m
