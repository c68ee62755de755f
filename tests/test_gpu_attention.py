"""GPU parity of the split-KV decode attention (kernels/decode_attention.py, ftk_decode_attention_bf16).

Against the CPU oracle (oracle/attention.py) on the same seeded inputs:
|y - ref| <= 2e-2 + 1e-2|ref|, and against float64 torch SDPA with the
reference's own bar (agent/verify_gpu.py:154-174: atol 0.03125, rtol 0.01),
at that test's shapes and magnitudes, with NaN in every unused cache slot.
Launch choices (split count, waves, loads in flight) only re-associate FP32
sums and move the point where p is rounded, so any two agree to within one
BF16 ulp (or 2^-8 where cancellation leaves a small output).
"""

import ctypes

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from conftest import to_bits
from oracle import attention, bf16

from kernels import _native
from kernels import decode_attention as A

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2

#: (batch, kv_heads, dim, capacity, valid): agent/verify_gpu.py:154-157.
REFERENCE_CASES = ((1, 8, 128, 1, 1), (1, 8, 128, 65, 1), (1, 8, 128, 65, 33), (1, 8, 128, 544, 513),
                   (4, 8, 128, 2080, 2048), (16, 8, 128, 640, 639), (2, 2, 64, 65, 65))


def _inputs(batch, kv_heads, dim, capacity, groups, magnitude, seed, device):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(batch, kv_heads * groups, 1, dim, generator=g) * magnitude).to(torch.bfloat16)
    k = (torch.randn(batch, kv_heads, capacity, dim, generator=g) * magnitude).to(torch.bfloat16)
    v = torch.randn(batch, kv_heads, capacity, dim, generator=g).to(torch.bfloat16)
    return q.to(device), k.to(device), v.to(device)


def _sdpa(q, k, v, valid, scale):
    groups = q.shape[1] // k.shape[1]
    kk = k[:, :, :valid].cpu().double().repeat_interleave(groups, dim=1)
    vv = v[:, :, :valid].cpu().double().repeat_interleave(groups, dim=1)
    return F.scaled_dot_product_attention(q.cpu().double(), kk, vv, scale=scale).squeeze(2).numpy()


def _oracle(q, k, v, position, scale, **kw):
    b, h, _, d = q.shape
    return attention.decode_attention(to_bits(q).reshape(b, h, d), to_bits(k), to_bits(v), position, scale, **kw)


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def one_ulp(a_bits, b_bits):
    """|a - b| <= one BF16 ulp of the larger, or 2^-8 absolute."""
    a, b = bf16.to_f32(a_bits).astype(np.float64), bf16.to_f32(b_bits).astype(np.float64)
    big = np.maximum(np.maximum(np.abs(a), np.abs(b)), 2.0 ** -20)
    ulp = 2.0 ** (np.floor(np.log2(big)) - 7)
    return bool(np.all(np.abs(a - b) <= np.maximum(ulp, 2.0 ** -8)))


def cfg(splits=0, waves=0, unroll=0, kind=0):
    return _native.AttnConfig(kind, splits, waves, unroll)


def _nan_tail(k, v, valid):
    k[:, :, valid:] = float("nan")
    v[:, :, valid:] = float("nan")


@pytest.mark.parametrize("batch,kv_heads,dim,capacity,valid", REFERENCE_CASES)
@pytest.mark.parametrize("magnitude", [1.0, 3.0])
def test_reference_cases_match_oracle_and_sdpa(cuda, batch, kv_heads, dim, capacity, valid, magnitude):
    q, k, v = _inputs(batch, kv_heads, dim, capacity, 4, magnitude, seed=17 * valid + capacity, device=cuda)
    scale = dim ** -0.5
    want_exact = _sdpa(q, k, v, valid, scale)
    want = _oracle(q, k, v, valid - 1, scale)
    _nan_tail(k, v, valid)
    position = torch.tensor([valid - 1], device=cuda, dtype=torch.int64)
    got = A.decode_attention(q, k, v, position, scale)
    assert got.shape == (batch, 1, kv_heads * 4, dim)
    assert torch.isfinite(got).all()
    bits = to_bits(got).reshape(batch, kv_heads * 4, dim)
    assert within(bits, want)
    g = bf16.to_f32(bits).astype(np.float64)
    assert np.all(np.abs(g - want_exact) <= 0.03125 + 0.01 * np.abs(want_exact))


@pytest.mark.parametrize("splits", [1, 2, 7, 64, 256, 500])
@pytest.mark.parametrize("kind,waves,unroll", [(_native.ATTN_ROWS, 4, 2), (_native.ATTN_ROWS, 4, 4),
                                               (_native.ATTN_ROWS, 8, 2), (_native.ATTN_ROWS, 8, 4),
                                               (_native.ATTN_ROWS, 4, 8), (_native.ATTN_QUAD, 4, 1),
                                               (_native.ATTN_QUAD, 4, 2), (_native.ATTN_QUAD, 8, 1),
                                               (_native.ATTN_QUAD, 8, 2)])
@pytest.mark.parametrize("groups", [2, 4])
def test_launch_choices_agree(cuda, splits, kind, waves, unroll, groups):
    if kind == _native.ATTN_ROWS and unroll == 8 and groups > 2:
        pytest.skip("8 rows in flight fit the registers with up to 2 query heads per KV head")
    batch, kv_heads, dim, capacity, valid = 1, 4, 128, 1000, 937
    q, k, v = _inputs(batch, kv_heads, dim, capacity, groups, 3.0, seed=23, device=cuda)
    scale = dim ** -0.5
    want = _oracle(q, k, v, valid - 1, scale)
    _nan_tail(k, v, valid)
    position = torch.tensor([valid - 1], device=cuda, dtype=torch.int64)
    p = A.plan(batch, kv_heads * groups, kv_heads, capacity, dim, cfg(splits, waves, unroll, kind))
    assert (p.kind, p.chunk, p.waves, p.unroll) == (kind, -(-capacity // splits), waves, unroll)
    q3 = q.view(batch, kv_heads * groups, dim)
    got = to_bits(A.attend(q3, k, v, position, scale, cfg(splits, waves, unroll, kind))).reshape(want.shape)
    base = to_bits(A.attend(q3, k, v, position, scale, cfg(1, 4, 2, _native.ATTN_ROWS))).reshape(want.shape)
    assert within(got, want)
    assert one_ulp(got, base)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 6, 7, 8])
def test_every_group_size(cuda, dim, groups):
    batch, kv_heads, capacity, valid = 2, 2, 300, 271
    q, k, v = _inputs(batch, kv_heads, dim, capacity, groups, 1.0, seed=100 + 10 * groups + dim, device=cuda)
    scale = dim ** -0.5
    want = _oracle(q, k, v, valid - 1, scale)
    _nan_tail(k, v, valid)
    position = torch.tensor([valid - 1], device=cuda, dtype=torch.int64)
    got = A.decode_attention(q, k, v, position, scale)
    assert within(to_bits(got).reshape(want.shape), want)
    q3 = q.view(batch, kv_heads * groups, dim)
    kinds = [_native.ATTN_ROWS] + ([_native.ATTN_QUAD] if dim == 128 and groups <= 4 else [])
    for kind in kinds:
        for splits in (1, 3):
            got = A.attend(q3, k, v, position, scale, cfg(splits, kind=kind))
            assert within(to_bits(got).reshape(want.shape), want), (kind, splits)


def test_one_valid_slot_returns_its_value_row(cuda):
    """Softmax weight exactly 1: the output is the value row, bit for bit, for any split count."""
    q, k, v = _inputs(3, 8, 128, 500, 4, 3.0, seed=31, device=cuda)
    _nan_tail(k, v, 1)
    position = torch.zeros(1, device=cuda, dtype=torch.int64)
    want = to_bits(v[:, :, 0]).repeat(4, axis=1)
    for splits in (0, 1, 5, 64):
        got = A.attend(q.view(3, 32, 128), k, v, position, 128 ** -0.5, cfg(splits))
        np.testing.assert_array_equal(to_bits(got).reshape(want.shape), want)


def test_position_past_capacity_reads_every_slot(cuda):
    q, k, v = _inputs(1, 8, 128, 200, 4, 1.0, seed=37, device=cuda)
    scale = 128 ** -0.5
    want = _oracle(q, k, v, 199, scale)
    got = A.decode_attention(q, k, v, torch.tensor([1000], device=cuda, dtype=torch.int64), scale)
    assert within(to_bits(got).reshape(want.shape), want)


def test_per_row_positions(cuda):
    """positions = B: row b reads slots 0..position[b] (the C ABI's per-row form)."""
    batch, kv_heads, dim, capacity = 4, 8, 128, 700
    q, k, v = _inputs(batch, kv_heads, dim, capacity, 4, 1.0, seed=41, device=cuda)
    rows = [0, 333, 699, 64]
    scale = dim ** -0.5
    wants = [_oracle(q[b:b + 1], k[b:b + 1], v[b:b + 1], rows[b], scale) for b in range(batch)]
    for b, r in enumerate(rows):
        k[b, :, r + 1:] = float("nan")
        v[b, :, r + 1:] = float("nan")
    position = torch.tensor(rows, device=cuda, dtype=torch.int64)
    got = A.attend(q.view(batch, 32, dim), k, v, position, scale)
    bits = to_bits(got).reshape(batch, 32, dim)
    for b in range(batch):
        assert within(bits[b:b + 1], wants[b]), b


def test_graph_replays_follow_the_device_position(cuda):
    """The length lives on the device: one captured graph serves every position."""
    q, k, v = _inputs(1, 8, 128, 1024, 4, 1.0, seed=43, device=cuda)
    scale = 128 ** -0.5
    position = torch.tensor([100], device=cuda, dtype=torch.int64)
    A.decode_attention(q, k, v, position, scale)  # sizes the workspace eagerly
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = A.decode_attention(q, k, v, position, scale)
    torch.cuda.synchronize()
    for pos in (100, 1023, 0, 517, 517):
        position.fill_(pos)
        graph.replay()
        torch.cuda.synchronize()
        eager = A.decode_attention(q, k, v, position, scale)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), pos
        want = _oracle(q, k, v, pos, scale)
        assert within(to_bits(out).reshape(want.shape), want), pos


def test_long_context_against_the_closed_form(cuda):
    """32K slots at Qwen3-8B heads: against float64 SDPA (the tile oracle would take minutes here)."""
    q, k, v = _inputs(1, 8, 128, 32768, 4, 1.0, seed=47, device=cuda)
    scale = 128 ** -0.5
    want = _sdpa(q, k, v, 30000, scale)
    _nan_tail(k, v, 30000)
    got = A.decode_attention(q, k, v, torch.tensor([29999], device=cuda, dtype=torch.int64), scale)
    g = bf16.to_f32(to_bits(got)).astype(np.float64).reshape(want.shape)
    assert np.all(np.abs(g - want) <= 0.03125 + 0.01 * np.abs(want))
