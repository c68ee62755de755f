"""Pin the decode-attention oracle (oracle/attention.py) against checks independent of it.

- torch's CPU scaled_dot_product_attention in float64 (a library routine; GQA
  by repeat_interleave, query head h reads KV head h // G), at the shapes and
  the tolerance of the reference's own test (agent/verify_gpu.py:154-174:
  atol 0.03125, rtol 0.01, magnitudes 1 and 3, unused slots NaN);
- one valid slot: softmax weight exactly 1, so the output is that value row;
- equal keys: equal weights, so integer-valued values average exactly;
- the split count and tile width only re-associate FP32 sums and move the
  BF16 rounding point of p, so every layout agrees to within one BF16 ulp;
- a transposed head mapping (h % Hkv) or a dropped log2(e) fails the first check.
"""

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from conftest import to_bits
from oracle import attention, bf16

#: (batch, kv_heads, dim, capacity, valid): agent/verify_gpu.py:154-157, capacities trimmed where
#: the pure-Python tile loop would take long (the kernel tests run the full ones).
REFERENCE_CASES = ((1, 8, 128, 1, 1), (1, 8, 128, 65, 1), (1, 8, 128, 65, 33), (1, 8, 128, 544, 513),
                   (2, 8, 128, 520, 500), (4, 8, 128, 160, 159), (2, 2, 64, 65, 65))


def _inputs(batch, kv_heads, dim, capacity, groups, magnitude, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(batch, kv_heads * groups, dim, generator=g) * magnitude).to(torch.bfloat16)
    k = (torch.randn(batch, kv_heads, capacity, dim, generator=g) * magnitude).to(torch.bfloat16)
    v = torch.randn(batch, kv_heads, capacity, dim, generator=g).to(torch.bfloat16)
    return q, k, v


def _sdpa(q, k, v, valid, scale):
    """float64 torch SDPA over slots [0, valid), GQA heads expanded by repeat_interleave."""
    groups = q.shape[1] // k.shape[1]
    kk = k[:, :, :valid].double().repeat_interleave(groups, dim=1)
    vv = v[:, :, :valid].double().repeat_interleave(groups, dim=1)
    out = F.scaled_dot_product_attention(q.double().unsqueeze(2), kk, vv, scale=scale)
    return out.squeeze(2).numpy()


@pytest.mark.parametrize("batch,kv_heads,dim,capacity,valid", REFERENCE_CASES)
@pytest.mark.parametrize("magnitude", [1.0, 3.0])
def test_oracle_matches_torch_sdpa(batch, kv_heads, dim, capacity, valid, magnitude):
    q, k, v = _inputs(batch, kv_heads, dim, capacity, 4, magnitude, seed=valid + capacity)
    scale = dim ** -0.5
    want = _sdpa(q, k, v, valid, scale)
    kb, vb = to_bits(k).copy(), to_bits(v).copy()
    kb[:, :, valid:] = 0x7FC0  # unused slots hold NaN: they must never be read into the result
    vb[:, :, valid:] = 0x7FC0
    got = bf16.to_f32(attention.decode_attention(to_bits(q), kb, vb, valid - 1, scale)).astype(np.float64)
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - want) <= 0.03125 + 0.01 * np.abs(want))
    # tighter than the bar: the FP32 path sits within a couple of BF16 roundings of the exact value
    assert np.max(np.abs(got - want)) < 0.02


def test_head_mapping_and_log2e_would_be_caught():
    """The closed-form check separates the right GQA mapping from h % Hkv, and exp2 without log2(e)."""
    q, k, v = _inputs(1, 4, 64, 48, 4, 3.0, seed=11)
    scale = 64 ** -0.5
    want = _sdpa(q, k, v, 48, scale)
    right = bf16.to_f32(attention.decode_attention(to_bits(q), to_bits(k), to_bits(v), 47, scale))
    assert np.max(np.abs(right - want)) < 0.02
    wrong_heads = torch.cat([q[:, i::4] for i in range(4)], dim=1)  # reorders heads like h % Hkv would
    moved = bf16.to_f32(attention.decode_attention(to_bits(wrong_heads), to_bits(k), to_bits(v), 47, scale))
    assert np.max(np.abs(moved - want)) > 0.1
    no_log2e = bf16.to_f32(attention.decode_attention(to_bits(q), to_bits(k), to_bits(v), 47,
                                                      scale / attention.LOG2E))
    assert np.max(np.abs(no_log2e - want)) > 0.05


def test_one_valid_slot_returns_its_value_row():
    q, k, v = _inputs(2, 2, 128, 40, 4, 3.0, seed=5)
    got = attention.decode_attention(to_bits(q), to_bits(k), to_bits(v), 0, 128 ** -0.5, splits=4)
    want = np.repeat(to_bits(v)[:, :, 0], 4, axis=1)
    np.testing.assert_array_equal(got, want)


def test_equal_keys_average_exactly():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 8, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 1, 64, generator=g).to(torch.bfloat16).expand(1, 2, 96, 64).contiguous()
    v = torch.randint(-8, 9, (1, 2, 96, 64), generator=g).to(torch.bfloat16)
    for valid, splits, block_n in ((96, 1, 32), (80, 3, 32), (37, 2, 16)):
        got = attention.decode_attention(to_bits(q), to_bits(k), to_bits(v), valid - 1, 0.125, block_n, splits)
        mean = v[:, :, :valid].double().mean(dim=2).repeat_interleave(4, dim=1)
        np.testing.assert_array_equal(got, bf16.from_f64(mean.numpy()))


def _ulp(x):
    """One BF16 ulp at |x| (8 significant bits)."""
    return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -20))) - 7)


def test_layouts_agree_within_bf16_rounding():
    q, k, v = _inputs(1, 2, 128, 300, 4, 3.0, seed=7)
    qb, kb, vb = to_bits(q), to_bits(k), to_bits(v)
    want = _sdpa(q, k, v, 291, 128 ** -0.5)
    base = bf16.to_f32(attention.decode_attention(qb, kb, vb, 290, 128 ** -0.5, 32, 1)).astype(np.float64)
    for block_n, splits in ((64, 1), (32, 8), (128, 3), (16, 32)):
        got = bf16.to_f32(attention.decode_attention(qb, kb, vb, 290, 128 ** -0.5, block_n, splits))
        # one BF16 ulp of the larger, or 2^-8 absolute where cancellation leaves a small output
        assert np.all(np.abs(got - base) <= np.maximum(_ulp(np.maximum(np.abs(got), np.abs(base))), 2.0 ** -8))
        assert np.max(np.abs(got - want)) < 0.0125


def test_default_splits_follows_the_reference_policy():
    # _default_config (decode_attention.py:152-157): block 32 below 16 groups, else 64;
    # min(32, cdiv(256, groups), cdiv(capacity, block)).
    assert attention.default_splits(1, 8, 4096) == 32
    assert attention.default_splits(16, 8, 640) == 2
    assert attention.default_splits(1, 8, 65) == 3
    assert attention.default_splits(4, 8, 2080) == 8
    assert attention.default_splits(1, 8, 1) == 1


def test_dense_reference_matches_torch_sdpa():
    q, k, v = _inputs(2, 2, 64, 50, 3, 1.0, seed=9)
    want = _sdpa(q, k, v, 41, 0.125)
    got = attention.dense_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), 41, 0.125)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
