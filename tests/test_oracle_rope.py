"""Pin the QK-norm + RoPE + cache oracle (oracle/rope.py) against checks independent of it.

- transformers' Qwen3RMSNorm (q_norm / k_norm) and apply_rotary_pos_emb, run by
  torch in BF16 on the CPU: the library formulation of the same function. The
  sum of squares may associate differently, so a few outputs may differ by one
  BF16 ulp; the rest are bit-equal. Dropping either product's rounding, or
  rounding x * inv_std after the gain, makes many outputs differ.
- the cache: exactly the slots position + t (or t in prefill) change; V is copied bit for bit;
- a Split's partials give the result of their rounded BF16 sum;
- the three phase modes (shared, per row, full tables + phases) agree when they name the same angles.
"""

import numpy as np
import pytest
import torch
from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb

from conftest import from_bits, to_bits
from oracle import bf16, rope


def _tables(positions, dim, theta=1_000_000.0):
    """BF16 cos/sin rows [len(positions), dim] of the Qwen3 rotary embedding."""
    inv = 1.0 / theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.tensor(positions, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _case(b, t, hq, hkv, d, cap, seed):
    g = torch.Generator().manual_seed(seed)
    packed = (torch.randn(b, t, (hq + 2 * hkv) * d, generator=g) * 2).to(torch.bfloat16)
    qg = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kg = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    keys = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16)
    values = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16)
    return packed, qg, kg, keys, values


def _hf(packed, qg, kg, eps, cos, sin, hq, hkv, d):
    """transformers' q_norm/k_norm and RoPE in torch BF16 on the CPU: (q [B,T,Hq,D], k [B,T,Hkv,D])."""
    b, t, _ = packed.shape
    q = packed[..., :hq * d].reshape(b, t, hq, d)
    k = packed[..., hq * d:(hq + hkv) * d].reshape(b, t, hkv, d)
    qn, kn = Qwen3RMSNorm(d, eps=eps), Qwen3RMSNorm(d, eps=eps)
    with torch.no_grad():
        qn.weight.copy_(qg.float())
        kn.weight.copy_(kg.float())
    qn, kn = qn.to(torch.bfloat16), kn.to(torch.bfloat16)
    with torch.no_grad():
        qe, ke = apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
    return qe.transpose(1, 2).contiguous(), ke.transpose(1, 2).contiguous()


def _ulps(a_bits, b_bits):
    return np.abs(a_bits.astype(np.int32) - b_bits.astype(np.int32))


@pytest.mark.parametrize("b,t,hq,hkv,d", [(1, 1, 32, 8, 128), (2, 3, 4, 2, 128), (3, 2, 8, 4, 64)])
def test_matches_transformers_bf16(b, t, hq, hkv, d):
    cap, position = 40, 17
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=b * 10 + t)
    cos, sin = _tables([position + i for i in range(t)], d)
    q, k_cache, v_cache = rope.qk_rope_cache(to_bits(packed), 1, to_bits(qg), to_bits(kg), 1e-6, 1e-6,
                                             to_bits(cos[None]), to_bits(sin[None]), [position],
                                             to_bits(keys), to_bits(values), hq)
    want_q, want_k = _hf(packed, qg, kg, 1e-6, cos[None], sin[None], hq, hkv, d)
    got_k = k_cache[:, :, position:position + t].transpose(0, 2, 1, 3)
    for got, want in ((q, to_bits(want_q)), (got_k, to_bits(want_k))):
        assert _ulps(got, want).max() <= 1
        assert np.mean(got == want) >= 0.999


def test_misplaced_roundings_would_be_caught():
    """Keeping either RoPE product in FP32, or the norm product before rounding, changes many outputs."""
    b, t, hq, hkv, d = 1, 2, 8, 2, 128
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, 8, seed=99)
    cos, sin = _tables([3, 4], d)
    x = bf16.to_f32(to_bits(packed)).reshape(b, t, -1, d)
    c, s = bf16.to_f32(to_bits(cos)), bf16.to_f32(to_bits(sin))
    good = rope.head_norm_rope(x[0, 0, 0], bf16.to_f32(to_bits(qg)), 1e-6, c[0], s[0])

    def fused_products(xv, gain, eps, cv, sv):
        inv = np.float32(1) / np.sqrt(np.mean(xv * xv, dtype=np.float32) + np.float32(eps), dtype=np.float32)
        w = bf16.round_f32(bf16.round_f32(xv * inv) * gain)
        rot = np.concatenate([-w[d // 2:], w[:d // 2]])
        return bf16.round_f32(w * cv + rot * sv)  # one rounding for the sum of FP32 products

    bad = fused_products(x[0, 0, 0], bf16.to_f32(to_bits(qg)), 1e-6, c[0], s[0])
    assert np.mean(good != bad) > 0.05


def test_cache_slots_and_value_copy():
    b, t, hq, hkv, d, cap = 2, 3, 4, 2, 128, 20
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=5)
    cos, sin = _tables([9, 10, 11], d)
    _, k_cache, v_cache = rope.qk_rope_cache(to_bits(packed), 1, to_bits(qg), to_bits(kg), 1e-6, 1e-6,
                                             to_bits(cos[None]), to_bits(sin[None]), [9], to_bits(keys),
                                             to_bits(values), hq)
    changed = np.any(k_cache != to_bits(keys), axis=-1)
    assert changed[:, :, 9:12].all() and not changed[:, :, :9].any() and not changed[:, :, 12:].any()
    v_slots = to_bits(packed).reshape(b, t, hq + 2 * hkv, d)[:, :, hq + hkv:].transpose(0, 2, 1, 3)
    np.testing.assert_array_equal(v_cache[:, :, 9:12], v_slots)
    untouched = np.ones(cap, bool)
    untouched[9:12] = False
    np.testing.assert_array_equal(v_cache[:, :, untouched], to_bits(values)[:, :, untouched])
    # prefill writes slots 0..T-1
    _, k_pre, _ = rope.qk_rope_cache(to_bits(packed), 1, to_bits(qg), to_bits(kg), 1e-6, 1e-6,
                                     to_bits(cos[None]), to_bits(sin[None]), [0, 1, 2], to_bits(keys),
                                     to_bits(values), hq, prefill=True)
    np.testing.assert_array_equal(k_pre[:, :, :3], k_cache[:, :, 9:12])


def test_split_partials_give_their_rounded_sum():
    b, t, hq, hkv, d = 1, 2, 4, 2, 64
    _, qg, kg, keys, values = _case(b, t, hq, hkv, d, 8, seed=7)
    g = torch.Generator().manual_seed(8)
    partial = torch.randn(3, b, t, (hq + 2 * hkv) * d, generator=g)
    rounded = (partial[0] + partial[1] + partial[2]).to(torch.bfloat16)
    cos, sin = _tables([2, 3], d)
    args = (to_bits(qg), to_bits(kg), 1e-6, 1e-5, to_bits(cos[None]), to_bits(sin[None]), [2],
            to_bits(keys), to_bits(values), hq)
    a = rope.qk_rope_cache(partial.numpy(), 3, *args)
    r = rope.qk_rope_cache(to_bits(rounded), 1, *args)
    for x, y in zip(a, r):
        np.testing.assert_array_equal(x, y)


def test_phase_modes_agree():
    b, t, hq, hkv, d, cap = 2, 2, 4, 2, 128, 32
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=13)
    pos = [5, 11]
    full_cos, full_sin = _tables(list(range(cap)), d)
    per_row = [full_cos[[p + i for p in pos for i in range(t)]], full_sin[[p + i for p in pos for i in range(t)]]]
    common = (to_bits(qg), to_bits(kg), 1e-6, 1e-6)
    rows = rope.qk_rope_cache(to_bits(packed), 1, *common, to_bits(per_row[0].reshape(b, t, d)),
                              to_bits(per_row[1].reshape(b, t, d)), pos, to_bits(keys), to_bits(values), hq,
                              rows=True)
    phases = np.tile(np.arange(t, dtype=np.int64), (b, 1))
    table = rope.qk_rope_cache(to_bits(packed), 1, *common, to_bits(full_cos), to_bits(full_sin), pos,
                               to_bits(keys), to_bits(values), hq, rows=True, phases=phases)
    for x, y in zip(rows, table):
        np.testing.assert_array_equal(x, y)
    # one row at a shared position: the shared-table mode gives the same bits
    shared = rope.qk_rope_cache(to_bits(packed[:1]), 1, *common, to_bits(full_cos[5:7][None]),
                                to_bits(full_sin[5:7][None]), [5], to_bits(keys[:1]), to_bits(values[:1]), hq)
    for x, y in zip(shared, rows):
        np.testing.assert_array_equal(x, y[:1])
