"""numpy restatement of the reference's fused Q/K head RMSNorm + RoPE + KV-cache update (test infrastructure only).

Only tests/ and __graft_entry__.smoke() use this module, as the checker.

Restates engine/kernels/qk_rope.py:13-94 (_qk_rope_cache) and :97-129
(qk_rope_cache). BF16 tensors are bit patterns (uint16); arithmetic is FP32
with the reference's cast placement, per (row, head) of D values:
  x        the packed QKV value (or the BF16 rounding of the FP32 sum of a
           Split's partials, engine/kernels/merged.py:37-45)
  inv_std  1 / sqrt(mean(x^2) + eps)               (eps of q_norm or k_norm)
  n        bf16(x * inv_std);  w = bf16(n * gain)   (qk_rope.py:41-45)
  rot      -w[c + D/2] for c < D/2, else w[c - D/2] (rotate_half)
  out      bf16( bf16(w * cos) + bf16(rot * sin) )  (qk_rope.py:58-61: both products rounded)
Query heads go to query[b, t, h]; key heads to keys[b, kv, pos]; the value
head is copied to values[b, kv, pos]. pos = t (prefill) or position + t
(decode; position[b] + t with per-row positions). The rotation phase is the
token (cos/sin [1, T, D]), the row (per-row tables [B, T, D]) or
position[b] + phases[b, t] in full [capacity, D] tables (qk_rope.py:47-57).

Parity pins (tests/test_oracle_rope.py): transformers' Qwen3RMSNorm and
apply_rotary_pos_emb evaluated by torch in BF16 on the CPU (library
routines), the cache slots written and untouched, and the phase modes
against each other.
"""

import numpy as np

from . import bf16

F32 = np.float32


def merged(packed, splits):
    """FP32 values of the packed QKV: BF16 bits as they are, or bf16(sum of FP32 partials) (merged.py:37-45)."""
    if splits == 1:
        return bf16.to_f32(packed)
    p = np.asarray(packed, F32)
    total = p[0].copy()
    for s in range(1, splits):
        total = (total + p[s]).astype(F32)
    return bf16.round_f32(total)


def head_norm_rope(x, gain, eps, cos, sin):
    """One head: FP32 x [D], BF16-valued gain/cos/sin [D] (FP32 arrays) -> FP32 of the BF16 result."""
    d = x.shape[-1]
    variance = (np.sum(x * x, dtype=F32) / F32(d)).astype(F32)
    inv_std = F32(1.0) / np.sqrt(variance + F32(eps), dtype=F32)
    normalized = bf16.round_f32(x * inv_std)
    weighted = bf16.round_f32(normalized * gain)
    half = d // 2
    rotated = np.concatenate([-weighted[half:], weighted[:half]]).astype(F32)
    direct = bf16.round_f32(weighted * cos)
    turn = bf16.round_f32(rotated * sin)
    return bf16.round_f32(direct + turn)


def qk_rope_cache(packed, splits, q_gain, k_gain, q_eps, k_eps, cos, sin, position, keys, values, q_heads,
                  prefill=False, rows=False, phases=None):
    """Returns (query bits [B, T, Hq, D], keys bits, values bits) after the cache update.

    packed: BF16 bits [B, T, (Hq + 2 Hkv) D] (splits = 1) or FP32 partials
    [splits, B, T, (Hq + 2 Hkv) D]. keys/values: BF16 bits [B, Hkv, C, D]
    (copied, then updated). cos/sin: BF16 bits, [1, T, D] shared, [B, T, D]
    with rows=True, or [capacity, D] tables with phases [B, T].
    """
    keys, values = np.array(keys, copy=True), np.array(values, copy=True)
    b_n, kv_heads, cap, d = keys.shape
    shape = np.shape(packed)[-3:] if splits > 1 else np.shape(packed)
    tokens = shape[1]
    x_all = merged(packed, splits).reshape(b_n, tokens, q_heads + 2 * kv_heads, d)
    qg, kg = bf16.to_f32(q_gain), bf16.to_f32(k_gain)
    c_tab, s_tab = bf16.to_f32(cos).reshape(-1, d), bf16.to_f32(sin).reshape(-1, d)
    pos = np.asarray(position, np.int64).reshape(-1)
    query = np.zeros((b_n, tokens, q_heads, d), np.uint16)
    for b in range(b_n):
        for t in range(tokens):
            row = b * tokens + t
            if phases is not None:
                phase = int(pos[b]) + int(np.asarray(phases)[b, t])
            else:
                phase = row if rows else t
            for h in range(q_heads + kv_heads):
                is_q = h < q_heads
                out = head_norm_rope(x_all[b, t, h], qg if is_q else kg, q_eps if is_q else k_eps,
                                     c_tab[phase], s_tab[phase])
                bits = bf16.round_bits(out)
                if is_q:
                    query[b, t, h] = bits
                    continue
                kv = h - q_heads
                slot = t if prefill else int(pos[b] if rows else pos[0]) + t
                keys[b, kv, slot] = bits
                values[b, kv, slot] = bf16.round_bits(x_all[b, t, q_heads + kv_heads + kv])
    return query, keys, values
