"""numpy restatement of the reference's split-KV GQA decode attention (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this
module, as the checker; the product path never calls it.

BF16 tensors cross this module as bit patterns (uint16 arrays). Arithmetic is
FP32, with the reference's cast placement:
  scores  s = f32(q . k) * f32(scale * log2(e))       (FP32 dot of BF16 operands)
  tile    m' = max(m, max s); p = exp2(s - m'); c = exp2(m - m')
          l = l * c + sum p;  acc = acc * c + bf16(p) . V
  merge   M = max_s m_s;  c_s = exp2(m_s - M);  out = bf16( sum acc_s c_s / sum l_s c_s )

Functions and the reference lines they restate:
  decode_partials   engine/kernels/decode_attention.py:31-99 (_decode_partials)
  decode_merge      engine/kernels/decode_attention.py:102-128 (_decode_merge)
  decode_attention  engine/kernels/decode_attention.py:131-149 (_attend), :229-258 (decode_attention)
  default_splits    engine/kernels/decode_attention.py:152-157 (_default_config's split count)
  dense_reference   the closed form the reference's own test compares with
                    (agent/verify_gpu.py:154-174: sdpa with a length mask)

Parity pins (tests/test_oracle_attention.py): torch's CPU
scaled_dot_product_attention in float64 (a library routine, GQA by
repeat_interleave) at the reference test's shapes and tolerance; one valid
token returns its value row bit for bit; equal keys return the exact mean of
integer-valued values; NaN in unused cache slots never reaches the result;
every split count and tile width agree to within BF16 rounding.
"""

import numpy as np

from . import bf16

F32 = np.float32
LOG2E = 1.4426950408889634


def scale_log2(scale):
    """The score multiplier: scale * log2(e) formed in double, used in FP32 (decode_attention.py:70)."""
    return F32(float(scale) * LOG2E)


def default_splits(batch, kv_heads, capacity, block_n=None):
    """_default_config's split count (decode_attention.py:152-157): min(32, cdiv(256, B*Hkv), cdiv(C, block_n))."""
    if block_n is None:
        block_n = 32 if batch * kv_heads < 16 else 64
    return min(32, -(-256 // (batch * kv_heads)), -(-capacity // block_n))


def decode_partials(q_bits, k_bits, v_bits, valid, scale, block_n, splits):
    """Per (row, KV head, split): FP32 partial numerators [G, D] and (max, denominator) [G, 2].

    q_bits [B, Hq, D]; k_bits, v_bits [B, Hkv, C, D]; `valid` cache slots
    (position + 1) are read. Returns partial [B*Hkv, S, G, D] and stats
    [B*Hkv, S, G, 2], FP32. Split s covers slots [s*chunk, min((s+1)*chunk, C, valid))
    in tiles of block_n slots (decode_attention.py:48-99).
    """
    q = bf16.to_f32(q_bits)
    k = bf16.to_f32(k_bits)
    v = bf16.to_f32(v_bits)
    b_n, hq, d = q.shape
    hkv, cap = k.shape[1], k.shape[2]
    g = hq // hkv
    chunk = -(-cap // splits)
    mul = scale_log2(scale)
    partial = np.zeros((b_n * hkv, splits, g, d), F32)
    stats = np.zeros((b_n * hkv, splits, g, 2), F32)
    for b in range(b_n):
        for h in range(hkv):
            query = q[b, h * g:(h + 1) * g]  # query heads h*G .. h*G+G-1 share KV head h
            for s in range(splits):
                begin = s * chunk
                end = min(begin + chunk, cap, valid)
                m = np.full(g, -np.inf, F32)
                l = np.zeros(g, F32)
                acc = np.zeros((g, d), F32)
                for start in range(begin, end, block_n):
                    stop = min(start + block_n, end)
                    key = k[b, h, start:stop]
                    scores = (np.matmul(query, key.T, dtype=F32) * mul).astype(F32)
                    m_new = np.maximum(m, scores.max(axis=1))
                    p = np.exp2(scores - m_new[:, None]).astype(F32)
                    c = np.exp2(m - m_new).astype(F32)
                    l = (l * c + p.sum(axis=1, dtype=F32)).astype(F32)
                    pv = np.matmul(bf16.round_f32(p), v[b, h, start:stop], dtype=F32)
                    acc = (acc * c[:, None] + pv).astype(F32)
                    m = m_new
                partial[b * hkv + h, s] = acc
                stats[b * hkv + h, s, :, 0] = m
                stats[b * hkv + h, s, :, 1] = l
    return partial, stats


def decode_merge(partial, stats, batch, q_heads):
    """bf16( sum_s acc_s exp2(m_s - M) / sum_s l_s exp2(m_s - M) ) per query head (decode_attention.py:102-128).

    Returns BF16 bits [B, Hq, D]. An empty split (m = -inf, l = 0) gets weight 0.
    """
    groups, splits, g, d = partial.shape
    m = stats[..., 0]
    l = stats[..., 1]
    top = m.max(axis=1, keepdims=True)
    with np.errstate(invalid="ignore"):
        c = np.exp2(m - top).astype(F32)
    c = np.where(np.isneginf(m), F32(0), c).astype(F32)
    den = (l * c).sum(axis=1, dtype=F32)
    num = (partial * c[..., None]).sum(axis=1, dtype=F32)
    out = (num / den[..., None]).astype(F32)
    return bf16.round_bits(out).reshape(batch, q_heads, d)


def decode_attention(q_bits, k_bits, v_bits, position, scale, block_n=32, splits=None):
    """Q [B, Hq, D] (a T = 1 decode query), KV [B, Hkv, C, D] -> BF16 bits [B, Hq, D].

    `position` is the index of the newest cache slot (position[0] of the
    reference's int64 [1] tensor); slots 0..position are read
    (decode_attention.py:46, :229-258).
    """
    b_n, hq, _ = np.shape(q_bits)
    hkv, cap = np.shape(k_bits)[1:3]
    if splits is None:
        splits = default_splits(b_n, hkv, cap, block_n)
    partial, stats = decode_partials(q_bits, k_bits, v_bits, int(position) + 1, scale, block_n, splits)
    return decode_merge(partial, stats, b_n, hq)


def dense_reference(q, k, v, valid, scale):
    """float64 softmax attention over slots [0, valid), GQA heads h -> h // (Hq / Hkv): the closed form.

    q [B, Hq, D], k, v [B, Hkv, C, D] as float arrays (any float dtype).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)[:, :, :valid]
    v = np.asarray(v, np.float64)[:, :, :valid]
    g = q.shape[1] // k.shape[1]
    k = np.repeat(k, g, axis=1)
    v = np.repeat(v, g, axis=1)
    s = np.einsum("bhd,bhtd->bht", q, k) * float(scale)
    s -= s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("bht,bhtd->bhd", w, v)

