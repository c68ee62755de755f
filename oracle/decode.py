"""numpy composition of one greedy decode step of a Qwen3 causal LM from this oracle's functions (test infrastructure only).

Only tests/ use this module, as the checker.

Restates engine/decode.py:215-297 (forward_last for one decode token per
row) with the packed layers of engine/layers.py:13-102. Per row b at
position p_b (slot p_b of the caches; the row attends to slots 0..p_b),
with h the layer output and r the residual stream:

  layer 0   n, r = embed_rms_norm(ids, E, ln1)               decode.py:227-229
  layer l   n, r = add_rms_norm(h, r, ln1)                   decode.py:236-243
            qkv  = project(n, [Wq; Wk; Wv])                   layers.py:23-26, :44
            q    = qk_rope_cache(qkv, ...) (K, V written)     layers.py:49-55; qk_rope.py:97-129
            a    = decode_attention(q, K, V, p_b, scaling)    layers.py:78-79
            o    = project(a, Wo)                              layers.py:86
            n, r = add_rms_norm(o, r, ln2)                     decode.py:258-261
            h    = project(swiglu(project(n, [Wg; Wu])), Wd)  layers.py:92-102
  final     n    = add_rms_norm(h, r, norm)                    decode.py:291-296
            logits = project(n, W_lm); ids = first argmax      decode.py:297; argmax.py:1-9

RoPE uses the full [capacity, D] cos/sin tables at phase p_b (the table
mode of qk_rope.py:47-57), which gives the same angles as the gathered
rows the reference passes at a shared position.

Parity pins (tests/test_oracle_decode.py): transformers' Qwen3ForCausalLM
evaluated by torch in float32 on the CPU (the library formulation of the
same model) on the same BF16 weights: logits within a tolerance set by
BF16 rounding, greedy ids equal wherever the float32 top-2 gap is clear of
it, and the cached keys and values against the library's own cache. Each
component function is pinned on its own in test_oracle.py,
test_oracle_rope.py and test_oracle_attention.py.
"""

import numpy as np

from . import attention, path, rope


def decode_step(weights, cfg, keys, values, token_ids, positions):
    """One decode token per row. Returns (ids int64 [B], logit bits [B, V]); updates keys/values in place.

    weights: BF16 bit arrays {"embed" [V, H], "norm" [H], "lm_head" [V, H],
    "cos"/"sin" [capacity, D], "layers": [{"ln1", "qkv", "q_norm",
    "k_norm", "o", "ln2", "gate_up", "down"}]}. cfg: {"q_heads",
    "kv_heads", "head_dim", "eps", "q_eps", "k_eps", "scaling"} (one eps for
    the layer norms; q_eps / k_eps for the head norms). keys / values: one
    [B, Hkv, C, D] bit array per layer. positions: one int per row.
    """
    hq, hkv, d = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    eps = cfg["eps"]
    pos = [int(p) for p in positions]
    batch = len(pos)
    phases = np.zeros((batch, 1), np.int64)
    h = r = None
    for index, lw in enumerate(weights["layers"]):
        if index == 0:
            n, r = path.embed_rms_norm(token_ids, weights["embed"], lw["ln1"], eps)
        else:
            n, r = path.add_rms_norm(h, r, lw["ln1"], eps)
        qkv = path.project(n, lw["qkv"])
        q, keys[index], values[index] = rope.qk_rope_cache(
            qkv.reshape(batch, 1, -1), 1, lw["q_norm"], lw["k_norm"], cfg["q_eps"], cfg["k_eps"],
            weights["cos"], weights["sin"], pos, keys[index], values[index], hq, rows=True, phases=phases)
        a = np.stack([attention.decode_attention(q[b], keys[index][b:b + 1], values[index][b:b + 1], pos[b],
                                                 cfg["scaling"])[0] for b in range(batch)])
        o = path.project(a.reshape(batch, hq * d), lw["o"])
        n, r = path.add_rms_norm(o, r, lw["ln2"], eps)
        h = path.project(path.paired_swiglu(n, lw["gate_up"]), lw["down"])
    n, _ = path.add_rms_norm(h, r, weights["norm"], eps)
    logits, ids, _ = path.lm_head_argmax(n, weights["lm_head"])
    return ids, logits
