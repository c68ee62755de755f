"""Pin the composed decode step (oracle/decode.py) against transformers' Qwen3ForCausalLM in float32 on the CPU.

Same BF16-valued weights; the oracle's prompt goes through one step per token
and its greedy tokens are appended, then the library model evaluates the whole
sequence at once. The oracle rounds to BF16 where the path does, so its logits
sit within |d| <= 2e-2 + 1e-2 |ref| of the float32 ones, and
its greedy ids equal theirs wherever the float32 top-2 gap is clear of that
bar. Its caches hold the library's keys (after q/k norm and RoPE) and values.
A wrong head mapping (each query head reading the other KV head of its pair)
fails the same bar: the comparison sees the wiring, not only the arithmetic.
"""

import numpy as np
import pytest
import torch

import qwen3_tiny as Q
from oracle import bf16, decode


def _generate(m, w, cfg, prompt, steps, capacity):
    batch, length = prompt.shape
    tokens = prompt.copy()
    layers = m.config.num_hidden_layers
    shape = (batch, cfg["kv_heads"], capacity, cfg["head_dim"])
    keys = [np.zeros(shape, np.uint16) for _ in range(layers)]
    values = [np.zeros(shape, np.uint16) for _ in range(layers)]
    logits = []
    for t in range(length + steps - 1):
        ids, step = decode.decode_step(w, cfg, keys, values, tokens[:, t], [t] * batch)
        logits.append(bf16.to_f32(step))
        if t >= length - 1:
            tokens = np.concatenate([tokens, ids[:, None]], axis=1)
    return tokens, np.stack(logits, 1), keys, values


@pytest.mark.parametrize("dims,batch", [(Q.SMALL, 2), (Q.QWEN3_06B, 1)])
def test_greedy_steps_match_transformers_float32(dims, batch):
    capacity, length, steps = 16, 6, 4
    m = Q.model(dims)
    cos, sin = Q.rope_tables(m, capacity)
    w, cfg = Q.weights(m, cos, sin)
    prompt = torch.randint(0, m.config.vocab_size, (batch, length), generator=torch.Generator().manual_seed(5))
    tokens, logits, keys, values = _generate(m, w, cfg, prompt.numpy(), steps, capacity)
    seq = torch.from_numpy(tokens[:, :length + steps - 1])
    with torch.no_grad():
        out = m(seq, use_cache=True)
    want = out.logits.numpy()
    assert Q.close(logits, want)
    ok, checked = Q.clear_ids_agree(tokens[:, length:], want[:, length - 1:], margin=0.05)
    assert ok and checked >= batch * steps // 2
    n = seq.shape[1]
    for layer in range(m.config.num_hidden_layers):
        cache = out.past_key_values.layers[layer]
        assert Q.close(bf16.to_f32(keys[layer][:, :, :n]), cache.keys.numpy())
        assert Q.close(bf16.to_f32(values[layer][:, :, :n]), cache.values.numpy())
        assert not keys[layer][:, :, n:].any() and not values[layer][:, :, n:].any()


def test_a_wrong_head_mapping_fails_the_bar():
    """Swap the two KV heads' K and V rows: every query head then reads the other head of its pair."""
    capacity, length = 12, 8
    m = Q.model()
    cos, sin = Q.rope_tables(m, capacity)
    w, cfg = Q.weights(m, cos, sin)
    hq, hkv, d = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    for lw in w["layers"]:
        qkv = lw["qkv"].reshape(hq + 2 * hkv, d, -1).copy()
        for base in (hq, hq + hkv):
            qkv[[base, base + 1]] = qkv[[base + 1, base]]
        lw["qkv"] = qkv.reshape(lw["qkv"].shape)
    prompt = torch.randint(0, m.config.vocab_size, (1, length), generator=torch.Generator().manual_seed(5))
    _, logits, _, _ = _generate(m, w, cfg, prompt.numpy(), 1, capacity)
    with torch.no_grad():
        want = m(prompt).logits.numpy()
    assert not Q.close(logits, want)
