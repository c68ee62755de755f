"""Small random Qwen3 causal LMs for the decode-step tests, and their weights as BF16 bit arrays.

Weights are drawn from a seeded generator and rounded to BF16 (so the float32
model and a BF16 copy hold the same values); norm gains are 1 + N(0, 0.1),
embeddings N(0, 1), projections transformers' N(0, 0.02) init.
"""

import numpy as np
import torch
from transformers import Qwen3Config, Qwen3ForCausalLM

from conftest import to_bits

#: (hidden, intermediate, q_heads, kv_heads, head_dim): a small model, and Qwen3-0.6B's and Qwen3-8B's
#: layer dimensions.
SMALL = (512, 1536, 8, 4, 128)
QWEN3_06B = (1024, 3072, 16, 8, 128)
QWEN3_8B = (4096, 12288, 32, 8, 128)


def model(dims=SMALL, vocab=4096, layers=2, seed=0):
    """A float32 Qwen3ForCausalLM on the CPU (eager attention) with BF16-valued weights."""
    hidden, inter, hq, hkv, d = dims
    cfg = Qwen3Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
                      num_attention_heads=hq, num_key_value_heads=hkv, head_dim=d, rms_norm_eps=1e-6,
                      rope_theta=1_000_000.0, tie_word_embeddings=False, max_position_embeddings=1024)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    m = Qwen3ForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.dim() == 1:
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g))
            elif "embed" in name:
                p.copy_(torch.randn(p.shape, generator=g))
            p.copy_(p.to(torch.bfloat16).float())
    return m


def rope_tables(m, capacity, device="cpu"):
    """The model's own BF16 cos/sin rows for positions 0..capacity-1: ([C, D], [C, D])."""
    with torch.no_grad():
        cos, sin = m.model.rotary_emb(torch.zeros(1, 1, 1, dtype=torch.bfloat16, device=device),
                                      torch.arange(capacity, device=device).unsqueeze(0))
    return cos[0], sin[0]


def weights(m, cos, sin):
    """(weights, cfg) for oracle.decode.decode_step: BF16 bits of every tensor the step reads."""
    base = m.model

    def bits(t):
        return to_bits(t.detach().to(torch.bfloat16))

    out = {"embed": bits(base.embed_tokens.weight), "norm": bits(base.norm.weight), "lm_head": bits(m.lm_head.weight),
           "cos": bits(cos), "sin": bits(sin), "layers": []}
    for layer in base.layers:
        a, mlp = layer.self_attn, layer.mlp
        out["layers"].append({
            "ln1": bits(layer.input_layernorm.weight), "ln2": bits(layer.post_attention_layernorm.weight),
            "qkv": bits(torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight])),
            "q_norm": bits(a.q_norm.weight), "k_norm": bits(a.k_norm.weight), "o": bits(a.o_proj.weight),
            "gate_up": bits(torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight])), "down": bits(mlp.down_proj.weight)})
    c = m.config
    cfg = {"q_heads": c.num_attention_heads, "kv_heads": c.num_key_value_heads, "head_dim": c.head_dim,
           "eps": c.rms_norm_eps, "q_eps": c.rms_norm_eps, "k_eps": c.rms_norm_eps, "scaling": c.head_dim ** -0.5}
    return out, cfg


def oracle_run(decode, w, cfg, tokens, batch, capacity, layers):
    """Teacher-forced oracle steps over ``tokens`` [B, T]: (ids [B, T], FP32 logits [B, T, V], keys, values)."""
    shape = (batch, cfg["kv_heads"], capacity, cfg["head_dim"])
    keys = [np.zeros(shape, np.uint16) for _ in range(layers)]
    values = [np.zeros(shape, np.uint16) for _ in range(layers)]
    ids, logits = [], []
    from oracle import bf16
    for t in range(tokens.shape[1]):
        step_ids, step_logits = decode.decode_step(w, cfg, keys, values, tokens[:, t], [t] * batch)
        ids.append(step_ids)
        logits.append(bf16.to_f32(step_logits))
    return np.stack(ids, 1), np.stack(logits, 1), keys, values


def close(got, want, atol=2e-2, rtol=1e-2):
    """|got - want| <= atol + rtol |want| everywhere (the path's elementwise bar)."""
    return bool(np.all(np.abs(np.asarray(got, np.float64) - want) <= atol + rtol * np.abs(want)))


def clear_ids_agree(got_ids, want_logits, margin):
    """Greedy ids equal the float32 argmax wherever its top-2 gap exceeds ``margin``; returns (ok, rows checked)."""
    top2 = np.sort(want_logits, axis=-1)[..., -2:]
    clear = (top2[..., 1] - top2[..., 0]) > margin
    return bool(np.all(np.asarray(got_ids)[clear] == want_logits.argmax(-1)[clear])), int(clear.sum())
