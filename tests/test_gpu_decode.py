"""Greedy decode steps of a small Qwen3 model through the library (fast-transformer_amd/decode.py), on the GPU.

The decoder runs a prompt one token per step and then generates; the oracle's
composed step (oracle/decode.py) is run teacher-forced on the same tokens.
Bars: logits within |d| <= 2e-2 + 1e-2 |ref| of the oracle's and of
transformers' float32 model on the same sequence (wider at Qwen3-8B's width,
where the logits are larger: see BARS); greedy ids equal to the oracle's
wherever its top-2 gap exceeds 2.5x the bar's atol; caches within the same bar
of the oracle's. A replayed graph of one step gives the eager results bit for bit.
"""

import copy

import numpy as np
import pytest
import torch

import qwen3_tiny as Q
from conftest import to_bits
from oracle import bf16, decode

import decode as D

pytestmark = pytest.mark.gpu


def _setup(dims, batch, capacity, seed=5, length=6):
    m = Q.model(dims)
    gpu = copy.deepcopy(m).to("cuda", torch.bfloat16)
    prompt = torch.randint(0, m.config.vocab_size, (batch, length), generator=torch.Generator().manual_seed(seed))
    return m, gpu, prompt


#: Bars (atol, rtol) against the oracle and against transformers' float32 model. At Qwen3-8B's
#: width the logits are ~4x larger (std 1.3) and BF16 rounding alone (transformers run in BF16)
#: moves them by up to 0.07 from float32, so that case takes a bar scaled to it.
BARS = {Q.SMALL: ((2e-2, 1e-2), (2e-2, 1e-2)), Q.QWEN3_06B: ((2e-2, 1e-2), (2e-2, 1e-2)),
        Q.QWEN3_8B: ((5e-2, 2e-2), (0.1, 2e-2))}


@pytest.mark.parametrize("dims,batch,fused", [(Q.SMALL, 1, True), (Q.SMALL, 2, True), (Q.SMALL, 2, False),
                                              (Q.QWEN3_06B, 1, True), (Q.QWEN3_06B, 4, True),
                                              (Q.QWEN3_8B, 2, True)])
def test_generate_matches_oracle_and_transformers(cuda, dims, batch, fused):
    capacity, steps = 24, 5
    m, gpu, prompt = _setup(dims, batch, capacity)
    dec = D.Decoder(gpu, batch, capacity, fused_rope=fused)
    assert dec.fused_rope == fused
    ids, logits = dec.generate(prompt, steps)
    torch.cuda.synchronize()
    length = prompt.shape[1]
    tokens = torch.cat([prompt, ids[:, :-1].cpu()], dim=1).numpy()
    w, cfg = Q.weights(m, dec.cos.cpu(), dec.sin.cpu())
    o_ids, o_logits, o_keys, o_values = Q.oracle_run(decode, w, cfg, tokens, batch, capacity,
                                                     m.config.num_hidden_layers)
    (oa, orl), (ta, trl) = BARS[dims]
    got = bf16.to_f32(to_bits(logits))
    assert Q.close(got, o_logits, oa, orl)
    ok, checked = Q.clear_ids_agree(ids.cpu().numpy(), o_logits[:, length - 1:], margin=2.5 * oa)
    assert ok and checked >= batch * steps // 2
    with torch.no_grad():
        want = m(torch.from_numpy(tokens)).logits.numpy()
    assert Q.close(got, want, ta, trl)
    n = tokens.shape[1]
    for layer in range(m.config.num_hidden_layers):
        k = bf16.to_f32(to_bits(dec.cache.keys[layer]))
        v = bf16.to_f32(to_bits(dec.cache.values[layer]))
        assert Q.close(k[:, :, :n], bf16.to_f32(o_keys[layer][:, :, :n]), oa, orl)
        assert Q.close(v[:, :, :n], bf16.to_f32(o_values[layer][:, :, :n]), oa, orl)
        assert not k[:, :, n:].any() and not v[:, :, n:].any()


@pytest.mark.parametrize("batch", [1, 3])
def test_graph_replays_give_the_eager_bits(cuda, batch):
    capacity, steps = 20, 6
    _, gpu, prompt = _setup(Q.SMALL, batch, capacity, seed=9)
    eager = D.Decoder(gpu, batch, capacity)
    e_ids, e_logits = eager.generate(prompt, steps)
    graphed = D.Decoder(gpu, batch, capacity)
    g_ids, g_logits = graphed.generate(prompt, steps, graph=True)
    torch.cuda.synchronize()
    assert torch.equal(e_ids, g_ids)
    assert torch.equal(e_logits, g_logits)
    n = prompt.shape[1] + steps - 1
    assert torch.equal(eager.cache.store[:, :, :, :, :n], graphed.cache.store[:, :, :, :, :n])
    # a second generation replays the same graph from position 0
    again_ids, again_logits = graphed.generate(prompt, steps, graph=True)
    torch.cuda.synchronize()
    assert torch.equal(again_ids, e_ids) and torch.equal(again_logits, e_logits)


@pytest.mark.parametrize("dims,batch", [(Q.SMALL, 2), (Q.QWEN3_8B, 1)])
def test_rope_in_the_attention_launch_matches_the_two_launches(cuda, dims, batch):
    """The head norms + RoPE in the attention prologue against the separate qk_rope_cache launch."""
    capacity, steps = 24, 5
    _, gpu, prompt = _setup(dims, batch, capacity, seed=11)
    fused = D.Decoder(gpu, batch, capacity)
    apart = D.Decoder(gpu, batch, capacity, fused_rope=False)
    assert fused.fused_rope and not apart.fused_rope
    f_ids, f_logits = fused.generate(prompt, steps)
    a_ids, a_logits = apart.generate(prompt, steps)
    torch.cuda.synchronize()
    (oa, orl), _ = BARS[dims]
    want = bf16.to_f32(to_bits(a_logits))
    assert Q.close(bf16.to_f32(to_bits(f_logits)), want, oa, orl)
    ok, checked = Q.clear_ids_agree(f_ids.cpu().numpy(), want[:, prompt.shape[1] - 1:], margin=2.5 * oa)
    assert ok and checked >= batch * steps // 2
    n = prompt.shape[1] + steps - 1
    k_f = bf16.to_f32(to_bits(fused.cache.store[:, :, :, :, :n]))
    k_a = bf16.to_f32(to_bits(apart.cache.store[:, :, :, :, :n]))
    assert Q.close(k_f, k_a, oa, orl)
