"""Greedy decode steps of a Qwen3 causal LM, one token per row, through this library's kernels.

The caller side of the path: engine/decode.py:165-297 (optimize_model,
KVCache, forward_last for a decode token) and engine/layers.py:13-102
(PackedAttention, PackedMLP), restated over the fused forms of ``kernels``.
One step, per row b at its device-side position p_b:

  layer 0   qkv, r = embed_rms_norm_linear(ids, E, ln1, W_qkv)   embedding gather + norm + QKV, one launch
  layer l   qkv    = rms_norm_linear(r, ln1, W_qkv)               norm + QKV, one launch
            a      = rope_attend(qkv, ...)                        head norms + RoPE, K, V into slot p_b,
                                                                  decode attention over slots 0..p_b
            r      = linear_residual(a, W_o, r)                   O, the residual add in its epilogue
            act    = gate_up_swiglu(r, W_gu, ln2)                 norm + gate/up + SwiGLU
            r      = linear_residual(act, W_down, r)              down, the residual add in its epilogue
  final     ids, logits = lm_head_argmax(r, W_lm, norm)           norm + lm_head + argmax

The reference adds each sublayer's output to the residual stream in the next
norm (add_rms_norm, decode.py:236-243, :258-261, :291-296); here the add runs
in the epilogue of the projection that produces it, which stores the same BF16
sum, so no norm prologue has to read a second [rows, H] stream. The head
norms, RoPE and the cache update run in the attention kernel's prologue
(rope_attend) where it takes the head layout (head_dim 128, at most 4 query
heads per KV head; otherwise qk_rope_cache and decode attention launch
apart). That is 5 launches per layer (6 with a merge of attention splits)
and one for the vocabulary. The weights are the model's own tensors (BF16, on the GPU),
packed once as the reference packs them ([Wq; Wk; Wv], [Wg; Wu],
layers.py:23-26, :92-95). Positions, input ids and the RoPE phase live on the
device, so one captured graph serves every step (``Decoder.capture``), the way
the reference replays its decode graph (decode.py:650-668).

A prompt is fed one token per step: each prompt token attends to the slots
before it, which is what a causal prefill computes. A batched prefill
(grouped SDPA over the whole prompt, layers.py:66-71) is not part of this
library.
"""

import torch

from kernels import _native
from kernels import argmax as _argmax
from kernels import decode_attention as _attention
from kernels import linear as _linear
from kernels import qk_rope as _rope
from kernels import swiglu as _swiglu


class KVCache:
    """Layer-local BF16 [batch, kv_heads, capacity, head_dim] caches in one allocation (engine/decode.py:176-213).

    ``store`` is [key/value, layer, B, Hkv, C, D]; ``keys[l]`` and
    ``values[l]`` are contiguous views of one layer.
    """

    def __init__(self, config, batch, capacity, device, dtype=torch.bfloat16):
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        shape = (batch, config.num_key_value_heads, capacity, head_dim)
        layers = config.num_hidden_layers
        self.store = torch.zeros((2, layers, *shape), dtype=dtype, device=device)
        self.keys = [self.store[0, layer] for layer in range(layers)]
        self.values = [self.store[1, layer] for layer in range(layers)]


class PackedLayer:
    """One decoder layer's weights as the step reads them (engine/layers.py:13-30, :92-98)."""

    def __init__(self, layer):
        attention, mlp = layer.self_attn, layer.mlp
        with torch.no_grad():
            self.qkv_weight = torch.cat((attention.q_proj.weight, attention.k_proj.weight,
                                         attention.v_proj.weight), dim=0).contiguous()
            self.gate_up_weight = torch.cat((mlp.gate_proj.weight, mlp.up_proj.weight), dim=0).contiguous()
        self.o_weight = attention.o_proj.weight.detach()
        self.down_weight = mlp.down_proj.weight.detach()
        self.input_norm = layer.input_layernorm
        self.post_norm = layer.post_attention_layernorm
        self.q_norm, self.k_norm = attention.q_norm, attention.k_norm
        self.q_heads = attention.q_proj.out_features // attention.head_dim
        self.scaling = attention.scaling


class Decoder:
    """Decode state for ``batch`` rows of a transformers Qwen3ForCausalLM held in BF16 on the GPU.

    ``token_ids`` [B] and ``position`` [B] (int64, on the device) are the
    step's inputs; ``step()`` returns (ids [B] int64, logits [B, V] BF16) and
    writes each layer's key and value at slot ``position[b]`` of row b.
    """

    def __init__(self, model, batch, capacity, fused_rope=True):
        base = model.model
        embed = base.embed_tokens.weight
        if embed.dtype != torch.bfloat16 or embed.device.type != "cuda":
            raise ValueError("the model must be BF16 on a GPU (model.to('cuda', torch.bfloat16))")
        _native.require_gpu(embed)
        self.batch, self.capacity = batch, capacity
        self.embed = embed.detach()
        self.lm_head = model.lm_head.weight.detach()
        self.norm = base.norm
        self.layers = [PackedLayer(layer) for layer in base.layers]
        self.cache = KVCache(model.config, batch, capacity, embed.device)
        device = embed.device
        with torch.no_grad():
            # Full tables [capacity, D]: the kernel reads row position[b] + phase on the device.
            cos, sin = base.rotary_emb(embed.new_empty((1, 1, embed.shape[1])),
                                       torch.arange(capacity, device=device).unsqueeze(0))
        self.cos, self.sin = cos[0].contiguous(), sin[0].contiguous()
        self.phases = torch.zeros((batch, 1), dtype=torch.int64, device=device)
        self.position = torch.zeros((batch,), dtype=torch.int64, device=device)
        self.token_ids = torch.zeros((batch,), dtype=torch.int64, device=device)
        self._graph = None
        first = self.layers[0]
        gains = [t for layer in self.layers for t in (layer.q_norm.weight, layer.k_norm.weight)]
        #: Head norms + RoPE in the attention launch (else the separate qk_rope_cache launch).
        self.fused_rope = bool(fused_rope) and _attention.rope_attention_supported(
            first.q_heads, self.cache.keys[0].shape[1], self.cache.keys[0].shape[3], capacity=capacity) and \
            all(t.is_contiguous() and t.data_ptr() % 16 == 0 for t in [self.cos, self.sin, self.cache.store, *gains])

    def step(self):
        """One decode token per row at ``position`` (engine/decode.py:215-297 for a one-token step)."""
        batch = self.batch
        residual = None
        for index, layer in enumerate(self.layers):
            eps = layer.input_norm.variance_epsilon
            if index == 0:
                qkv, residual = _linear.embed_rms_norm_linear(self.token_ids, self.embed, layer.input_norm.weight,
                                                              eps, layer.qkv_weight)
            else:
                qkv = _linear.rms_norm_linear(residual, layer.input_norm.weight, eps, layer.qkv_weight)
            keys, values = self.cache.keys[index], self.cache.values[index]
            if self.fused_rope:
                attention = _attention.rope_attend(qkv, layer.q_norm, layer.k_norm, self.cos, self.sin,
                                                   self.position, keys, values, layer.q_heads, layer.scaling,
                                                   phases=self.phases)
            else:
                query = _rope.qk_rope_cache(qkv.view(batch, 1, -1), layer.q_norm, layer.k_norm, self.cos, self.sin,
                                            self.position, keys, values, layer.q_heads, rows=True,
                                            phases=self.phases)
                attention = _attention.attend(query.reshape(batch, layer.q_heads, -1), keys, values,
                                              self.position, layer.scaling)
            residual = _linear.linear_residual(attention.view(batch, -1), layer.o_weight, residual)
            act = _swiglu.gate_up_swiglu(residual, layer.gate_up_weight, layer.post_norm.weight,
                                         layer.post_norm.variance_epsilon)
            residual = _linear.linear_residual(act, layer.down_weight, residual)
        return _argmax.lm_head_argmax(residual, self.lm_head, self.norm.weight, self.norm.variance_epsilon)

    def advance(self, ids):
        """Feed ``ids`` as the next tokens and move every row one slot on (device-side, capturable)."""
        self.token_ids.copy_(ids)
        self.position.add_(1)

    def capture(self):
        """Record ``step`` + ``advance`` in one graph; returns the graph's (ids, logits) outputs.

        One eager step first sizes the workspaces the kernels share (capture
        allocates nothing of its own); it writes slot ``position`` of the
        caches, which the next real step at that position rewrites.
        """
        self.step()
        stream = torch.cuda.Stream(device=self.embed.device)
        stream.wait_stream(torch.cuda.current_stream(self.embed.device))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                ids, logits = self.step()
                self.advance(ids)
        torch.cuda.current_stream(self.embed.device).wait_stream(stream)
        self._graph = (graph, ids, logits)
        return ids, logits

    def generate(self, prompt, steps, graph=False):
        """Greedy continuation of ``prompt`` [B, P] int64: ([B, steps] ids, [B, P + steps - 1, V] logits).

        The prompt goes through one step per token (positions 0..P-1); the
        last of them gives the first new token, and ``steps - 1`` more steps
        follow. ``graph`` replays one captured step instead of launching each.
        """
        batch, length = prompt.shape
        if batch != self.batch:
            raise ValueError(f"prompt has {batch} rows, the decoder {self.batch}")
        if length < 1 or steps < 1 or length + steps - 1 > self.capacity:
            raise ValueError(f"{length} prompt tokens + {steps} steps do not fit {self.capacity} cache slots")
        prompt = prompt.to(self.token_ids.device)
        if graph and self._graph is None:
            self.position.zero_()
            self.token_ids.copy_(prompt[:, 0])
            self.capture()
        self.position.zero_()
        out, logits = [], []
        for t in range(length + steps - 1):
            if t < length:
                self.token_ids.copy_(prompt[:, t])
            if graph:
                g, ids, step_logits = self._graph
                g.replay()
            else:
                ids, step_logits = self.step()
                self.advance(ids)
            logits.append(step_logits.clone())
            if t >= length - 1:
                out.append(ids.clone())
        return torch.stack(out, dim=1), torch.stack(logits, dim=1)
