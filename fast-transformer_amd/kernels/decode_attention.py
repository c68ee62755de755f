"""Dense GQA decode attention with a device-side length and split-KV softmax reduction, on libftk.

Drop-in for engine/kernels/decode_attention.py:229-258 (``decode_attention``):
the same signature, shapes, assertions and output layout. BF16 Q/K/V, FP32
scores and sums, p rounded to BF16 before it weights V, BF16 output. Every
cache slot up to ``position`` contributes; later slots are never read into
the result. No host synchronization: the length is read on the device, so a
captured graph replays for every position.

Each (row, KV head) pair's slots are cut into intervals ("splits"); a
workgroup attends to one interval and writes FP32 partials, and a second
kernel merges them (engine/kernels/decode_attention.py:31-149). With one
interval the first kernel writes the output itself. The split count is the
planner's, for MI355X: about two workgroups per CU, at least one load step
per wave (``ftk_plan_decode_attention``); ``config`` overrides it.
"""

import ctypes

import torch

from kernels import _native

#: Query heads per KV head the kernels take (Qwen3 models have 1..8).
MAX_GROUP = 8

#: Per-shape launch choices, frozen before capture (engine/kernels/decode_attention.py:185 ``_CONFIGS``).
_CONFIGS = {}


def plan(batch, query_heads, kv_heads, capacity, dim, config=None, compute_units=None):
    """The launch ``decode_attention`` makes for this shape (an ``AttnPlan``)."""
    cus = compute_units if compute_units is not None else _native.lib().ftk_device_compute_units()
    out = _native.AttnPlan()
    cfg = ctypes.byref(config) if config is not None else None
    _native.call("ftk_plan_decode_attention", batch, query_heads, kv_heads, capacity, dim, cus, cfg,
                 ctypes.byref(out))
    return out


def attend(query, key, value, position, scale, config=None):
    """The launch itself: query [B, Hq, D] view, cache [B, Hkv, C, D], position int64 [1] or [B]."""
    batch, query_heads, dim = query.shape
    kv_heads, capacity = key.shape[1:3]
    out = torch.empty((batch, 1, query_heads, dim), device=query.device, dtype=query.dtype)
    cfg = ctypes.byref(config) if config is not None else None
    need = int(_native.lib().ftk_decode_attention_workspace_bytes(batch, query_heads, kv_heads, capacity, dim, cfg))
    if need < 0:
        raise ValueError(f"decode attention does not take this shape: {tuple(key.shape)} with {query_heads} heads")
    ws = _native.workspace(query.device, need, "attention") if need > 0 else None
    _native.call("ftk_decode_attention_bf16", _native.ptr(query), _native.ptr(key), _native.ptr(value),
                 _native.ptr(position), position.numel(), _native.ptr(out), batch, query_heads, kv_heads, capacity,
                 dim, float(scale), _native.ptr(ws), ws.numel() if ws is not None else 0, cfg,
                 _native.stream_of(query))
    return out


#: Head dimension and query heads per KV head the fused RoPE prologue takes (the QUAD kind).
ROPE_DIM, ROPE_MAX_GROUP = 128, 4


def _aligned(*tensors):
    return all(t.data_ptr() % 16 == 0 for t in tensors)


def rope_attention_supported(query_heads, kv_heads, dim, config=None, capacity=None):
    """Whether ``rope_attend`` takes this head layout: D = 128, at most 4 query heads per KV head, and
    (when given) a cache whose byte offsets fit 32 bits (up to 2^32 / 256 - 512 slots)."""
    if config is not None and config.kind not in (0, _native.ATTN_QUAD):
        return False
    if capacity is not None and (capacity + 512) * dim * 2 > 0xFFFFFFFF:
        return False
    return dim == ROPE_DIM and query_heads % kv_heads == 0 and query_heads // kv_heads <= ROPE_MAX_GROUP


def rope_attend(packed, q_norm, k_norm, cos, sin, position, keys, values, q_heads, scale, phases=None,
                config=None):
    """One decode token per row: qk_rope_cache (decode form) and decode_attention in one launch (plus the merge).

    Replaces engine/layers.py:51-55 then :76 for a one-token step: packed
    BF16 QKV [B, (Hq + 2 Hkv) D] (or [B, 1, ...]); q_norm / k_norm the head
    norms; cos / sin whole BF16 tables [table_rows, D], row b rotated at
    position[b] + phases[b] (``phases`` [B] or [B, 1] int64, or None for 0);
    position int64 [1] or [B]. Writes row b's key and value heads into
    ``keys`` / ``values`` [B, Hkv, C, D] at slot position[b] and returns the
    attention output [B, 1, Hq, D] over slots 0..position[b]. The same
    roundings as the two launches; FP32 sums in another order, so results
    agree with them within a BF16 ulp. Needs ``rope_attention_supported``
    and 16-byte aligned tensors (ValueError otherwise).
    """
    batch, kv_heads, capacity, dim = keys.shape
    width = (q_heads + 2 * kv_heads) * dim
    assert packed.dtype == keys.dtype == values.dtype == cos.dtype == sin.dtype == torch.bfloat16
    assert packed.numel() == batch * width and packed.shape[0] == batch and packed.shape[-1] == width
    assert packed.is_contiguous() and keys.is_contiguous() and values.is_contiguous()
    assert values.shape == keys.shape
    assert cos.shape == sin.shape and cos.shape[-1] == dim and cos.is_contiguous() and sin.is_contiguous()
    assert position.dtype == torch.int64 and position.numel() in (1, batch)
    if phases is not None:
        assert phases.dtype == torch.int64 and phases.numel() == batch and phases.is_contiguous()
    if not rope_attention_supported(q_heads, kv_heads, dim, config, capacity):
        raise ValueError(f"the fused RoPE attention takes D = {ROPE_DIM} and at most {ROPE_MAX_GROUP} query heads "
                         f"per KV head, got D = {dim}, {q_heads} / {kv_heads} heads")
    q_weight, k_weight = q_norm.weight.contiguous(), k_norm.weight.contiguous()
    _native.require_gpu(packed, keys, values, cos, sin, position, q_weight, k_weight)
    if not _aligned(packed, keys, values, cos, sin, q_weight, k_weight):
        raise ValueError("the fused RoPE attention needs 16-byte aligned tensors")
    out = torch.empty((batch, 1, q_heads, dim), device=packed.device, dtype=packed.dtype)
    cfg = ctypes.byref(config) if config is not None else None
    need = int(_native.lib().ftk_decode_attention_workspace_bytes(batch, q_heads, kv_heads, capacity, dim, cfg))
    if need < 0:
        raise ValueError(f"decode attention does not take this shape: {tuple(keys.shape)} with {q_heads} heads")
    ws = _native.workspace(packed.device, need, "attention") if need > 0 else None
    _native.call("ftk_rope_decode_attention_bf16", _native.ptr(packed), _native.ptr(q_weight),
                 _native.ptr(k_weight), float(q_norm.variance_epsilon), float(k_norm.variance_epsilon),
                 _native.ptr(cos), _native.ptr(sin), cos.numel() // dim, _native.ptr(position), position.numel(),
                 _native.ptr(phases), _native.ptr(keys), _native.ptr(values), _native.ptr(out), batch, q_heads,
                 kv_heads, capacity, dim, float(scale), _native.ptr(ws), ws.numel() if ws is not None else 0, cfg,
                 _native.stream_of(packed))
    return out


def decode_attention(query, key, value, position, scale):
    """Q [B,Hq,1,D], KV [B,Hkv,C,D] -> [B,1,Hq,D]."""
    batch, query_heads, tokens, dim = query.shape
    kv_heads, capacity = key.shape[1:3]
    assert tokens == 1 and query_heads % kv_heads == 0
    assert query.dtype == key.dtype == value.dtype == torch.bfloat16
    assert query.is_contiguous() and key.is_contiguous() and value.is_contiguous()
    assert value.shape == key.shape and key.shape[0] == batch and key.shape[3] == dim
    assert dim in (64, 128) and position.shape == (1,) and position.dtype == torch.int64
    if query_heads // kv_heads > MAX_GROUP:
        raise ValueError(f"at most {MAX_GROUP} query heads per KV head, got {query_heads // kv_heads}")
    _native.require_gpu(query, key, value, position)
    shape = (query.device, batch, query_heads, kv_heads, capacity, dim)
    return attend(query.view(batch, query_heads, dim), key, value, position, scale, _CONFIGS.get(shape))
