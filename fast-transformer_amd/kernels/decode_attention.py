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


def block_attention(query, key, value, position, scale, chain):
    """Verify-block attention (engine/kernels/decode_attention.py:637-680): outside this library.

    The name exists so that engine/layers.py:7 imports; a speculative verify
    pass (the only caller, engine/layers.py:62-68) raises here. One-token decode
    steps use ``decode_attention``.
    """
    raise NotImplementedError("verify-block attention (speculative decoding) is outside this library; "
                              "decode one token per step with decode_attention")


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
