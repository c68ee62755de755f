"""Q/K head RMSNorm, RoPE and the in-place KV-cache update, on libftk.

Drop-in for engine/kernels/qk_rope.py:97-129 (``qk_rope_cache``): the same
signature, assertions, outputs and cache writes. One wave per (row, head)
normalises the head with its q_norm / k_norm gain, rotates it with the
BF16 cos/sin rows (both RoPE products rounded to BF16 before their BF16
sum, as the native function does), writes query heads to a token-major
query and key heads, plus the copied value heads, into the caches at the
step's slot. The packed QKV may be a ``Split`` (its FP32 partials are summed
and rounded first). Slots outside the cache and phases outside the tables are
skipped on the device, since the host cannot see the device-side position.
"""

import torch

from kernels import _native
from kernels.merged import source


def qk_rope_cache(packed, q_norm, k_norm, cos, sin, position, keys, values, q_heads, prefill=False, rows=False,
                  phases=None):
    """Normalise and rotate the query and key heads of ``packed`` [B, T, (Hq + 2 Hkv) D] and write
    the key and value heads into the [B, Hkv, C, D] caches.

    Without ``rows`` one [1, T, D] cos/sin pair serves every batch row; with ``rows`` each row has
    its own (or, with ``phases``, its own offsets into whole tables). Prefill fills slots [0, T);
    a decode step fills the T slots from the position held on the device. The result is the
    queries as [B, Hq, T, D], a view of token-major storage that is contiguous for T = 1.
    """
    batch, kv_heads, capacity, dim = keys.shape
    packed, splits, count, shape = source(packed)
    tokens = shape[1]
    assert keys.dtype == values.dtype == torch.bfloat16
    assert packed.dtype == (torch.bfloat16 if splits == 1 else torch.float32)
    assert packed.is_contiguous() and keys.is_contiguous() and values.is_contiguous()
    assert shape == (batch, tokens, (q_heads + 2 * kv_heads) * dim)
    assert 0 < tokens <= capacity
    assert values.shape == keys.shape and dim % 2 == 0
    assert not (rows and prefill)
    table = phases is not None
    if table:
        assert rows and phases.shape == (batch, tokens) and phases.is_contiguous() and phases.dtype == torch.int64
        assert cos.shape == sin.shape and cos.shape[-1] == dim and cos.numel() // dim >= capacity
    else:
        assert cos.numel() == sin.numel() == (batch if rows else 1) * tokens * dim
    assert cos.is_contiguous() and sin.is_contiguous()
    assert position.shape == ((tokens,) if prefill else (batch,) if rows else (1,))
    assert position.dtype == torch.int64
    if dim not in (64, 128):
        raise ValueError(f"head_dim {dim}: these kernels take 64 or 128")
    _native.require_gpu(packed, keys, values, cos, sin, position, q_norm.weight, k_norm.weight)
    query = torch.empty((batch, tokens, q_heads, dim), device=packed.device, dtype=keys.dtype)
    mode = (_native.ROPE_PREFILL if prefill else 0) | (_native.ROPE_ROWS if rows else 0) | \
        (_native.ROPE_TABLE if table else 0)
    q_weight, k_weight = q_norm.weight.contiguous(), k_norm.weight.contiguous()
    _native.call("ftk_qk_rope_cache_bf16", _native.ptr(packed), splits, count if splits > 1 else 0,
                 _native.ptr(q_weight), _native.ptr(k_weight), float(q_norm.variance_epsilon),
                 float(k_norm.variance_epsilon), _native.ptr(cos), _native.ptr(sin), cos.numel() // dim,
                 _native.ptr(position), _native.ptr(phases), _native.ptr(query), _native.ptr(keys),
                 _native.ptr(values), batch, tokens, q_heads, kv_heads, capacity, dim, mode,
                 _native.stream_of(packed))
    return query.transpose(1, 2)
