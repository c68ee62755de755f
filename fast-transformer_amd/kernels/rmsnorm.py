"""Qwen3 RMSNorm with the reference's BF16 cast boundaries (engine/kernels/rmsnorm.py:1-162).

``rms_norm(x, weight, eps)``, ``add_rms_norm(x, residual, weight, eps)`` and
``embed_rms_norm(token_ids, table, weight, eps)`` keep
the reference's signatures, errors and outputs: the normalised value is rounded
to BF16 before the gain multiply (rmsnorm.py:35-46), the residual sum is a
BF16 add (rmsnorm.py:86-95), inputs are never mutated. ``add_rms_norm``
accepts a ``Split`` like the reference. The fused RMSNorm prologue of the
projections is ``kernels.linear.rms_norm_linear`` (with the residual side:
``add_rms_norm_linear``, ``embed_rms_norm_linear``) and the ``norm_weight`` /
``residual`` arguments of ``kernels.swiglu.gate_up_swiglu`` /
``kernels.argmax.lm_head_argmax``.
"""

import torch

from kernels import _native
from kernels.merged import source

#: Kept for signature parity with rmsnorm.py:15; the HIP kernels loop, so any width works.
MAX_BLOCK = 8192


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dimension, matching ``Qwen3RMSNorm.forward`` (rmsnorm.py:49-72)."""
    _native.require_gpu(x, weight)
    shape = x.shape
    rows = x.reshape(-1, shape[-1]).contiguous()
    n_rows, n_cols = rows.shape
    if weight.numel() != n_cols:
        raise ValueError(f"norm weight has {weight.numel()} elements for {n_cols} columns")
    out = torch.empty_like(rows)
    if n_rows == 0:
        return out.reshape(shape)
    _native.call("ftk_rms_norm_bf16", _native.ptr(rows), rows.stride(0), _native.ptr(weight.contiguous()),
                 _native.ptr(out), n_rows, n_cols, float(eps), _native.stream_of(rows))
    return out.reshape(shape)


def add_rms_norm(x, residual, weight, eps):
    """``(rms_norm(s), s)`` for the BF16 sum ``s = x + residual``; neither input is written.

    ``x`` may be a ``Split`` (its partials are summed and rounded before the add). Signature,
    assertions and outputs of engine/kernels/rmsnorm.py:98-125.
    """
    x_data, splits, count, shape = source(x)
    assert shape == tuple(residual.shape)
    assert residual.dtype == weight.dtype == torch.bfloat16
    assert x_data.dtype == (torch.bfloat16 if splits == 1 else torch.float32)
    _native.require_gpu(x_data, residual, weight)
    width = shape[-1]
    x_rows = x_data.reshape(-1, width).contiguous() if splits == 1 else x_data.contiguous()
    residual_rows = residual.reshape(-1, width).contiguous()
    out = torch.empty_like(residual_rows)
    summed = torch.empty_like(residual_rows)
    rows = residual_rows.shape[0]
    if rows == 0:
        return out.reshape(shape), summed.reshape(shape)
    # splits == 1 is a BF16 tensor (C ABI: 0 splits); otherwise FP32 partials [S, rows * width].
    _native.call("ftk_add_rms_norm_bf16", _native.ptr(x_rows), 0 if splits == 1 else splits,
                 count if splits > 1 else 0, _native.ptr(residual_rows), _native.ptr(weight.contiguous()),
                 _native.ptr(out), _native.ptr(summed), rows, width, float(eps), _native.stream_of(residual_rows))
    return out.reshape(shape), summed.reshape(shape)


def embed_rms_norm(token_ids, table, weight, eps):
    """(normalized, hidden) for the embedding rows of ``token_ids`` in one launch (rmsnorm.py:145-162).

    ``hidden`` is the gathered rows (the residual stream), ``normalized`` their
    RMSNorm. int64 ids and a contiguous table, as the reference requires.
    """
    _native.require_gpu(token_ids, table, weight)
    ids = token_ids.reshape(-1).contiguous()
    if not table.is_contiguous() or ids.dtype != torch.int64:
        raise ValueError("embed_rms_norm takes int64 token ids and a contiguous [rows, hidden] table")
    n_cols = table.shape[1]
    hidden = torch.empty((ids.numel(), n_cols), dtype=table.dtype, device=table.device)
    out = torch.empty_like(hidden)
    shape = (*token_ids.shape, n_cols)
    if ids.numel() == 0:
        return out.reshape(shape), hidden.reshape(shape)
    _native.call("ftk_embed_rms_norm_bf16", _native.ptr(ids), 8, _native.ptr(table), _native.ptr(weight.contiguous()),
                 _native.ptr(out), _native.ptr(hidden), ids.numel(), n_cols, float(eps), _native.stream_of(table))
    return out.reshape(shape), hidden.reshape(shape)
