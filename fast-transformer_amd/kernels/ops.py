"""The path's operators as torch custom ops: ``torch.ops.ftk.*``.

Each op calls the same libftk.so entry point as the Python function it is
named after (include/ftk.h, through ``kernels._native``), so eager results
are identical. A fake (meta) implementation gives the output shapes without
running anything, so the ops trace under ``torch.compile`` / ``torch.export``
and take part in FakeTensor shape propagation. Mutated arguments are declared
(``qk_rope_cache`` and ``rope_attend`` write the KV caches in place).

    import kernels.ops  # registers the ops
    y = torch.ops.ftk.rms_norm_linear(x, gamma, 1e-6, w)

Registered:
  ftk::linear(x, weight)                                    engine/kernels/linear.py:489-523
  ftk::linear_residual(x, weight, residual)                 linear + the add of rmsnorm.py:86-95 in its epilogue
  ftk::rms_norm_linear(x, norm_weight, eps, weight)         rmsnorm.py:49-72 + linear
  ftk::add_rms_norm_linear(x, residual, norm_weight, eps, weight) -> (y, summed)
  ftk::gate_up_swiglu(x, gate_up_weight, norm_weight?, eps) swiglu.py:13-40 fused into the projection
  ftk::lm_head_argmax(x, weight, norm_weight?, eps) -> (ids, logits)   argmax.py:73-167
  ftk::rms_norm(x, weight, eps)                             rmsnorm.py:49-72
  ftk::add_rms_norm(x, residual, weight, eps) -> (normalized, summed)   rmsnorm.py:98-125
  ftk::swiglu(packed)                                       swiglu.py:27-40
  ftk::argmax(logits)                                       argmax.py:51-70
  ftk::decode_attention(query, key, value, position, scale) decode_attention.py:229-258
  ftk::qk_rope_cache(packed, q_weight, k_weight, q_eps, k_eps, cos, sin, position, keys!, values!, q_heads)
                                                            qk_rope.py:97-129 (one decode step)
  ftk::rope_attend(packed, q_weight, k_weight, q_eps, k_eps, cos, sin, position, keys!, values!, q_heads, scale,
                   phases?)                                 both of the above in one launch (layers.py:51-55, :76)
"""

from typing import Optional, Tuple

import torch
from torch import Tensor

from kernels import argmax as _argmax
from kernels import decode_attention as _attention
from kernels import linear as _linear
from kernels import qk_rope as _rope
from kernels import rmsnorm as _rmsnorm
from kernels import swiglu as _swiglu


class _Norm:
    def __init__(self, weight, eps):
        self.weight, self.variance_epsilon = weight, eps


@torch.library.custom_op("ftk::linear", mutates_args=())
def linear(x: Tensor, weight: Tensor) -> Tensor:
    return _linear.linear(x, weight)


@linear.register_fake
def _(x, weight):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


@torch.library.custom_op("ftk::linear_residual", mutates_args=())
def linear_residual(x: Tensor, weight: Tensor, residual: Tensor) -> Tensor:
    return _linear.linear_residual(x, weight, residual)


@linear_residual.register_fake
def _(x, weight, residual):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


@torch.library.custom_op("ftk::rms_norm_linear", mutates_args=())
def rms_norm_linear(x: Tensor, norm_weight: Tensor, eps: float, weight: Tensor) -> Tensor:
    return _linear.rms_norm_linear(x, norm_weight, eps, weight)


@rms_norm_linear.register_fake
def _(x, norm_weight, eps, weight):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


@torch.library.custom_op("ftk::add_rms_norm_linear", mutates_args=())
def add_rms_norm_linear(x: Tensor, residual: Tensor, norm_weight: Tensor, eps: float,
                        weight: Tensor) -> Tuple[Tensor, Tensor]:
    return _linear.add_rms_norm_linear(x, residual, norm_weight, eps, weight)


@add_rms_norm_linear.register_fake
def _(x, residual, norm_weight, eps, weight):
    return x.new_empty((*x.shape[:-1], weight.shape[0])), torch.empty_like(x)


@torch.library.custom_op("ftk::gate_up_swiglu", mutates_args=())
def gate_up_swiglu(x: Tensor, gate_up_weight: Tensor, norm_weight: Optional[Tensor], eps: float) -> Tensor:
    return _swiglu.gate_up_swiglu(x, gate_up_weight, norm_weight, eps)


@gate_up_swiglu.register_fake
def _(x, gate_up_weight, norm_weight, eps):
    return x.new_empty((*x.shape[:-1], gate_up_weight.shape[0] // 2))


@torch.library.custom_op("ftk::lm_head_argmax", mutates_args=())
def lm_head_argmax(x: Tensor, weight: Tensor, norm_weight: Optional[Tensor], eps: float) -> Tuple[Tensor, Tensor]:
    ids, logits = _argmax.lm_head_argmax(x, weight, norm_weight, eps, logits=True)
    return ids, logits


@lm_head_argmax.register_fake
def _(x, weight, norm_weight, eps):
    return (x.new_empty(x.shape[:-1], dtype=torch.int64), x.new_empty((*x.shape[:-1], weight.shape[0])))


@torch.library.custom_op("ftk::rms_norm", mutates_args=())
def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    return _rmsnorm.rms_norm(x, weight, eps)


@rms_norm.register_fake
def _(x, weight, eps):
    return torch.empty_like(x)


@torch.library.custom_op("ftk::add_rms_norm", mutates_args=())
def add_rms_norm(x: Tensor, residual: Tensor, weight: Tensor, eps: float) -> Tuple[Tensor, Tensor]:
    normalized, summed = _rmsnorm.add_rms_norm(x, residual, weight, eps)
    return normalized, summed


@add_rms_norm.register_fake
def _(x, residual, weight, eps):
    return torch.empty_like(x), torch.empty_like(x)


@torch.library.custom_op("ftk::swiglu", mutates_args=())
def swiglu(packed: Tensor) -> Tensor:
    return _swiglu.swiglu(packed)


@swiglu.register_fake
def _(packed):
    return packed.new_empty((*packed.shape[:-1], packed.shape[-1] // 2))


@torch.library.custom_op("ftk::argmax", mutates_args=())
def argmax(logits: Tensor) -> Tensor:
    return _argmax.argmax(logits)


@argmax.register_fake
def _(logits):
    return logits.new_empty(logits.shape[:-1], dtype=torch.int64)


@torch.library.custom_op("ftk::decode_attention", mutates_args=())
def decode_attention(query: Tensor, key: Tensor, value: Tensor, position: Tensor, scale: float) -> Tensor:
    return _attention.decode_attention(query, key, value, position, scale)


@decode_attention.register_fake
def _(query, key, value, position, scale):
    batch, heads, _, dim = query.shape
    return query.new_empty((batch, 1, heads, dim))


@torch.library.custom_op("ftk::qk_rope_cache", mutates_args=("keys", "values"))
def qk_rope_cache(packed: Tensor, q_weight: Tensor, k_weight: Tensor, q_eps: float, k_eps: float, cos: Tensor,
                  sin: Tensor, position: Tensor, keys: Tensor, values: Tensor, q_heads: int) -> Tensor:
    query = _rope.qk_rope_cache(packed, _Norm(q_weight, q_eps), _Norm(k_weight, k_eps), cos, sin, position, keys,
                                values, q_heads)
    return query.transpose(1, 2).contiguous()  # token-major [B, T, Hq, D]: an op returns a fresh tensor


@qk_rope_cache.register_fake
def _(packed, q_weight, k_weight, q_eps, k_eps, cos, sin, position, keys, values, q_heads):
    batch, tokens = packed.shape[:2]
    return packed.new_empty((batch, tokens, q_heads, keys.shape[-1]), dtype=keys.dtype)


@torch.library.custom_op("ftk::rope_attend", mutates_args=("keys", "values"))
def rope_attend(packed: Tensor, q_weight: Tensor, k_weight: Tensor, q_eps: float, k_eps: float, cos: Tensor,
                sin: Tensor, position: Tensor, keys: Tensor, values: Tensor, q_heads: int, scale: float,
                phases: Optional[Tensor] = None) -> Tensor:
    return _attention.rope_attend(packed, _Norm(q_weight, q_eps), _Norm(k_weight, k_eps), cos, sin, position, keys,
                                  values, q_heads, scale, phases=phases)


@rope_attend.register_fake
def _(packed, q_weight, k_weight, q_eps, k_eps, cos, sin, position, keys, values, q_heads, scale, phases=None):
    return packed.new_empty((packed.shape[0], 1, q_heads, keys.shape[-1]), dtype=keys.dtype)
