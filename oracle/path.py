"""numpy restatement of the decode-time skinny BF16 projection path (test infrastructure only).

Every tensor crosses this module as BF16 *bit patterns* (uint16 arrays) or
FP32 arrays; nothing here uses torch. Cast placement follows the reference
exactly; reduction order does not matter (the reference promises only FP32
accumulation and one rounding, engine/kernels/linear.py:1-6).

Functions and the reference lines they restate:
  project          engine/kernels/linear.py:27-47 (_gemv), :50-78 (_skinny_gemm),
                   engine/kernels/gemm.py:1-17; agent/local_cpu/shim/references.py:313-328
  project_exact    the fp64 golden of agent/local_cpu/interp/run_numeric.py:51
  merge_splits     engine/kernels/merged.py:37-45, engine/kernels/linear.py:81-93
  rms_norm         engine/kernels/rmsnorm.py:21-46 (HF Qwen3RMSNorm cast order)
  add_rms_norm     engine/kernels/rmsnorm.py:75-95
  swiglu           engine/kernels/swiglu.py:13-24
  paired_swiglu    agent/local_cpu/shim/references.py:356-364 (fused gate/up form)
  argmax_first     engine/kernels/argmax.py:1-9, :19-48
  lm_head_argmax   engine/kernels/argmax.py:73-106, :132-167; engine/decode.py:264-278
"""

import numpy as np

from . import bf16

F32 = np.float32


def _f32(bits):
    return bf16.to_f32(bits)


def project(x_bits, w_bits):
    """y[m, n] = bf16( sum_k f32(x[m, k]) * f32(w[n, k]) ), FP32 accumulation, one rounding.

    x_bits [M, K], w_bits [N, K] (PyTorch Linear layout, K contiguous) -> [M, N] bits.
    (engine/kernels/linear.py:27-47, :50-78; agent/local_cpu/shim/references.py:313-328)
    """
    x = _f32(x_bits).reshape(-1, np.shape(x_bits)[-1])
    w = _f32(w_bits)
    y = np.matmul(x, w.T, dtype=F32)
    return bf16.round_bits(y).reshape(*np.shape(x_bits)[:-1], np.shape(w_bits)[0])


def project_exact(x_bits, w_bits):
    """fp64 product x @ w.T (no rounding): the golden the reference measures ulps against."""
    x = _f32(x_bits).astype(np.float64).reshape(-1, np.shape(x_bits)[-1])
    w = _f32(w_bits).astype(np.float64)
    return (x @ w.T).reshape(*np.shape(x_bits)[:-1], np.shape(w_bits)[0])


def merge_splits(partial):
    """bf16( p[0] + p[1] + ... + p[S-1] ) with FP32 adds in split order.

    partial: FP32 [S, ...]. (engine/kernels/merged.py:37-45; the merge launch
    engine/kernels/linear.py:81-93 sums the same partials.)
    """
    p = np.asarray(partial, dtype=F32)
    total = p[0].copy()
    for s in range(1, p.shape[0]):
        total = (total + p[s]).astype(F32)
    return bf16.round_bits(total)


def _row_scale(v, eps):
    """rsqrt(mean(v^2) + eps) per row, FP32 (the sum itself is taken exactly, then rounded to FP32)."""
    ms = (np.sum(v.astype(np.float64) ** 2, axis=-1, keepdims=True) / v.shape[-1]).astype(F32)
    return (F32(1.0) / np.sqrt((ms + F32(eps)).astype(F32))).astype(F32)


def rms_norm(x_bits, gamma_bits, eps):
    """Qwen3 RMSNorm: y = bf16( f32(bf16(v * rsqrt(mean(v^2) + eps))) * f32(gamma) ).

    The normalised value is rounded to BF16 *before* the gamma multiply
    (engine/kernels/rmsnorm.py:35-46, agent/local_cpu/shim/references.py:42-48).
    """
    v = _f32(x_bits)
    scale = _row_scale(v, eps)
    normed = bf16.round_f32((v * scale).astype(F32))
    return bf16.round_bits((normed * _f32(gamma_bits)).astype(F32))


def add_rms_norm(x_bits, residual_bits, gamma_bits, eps):
    """(normalised, summed): s = bf16(f32(x) + f32(r)), then rms_norm(s).

    (engine/kernels/rmsnorm.py:75-95, :98-125; agent/local_cpu/shim/references.py:51-64)
    """
    summed = bf16.round_bits((_f32(x_bits) + _f32(residual_bits)).astype(F32))
    return rms_norm(summed, gamma_bits, eps), summed


def embed_rms_norm(token_ids, table_bits, gamma_bits, eps):
    """(normalised, hidden): hidden = table[token_ids] (the residual stream), then rms_norm(hidden).

    (engine/kernels/rmsnorm.py:128-162: the gathered row is stored unchanged and
    normalised with the cast order of :35-46.)
    """
    hidden = np.asarray(table_bits)[np.asarray(token_ids, dtype=np.int64)]
    return rms_norm(hidden, gamma_bits, eps), hidden


def silu_bf16(g):
    """bf16( g / (1 + exp(-g)) ) for FP32 g, every step an FP32 operation.

    exp is taken in fp64 and rounded once to FP32 (a correctly rounded FP32 exp);
    the add and the divide are FP32. (engine/kernels/swiglu.py:20-24)
    """
    g = np.asarray(g, dtype=F32)
    with np.errstate(over="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(F32)
    den = (F32(1.0) + e).astype(F32)
    with np.errstate(over="ignore", invalid="ignore"):
        return bf16.round_f32((g / den).astype(F32))


def swiglu(packed_bits):
    """out = bf16( f32(bf16(silu(gate))) * f32(up) ); gate = [..., :I], up = [..., I:].

    (engine/kernels/swiglu.py:13-24, agent/local_cpu/shim/references.py:133-140)
    """
    p = _f32(packed_bits)
    width = p.shape[-1] // 2
    gate, up = p[..., :width], p[..., width:]
    return bf16.round_bits((silu_bf16(gate) * up).astype(F32))


def paired_swiglu(x_bits, w_bits):
    """Fused gate/up projection + SwiGLU over ``w = cat(W_gate, W_up)`` [2I, K].

    gate and up are each rounded to BF16 from their FP32 sums before the SiLU
    (agent/local_cpu/shim/references.py:356-364; packing engine/layers.py:92-95).
    """
    gu = project(x_bits, w_bits)
    return swiglu(gu)


def argmax_first(logit_bits):
    """Index of the maximum BF16 logit along the last axis, lowest index on ties (int64).

    BF16 -> FP32 is exact, so comparing FP32 values compares the BF16 logits.
    A NaN counts as the maximum (torch.argmax / numpy.argmax rule).
    (engine/kernels/argmax.py:1-9, :19-48; agent/local_cpu/shim/references.py:67-87)
    """
    return np.argmax(_f32(logit_bits), axis=-1).astype(np.int64)


def lm_head_argmax(x_bits, w_bits, gamma_bits=None, eps=1e-6):
    """(logit bits [M, V], ids int64 [M], top FP32 [M]) for the final norm + lm_head + greedy argmax.

    (engine/decode.py:264-278; engine/kernels/argmax.py:73-106, :132-167)
    """
    xn = x_bits if gamma_bits is None else rms_norm(x_bits, gamma_bits, eps)
    logits = project(xn, w_bits)
    ids = argmax_first(logits)
    top = np.take_along_axis(_f32(logits), ids[..., None], axis=-1)[..., 0]
    return logits, ids, top


def norm_project(x_bits, gamma_bits, eps, w_bits):
    """rms_norm prologue then projection: the QKV / lm_head input path of engine/decode.py:240-278."""
    return project(rms_norm(x_bits, gamma_bits, eps), w_bits)


def add_norm_project(x_bits, residual_bits, gamma_bits, eps, w_bits):
    """(projection of add_rms_norm(x, r), the BF16 sum): the residual side of the prologue
    (engine/decode.py:240-261 add_rms_norm then the layer's projection)."""
    normed, summed = add_rms_norm(x_bits, residual_bits, gamma_bits, eps)
    return project(normed, w_bits), summed


def gate_up_swiglu(x_bits, w_bits, gamma_bits=None, eps=1e-6):
    """Optional rms_norm prologue, then the fused gate/up + SwiGLU (engine/layers.py:99-102)."""
    xn = x_bits if gamma_bits is None else rms_norm(x_bits, gamma_bits, eps)
    return paired_swiglu(xn, w_bits)
