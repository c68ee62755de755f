"""SwiGLU from packed gate/up, preserving SiLU's BF16 output (engine/kernels/swiglu.py:1-40).

``swiglu(packed)``: out = bf16( f32(bf16(silu(gate))) * f32(up) ) for packed
[..., 2I] BF16 (or a ``Split``), gate = [..., :I], up = [..., I:].

``gate_up_swiglu(x, gate_up_weight, norm_weight=None, eps=1e-6)`` is the fused
form of engine/layers.py:99-102 (``swiglu(linear(x, gate_up_weight))``): one
kernel streams gate row j and up row I + j of cat(W_gate, W_up), rounds both
sums to BF16 and applies SwiGLU in its epilogue; with ``norm_weight`` it also
folds the post-attention RMSNorm into its prologue.
"""

import torch

from kernels import _native
from kernels.merged import source


def swiglu(packed):
    """Contiguous BF16 [..., 2*I] gate/up input (or a Split); new contiguous [..., I] output."""
    data, splits, count, shape = source(packed)
    _native.require_gpu(data)
    width = shape[-1] // 2
    output = torch.empty((*shape[:-1], width), device=data.device, dtype=torch.bfloat16)
    rows = output.numel() // width
    if rows == 0:
        return output
    data = data.contiguous()
    # FP32 data is a Split's partials, one plane included (summed and rounded once);
    # BF16 data is read as stored.
    partials = data.dtype == torch.float32
    _native.call("ftk_swiglu_bf16", _native.ptr(data), splits if partials else 0, count if partials else 0,
                 _native.ptr(output), rows, width, _native.stream_of(data))
    return output


def gate_up_swiglu(x, gate_up_weight, norm_weight=None, eps=1e-6, config=None, residual=None, sumsq=None):
    """swiglu(rms_norm?(x [+ residual]) @ gate_up_weight.T) in one projection kernel; [..., I] BF16.

    With ``residual`` the prologue is add_rms_norm (engine/kernels/rmsnorm.py:75-125,
    the post-attention norm of engine/decode.py:258-261) and the result is
    ``(activation, x + residual)``: the sum is the next residual stream. ``sumsq``: a
    ``kernels.linear.SumSq`` that may hold x's sums of squares for the norm.
    """
    _native.require_gpu(x, gate_up_weight, norm_weight, residual)
    if residual is not None and norm_weight is None:
        raise ValueError("a residual needs the norm it feeds (norm_weight)")
    from torch.nn import functional as F

    from kernels.linear import _as_config, _choice, _fusable, fused_project, linear, prefer_native
    from kernels.rmsnorm import rms_norm

    shape = x.shape
    flat = x.reshape(-1, shape[-1]).contiguous()
    m, k = flat.shape
    n = gate_up_weight.shape[0]
    if n % 2:
        raise ValueError("gate_up_weight must stack gate and up rows: an even row count")
    out = torch.empty((m, n // 2), device=x.device, dtype=torch.bfloat16)
    res = None if residual is None else residual.reshape(-1, shape[-1]).contiguous()
    summed = None if residual is None else torch.empty_like(res)
    if m == 0:
        act = out.reshape(*shape[:-1], n // 2)
        return act if residual is None else (act, summed.reshape(shape))
    if config is None and residual is None and _fusable(flat, gate_up_weight, norm_weight):
        # selected like a plain projection, under its own key (kernels/linear.py _choice)
        def run(choice, w, inp=flat):
            y = torch.empty((inp.shape[0], w.shape[0] // 2), device=inp.device, dtype=torch.bfloat16)
            st = fused_project(inp, w, _native.EPI_SWIGLU, y, norm_weight, eps, config=_as_config(choice),
                               sumsq=sumsq)
            return y if st == _native.FTK_OK else None

        def native(w, inp=flat):
            return swiglu(F.linear(inp if norm_weight is None else rms_norm(inp, norm_weight, eps), w))

        choice = _choice("swiglu", flat, gate_up_weight, run, native, _native.EPI_SWIGLU, norm_weight is not None)
        if choice == "native":
            # the form selection timed: torch's GEMM itself, never a second selection by linear()
            return native(gate_up_weight).reshape(*shape[:-1], n // 2)
        status = fused_project(flat, gate_up_weight, _native.EPI_SWIGLU, out, norm_weight, eps,
                               config=_as_config(choice), sumsq=sumsq)
    else:
        status = _native.FTK_ERR_UNSUPPORTED if prefer_native(m, config) else \
            fused_project(flat, gate_up_weight, _native.EPI_SWIGLU, out, norm_weight, eps, residual=res,
                          summed=summed, config=config, sumsq=sumsq)
    if status != _native.FTK_OK:
        from kernels.rmsnorm import add_rms_norm, rms_norm
        if residual is not None:
            xn, summed = add_rms_norm(x, residual, norm_weight, eps)
            return swiglu(linear(xn, gate_up_weight)), summed
        xn = x if norm_weight is None else rms_norm(x, norm_weight, eps)
        return swiglu(linear(xn, gate_up_weight))
    act = out.reshape(*shape[:-1], n // 2)
    return act if residual is None else (act, summed.reshape(shape))
