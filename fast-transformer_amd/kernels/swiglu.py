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
    data = data.contiguous()
    _native.call("ftk_swiglu_bf16", _native.ptr(data), 0 if splits == 1 else splits, count if splits > 1 else 0,
                 _native.ptr(output), rows, width, _native.stream_of(data))
    return output


def gate_up_swiglu(x, gate_up_weight, norm_weight=None, eps=1e-6, config=None):
    """swiglu(rms_norm?(x) @ gate_up_weight.T) in one projection kernel; [..., I] BF16."""
    _native.require_gpu(x, gate_up_weight, norm_weight)
    shape = x.shape
    flat = x.reshape(-1, shape[-1]).contiguous()
    m, k = flat.shape
    n = gate_up_weight.shape[0]
    if n % 2:
        raise ValueError("gate_up_weight must stack gate and up rows: an even row count")
    out = torch.empty((m, n // 2), device=x.device, dtype=torch.bfloat16)
    ws = _native.project_workspace(x.device, m, n, k, _native.EPI_SWIGLU, config, prologue=norm_weight is not None)
    status = _native.try_call(
        "ftk_project_bf16", _native.ptr(flat), _native.ptr(norm_weight), float(eps), _native.ptr(gate_up_weight),
        _native.ptr(out), m, n, k, _native.EPI_SWIGLU, None, 0, None, _native.ptr(ws), ws.numel(), config,
        _native.stream_of(flat))
    if status == _native.FTK_ERR_UNSUPPORTED:
        from kernels.linear import linear
        from kernels.rmsnorm import rms_norm
        xn = x if norm_weight is None else rms_norm(x, norm_weight, eps)
        return swiglu(linear(xn, gate_up_weight))
    if status != _native.FTK_OK:
        raise _native.FtkError("ftk_project_bf16", status)
    return out.reshape(*shape[:-1], n // 2)
