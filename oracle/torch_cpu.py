"""The reference's native torch formulation of the path, on the CPU (test infrastructure only).

This is what the reference falls back to and measures itself against:
BF16 ``torch.nn.functional.linear`` (engine/kernels/linear.py:456-458,
:492-493, :517-518), Qwen3's RMSNorm with native cast placement
(engine/kernels/rmsnorm.py:35-46; agent/local_cpu/interp/run_numeric.py:16-18),
``F.silu(gate) * up`` (run_numeric.py:30) and ``torch.argmax`` of BF16 logits
(engine/kernels/argmax.py:56-57). It is timed as the CPU baseline in bench.py
and used in tests as a second opinion beside the numpy oracle.
"""

import torch
from torch.nn import functional as F


def linear(x, w):
    """BF16 x @ w.T (the reference's native fallback)."""
    return F.linear(x, w)


def rms_norm(x, gamma, eps):
    v = x.float()
    v = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)
    return gamma * v.to(x.dtype)


def add_rms_norm(x, residual, gamma, eps):
    summed = x + residual
    return rms_norm(summed, gamma, eps), summed


def swiglu(packed):
    gate, up = packed.chunk(2, dim=-1)
    return F.silu(gate) * up


def gate_up_swiglu(x, w, gamma=None, eps=1e-6):
    xn = x if gamma is None else rms_norm(x, gamma, eps)
    return swiglu(F.linear(xn, w))


def lm_head_argmax(x, w, gamma=None, eps=1e-6):
    xn = x if gamma is None else rms_norm(x, gamma, eps)
    logits = F.linear(xn, w)
    return logits, logits.argmax(-1)


def layer_projections(h, attn, layer, eps):
    """One decode layer's projection set at the reference's cast placement.

    h: residual stream [M, H]; attn: attention output [M, Hq*D] (attention itself is
    outside the path); layer: dict of BF16 weights (qkv, o, gate_up, down) and norm
    gains (ln1, ln2). Returns (qkv, o, act, down) outputs. Mirrors engine/decode.py:240-261
    with engine/layers.py:44, :86, :101-102.
    """
    qkv = F.linear(rms_norm(h, layer["ln1"], eps), layer["qkv"])
    o = F.linear(attn, layer["o"])
    act = gate_up_swiglu(o, layer["gate_up"], layer["ln2"], eps)
    down = F.linear(act, layer["down"])
    return qkv, o, act, down
