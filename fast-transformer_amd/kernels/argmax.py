"""Greedy token ids from BF16 logits, lowest index on ties (engine/kernels/argmax.py:1-167).

``argmax(logits, block=8192, top=None)``, ``fused_argmax(x, weight, ...)`` and
``greedy_tokens(x, weight, linear, top=None)`` keep the reference's
signatures and int64 results. Ties resolve to the lowest index and NaN counts
as the maximum, torch.argmax's rule; BF16 -> FP32 is exact, so the answer is
identical to torch.argmax of the BF16 logits.

Device scheme (the reference's two stages, argmax.py:19-48): each workgroup
reduces its logits to a 64-bit key per row (orderable BF16 value << 32 |
~index) and stores it; a second small kernel takes the max over the
workgroups and writes the ids. max is order-independent, so results are
deterministic, and no workgroup ever waits on another.

``lm_head_argmax`` is the fused final-norm + lm_head + argmax kernel: the
vocabulary GEMV rounds each logit to BF16 and reduces it in its epilogue,
optionally writing the logits and the winning FP32 logit (``top``).
"""

import torch

from kernels import _native


def argmax(logits, block=8192, top=None):
    """int64 argmax over the last dimension of BF16 logits [..., V]; with ``top`` also the winning logit (FP32)."""
    if logits.dtype != torch.bfloat16:
        return logits.argmax(dim=-1)
    _native.require_gpu(logits, top)
    logits = logits.contiguous()
    vocab = logits.shape[-1]
    rows = logits.numel() // vocab
    out = torch.empty(logits.shape[:-1], dtype=torch.int64, device=logits.device)
    if rows == 0:
        return out
    ws = _native.argmax_workspace(logits.device, rows, vocab)
    if top is not None and (top.dtype != torch.float32 or not top.is_contiguous() or top.numel() < rows):
        raise ValueError("top must be a contiguous FP32 tensor with one slot per row")
    _native.call("ftk_argmax_bf16", _native.ptr(logits), rows, vocab, _native.ptr(out), 8, _native.ptr(top),
                 _native.ptr(ws), ws.numel(), _native.stream_of(logits))
    return out


def lm_head_argmax(x, weight, norm_weight=None, eps=1e-6, logits=True, top=None, ids_dtype=torch.int64,
                   config=None, residual=None, sumsq=None):
    """(ids, logits or None): greedy ids of rms_norm?(x [+ residual]) @ weight.T in one projection kernel.

    Ties go to the lowest index of the BF16-rounded logits. ``residual`` makes
    the prologue the final add_rms_norm of engine/decode.py:264-265 (its sum is
    not needed afterwards). Shapes the fused kernel does not take run the norm,
    projection and argmax kernels in turn. ``sumsq``: a ``kernels.linear.SumSq`` that may
    hold x's sums of squares for the norm.
    """
    _native.require_gpu(x, weight, norm_weight, top, residual)
    if residual is not None and norm_weight is None:
        raise ValueError("a residual needs the norm it feeds (norm_weight)")
    from torch.nn import functional as F

    from kernels.linear import _as_config, _choice, _fusable, fused_project, linear, prefer_native
    from kernels.rmsnorm import add_rms_norm, rms_norm

    shape = x.shape
    flat = x.reshape(-1, shape[-1]).contiguous()
    m, k = flat.shape
    v = weight.shape[0]
    ids = torch.empty(shape[:-1], dtype=ids_dtype, device=x.device)
    out = torch.empty((*shape[:-1], v), dtype=torch.bfloat16, device=x.device) if logits else None
    if top is not None and (top.dtype != torch.float32 or not top.is_contiguous() or top.numel() < m):
        raise ValueError("top must be a contiguous FP32 tensor with one slot per row")
    if m == 0:
        return ids, out
    res = None if residual is None else residual.reshape(-1, shape[-1]).contiguous()
    if config is None and residual is None and _fusable(flat, weight, norm_weight):
        # selected like a plain projection, under its own key (kernels/linear.py _choice); the
        # agreement check compares the logits
        def run(choice, w, inp=flat):
            lg = torch.empty((inp.shape[0], w.shape[0]), device=inp.device, dtype=torch.bfloat16)
            tok = torch.empty((inp.shape[0],), device=inp.device, dtype=ids_dtype)
            st = fused_project(inp, w, _native.EPI_ARGMAX, lg, norm_weight, eps, ids=tok, config=_as_config(choice),
                               sumsq=sumsq)
            return lg if st == _native.FTK_OK else None

        def native_logits(w, inp=flat):
            return F.linear(inp if norm_weight is None else rms_norm(inp, norm_weight, eps), w)

        def native(w, inp=flat):
            return argmax(native_logits(w, inp))

        choice = _choice("argmax", flat, weight, run, native, _native.EPI_ARGMAX, norm_weight is not None,
                         compare=native_logits)
        if choice == "native":
            # the form selection timed: torch's GEMM itself, never a second selection by linear()
            full = native_logits(weight)
            return argmax(full, top=top).to(ids_dtype), (full.reshape(*shape[:-1], v) if logits else None)
        status = fused_project(flat, weight, _native.EPI_ARGMAX, out, norm_weight, eps, ids=ids, top=top,
                               config=_as_config(choice), sumsq=sumsq)
    else:
        status = _native.FTK_ERR_UNSUPPORTED if prefer_native(m, config) else \
            fused_project(flat, weight, _native.EPI_ARGMAX, out, norm_weight, eps, residual=res, ids=ids, top=top,
                          config=config, sumsq=sumsq)
    if status != _native.FTK_OK:
        if residual is not None:
            xn = add_rms_norm(x, residual, norm_weight, eps)[0]
        else:
            xn = x if norm_weight is None else rms_norm(x, norm_weight, eps)
        full = linear(xn, weight)
        return argmax(full, top=top).to(ids_dtype), (full if logits else None)
    return ids, out


def fused_applies(rows, k, n):
    """Whether the fused lm_head + argmax kernel takes this shape."""
    p = _native.Plan()
    return _native.lib().ftk_plan_project(rows, n, k, _native.EPI_ARGMAX, 256, None, p) == _native.FTK_OK


def fused_argmax(x, weight, block_n=64, block_k=128):
    """argmax(x @ weight.T) for <= 32 BF16 rows without materializing the logits; None if not applicable.

    (argmax.py:112-129.) ``block_n``/``block_k`` are accepted for signature parity;
    the HIP kernel needs neither N nor K to be a multiple of anything but K % 8.
    """
    rows = x.numel() // x.shape[-1]
    if rows > _native.MAX_ROWS or x.dtype != torch.bfloat16 or not weight.is_contiguous():
        return None
    if not fused_applies(rows, x.shape[-1], weight.shape[0]):
        return None
    return lm_head_argmax(x, weight, logits=False)[0]


def greedy_tokens(x, weight, linear, top=None):
    """Greedy token per row of x @ weight.T (argmax.py:132-167).

    With ``top`` the caller also wants the logits and the winning logit:
    returns (ids, logits). When ``linear`` is this package's projection, the
    fused lm_head kernel does both in one launch; any other ``linear`` is
    honoured by projecting with it and calling ``argmax``.
    """
    from kernels import linear as _linear_module

    if linear is _linear_module.linear:
        ids, logits = lm_head_argmax(x, weight, logits=top is not None, top=top)
        return (ids, logits) if top is not None else ids
    logits = linear(x, weight)
    if top is not None:
        return argmax(logits, top=top), logits
    return argmax(logits)
