"""BF16 skinny projections y = x @ W.T for M <= 32 rows, on gfx950 HIP kernels.

Drop-in for engine/kernels/linear.py: ``linear(x, weight, split_ok=False)``,
``keep_native(rows, weight)`` and ``MAX_ROWS`` keep the reference's names,
argument meaning and fallback rule (linear.py:484-523). FP32 accumulation and
one rounding to BF16 (linear.py:1-6). Under them:

  * M = 1 (and plain projections to M = 4): an HBM-streaming GEMV (x slice in
    registers, 16-byte non-temporal weight loads, v_dot2_f32_bf16, DPP reductions);
  * M = 2..16: MFMA kinds (4x4x4 blocks fed straight from 4-row x 256-byte
    loads, or 16x16x32 tiles fed through LDS), as the C library's planner picks;
    ragged K or an unaligned pointer takes a generic kernel with scalar loads;
  * M = 17..32: torch's native GEMM by default (hipBLASLt measured faster there),
    the way the reference keeps cuBLAS unless a timed kind beats it; the fused
    forms run their norm / epilogue kernels around it. An explicit config, or
    the first-use timing of the candidates (on unless FTK_TUNE=0), still
    launches these kernels at any M.

``split_ok`` is accepted for signature compatibility. The result is always a
contiguous BF16 tensor, which the reference allows ("may be" a Split,
linear.py:490): split-K is finished inside the kernel.

Beyond the reference's surface, the fused forms of the path live here too:
``rms_norm_linear`` (RMSNorm prologue + projection), and in swiglu.py /
argmax.py the SwiGLU and greedy-argmax epilogues.
"""

import ctypes
import os
import statistics
import time

import torch
from torch.nn import functional as F

from kernels import _native
from kernels.tune import knobs, register

#: Verify blocks of up to 32 rows still read each weight once per step (linear.py:340-343).
MAX_ROWS = _native.MAX_ROWS

#: Frozen launch choices by shape key (see the selection section below): None = planner default,
#: "native" = torch's GEMM (keep_native), or a launch tuple. _VALIDATED: the timed candidates.
_CHOICES = {}
_VALIDATED = {}
#: Time the candidate launch shapes of each shape at its first eager use, as linear.py:494-511
#: always does. On by default; FTK_TUNE=0 (or ``TUNE = False``) keeps the planner's defaults, which
#: come from the same kind of timing, done once on MI355X.
TUNE = os.environ.get("FTK_TUNE", "1") != "0"

#: From this many rows the planner's default is torch's native GEMM (hipBLASLt), as the reference
#: keeps cuBLAS unless a timed kind beats it (linear.py:455-475). Measured on MI355X at Qwen3-8B
#: shapes: at 32 rows hipBLASLt is 1.6-2.7x faster than these kernels; at 16 and fewer rows these
#: kernels are faster on every projection (1.09x for down at 16 rows, up to 2.1x for O).
NATIVE_FROM_ROWS = 17


def prefer_native(rows, config=None):
    """Whether a call with no explicit launch choice goes to the native GEMM (plus separate norm /
    epilogue kernels for the fused forms)."""
    return config is None and rows >= NATIVE_FROM_ROWS


def _fusable(flat, weight, norm_weight=None):
    """Whether the fused kernels take these operands (K % 8 == 0, 16-byte aligned): only then is
    there a kernel choice to select."""
    ptrs = [flat.data_ptr(), weight.data_ptr()] + ([] if norm_weight is None else [norm_weight.data_ptr()])
    return flat.shape[1] % 8 == 0 and all(p % 16 == 0 for p in ptrs)


def _as_rows(x):
    rows = x.numel() // x.shape[-1]
    return x.reshape(rows, x.shape[-1]).contiguous()


class SumSq:
    """The RMSNorm statistics of a row stream, handed from the projection that writes the rows to the
    norm that reads them next (``ftk_rows.sumsq_out`` / ``sumsq``; the RING kind, 2..16 rows).

    A projection given this object without a norm (``linear_sumsq``, ``project``, ``linear_residual``)
    writes, beside its output ``y`` [M, N], the FP32 sums of the squares of each row's stored BF16
    values by 16-column part. A later norm-prologue call over that same ``y`` (``rms_norm_linear``,
    ``gate_up_swiglu``, ``lm_head_argmax`` given the object) sums those parts instead of reading the
    rows: its kernel need not wait for every row of x before its first products. The sums are used
    only while they describe the call's x: the same tensor (address and shape; the object keeps its
    storage alive), unchanged since it was written (version counter). Otherwise, or where either
    launch is not RING, the norm reads x as usual. One object serves a whole decode step: each producer overwrites the
    sums, and each norm reads the sums of its own input.
    """

    def __init__(self):
        self._buf = None
        self._src = None

    def _out(self, y):
        """Buffer for the sums of ``y`` [M, N]; the previous sums stop counting."""
        self._src = None
        need = y.shape[0] * ((y.shape[1] + 15) // 16)
        buf = self._buf
        if buf is None or buf.device != y.device or buf.numel() < need:
            if y.is_cuda and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("SumSq buffers must be sized during eager warmup, before graph capture")
            if buf is not None:
                _native._RETIRED.append(buf)  # a captured graph may hold its address
            buf = self._buf = torch.empty(max(need, 4096), dtype=torch.float32, device=y.device)
        return buf

    def _wrote(self, y):
        # Holding y's storage keeps its address from being handed to another tensor meanwhile.
        self._src = (y.untyped_storage(), y.data_ptr(), tuple(y.shape), y._version, y.device)

    def _of(self, x):
        """The sums of ``x`` [M, K], or None where they do not describe it."""
        src = self._src
        if src is None or (x.data_ptr(), tuple(x.shape), x._version, x.device) != src[1:]:
            return None
        return self._buf


def fused_project(x, weight, epilogue, out, norm_weight=None, eps=1e-6, residual=None, x_ids=None, summed=None,
                  ids=None, top=None, config=None, sumsq=None):
    """One projection launch with its fused prologue / epilogue (ftk_project_rows_bf16).

    ``x`` is [M, K] (or, with ``x_ids``, the [rows, K] table they index);
    ``residual`` [M, K] is added before the norm and ``summed`` [M, K] receives
    the rows the norm read. ``sumsq`` (a ``SumSq``): with the norm, its sums of x
    replace the norm's read of x where they describe x; without it (the STORE
    epilogue), the call writes the sums of ``out``. Returns the C status: FTK_OK, or
    FTK_ERR_UNSUPPORTED when the shape / alignment has no fused kernel (the
    caller then composes the separate kernels). Raises on anything else.
    """
    m = x_ids.numel() if x_ids is not None else x.shape[0]
    k = x.shape[1]
    n = weight.shape[0]
    sq_in = sq_out = None
    if sumsq is not None:
        if norm_weight is not None:
            if residual is None and summed is None and x_ids is None:
                sq_in = sumsq._of(x)
        elif epilogue == _native.EPI_STORE:
            sq_out = sumsq._out(out)
    ws = _native.project_workspace(x.device, m, n, k, epilogue, config, prologue=norm_weight is not None,
                                   residual=residual is not None)
    ids_bytes = 0 if ids is None else {torch.int64: 8, torch.int32: 4}[ids.dtype]

    def call(sq_in, sq_out):
        rows = None
        if residual is not None or summed is not None or x_ids is not None or sq_in is not None or sq_out is not None:
            x_ids_bytes = 0 if x_ids is None else {torch.int64: 8, torch.int32: 4}[x_ids.dtype]
            table_rows = x.shape[0] if x_ids is not None else 0
            rows = ctypes.byref(_native.Rows(_native.ptr(residual), _native.ptr(summed), _native.ptr(x_ids),
                                             x_ids_bytes, table_rows, _native.ptr(sq_in), _native.ptr(sq_out)))
        return _native.try_call(
            "ftk_project_rows_bf16", _native.ptr(x), rows, _native.ptr(norm_weight), float(eps),
            _native.ptr(weight), _native.ptr(out), m, n, k, epilogue, _native.ptr(ids), ids_bytes,
            _native.ptr(top), _native.ptr(ws), ws.numel(), config, _native.stream_of(x))

    status = call(sq_in, sq_out)
    if status == _native.FTK_ERR_UNSUPPORTED and (sq_in is not None or sq_out is not None):
        status = call(None, None)  # not a RING launch: the norm reads x, no sums are written
    elif status == _native.FTK_OK and sq_out is not None:
        sumsq._wrote(out)
    if status not in (_native.FTK_OK, _native.FTK_ERR_UNSUPPORTED):
        raise _native.FtkError("ftk_project_rows_bf16", status)
    return status


def project(x, weight, config=None, out=None, sumsq=None):
    """y[M, N] = x[M, K] @ weight[N, K].T on the GPU (the device work of _project, linear.py:178-314).

    ``config`` is a ``_native.Config`` (None = planner default). ``sumsq`` (a ``SumSq``) receives
    the rows' sums of squares for the norm that reads y next. Raises on any unsupported input;
    there is no fallback here.
    """
    _native.require_gpu(x, weight)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("project takes BF16 x and weight")
    if not weight.is_contiguous():
        raise ValueError("project takes a contiguous [N, K] weight")
    m, k = x.shape
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError(f"x has K={k}, weight has K={weight.shape[1]}")
    if out is None:
        out = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
    if m == 0:
        return out
    status = fused_project(x, weight, _native.EPI_STORE, out, config=config, sumsq=sumsq)
    if status == _native.FTK_ERR_UNSUPPORTED:
        if config is not None:
            raise _native.FtkError("ftk_project_rows_bf16", status)
        # unaligned pointers: the generic kind takes any alignment
        _native.call("ftk_linear_bf16", _native.ptr(x), _native.ptr(weight), _native.ptr(out), m, n, k,
                     _native.stream_of(x))
    return out


def rms_norm_linear(x, norm_weight, eps, weight, config=None, sumsq=None):
    """rms_norm(x, norm_weight, eps) @ weight.T with the norm folded into the projection's prologue.

    Cast order of engine/kernels/rmsnorm.py:35-46 (normalised value rounded to
    BF16 before the gain multiply). Shapes no fused kernel takes (K % 8 != 0,
    unaligned) run the separate norm kernel, then ``linear``. ``sumsq``: a ``SumSq``
    that may hold x's sums of squares (written by the projection that produced x).
    """
    _native.require_gpu(x, norm_weight, weight)
    from kernels.rmsnorm import rms_norm

    shape = x.shape
    flat = _as_rows(x)
    m, k = flat.shape
    n = weight.shape[0]
    if m == 0:
        return torch.empty((*shape[:-1], n), device=x.device, dtype=torch.bfloat16)

    def fused(cfg, w, inp=flat):
        y = torch.empty((inp.shape[0], w.shape[0]), device=inp.device, dtype=torch.bfloat16)
        status = fused_project(inp, w, _native.EPI_STORE, y, norm_weight, eps, config=cfg, sumsq=sumsq)
        return y if status == _native.FTK_OK else None

    if config is None and _fusable(flat, weight, norm_weight):
        def native(w, inp=flat):
            return F.linear(rms_norm(inp, norm_weight, eps), w)

        choice = _choice("norm", flat, weight, lambda c, w, inp=flat: fused(_as_config(c), w, inp), native,
                         prologue=True)
        if choice == "native":
            # the form selection timed: torch's GEMM itself, never a second selection by linear()
            return native(weight).reshape(*shape[:-1], n)
        out = fused(_as_config(choice), weight)
    else:
        out = None if prefer_native(m, config) else fused(config, weight)
    if out is None:
        return linear(rms_norm(x, norm_weight, eps), weight)
    return out.reshape(*shape[:-1], n)


def add_rms_norm_linear(x, residual, norm_weight, eps, weight, config=None):
    """(add_rms_norm(x, residual)[0] @ weight.T, x + residual) in one launch.

    The residual side of the prologue (engine/kernels/rmsnorm.py:75-125, the
    calls at engine/decode.py:240-261): s = bf16(x + residual) is normalised
    and projected, and s is returned as the next residual. Inputs are not
    modified. Shapes without a fused kernel run add_rms_norm, then ``linear``.
    """
    _native.require_gpu(x, residual, norm_weight, weight)
    if tuple(x.shape) != tuple(residual.shape):
        raise ValueError("x and residual must have the same shape")
    shape = x.shape
    flat, res = _as_rows(x), _as_rows(residual)
    m, k = flat.shape
    n = weight.shape[0]
    out = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
    summed = torch.empty_like(res)
    if m == 0:
        return out.reshape(*shape[:-1], n), summed.reshape(shape)
    status = _native.FTK_ERR_UNSUPPORTED if prefer_native(m, config) else \
        fused_project(flat, weight, _native.EPI_STORE, out, norm_weight, eps, residual=res, summed=summed,
                      config=config)
    if status != _native.FTK_OK:
        from kernels.rmsnorm import add_rms_norm
        normed, summed = add_rms_norm(x, residual, norm_weight, eps)
        return linear(normed, weight), summed
    return out.reshape(*shape[:-1], n), summed.reshape(shape)


def embed_rms_norm_linear(token_ids, table, norm_weight, eps, weight, config=None):
    """(embed_rms_norm(token_ids, table)[0] @ weight.T, the embedding rows) in one launch.

    The first layer's input (engine/kernels/rmsnorm.py:128-162, engine/decode.py:229):
    row m = table[token_ids[m]], normalised and projected; the gathered rows are
    returned as the residual stream. ``token_ids`` int64 or int32.
    """
    _native.require_gpu(token_ids, table, norm_weight, weight)
    ids = token_ids.reshape(-1).contiguous()
    k = table.shape[1]
    n = weight.shape[0]
    out = torch.empty((ids.numel(), n), device=table.device, dtype=torch.bfloat16)
    hidden = torch.empty((ids.numel(), k), device=table.device, dtype=torch.bfloat16)
    if ids.numel() == 0:
        return out.reshape(*token_ids.shape, n), hidden.reshape(*token_ids.shape, k)
    status = _native.FTK_ERR_UNSUPPORTED if prefer_native(ids.numel(), config) else \
        fused_project(table.contiguous(), weight, _native.EPI_STORE, out, norm_weight, eps, x_ids=ids,
                      summed=hidden, config=config)
    if status != _native.FTK_OK:
        from kernels.rmsnorm import embed_rms_norm
        normed, hidden = embed_rms_norm(token_ids, table, norm_weight, eps)
        return linear(normed, weight), hidden
    return out.reshape(*token_ids.shape, n), hidden.reshape(*token_ids.shape, k)


# ---- selection: each shape's launch choice, timed once during eager warmup ----------------------
#
# The reference's policy (engine/kernels/linear.py:317-486): on a shape's first use, outside graph
# capture, time the candidate layouts that pass an operator sanity check against the native GEMM
# on cold weights; a kind must beat the best so far by 1.5 %, and the winner is checked against
# native once more. The three fastest are registered as a knob, which ``refine`` re-judges inside
# a captured step. Here the candidates are this library's launch shapes (kind, rows_per_wave,
# unroll, groups_per_cu, waves) for the planner, plus its default; "native" is torch's GEMM with
# this library's norm / SwiGLU / argmax kernels around it. The fused forms are selected the same
# way as plain projections, each under its own key.

#: Selection budgets per shape and per process, as the reference's _SHAPE_SECONDS and
#: _PROCESS_SECONDS (linear.py:345-348). Past the process budget a shape is not timed: a verify
#: block (5..MAX_ROWS rows) takes a choice already validated for the same weight at another row
#: count (_inherit), any other shape its untuned default. FTK_TUNE_SECONDS sets the process budget.
SHAPE_SECONDS = 6.0
PROCESS_SECONDS = float(os.environ.get("FTK_TUNE_SECONDS", "28"))
_TUNING_DEADLINE = None
#: Seconds this process has spent timing candidates, and the shapes past the budget.
tuning_seconds = 0.0
inherited = {}
#: Weight bytes cycled through per timing graph: distinct copies, so no call is served from the
#: 256 MB MALL (the MI355X counterpart of _cold_graph_time's 128 MiB flush, linear.py:317-337).
COLD_BYTES = 768 << 20


def _key(op, device, rows, n, k):
    """Plain projections keep the reference's key (linear.py:446); fused forms prefix their operation."""
    return (device, rows, n, k) if op == "linear" else (op, device, rows, n, k)


def _as_config(choice):
    return None if choice is None or choice == "native" else _native.Config(*choice)


def _candidates(m, n, k, epilogue=_native.EPI_STORE, prologue=False):
    """Launch shapes worth timing for one (M, N, K): the planner accepts each for this epilogue."""
    if k % 8:
        return []
    configs = []
    if m <= 4:
        for rpw, unroll, kw in ((2, 4, 1), (4, 2, 1), (2, 2, 2), (2, 4, 2), (1, 1, 4), (2, 2, 4)):
            configs.append((_native.KIND_GEMV, rpw, unroll, 8, kw))
    if m <= 8:
        for rpw in (1, 2, 4, 8):
            for kw in (1, 2, 4, 8):
                for gpc in (2, 16, 32):
                    configs.append((_native.KIND_STREAM, rpw, 0, gpc, kw))
    if 2 <= m <= 16:
        for rows in (4, 8, 16, 24):
            for kw in (4, 8):
                for gpc in (1, 32):
                    configs.append((_native.KIND_QUAD, rows, 0, gpc, kw))
    if 2 <= m <= 16 or (m == 1 and epilogue == _native.EPI_ARGMAX):
        for rows in (12, 16, 24):
            for depth in (2, 3):
                for gpc in (1, 2):
                    configs.append((_native.KIND_RING, rows, depth, gpc, 8))
    if m >= 5:
        for rows in (16, 32):
            for unroll in (2, 3, 4):
                for gpc in (1, 2):
                    configs.append((_native.KIND_STAGE, rows, unroll, gpc, 8))
        for rows in (16, 32):
            for kw, unroll in ((8, 4), (8, 8), (16, 4)):
                configs.append((_native.KIND_MFMA_STREAM, rows, unroll, 1, kw))
    for rows, unroll, waves in ((16, 4, 4), (16, 8, 8), (32, 4, 8), (64, 2, 4)):
        configs.append((_native.KIND_MFMA, rows, unroll, 0, waves))
    p = _native.Plan()
    flags = epilogue | (_native.PLAN_PROLOGUE if prologue else 0)
    return [c for c in configs if _native.lib().ftk_plan_project(m, n, k, flags, 256, _native.Config(*c), p)
            == _native.FTK_OK]


def _cold_us(fn, weights, reps=5):
    """Median µs of one call of ``fn(w)``, timed over graph replays that cycle through ``weights``
    (distinct copies, so every call streams its weight from HBM)."""
    for w in weights[:2]:
        fn(w)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for w in weights:
                fn(w)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(reps):
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3 / len(weights))
    return statistics.median(times)


def _agrees(got, reference):
    """Operator sanity check against the native GEMM's output: |Δ| <= 0.016 |ref| + 0.001 (linear.py:399-409)."""
    got, ref = got.float(), reference.float()
    return bool(((got - ref).abs() <= ref.abs() * 0.016 + 0.001).all())


def _choose(op, x, weight, run, native, epilogue=_native.EPI_STORE, prologue=False, compare=None):
    """Time the candidates of one shape once, eagerly (linear.py:436-481); returns the choice.

    ``run(choice, w, inp)`` computes the operation with a launch choice (None = planner default)
    on weight ``w`` and input ``inp``; ``native(w, inp)`` is the native-GEMM form, and
    ``compare(w, inp)`` (default ``native``) its output in the form ``run`` returns (the logits,
    for lm_head + argmax). Every candidate, the planner default included, must agree with the
    native output on a fixed probe input before it is timed (linear.py:452-453).
    """
    global _TUNING_DEADLINE, tuning_seconds
    m, k = x.shape
    n = weight.shape[0]
    key = _key(op, x.device, m, n, k)
    started = time.monotonic()
    if _TUNING_DEADLINE is None:
        _TUNING_DEADLINE = started + PROCESS_SECONDS
    if started >= _TUNING_DEADLINE:
        return _inherit(op, x, weight, run, native, compare)
    copies = max(2, min(16, -(-COLD_BYTES // max(1, weight.numel() * weight.element_size()))))
    weights = [weight] + [weight.clone() for _ in range(copies - 1)]
    generator = torch.Generator(device=x.device).manual_seed(1729)
    probe = torch.randn(x.shape, device=x.device, dtype=x.dtype, generator=generator)
    if run(None, weight, probe) is None:
        return "native"
    reference = (compare or native)(weight, probe).clone()
    deadline = min(_TUNING_DEADLINE, time.monotonic() + SHAPE_SECONDS)
    native_us = _cold_us(native, weights)
    best_us, best = native_us, "native"
    validated = [(native_us, "native")]
    for choice in [None] + _candidates(m, n, k, epilogue, prologue):
        if time.monotonic() >= deadline:
            break
        got = run(choice, weight, probe)
        if got is None or not _agrees(got, reference):
            continue
        us = _cold_us(lambda w, c=choice: run(c, w), weights)
        validated.append((us, choice))
        if us < best_us * 0.985:
            best_us, best = us, choice
    if best != "native":
        # recheck both, so clock ramp-up cannot favour a late candidate (linear.py:470-475)
        native_us = _cold_us(native, weights)
        best_us = _cold_us(lambda w: run(best, w), weights)
        if best_us >= native_us * 0.985:
            best = "native"
    if best not in ("native", None):
        # the same recheck against the planner default: a launch shape must keep its 1.5 % lead
        # over it on a second timing, or the default stays (timing noise does not switch kernels)
        default_us = _cold_us(lambda w: run(None, w), weights)
        if _cold_us(lambda w: run(best, w), weights) >= default_us * 0.985:
            best = None
    validated.sort(key=lambda item: item[0])
    _VALIDATED[key] = validated
    del weights
    tuning_seconds += time.monotonic() - started
    return best


def _inherit(op, x, weight, run, native, compare=None):
    """The choice of a shape past the process budget (linear.py:412-433).

    A verify block (5..MAX_ROWS rows) takes a launch choice already frozen for the same operation
    and weight shape at another row count above 4, if it agrees with the native GEMM's output on a
    probe input (the launch must also exist at this row count). Otherwise, and for other row
    counts, the shape takes its untuned default. The captured step's ``refine`` still re-judges it.
    """
    m, k = x.shape
    n = weight.shape[0]
    key = _key(op, x.device, m, n, k)
    default = "native" if prefer_native(m) else None
    inherited[key] = default
    _VALIDATED[key] = [(0.0, default)]
    if m <= 4 or m > MAX_ROWS:
        return default
    generator = torch.Generator(device=x.device).manual_seed(1729)
    probe = torch.randn(x.shape, device=x.device, dtype=x.dtype, generator=generator)
    if run(None, weight, probe) is None:
        return default
    reference = (compare or native)(weight, probe).clone()
    for other, choice in list(_CHOICES.items()):
        if choice in (None, "native") or _key(op, x.device, other[-3], n, k) != other:
            continue  # a default, or another operation, device or weight shape
        if other[-3] <= 4:
            continue
        try:
            got = run(choice, weight, probe)
        except _native.FtkError:
            continue  # the launch does not exist at this row count
        if got is None or not _agrees(got, reference):
            continue
        _VALIDATED[key] = [(0.0, choice), (1.0, default)]
        inherited[key] = choice
        return choice
    return default


def _choice(op, x, weight, run, native, epilogue=_native.EPI_STORE, prologue=False, compare=None):
    """The frozen launch choice of a call with no explicit config, selected on first use when tuning is on.

    A first use during graph capture raises RuntimeError, as linear.py:497-498 does. A "native"
    choice means the caller runs ``native`` itself (torch's GEMM), the form that was timed."""
    m, k = x.shape
    n = weight.shape[0]
    key = _key(op, x.device, m, n, k)
    if key not in _CHOICES:
        if TUNE:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("projection selection must finish during eager warmup")
            _CHOICES[key] = _choose(op, x, weight, run, native, epilogue, prologue, compare)
            # Re-judging order = weight traffic per step: the vocabulary projection runs once per
            # step, every other projection once per layer (linear.py:515-520). The planner default
            # always stays an option, so a captured step can fall back to it.
            traffic = n * k // (36 if n > 65536 else 1)
            options = [c for _, c in _VALIDATED[key]][:3]
            if None not in options:
                options.append(None)
            if _CHOICES[key] not in options:
                options.insert(0, _CHOICES[key])
            register(key, m, traffic, options, lambda: _CHOICES[key],
                     lambda choice: _CHOICES.__setitem__(key, choice))
        else:
            _CHOICES[key] = "native" if prefer_native(m) else None
    return _CHOICES[key]


def refine(step_seconds, rows, seconds=10.0):
    """Keep a frozen choice's alternative only if the whole captured step gets faster
    (engine/decode.py:556-583, DecodeState.refine).

    ``step_seconds()`` captures the step with the choices in force and returns its replay time.
    Knobs of batch size ``rows`` are re-judged heaviest first; each alternative option is put in
    force, the step is captured and timed again, and the option stays only if the step is at
    least 1 % faster. Every option already passed the operator check, so only speed is decided.
    Returns the step time with the final choices; the caller captures its final graph after this.
    """
    deadline = time.monotonic() + seconds
    best = step_seconds()
    for knob in knobs(rows):
        chosen = knob.get()
        for option in knob.options:
            if option == chosen or time.monotonic() >= deadline:
                continue
            knob.select(option)
            elapsed = step_seconds()
            if elapsed < best * 0.99:
                best, chosen = elapsed, option
        knob.select(chosen)
    return best


def linear_residual(x, weight, residual, config=None, sumsq=None):
    """bf16(linear(x, weight) + residual): a projection whose output joins the residual stream.

    The add of add_rms_norm (engine/kernels/rmsnorm.py:86-95) runs in the projection's epilogue
    (ftk_project_add_bf16). Where engine/decode.py:236-243 / :258-261 add the O and down outputs to
    the residual, the result is add_rms_norm's ``summed`` bit for bit, so the next norm reads it as a
    plain x and no prologue reads the residual again. Neither input is modified. Every row count
    runs this library's kernels (the MFMA kind from 17 rows). ``sumsq`` (a ``SumSq``) receives the
    new stream's sums of squares for the norm that reads it next (ftk_project_add_rows_bf16).
    """
    _native.require_gpu(x, weight, residual)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or residual.dtype != torch.bfloat16:
        raise ValueError("linear_residual takes BF16 x, weight and residual")
    if not weight.is_contiguous():
        raise ValueError("linear_residual takes a contiguous [N, K] weight")
    n, k = weight.shape
    if x.shape[-1] != k:
        raise ValueError(f"x has K={x.shape[-1]}, weight has K={k}")
    if tuple(residual.shape) != (*x.shape[:-1], n):
        raise ValueError(f"residual must be {(*x.shape[:-1], n)}, got {tuple(residual.shape)}")
    flat = _as_rows(x)
    res = residual.reshape(-1, n).contiguous()
    m = flat.shape[0]
    out = torch.empty((m, n), device=x.device, dtype=torch.bfloat16)
    if m == 0:
        return out.reshape(*x.shape[:-1], n)
    cfg = ctypes.byref(config) if config is not None else None
    if sumsq is not None:
        rows = _native.Rows(None, None, None, 0, 0, None, _native.ptr(sumsq._out(out)))
        status = _native.try_call("ftk_project_add_rows_bf16", _native.ptr(flat), ctypes.byref(rows),
                                  _native.ptr(weight), _native.ptr(res), _native.ptr(out), m, n, k, cfg,
                                  _native.stream_of(flat))
        if status == _native.FTK_OK:
            sumsq._wrote(out)
            return out.reshape(*x.shape[:-1], n)
        if status != _native.FTK_ERR_UNSUPPORTED:  # not a RING launch: no sums, the call below
            raise _native.FtkError("ftk_project_add_rows_bf16", status)
    _native.call("ftk_project_add_bf16", _native.ptr(flat), _native.ptr(weight), _native.ptr(res), _native.ptr(out),
                 m, n, k, cfg, _native.stream_of(flat))
    return out.reshape(*x.shape[:-1], n)


def keep_native(rows, weight):
    """Leave a shape on torch's native GEMM without tuning it (linear.py:484-486)."""
    _CHOICES.setdefault((weight.device, rows, weight.shape[0], weight.shape[1]), "native")


def linear(x, weight, split_ok=False):
    """x @ weight.T in BF16 (linear.py:489-523). ``split_ok`` is accepted; the result is always BF16."""
    return _linear(x, weight, None)


def linear_sumsq(x, weight, sumsq):
    """``linear(x, weight)`` whose output an RMSNorm reads next: the launch also writes the output
    rows' sums of squares into ``sumsq`` (a ``SumSq``), where it is a RING launch. Not a reference
    call: the reference's norm reads its input rows (engine/kernels/rmsnorm.py:21-46)."""
    return _linear(x, weight, sumsq)


def _linear(x, weight, sumsq):
    rows = x.numel() // x.shape[-1]
    if rows > MAX_ROWS or x.dtype != torch.bfloat16 or not weight.is_contiguous():
        return F.linear(x, weight)
    _native.require_gpu(x, weight)
    if rows == 0:
        return x.new_empty((*x.shape[:-1], weight.shape[0]))
    flat = _as_rows(x)

    def run(choice, w, inp=flat):
        return project(inp, w, _as_config(choice))

    choice = _choice("linear", flat, weight, run, lambda w, inp=flat: F.linear(inp, w))
    if choice == "native":
        return F.linear(x, weight)
    out = project(flat, weight, _as_config(choice), sumsq=sumsq)
    return out.reshape(*x.shape[:-1], weight.shape[0])


def plan(m, n, k, epilogue=_native.EPI_STORE, compute_units=256, config=None, prologue=False, residual=False):
    """The launch the C planner makes for a shape (host only; no device needed). ``residual``: the
    prologue adds a residual (add_rms_norm_linear and the residual forms of the fused calls)."""
    p = _native.Plan()
    flags = epilogue | (_native.PLAN_PROLOGUE if prologue else 0) | (_native.PLAN_RESIDUAL if residual else 0)
    _native.call("ftk_plan_project", m, n, k, flags, compute_units, config, p)
    return p
