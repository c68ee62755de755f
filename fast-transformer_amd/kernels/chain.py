"""Projection chains: a list of dependent M = 1 projections run by one cooperative launch.

A decode step in the reference is a captured graph of separate launches (engine/decode.py:650-668),
overlapped on H100 by programmatic dependent launch (engine/kernels/pdl.py). On MI355X every kernel
boundary in a graph costs the tail of one launch plus the start of the next, and gfx950 has no
dependent launch. A chain (ftk_chain_*, csrc/ftk_chain.hip) instead runs the layer's projections --
the calls of engine/layers.py:44, :86, :101-102 with the norms and residual adds of
engine/decode.py:229-261 -- inside one launch: every workgroup (one per CU) issues its next weight
window before it waits for that stage's input, and outputs travel between workgroups as tagged
words. Per stage the arithmetic is that of ``linear`` / ``rms_norm_linear`` / ``gate_up_swiglu`` /
``linear_residual``.

    chain = ProjectionChain(eps)
    q = chain.add(w_qkv, x=hidden, norm_weight=ln1)                 # QKV on rms_norm(hidden)
    o = chain.add(w_o, x=attn_out, residual=hidden, after=q)         # O + residual, after QKV
    g = chain.add(w_gate_up, source=o, norm_weight=ln2, swiglu=True)
    d = chain.add(w_down, source=g, residual_source=o)
    chain.prepare()                                                  # once, outside capture
    chain.launch()                                                   # on the current stream
    chain.output(d)                                                  # the new residual stream

Inputs and outputs are baked in at ``prepare``: a launch reads and writes the same tensors every
time (as a captured graph does). ``status()`` synchronizes and raises if a bounded wait inside the
kernel expired.
"""

import ctypes

import torch

from kernels import _native


class ChainError(RuntimeError):
    pass


class ProjectionChain:
    """A list of M = 1 projections whose inputs may be earlier stages' outputs."""

    def __init__(self, eps=1e-6):
        self.eps = float(eps)
        self._stages = []    # _native.ChainStage
        self._keep = []      # tensors the stages point at
        self._outputs = []   # per stage: its BF16 output tensor (or None)
        self._chain = None
        self._workspace = None
        self.device = None

    def __len__(self):
        return len(self._stages)

    def add(self, weight, *, x=None, source=None, norm_weight=None, swiglu=False, residual=None,
            residual_source=None, after=None, output=True):
        """Append a stage; returns its index.

        ``weight`` [N, K] BF16 (cat(gate, up) with ``swiglu``). The input row is ``x`` ([K] or
        [1, K] BF16) or the output of stage ``source``; ``norm_weight`` adds the RMSNorm prologue.
        ``residual`` ([N] BF16) or ``residual_source`` (a stage) is added in the epilogue:
        y = bf16(bf16(x W^T) + r). ``after`` names a stage that must have finished first (work
        outside the chain between them, such as attention). ``output`` allocates the stage's BF16
        output tensor (``output(i)``); later stages read their inputs from the chain either way.
        """
        if self._chain is not None:
            raise ChainError("the chain is prepared; build a new one to change it")
        if (x is None) == (source is None):
            raise ValueError("give exactly one of x and source")
        if residual is not None and residual_source is not None:
            raise ValueError("give at most one of residual and residual_source")
        if swiglu and (residual is not None or residual_source is not None):
            raise ValueError("a SwiGLU stage takes no residual")
        tensors = [t for t in (weight, x, norm_weight, residual) if t is not None]
        _native.require_gpu(*tensors)
        device = weight.device
        if self.device is None:
            self.device = device
        if any(t.device != self.device for t in tensors):
            raise ValueError("every tensor of a chain lives on one device")
        if any(t.dtype != torch.bfloat16 for t in tensors):
            raise ValueError("chain stages take BF16 tensors")
        if not weight.is_contiguous():
            raise ValueError("chain stages take a contiguous [N, K] weight")
        n, k = weight.shape
        for name, idx in (("source", source), ("residual_source", residual_source), ("after", after)):
            if idx is not None and not 0 <= idx < len(self._stages):
                raise ValueError(f"{name} must name an earlier stage, got {idx}")
        if x is not None:
            x = x.reshape(-1).contiguous()
            if x.numel() != k:
                raise ValueError(f"x has {x.numel()} elements, the weight has K={k}")
        if norm_weight is not None:
            norm_weight = norm_weight.reshape(-1).contiguous()
            if norm_weight.numel() != k:
                raise ValueError(f"norm_weight has {norm_weight.numel()} elements for K={k}")
        width = n // 2 if swiglu else n
        if residual is not None:
            residual = residual.reshape(-1).contiguous()
            if residual.numel() != width:
                raise ValueError(f"residual has {residual.numel()} elements for {width} outputs")
        out = torch.empty((1, width), dtype=torch.bfloat16, device=self.device) if output else None
        st = _native.ChainStage(
            _native.ptr(weight), _native.ptr(norm_weight), _native.ptr(x), _native.ptr(residual), _native.ptr(out),
            n, k, _native.EPI_SWIGLU if swiglu else _native.EPI_STORE,
            -1 if source is None else source, -1 if residual_source is None else residual_source,
            -1 if after is None else after)
        self._stages.append(st)
        self._keep.extend(t for t in (weight, x, norm_weight, residual) if t is not None)
        self._outputs.append(out)
        return len(self._stages) - 1

    def output(self, index):
        """The BF16 [1, N_out] output tensor of stage ``index`` (None if it was added with output=False)."""
        return self._outputs[index]

    def _array(self):
        return (_native.ChainStage * len(self._stages))(*self._stages)

    def plan(self, compute_units=256):
        """(shape ids, tile counts) per stage on ``compute_units`` CUs (host only)."""
        n = len(self._stages)
        shapes, tiles = (ctypes.c_int * n)(), (ctypes.c_int * n)()
        _native.call("ftk_chain_plan", self._array(), n, compute_units, shapes, tiles)
        return list(shapes), list(tiles)

    def prepare(self):
        """Plan every stage and write the chain's device program (synchronous; not during capture)."""
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("prepare a chain during eager warmup, before graph capture")
        if not self._stages:
            raise ValueError("an empty chain")
        arr = self._array()
        n = len(self._stages)
        with torch.cuda.device(self.device):
            need = int(_native.lib().ftk_chain_workspace_bytes(arr, n))
            if need < 0:
                raise ChainError("ftk_chain_workspace_bytes: the chain has an invalid or unsupported stage")
            ws = torch.zeros(need + 256, dtype=torch.uint8, device=self.device)
            offset = (-ws.data_ptr()) % 256
            chain = _native.Chain()
            _native.call("ftk_chain_prepare", arr, n, self.eps, ctypes.c_void_p(ws.data_ptr() + offset), need,
                         ctypes.byref(chain))
        self._workspace, self._chain = ws, chain
        return self

    def launch(self):
        """Enqueue one run of the chain on the current stream (capture-safe)."""
        if self._chain is None:
            raise ChainError("prepare the chain before launching it")
        _native.call("ftk_chain_launch", ctypes.byref(self._chain),
                     ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))

    def status(self):
        """Synchronize; raise ChainError if a bounded wait of some launch expired."""
        code = _native.lib().ftk_chain_status(ctypes.byref(self._chain))
        if code < 0:
            raise ChainError(f"ftk_chain_status: HIP error {_native.lib().ftk_last_hip_error()}")
        if code > 0:
            raise ChainError(f"a chain launch stopped: the wait of stage {code - 1} expired "
                             "(prepare the chain again to reuse it)")

    def stamps(self):
        """Real-time clock stamps (100 MHz) of the last launch, per workgroup:
        ([stages][grid] stage begins, [stages][grid] input ready (0: no tile), [stages][grid] stage ends,
        [grid] kernel starts)."""
        n, g = self._chain.stages, self._chain.grid
        buf = (ctypes.c_int64 * ((3 * n + 1) * g))()
        _native.call("ftk_chain_stamps", ctypes.byref(self._chain), buf)
        flat = list(buf)
        rows = [flat[r * g:(r + 1) * g] for r in range(3 * n)]
        return rows[0::3], rows[1::3], rows[2::3], flat[3 * n * g:]

    def stage_us(self):
        """Per-stage time of the last launch (µs): when the last workgroup finished each stage, minus
        when the last one finished the stage before (the first stage from the earliest start)."""
        _, _, ends, starts = self.stamps()
        prev = min(starts)
        out = []
        for stage in ends:
            last = max(stage)
            out.append((last - prev) / 100.0)
            prev = last
        return out


def decode_layers(layers, hidden, attn, eps, residual_epilogue=False, attention_fence=True, outputs="all"):
    """The M = 1 projection set of a stack of decode layers as one chain.

    ``layers``: dicts with the BF16 weights ``qkv``, ``o``, ``gate_up``, ``down`` and norm gains
    ``ln1``, ``ln2``. ``hidden`` [1, H] is the first layer's input; ``attn`` [1, Hq D] (or one per
    layer) stands for the attention output O reads.

    - ``residual_epilogue=False``: QKV(rms_norm(h)), O(attn), gate/up + SwiGLU on rms_norm(O's
      output), down -> the next layer's h (the projection set of engine/layers.py:44, :86,
      :101-102 without the residual stream).
    - ``residual_epilogue=True``: the decode data flow of engine/decode.py:229-261 with the
      residual adds in the O and down epilogues: QKV(rms_norm(r)), r = O(attn) + r,
      gate/up + SwiGLU on rms_norm(r), r = down(act) + r; ``hidden`` is the residual stream.

    ``attention_fence``: O starts only after its layer's QKV has finished, as it would with the
    attention between them. ``outputs``: "all" keeps every stage's output, "qkv" the QKV outputs
    and the last stage's. Returns (chain, {"qkv": [...], "o": [...], "act": [...], "down": [...]})
    with the stage indices.
    """
    chain = ProjectionChain(eps)
    idx = {"qkv": [], "o": [], "act": [], "down": []}
    prev = None
    attns = attn if isinstance(attn, (list, tuple)) else [attn] * len(layers)
    last_layer = len(layers) - 1
    for i, (lw, a) in enumerate(zip(layers, attns)):
        keep = outputs == "all"
        src = dict(x=hidden) if prev is None else dict(source=prev)
        q = chain.add(lw["qkv"], norm_weight=lw["ln1"], output=keep or outputs == "qkv", **src)
        fence = dict(after=q) if attention_fence else {}
        if residual_epilogue:
            res = dict(residual=hidden) if prev is None else dict(residual_source=prev)
            o = chain.add(lw["o"], x=a, output=keep, **res, **fence)
        else:
            o = chain.add(lw["o"], x=a, output=keep, **fence)
        g = chain.add(lw["gate_up"], source=o, norm_weight=lw["ln2"], swiglu=True, output=keep)
        res = dict(residual_source=o) if residual_epilogue else {}
        d = chain.add(lw["down"], source=g, output=keep or i == last_layer, **res)
        for key, v in (("qkv", q), ("o", o), ("act", g), ("down", d)):
            idx[key].append(v)
        prev = d
    return chain, idx
