"""ctypes binding of libftk.so, the gfx950 HIP library behind every kernel in this package.

The library's C ABI is declared in include/ftk.h. Tensors cross it as raw
device pointers, streams as hipStream_t handles taken from torch's current
stream. There is no fallback: if the library is missing or fails to load,
every call raises.
"""

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).with_name("libftk.so")

FTK_OK, FTK_ERR_INVALID, FTK_ERR_UNSUPPORTED, FTK_ERR_WORKSPACE, FTK_ERR_HIP, FTK_ERR_TOO_LARGE = range(6)
STATIC_SCRATCH_BYTES = 1 << 20  # FTK_STATIC_SCRATCH_BYTES
EPI_STORE, EPI_SWIGLU, EPI_ARGMAX = range(3)
PLAN_PROLOGUE = 0x100  # FTK_PLAN_PROLOGUE
PLAN_RESIDUAL = 0x200  # FTK_PLAN_RESIDUAL
KIND_AUTO, KIND_GEMV, KIND_MFMA, KIND_GENERIC, KIND_STREAM, KIND_MFMA_STREAM, KIND_QUAD, KIND_STAGE, KIND_RING = range(9)
ATTN_AUTO, ATTN_ROWS, ATTN_QUAD = range(3)
ROPE_PREFILL, ROPE_ROWS, ROPE_TABLE = 0x1, 0x2, 0x4
MAX_ROWS = 32

_c_void_p, _i64, _int, _float = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float


class Config(ctypes.Structure):
    """ftk_config: a launch choice (kind, rows_per_wave, unroll, groups_per_cu, waves); zeros = planner default."""

    _fields_ = [("kind", _int), ("rows_per_wave", _int), ("unroll", _int), ("groups_per_cu", _int),
                ("waves", _int)]

    def key(self):
        return (self.kind, self.rows_per_wave, self.unroll, self.groups_per_cu, self.waves)

    def __repr__(self):
        return f"Config{self.key()}"


class Plan(ctypes.Structure):
    _fields_ = [("kind", _int), ("rows_per_wave", _int), ("unroll", _int), ("waves", _int), ("grid", _int),
                ("tiles", _int),
                ("threads", _int), ("lds_bytes", _i64), ("splits", _int), ("k_slice", _int),
                ("workspace_bytes", _i64)]


class Rows(ctypes.Structure):
    """ftk_rows: the prologue's residual, stored sum and gathered row indices, and the norm's sums of
    squares handed between RING launches (sumsq in, sumsq_out written) (NULL = absent)."""

    _fields_ = [("residual", _c_void_p), ("sum", _c_void_p), ("x_ids", _c_void_p), ("x_ids_bytes", _int),
                ("x_rows", _i64), ("sumsq", _c_void_p), ("sumsq_out", _c_void_p)]


class AttnConfig(ctypes.Structure):
    """ftk_attn_config: a decode-attention launch choice (kind, splits, waves, unroll); zeros = planner default."""

    _fields_ = [("kind", _int), ("splits", _int), ("waves", _int), ("unroll", _int)]

    def key(self):
        return (self.kind, self.splits, self.waves, self.unroll)

    def __repr__(self):
        return f"AttnConfig{self.key()}"


class AttnPlan(ctypes.Structure):
    _fields_ = [("kind", _int), ("splits", _int), ("chunk", _int), ("waves", _int), ("unroll", _int),
                ("grid", _int), ("workspace_bytes", _i64)]


# name -> (restype, argtypes), exactly the declarations of include/ftk.h
SIGNATURES = {
    "ftk_version": (ctypes.c_char_p, []),
    "ftk_status_string": (ctypes.c_char_p, [_int]),
    "ftk_last_hip_error": (_int, []),
    "ftk_device_compute_units": (_int, []),
    "ftk_persistent_programs": (_int, [_int, _int]),
    "ftk_ring_tile": (_int, [_int, _int, _int, _int]),
    "ftk_linear_bf16": (_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "ftk_rms_norm_linear_bf16": (_int, [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                        _c_void_p]),
    "ftk_gate_up_swiglu_bf16": (_int, [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                       _c_void_p]),
    "ftk_lm_head_argmax_bf16": (_int, [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _c_void_p, _int,
                                       _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p]),
    "ftk_lm_head_argmax_static_bf16": (_int, [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _c_void_p, _int,
                                              _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "ftk_project_bf16": (_int, [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _i64, _i64, _i64, _int,
                                _c_void_p, _int, _c_void_p, _c_void_p, _i64, ctypes.POINTER(Config), _c_void_p]),
    "ftk_project_add_bf16": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                    ctypes.POINTER(Config), _c_void_p]),
    "ftk_project_add_rows_bf16": (_int, [_c_void_p, ctypes.POINTER(Rows), _c_void_p, _c_void_p, _c_void_p, _i64,
                                         _i64, _i64, ctypes.POINTER(Config), _c_void_p]),
    "ftk_project_rows_bf16": (_int, [_c_void_p, ctypes.POINTER(Rows), _c_void_p, _float, _c_void_p, _c_void_p,
                                     _i64, _i64, _i64, _int, _c_void_p, _int, _c_void_p, _c_void_p, _i64,
                                     ctypes.POINTER(Config), _c_void_p]),
    "ftk_rms_norm_bf16": (_int, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _float, _c_void_p]),
    "ftk_embed_rms_norm_bf16": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
                                       _float, _c_void_p]),
    "ftk_add_rms_norm_bf16": (_int, [_c_void_p, _int, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                     _i64, _float, _c_void_p]),
    "ftk_swiglu_bf16": (_int, [_c_void_p, _int, _i64, _c_void_p, _i64, _i64, _c_void_p]),
    "ftk_argmax_bf16": (_int, [_c_void_p, _i64, _i64, _c_void_p, _int, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "ftk_merge_splits_bf16": (_int, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "ftk_argmax_workspace_bytes": (_i64, [_i64, _i64]),
    "ftk_project_workspace_bytes": (_i64, [_i64, _i64, _i64, _int, ctypes.POINTER(Config)]),
    "ftk_decode_attention_bf16": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _c_void_p, _i64, _i64,
                                         _i64, _i64, _i64, ctypes.c_double, _c_void_p, _i64,
                                         ctypes.POINTER(AttnConfig), _c_void_p]),
    "ftk_rope_decode_attention_bf16": (_int, [_c_void_p, _c_void_p, _c_void_p, _float, _float, _c_void_p, _c_void_p,
                                              _i64, _c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                              _i64, _i64, _i64, _i64, _i64, ctypes.c_double, _c_void_p, _i64,
                                              ctypes.POINTER(AttnConfig), _c_void_p]),
    "ftk_decode_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(AttnConfig)]),
    "ftk_plan_decode_attention": (_int, [_i64, _i64, _i64, _i64, _i64, _int, ctypes.POINTER(AttnConfig),
                                         ctypes.POINTER(AttnPlan)]),
    "ftk_qk_rope_cache_bf16": (_int, [_c_void_p, _int, _i64, _c_void_p, _c_void_p, _float, _float, _c_void_p,
                                      _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                      _i64, _i64, _i64, _i64, _i64, _i64, _int, _c_void_p]),
    "ftk_plan_project": (_int, [_i64, _i64, _i64, _int, _int, ctypes.POINTER(Config), ctypes.POINTER(Plan)]),
    "ftk_stream_read": (_int, [_c_void_p, _i64, _c_void_p, _int, _int, _c_void_p]),
    "ftk_plan_coverage": (_int, [ctypes.POINTER(Plan), _i64, _int, ctypes.POINTER(ctypes.c_int32), _i64,
                                 ctypes.POINTER(_i64)]),
}

_LIB = None
_LOCK = threading.Lock()


class FtkError(RuntimeError):
    def __init__(self, name, status, hip_error=0):
        self.status, self.hip_error = status, hip_error
        text = lib().ftk_status_string(status).decode()
        extra = f" (hipError {hip_error})" if status == FTK_ERR_HIP else ""
        super().__init__(f"{name}: {text}{extra}")


def lib():
    """The loaded library (loaded once). Raises if libftk.so is missing: there is no fallback."""
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `python fast-transformer_amd/build.py` "
                        "(or __graft_entry__.build()); these kernels have no fallback")
                # torch first: the library must bind to the HIP runtime torch already loaded.
                handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
                for name, (restype, argtypes) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype, fn.argtypes = restype, argtypes
                _LIB = handle
    return _LIB


def call(name, *args):
    """Call an ftk entry point; raise FtkError on any status but FTK_OK."""
    status = getattr(lib(), name)(*args)
    if status != FTK_OK:
        raise FtkError(name, status, lib().ftk_last_hip_error() if status == FTK_ERR_HIP else 0)


def try_call(name, *args):
    """Call an ftk entry point; return its status, raising only on launch failure."""
    status = getattr(lib(), name)(*args)
    if status == FTK_ERR_HIP:
        raise FtkError(name, status, lib().ftk_last_hip_error())
    return status


def stream_of(tensor):
    """hipStream_t of torch's current stream on the tensor's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)


def ptr(tensor):
    return ctypes.c_void_p(tensor.data_ptr()) if tensor is not None else None


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("these kernels run on the GPU: got a tensor on " + str(t.device))


_WORKSPACES = {}
#: Every workspace ever handed to a kernel stays alive: a captured graph keeps its address.
_RETIRED = []


def workspace(device, need, purpose):
    """Per-device, per-purpose scratch buffer of at least ``need`` bytes, zeroed when allocated.

    The kernels keep per-call scratch there (RMSNorm row scales, per-workgroup
    argmax keys). The argmax key words must be zero when a call starts; every
    call leaves the words it used zero again. A buffer only grows, outside
    graph capture; a replaced buffer is kept alive for graphs that captured its
    address.
    """
    key = (device, purpose)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the kernels' workspace must be sized during eager warmup, before graph capture")
        size = max(int(need), 1 << 20, 2 * (ws.numel() if ws is not None else 0))
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def argmax_workspace(device, rows, vocab):
    """Workspace of the standalone argmax for ``rows`` rows of ``vocab`` logits."""
    return workspace(device, int(lib().ftk_argmax_workspace_bytes(rows, vocab)), "argmax")


def project_workspace(device, m, n, k, epilogue, config=None, prologue=False, residual=False):
    """Workspace of one projection call (row scales, argmax keys); ``prologue``: the call has gamma;
    ``residual``: its prologue adds a residual, which the planner plans on other kinds and grids."""
    flags = epilogue | (PLAN_PROLOGUE if prologue else 0) | (PLAN_RESIDUAL if residual else 0)
    return workspace(device, int(lib().ftk_project_workspace_bytes(m, n, k, flags, config)), "project")
