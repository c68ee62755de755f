"""The lm_head + argmax entry point that allocates nothing (ftk_lm_head_argmax_static_bf16),
called through the C ABI and checked against the workspace entry point (ftk_lm_head_argmax_bf16):
same ids, logits and top logits bit for bit, on calls in a row (each smaller than the one before;
the first two on the RING kind, whose walks claim their last tiles from a counter in the static
scratch that the previous call left at zero), and a call beyond its static scratch rejected
before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits

from kernels import _native

pytestmark = pytest.mark.gpu


def _inputs(m, v, k, seed, device):
    x = seeded((m, k), seed, device=device)
    w = seeded((v, k), seed + 1, scale=0.02, device=device)
    gamma = seeded((k,), seed + 2, scale=0.1, shift=1.0, device=device)
    return x, w, gamma


def _outputs(m, v, device, ids_dtype):
    logits = torch.full((m, v), -1.0, device=device, dtype=torch.bfloat16)
    ids = torch.full((m,), -7, device=device, dtype=ids_dtype)
    top = torch.full((m,), float("nan"), device=device, dtype=torch.float32)
    return logits, ids, top


def _run(name, x, w, gamma, logits, ids, top, workspace=None):
    m, k = x.shape
    v = w.shape[0]
    ids_bytes = ids.element_size()
    args = [_native.ptr(x), _native.ptr(gamma), 1e-6, _native.ptr(w), _native.ptr(logits), _native.ptr(ids),
            ids_bytes, _native.ptr(top), m, v, k]
    if name == "ftk_lm_head_argmax_bf16":
        args += [_native.ptr(workspace), workspace.numel()]
    return getattr(_native.lib(), name)(*args, _native.stream_of(x))


def test_static_scratch_matches_the_workspace_entry_point(cuda):
    # calls in a row, each smaller: fewer rows, then a smaller vocabulary and no prologue gain
    cases = ((4, 151936, 4096, torch.int32, True), (1, 151936, 4096, torch.int64, True),
             (1, 50000, 2048, torch.int64, False))
    for m, v, k, ids_dtype, with_gamma in cases:
        print(f"static scratch lm_head case M={m} V={v} K={k} ids={ids_dtype}", flush=True)
        x, w, gamma = _inputs(m, v, k, 7000 + m, cuda)
        if not with_gamma:
            gamma = None
        need = int(_native.lib().ftk_project_workspace_bytes(m, v, k, _native.EPI_ARGMAX | _native.PLAN_PROLOGUE,
                                                             None))
        assert 0 < need <= _native.STATIC_SCRATCH_BYTES
        workspace = torch.zeros(need, dtype=torch.uint8, device=cuda)
        want = _outputs(m, v, cuda, ids_dtype)
        assert _run("ftk_lm_head_argmax_bf16", x, w, gamma, *want, workspace=workspace) == _native.FTK_OK
        got = _outputs(m, v, cuda, ids_dtype)
        assert _run("ftk_lm_head_argmax_static_bf16", x, w, gamma, *got) == _native.FTK_OK
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_bits(got[0]), to_bits(want[0]))
        np.testing.assert_array_equal(got[1].cpu().numpy(), want[1].cpu().numpy())
        np.testing.assert_array_equal(got[2].cpu().numpy().view(np.uint32), want[2].cpu().numpy().view(np.uint32))
        # and the ids are the first maximum of the BF16 logits
        np.testing.assert_array_equal(got[1].cpu().numpy(), torch.argmax(got[0].float().cpu(), -1).numpy())


def test_static_scratch_rejects_a_call_beyond_its_size(cuda):
    m, v, k = 32, 151936, 4096
    need = int(_native.lib().ftk_project_workspace_bytes(m, v, k, _native.EPI_ARGMAX, None))
    assert need > _native.STATIC_SCRATCH_BYTES
    x, w, _ = _inputs(m, 1, k, 7100, cuda)
    w = torch.empty((v, k), device=cuda, dtype=torch.bfloat16)
    logits, ids, top = _outputs(m, v, cuda, torch.int32)
    status = _run("ftk_lm_head_argmax_static_bf16", x, w, None, logits, ids, top)
    assert status == _native.FTK_ERR_TOO_LARGE
    assert b"static" in _native.lib().ftk_status_string(status)
    torch.cuda.synchronize()
    assert bool((ids == -7).all())  # nothing was launched
