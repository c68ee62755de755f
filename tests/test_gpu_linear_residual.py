"""GPU parity of the projection with the residual add in its epilogue (linear_residual, ftk_project_add_bf16).

The stored value is bf16(f32(bf16(x @ W^T)) + f32(residual)), the `summed` output of
add_rms_norm (engine/kernels/rmsnorm.py:86-95) applied to the projection's output:
- bit for bit the kernel's own projection (same launch choice) followed by that add,
  for every kind (STREAM, QUAD, STAGE, MFMA_STREAM, GEMV, MFMA, generic), row counts
  1..32 and ragged N;
- within 2e-2 + 1e-2|ref| of the oracle's projection followed by the same add;
- add_rms_norm's `summed` bit for bit (the standalone kernel on the projection's output);
- in place (y = residual) through the C ABI, and in a replayed graph.
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import linear as L
from kernels import rmsnorm as RN

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _cfg(kind, rows, unroll, gpc, waves):
    return _native.Config(kind, rows, unroll, gpc, waves)


#: (kind config, row counts it takes) at K = 4096.
CONFIGS = [
    (None, (1, 3, 5, 8, 16, 17, 32)),
    (_cfg(_native.KIND_STREAM, 2, 0, 0, 4), (1, 2, 4)),
    (_cfg(_native.KIND_STREAM, 4, 0, 0, 4), (5, 8)),
    (_cfg(_native.KIND_QUAD, 8, 0, 0, 8), (2, 5, 8, 16)),
    (_cfg(_native.KIND_STAGE, 16, 2, 0, 8), (5, 9, 16)),
    (_cfg(_native.KIND_RING, 16, 2, 0, 8), (2, 5, 9, 16)),
    (_cfg(_native.KIND_MFMA_STREAM, 16, 4, 0, 8), (5, 16)),
    (_cfg(_native.KIND_GEMV, 2, 2, 0, 2), (1, 4)),
    (_cfg(_native.KIND_MFMA, 16, 4, 0, 4), (1, 16, 32)),
    (_cfg(_native.KIND_GENERIC, 0, 0, 0, 0), (1, 7, 32)),
]


def _inputs(m, n, k, seed, device):
    x = seeded((m, k), seed=seed, device=device)
    w = seeded((n, k), seed=seed + 1, scale=0.02, device=device)
    r = seeded((m, n), seed=seed + 2, device=device)
    return x, w, r


def _add(y, r):
    return (y.float() + r.float()).to(torch.bfloat16)


def _case_ids():
    return [f"{'default' if c is None else c.kind}-{m}" for c, ms in CONFIGS for m in ms]


@pytest.mark.parametrize("config,m", [(c, m) for c, ms in CONFIGS for m in ms], ids=_case_ids())
@pytest.mark.parametrize("n", [1536, 1000])
def test_matches_the_projection_then_the_add(cuda, config, m, n):
    k = 4096
    x, w, r = _inputs(m, n, k, seed=7000 + m + n, device=cuda)
    if config is not None:
        p = _native.Plan()
        assert _native.lib().ftk_plan_project(m, n, k, _native.EPI_STORE, 256, ctypes.byref(config), p) \
            == _native.FTK_OK or config.kind == _native.KIND_GENERIC
    got = L.linear_residual(x, w, r, config=config)
    y = L.project(x, w, config) if config is not None else L.linear(x, w)
    if config is None and m >= L.NATIVE_FROM_ROWS:
        y = L.project(x, w)  # the epilogue form always runs this library's kernels
    assert torch.equal(got, _add(y, r))
    want = bf16.round_bits(bf16.to_f32(path.project(to_bits(x), to_bits(w))) + bf16.to_f32(to_bits(r)))
    g, wf = bf16.to_f32(to_bits(got)).astype(np.float64), bf16.to_f32(want).astype(np.float64)
    assert np.all(np.abs(g - wf) <= ATOL + RTOL * np.abs(wf))
    assert np.mean(to_bits(got) == want) >= 0.99


@pytest.mark.parametrize("m", [1, 5, 16])
def test_equals_add_rms_norm_summed(cuda, m):
    """The stored value is what add_rms_norm hands on as the residual stream."""
    n, k = 4096, 4096
    x, w, r = _inputs(m, n, k, seed=7100 + m, device=cuda)
    gamma = torch.ones(n, device=cuda, dtype=torch.bfloat16)
    _, summed = RN.add_rms_norm(L.project(x, w), r, gamma, 1e-6)
    assert torch.equal(L.linear_residual(x, w, r), summed)


def test_in_place_through_the_c_abi(cuda):
    m, n, k = 5, 4096, 12288
    x, w, r = _inputs(m, n, k, seed=7200, device=cuda)
    want = L.linear_residual(x, w, r)
    y = r.clone()
    _native.call("ftk_project_add_bf16", _native.ptr(x), _native.ptr(w), _native.ptr(y), _native.ptr(y), m, n, k,
                 None, _native.stream_of(x))
    assert torch.equal(y, want)


def test_inputs_are_not_modified_and_shapes_are_kept(cuda):
    x, w, r = _inputs(6, 2048, 4096, seed=7300, device=cuda)
    x3, r3 = x.view(2, 3, 4096), r.view(2, 3, 2048)
    x0, r0 = x3.clone(), r3.clone()
    out = L.linear_residual(x3, w, r3)
    assert out.shape == (2, 3, 2048) and out.is_contiguous()
    assert torch.equal(x3, x0) and torch.equal(r3, r0)
    assert torch.equal(out.view(6, 2048), L.linear_residual(x, w, r))


def test_ragged_k_and_unaligned_pointers_take_the_generic_kind(cuda):
    m, n, k = 3, 700, 1001
    x, w, r = _inputs(m, n, k, seed=7400, device=cuda)
    got = L.linear_residual(x, w, r)
    assert torch.equal(got, _add(L.project(x, w), r))
    big = seeded((m, k + 1), seed=7410, device=cuda)
    xs = big[:, 1:]  # rows 2-byte aligned only
    assert torch.equal(L.linear_residual(xs, w, r), _add(L.project(xs.contiguous(), w), r))


def test_graph_replays_match_eager(cuda):
    m, n, k = 1, 4096, 4096
    x, w, r = _inputs(m, n, k, seed=7500, device=cuda)
    eager = L.linear_residual(x, w, r)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = L.linear_residual(x, w, r)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        torch.cuda.synchronize()
