"""GPU tests of the one-launch greedy argmax (lm_head + argmax, engine/kernels/argmax.py:112-129).

The STREAM kind (at M = 1 the default without the norm prologue, or where RING's claimed tail does
not apply) gathers the workgroups' keys in one extra workgroup of the projection launch; the other
kinds keep the second, finalize launch. Both forms share the key region of the projection
workspace, which is zero between calls. Checked here:
- ids equal the first maximum of the kernel's own BF16 logits (and top equals that logit), through
  every kind in one sequence of calls sharing the workspace, and the key region is zero after each;
- exact ties take the lowest index and a NaN logit wins, through the gathered form (M = 1) and the
  two-launch RING form (M = 5, 16) alike;
- a captured graph of a gathered (STREAM, M = 1) and a two-launch (M = 5) call replays to the
  eager ids every time, with another two-launch call between the replays.
"""

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import argmax as A
from kernels import linear as L

pytestmark = pytest.mark.gpu

V, K = 151936, 4096
STREAM = _native.Config(_native.KIND_STREAM, 0, 0, 0, 0)  # the STREAM kind's default launch shape


def _gathered(m, config=None, prologue=True):
    p = L.plan(m, V, K, _native.EPI_ARGMAX, config=config, prologue=prologue)
    return p.kind == _native.KIND_STREAM and (m == 1 or p.grid <= p.threads), p


def _keys_zero(device, m, grid):
    ws = _native._WORKSPACES[(device, "project")]
    region = ws[256:256 + 8 * m * grid]
    return bool((region == 0).all())


@pytest.fixture(scope="module")
def head(cuda):
    w = seeded((V, K), seed=300, scale=0.02, device=cuda)
    g = seeded((K,), seed=301, scale=0.1, shift=1.0, device=cuda)
    return w, g


def _check(ids, top, logits, m):
    got = to_bits(logits).reshape(m, V)
    want = path.argmax_first(got)
    assert np.array_equal(ids.cpu().numpy(), want)
    assert np.array_equal(top.cpu().numpy(), bf16.to_f32(got)[np.arange(m), want])


def test_every_kind_in_one_sequence_shares_the_workspace(cuda, head):
    w, g = head
    cases = [(1, STREAM), (5, None), (2, None), (1, _native.Config(_native.KIND_GEMV, 2, 2, 8, 4)), (16, None),
             (1, None), (8, _native.Config(_native.KIND_QUAD, 16, 0, 1, 8)), (5, None), (1, STREAM), (1, None)]
    kinds = set()
    for i, (m, config) in enumerate(cases):
        x = seeded((m, K), seed=310 + i, device=cuda)
        top = torch.empty(m, dtype=torch.float32, device=cuda)
        ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, top=top, config=config)
        torch.cuda.synchronize()
        gathered, p = _gathered(m, config)
        kinds.add(gathered)
        print(f"case {i}: M={m} kind {p.kind} grid {p.grid} gathered {gathered}", flush=True)
        _check(ids, top, logits, m)
        assert _keys_zero(cuda, m, p.grid), f"case {i}: key words left behind"
    assert kinds == {True, False}


@pytest.mark.parametrize("m", [1, 5, 16])
def test_gathered_ties_take_the_lowest_index_and_nan_wins(cuda, head, m):
    w, g = head
    assert _gathered(m, prologue=False)[0] == (m == 1)
    x = seeded((1, K), seed=320, device=cuda).expand(m, K).contiguous()
    w2 = w.clone()
    best = (x[0].float() * 10).to(torch.bfloat16) / 10
    for row in (150001, 70000, 9001):
        w2[row] = best
    ids, logits = A.lm_head_argmax(x, w2, logits=True)
    assert ids.tolist() == [9001] * m
    w2[120000, 7] = float("nan")
    w2[130000, 9] = float("nan")
    ids = A.lm_head_argmax(x, w2, logits=False)[0]
    assert ids.tolist() == [120000] * m


def test_graph_of_gathered_and_two_launch_calls_replays_to_the_eager_ids(cuda, head):
    w, g = head
    xs = {m: seeded((m, K), seed=330 + m, device=cuda) for m in (1, 5)}
    tops = {m: torch.empty(m, dtype=torch.float32, device=cuda) for m in (1, 5)}
    cfgs = {1: STREAM, 5: None}
    assert _gathered(1, STREAM)[0] and not _gathered(5)[0]
    eager = {m: A.lm_head_argmax(xs[m], w, g, 1e-6, logits=False, top=tops[m], config=cfgs[m])[0].clone()
             for m in (1, 5)}
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = {m: A.lm_head_argmax(xs[m], w, g, 1e-6, logits=False, top=tops[m], config=cfgs[m])[0]
                   for m in (1, 5)}
    torch.cuda.synchronize()
    other = seeded((2, K), seed=340, device=cuda)
    for r in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for m in (1, 5):
            assert torch.equal(out[m], eager[m]), (r, m)
        A.lm_head_argmax(other, w, g, 1e-6, logits=False)  # a two-launch call between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("m", [2, 5, 8])
def test_stream_multi_row_gather_equals_two_launch_form(cuda, m):
    """Several x rows on the STREAM kind with at most one key word per gathering lane (4096 rows
    walked by 256 workgroups): one launch whose gatherer reads every walker's M words at once, the
    same logits and ids as the two-launch form of the same kernel (1024 workgroups, more than one
    word per lane), and the key region zero afterwards."""
    v, k = 4096, 4096
    cfg = _native.Config(_native.KIND_STREAM, 2, 0, 1, 4)
    p = L.plan(m, v, k, _native.EPI_ARGMAX, config=cfg, prologue=True)
    assert p.kind == _native.KIND_STREAM and p.grid <= p.threads
    x = seeded((m, k), seed=350 + m, device=cuda)
    w = seeded((v, k), seed=351, scale=0.02, device=cuda)
    g = seeded((k,), seed=352, scale=0.1, shift=1.0, device=cuda)
    w[1234] = w[77]  # an exact tie: the lower index wins
    top = torch.empty(m, dtype=torch.float32, device=cuda)
    ids, logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True, top=top, config=cfg)
    torch.cuda.synchronize()
    assert _keys_zero(cuda, m, p.grid)
    got = to_bits(logits).reshape(m, v)
    want = path.argmax_first(got)
    assert np.array_equal(ids.cpu().numpy(), want)
    assert np.array_equal(top.cpu().numpy(), bf16.to_f32(got)[np.arange(m), want])
    two = _native.Config(_native.KIND_STREAM, 2, 0, 4, 4)
    p2 = L.plan(m, v, k, _native.EPI_ARGMAX, config=two, prologue=True)
    assert p2.kind == _native.KIND_STREAM and p2.grid > p2.threads  # the finalize launch
    ids_2, logits_2 = A.lm_head_argmax(x, w, g, 1e-6, logits=True, config=two)
    assert torch.equal(logits, logits_2) and torch.equal(ids, ids_2)
