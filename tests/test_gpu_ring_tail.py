"""GPU tests of the RING kind's claimed tail: where a workgroup walks kRingTailMinTiles (16) or
more tiles (lm_head + argmax with the norm prologue, at 1..16 rows), the last eighth of the tiles is claimed from a counter
in the projection workspace, two tiles ahead of use, so that the workgroups that run ahead take
more of them.

Checked on the default launches:
- several calls in a row (different x each), logits against the CPU oracle (|y - ref| <=
  2e-2 + 1e-2|ref|), ids equal to the greedy id of the kernel's own logits and to the oracle's
  where the top two logits are clearly apart, top values equal to the winning logits;
- a vocabulary whose last tile is ragged;
- the counter back at zero after every call (the launch's last claim resets it), so the next call
  starts from the first tail tile;
- a captured graph of the call, replayed three times with eager calls in between, equal to the
  eager call every time.
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

ATOL, RTOL = 2e-2, 1e-2
EPS = 1e-6
K = 4096
CLAIM_WORD = 128 // 4  # u32 index of the counter in the projection workspace


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return not (np.abs(g - w) > ATOL + RTOL * np.abs(w)).any()


def claim_word(device):
    ws = _native._WORKSPACES[(device, "project")]
    return int(ws[: 4 * (CLAIM_WORD + 1)].view(torch.int32)[CLAIM_WORD].item())


@pytest.fixture(scope="module")
def head(cuda):
    v = 65536 + 40  # 4099 16-row tiles, the last one ragged
    return (seeded((v, K), seed=9101, scale=0.02, device=cuda), seeded((K,), seed=9102, scale=0.1, shift=1.0,
                                                                         device=cuda))


@pytest.mark.parametrize("m", [1, 2, 4, 5, 16])
def test_claimed_tail_calls_in_a_row_match_the_oracle(cuda, head, m):
    w, g = head
    p = L.plan(m, w.shape[0], K, _native.EPI_ARGMAX, prologue=True)
    assert p.kind == _native.KIND_RING and p.tiles >= 16 * p.grid, (p.kind, p.tiles, p.grid)
    wb, gb = to_bits(w), to_bits(g)
    for call in range(3):
        x = seeded((m, K), seed=9200 + 10 * m + call, device=cuda)
        top = torch.empty(m, dtype=torch.float32, device=cuda)
        ids, logits = A.lm_head_argmax(x, w, g, EPS, logits=True, top=top)
        torch.cuda.synchronize()
        assert claim_word(cuda) == 0, f"call {call}: the counter was left at {claim_word(cuda)}"
        want_logits, want_ids, _ = path.lm_head_argmax(to_bits(x), wb, gb, EPS)
        got_logits = to_bits(logits)
        assert within(got_logits, want_logits), f"call {call}"
        ids = ids.cpu().numpy()
        assert np.array_equal(ids, path.argmax_first(got_logits)), f"call {call}"
        v_sorted = np.sort(bf16.to_f32(want_logits).astype(np.float64), axis=-1)
        clear = (v_sorted[:, -1] - v_sorted[:, -2]) > 1e-2
        assert np.array_equal(ids[clear], want_ids[clear]), f"call {call}"
        assert np.array_equal(top.cpu().numpy(), bf16.to_f32(got_logits)[np.arange(m), ids]), f"call {call}"


@pytest.mark.parametrize("m", [1, 5])
def test_claimed_tail_graph_replays_equal_eager(cuda, head, m):
    w, g = head
    x = seeded((m, K), seed=9300, device=cuda)
    want_ids, want_logits = A.lm_head_argmax(x, w, g, EPS, logits=True, ids_dtype=torch.int32)
    want_ids, want_logits = want_ids.clone(), want_logits.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        A.lm_head_argmax(x, w, g, EPS, logits=True, ids_dtype=torch.int32)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            ids, logits = A.lm_head_argmax(x, w, g, EPS, logits=True, ids_dtype=torch.int32)
    torch.cuda.synchronize()
    other = seeded((m, K), seed=9301, device=cuda)
    for i in range(3):
        ids.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids, want_ids) and torch.equal(logits, want_logits), f"replay {i}"
        assert claim_word(cuda) == 0
        A.lm_head_argmax(other, w, g, EPS, logits=False)  # an eager call between replays
        torch.cuda.synchronize()
        assert claim_word(cuda) == 0
