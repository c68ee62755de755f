"""The kernels capture into a graph: replays (with eager work and synchronizations
between them, and fresh inputs copied in place) equal the eager results, every time.
The argmax workspace is cleared by the kernels themselves, so replays need no memset node."""

import pytest
import torch

from conftest import seeded

from kernels import argmax as A
from kernels import linear as L
from kernels import rmsnorm as R
from kernels import swiglu as S

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(cuda):
    h, i, v, q = 1024, 3072, 8192, 2048
    x = seeded((1, h), seed=1, device=cuda)
    g1 = seeded((h,), seed=2, scale=0.1, shift=1.0, device=cuda)
    w_qkv = seeded((4096, h), seed=3, scale=0.02, device=cuda)
    w_gu = seeded((2 * i, h), seed=4, scale=0.02, device=cuda)
    w_down = seeded((h, i), seed=5, scale=0.02, device=cuda)
    w_head = seeded((v, h), seed=6, scale=0.02, device=cuda)
    attn = seeded((1, q), seed=7, device=cuda)
    w_o = seeded((h, q), seed=8, scale=0.02, device=cuda)

    def step():
        qkv = L.rms_norm_linear(x, g1, 1e-6, w_qkv)
        o = L.linear(attn, w_o)
        normed, summed = R.add_rms_norm(o, x, g1, 1e-6)
        act = S.gate_up_swiglu(normed, w_gu)
        down = L.linear(act, w_down)
        ids, logits = A.lm_head_argmax(down, w_head, g1, 1e-6, logits=True)
        return qkv, summed, act, down, ids, logits

    step()  # eager warmup: selection and workspaces outside capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            outs = step()
    torch.cuda.current_stream().wait_stream(stream)
    for seed in (11, 12, 13):
        x.copy_(seeded((1, h), seed=seed, device=cuda))
        attn.copy_(seeded((1, q), seed=seed + 100, device=cuda))
        eager = step()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, eager):
            assert torch.equal(got, want)
