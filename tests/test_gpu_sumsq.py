"""GPU parity of the norm's sums of squares handed between RING launches (``ftk_rows.sumsq_out`` /
``sumsq``, ``kernels.linear.SumSq``): a projection that writes a row stream also writes its rows'
sums of squares by 16-column part, and the next RMSNorm-prologue projection over that stream sums
those parts instead of reading the rows.

Checked at 5, 8 and 16 rows (the RING kind's rows) at Qwen3-8B widths:
- the written sums against float64 sums of the stored BF16 values, with the stored values equal to
  the same call's without the sums (plain and residual-add producers);
- every consumer (QKV, gate/up + SwiGLU, lm_head + argmax) against the CPU oracle with
  |y - ref| <= 2e-2 + 1e-2|ref| (>= 99 % bit-equal), and against the same call without the sums
  (at most one BF16 ulp apart, two after SwiGLU: the sums' order differs from the row read's);
- the rules that keep stale sums out: an in-place change of the rows, another tensor, a producer
  launch that is not RING;
- a captured two-layer chain passing the sums along, replayed three times with eager work in
  between, equal to the eager chain every time; a sums buffer first needed under capture raises.
"""

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import argmax as A
from kernels import linear as L
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
EPS = 1e-6
H, QKV, I, V = 4096, 6144, 12288, 16384


def check(got, want):
    got_bits = to_bits(got)
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want).astype(np.float64)
    bad = np.abs(g - w) > ATOL + RTOL * np.abs(w)
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tolerance, first at {np.argwhere(bad)[:4].tolist()}"
    assert np.mean(got_bits == want) >= 0.99


def within_ulps(a, b, ulps):
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    assert (ai - bi).abs().max().item() <= ulps


def sums_of(ss, y):
    buf = ss._of(y)
    assert buf is not None, "the producer wrote no sums for its output"
    m, n = y.shape
    return buf[: m * (n // 16)].view(m, n // 16).double()


def exact_sums(y):
    m, n = y.shape
    return (y.double() ** 2).view(m, n // 16, 16).sum(-1)


@pytest.fixture(scope="module")
def weights(cuda):
    return {
        "g1": seeded((H,), seed=8101, scale=0.1, shift=1.0, device=cuda),
        "qkv": seeded((QKV, H), seed=8102, scale=0.02, device=cuda),
        "o": seeded((H, H), seed=8103, scale=0.02, device=cuda),
        "g2": seeded((H,), seed=8104, scale=0.1, shift=1.0, device=cuda),
        "gate_up": seeded((2 * I, H), seed=8105, scale=0.02, device=cuda),
        "down": seeded((H, I), seed=8106, scale=0.02, device=cuda),
        "gf": seeded((H,), seed=8107, scale=0.1, shift=1.0, device=cuda),
        "head": seeded((V, H), seed=8108, scale=0.02, device=cuda),
    }


@pytest.mark.parametrize("m", [5, 8, 16])
def test_producers_write_the_sums_of_what_they_store(cuda, weights, m):
    w = weights
    act = seeded((m, I), seed=8200 + m, device=cuda)
    assert L.plan(m, H, I).kind == _native.KIND_RING
    ss = L.SumSq()
    y = L.linear_sumsq(act, w["down"], ss)
    torch.cuda.synchronize()
    want = exact_sums(y)
    assert torch.allclose(sums_of(ss, y), want, rtol=1e-6, atol=0)
    assert torch.equal(y, L.linear(act, w["down"]))

    res = seeded((m, H), seed=8300 + m, device=cuda)
    y2 = L.linear_residual(act, w["down"], res, sumsq=ss)
    torch.cuda.synchronize()
    assert ss._of(y) is None  # the second producer's sums replaced the first's
    assert torch.allclose(sums_of(ss, y2), exact_sums(y2), rtol=1e-6, atol=0)
    assert torch.equal(y2, L.linear_residual(act, w["down"], res))


@pytest.mark.parametrize("m", [5, 8, 16])
def test_consumers_match_the_oracle(cuda, weights, m):
    w = weights
    bits = {name: to_bits(t) for name, t in w.items()}
    ss = L.SumSq()
    act = seeded((m, I), seed=8400 + m, device=cuda)
    h = L.linear_sumsq(act, w["down"], ss)
    hb = to_bits(h)

    assert L.plan(m, QKV, H, prologue=True).kind == _native.KIND_RING
    got = L.rms_norm_linear(h, w["g1"], EPS, w["qkv"], sumsq=ss)
    check(got, path.norm_project(hb, bits["g1"], EPS, bits["qkv"]))
    within_ulps(got, L.rms_norm_linear(h, w["g1"], EPS, w["qkv"]), 1)

    got = S.gate_up_swiglu(h, w["gate_up"], w["g2"], EPS, sumsq=ss)
    check(got, path.gate_up_swiglu(hb, bits["gate_up"], bits["g2"], EPS))
    within_ulps(got, S.gate_up_swiglu(h, w["gate_up"], w["g2"], EPS), 2)

    assert L.plan(m, V, H, epilogue=_native.EPI_ARGMAX, prologue=True).kind == _native.KIND_RING
    ids, logits = A.lm_head_argmax(h, w["head"], w["gf"], EPS, logits=True, sumsq=ss)
    want_logits, want_ids, _ = path.lm_head_argmax(hb, bits["head"], bits["gf"], EPS)
    check(logits, want_logits)
    # the greedy id of the kernel's own logits (an ulp of difference may move a near-tie)
    assert np.array_equal(ids.cpu().numpy(), path.argmax_first(to_bits(logits)))
    assert ss._of(h) is not None  # consumers leave the sums in place
    torch.cuda.synchronize()


def test_stale_sums_are_not_used(cuda, weights):
    w = weights
    m = 8
    ss = L.SumSq()
    act = seeded((m, I), seed=8500, device=cuda)
    y = L.linear_sumsq(act, w["down"], ss)
    assert ss._of(y) is not None
    assert ss._of(y.clone()) is None  # another tensor
    assert ss._of(y[:4]) is None  # other rows
    y.mul_(2)  # the rows change in place: the sums no longer describe them
    assert ss._of(y) is None
    got = L.rms_norm_linear(y, w["g1"], EPS, w["qkv"], sumsq=ss)
    assert torch.equal(got, L.rms_norm_linear(y, w["g1"], EPS, w["qkv"]))
    check(got, path.norm_project(to_bits(y), to_bits(w["g1"]), EPS, to_bits(w["qkv"])))


@pytest.mark.parametrize("m", [1, 4])
def test_no_sums_where_the_producer_is_not_ring(cuda, weights, m):
    w = weights
    assert L.plan(m, H, I).kind != _native.KIND_RING
    ss = L.SumSq()
    act = seeded((m, I), seed=8600 + m, device=cuda)
    y = L.linear_sumsq(act, w["down"], ss)
    assert ss._of(y) is None
    check(y, path.project(to_bits(act), to_bits(w["down"])))
    got = L.rms_norm_linear(y, w["g1"], EPS, w["qkv"], sumsq=ss)
    assert torch.equal(got, L.rms_norm_linear(y, w["g1"], EPS, w["qkv"]))


def test_captured_chain_replays_equal_eager(cuda, weights):
    w = weights
    m = 5
    attn = seeded((m, H), seed=8700, device=cuda)
    h0 = seeded((m, H), seed=8701, device=cuda)
    ss = L.SumSq()

    def chain():
        h = h0
        for _ in range(2):
            L.rms_norm_linear(h, w["g1"], EPS, w["qkv"], sumsq=ss)
            o = L.linear_sumsq(attn, w["o"], ss)
            act = S.gate_up_swiglu(o, w["gate_up"], w["g2"], EPS, sumsq=ss)
            h = L.linear_sumsq(act, w["down"], ss)
        return h

    want = chain().clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        chain()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = chain()
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        L.linear(attn, w["o"])  # eager work between replays
        torch.cuda.synchronize()


def test_a_buffer_first_needed_under_capture_raises(cuda, weights):
    act = seeded((5, I), seed=8800, device=cuda)
    L.linear_sumsq(act, weights["down"], L.SumSq())  # the shape itself warmed eagerly
    fresh = L.SumSq()  # its buffer would be allocated inside the graph
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="eager warmup"):
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                L.linear_sumsq(act, weights["down"], fresh)
    torch.cuda.synchronize()
