"""GPU parity of projection chains (ftk_chain_*, csrc/ftk_chain.hip; kernels/chain.py).

A chain runs a stack of M = 1 decode-layer projections in one cooperative launch. Each stage is
checked against the oracle applied to that stage's own input as the chain produced it (so every
stage meets the per-operation bar, 2e-2 + 1e-2 |ref|, with no error carried over):
- QKV: rms_norm prologue then projection (engine/kernels/rmsnorm.py:35-46, engine/layers.py:44);
- O: projection, plus the residual add of engine/kernels/rmsnorm.py:86-95 in the residual flow;
- gate/up + SwiGLU on the normalised O output (engine/layers.py:99-102, swiglu.py:20-24);
- down: projection (plus the residual add).
Replays of a captured chain equal the eager launch bit for bit, fresh inputs are picked up by
every launch, and no bounded wait ever expires (status 0).
"""

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import chain as CH
from kernels import linear as L
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

ATOL, RTOL, EPS = 2e-2, 1e-2, 1e-6

SHAPES = {  # hidden, intermediate, attention width (q heads x 128), QKV rows
    "0.6B": (1024, 3072, 2048, 4096),
    "8B": (4096, 12288, 4096, 6144),
}


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ATOL + RTOL * np.abs(w)))


def add_bits(a_bits, b_bits):
    """bf16(f32(a) + f32(b)): the residual add (engine/kernels/rmsnorm.py:86-88)."""
    return bf16.round_bits(bf16.to_f32(a_bits) + bf16.to_f32(b_bits))


def make_layers(model, n, seed, device):
    h, i, q, qkv = SHAPES[model]
    layers = []
    for l in range(n):
        s = seed + 10 * l
        layers.append(dict(qkv=seeded((qkv, h), s, scale=0.02, device=device),
                           o=seeded((h, q), s + 1, scale=0.02, device=device),
                           gate_up=seeded((2 * i, h), s + 2, scale=0.02, device=device),
                           down=seeded((h, i), s + 3, scale=0.02, device=device),
                           ln1=seeded((h,), s + 4, scale=0.1, shift=1.0, device=device),
                           ln2=seeded((h,), s + 5, scale=0.1, shift=1.0, device=device)))
    return layers


def check_stages(chain, idx, layers, hidden, attn, residual):
    for i, lw in enumerate(layers):
        h_in = to_bits(hidden) if i == 0 else to_bits(chain.output(idx["down"][i - 1]))
        qkv = to_bits(chain.output(idx["qkv"][i]))
        assert within(qkv, path.norm_project(h_in.reshape(1, -1), to_bits(lw["ln1"]), EPS, to_bits(lw["qkv"]))), \
            f"layer {i} qkv"
        o = to_bits(chain.output(idx["o"][i]))
        want_o = path.project(to_bits(attn), to_bits(lw["o"]))
        if residual:
            want_o = add_bits(want_o, h_in.reshape(1, -1))
        assert within(o, want_o), f"layer {i} o"
        act = to_bits(chain.output(idx["act"][i]))
        assert within(act, path.gate_up_swiglu(o, to_bits(lw["gate_up"]), to_bits(lw["ln2"]), EPS)), f"layer {i} act"
        down = to_bits(chain.output(idx["down"][i]))
        want_d = path.project(act, to_bits(lw["down"]))
        if residual:
            want_d = add_bits(want_d, o)
        assert within(down, want_d), f"layer {i} down"


@pytest.mark.parametrize("model,n_layers", [("0.6B", 3), ("8B", 1)])
@pytest.mark.parametrize("residual", [False, True])
def test_chain_stages_match_oracle(cuda, model, n_layers, residual):
    print(f"chain parity {model} layers={n_layers} residual={residual}", flush=True)
    h, _, q, _ = SHAPES[model]
    layers = make_layers(model, n_layers, 100, cuda)
    hidden = seeded((1, h), 1, device=cuda)
    attn = seeded((1, q), 2, device=cuda)
    chain, idx = CH.decode_layers(layers, hidden, attn, EPS, residual_epilogue=residual)
    chain.prepare()
    chain.launch()
    chain.status()
    check_stages(chain, idx, layers, hidden, attn, residual)


def test_chain_agrees_with_the_single_launch_kernels(cuda):
    """The same projections as separate launches (STREAM kind): within one BF16 ulp almost everywhere."""
    h, _, q, _ = SHAPES["8B"]
    layers = make_layers("8B", 1, 300, cuda)
    hidden = seeded((1, h), 3, device=cuda)
    attn = seeded((1, q), 4, device=cuda)
    chain, idx = CH.decode_layers(layers, hidden, attn, EPS)
    chain.prepare()
    chain.launch()
    chain.status()
    lw = layers[0]
    qkv = L.rms_norm_linear(hidden, lw["ln1"], EPS, lw["qkv"])
    o = L.linear(attn, lw["o"])
    act = S.gate_up_swiglu(chain.output(idx["o"][0]), lw["gate_up"], lw["ln2"], EPS)
    down = L.linear(chain.output(idx["act"][0]), lw["down"])
    for name, single, got in (("qkv", qkv, idx["qkv"][0]), ("o", o, idx["o"][0]), ("act", act, idx["act"][0]),
                              ("down", down, idx["down"][0])):
        a = bf16.to_f32(to_bits(single)).astype(np.float64)
        b = bf16.to_f32(to_bits(chain.output(got))).astype(np.float64)
        same = np.mean(a == b)
        assert same >= 0.97, f"{name}: only {same:.3f} identical to the single launches"
        assert np.all(np.abs(a - b) <= 2.0 ** -7 * np.maximum(np.abs(a), 2.0 ** -10) + 1e-6), name


def test_chain_picks_up_fresh_inputs_every_launch(cuda):
    h, _, q, _ = SHAPES["0.6B"]
    layers = make_layers("0.6B", 2, 500, cuda)
    hidden = seeded((1, h), 5, device=cuda)
    attn = seeded((1, q), 6, device=cuda)
    chain, idx = CH.decode_layers(layers, hidden, attn, EPS, residual_epilogue=True)
    chain.prepare()
    for trial in range(3):
        hidden.copy_(seeded((1, h), 50 + trial, device=cuda))
        attn.copy_(seeded((1, q), 60 + trial, device=cuda))
        chain.launch()
        chain.status()
        check_stages(chain, idx, layers, hidden, attn, residual=True)


def test_chain_graph_replays_match_eager(cuda):
    h, _, q, _ = SHAPES["0.6B"]
    layers = make_layers("0.6B", 4, 700, cuda)
    hidden = seeded((1, h), 7, device=cuda)
    attn = seeded((1, q), 8, device=cuda)
    chain, idx = CH.decode_layers(layers, hidden, attn, EPS, residual_epilogue=True)
    chain.prepare()
    chain.launch()
    chain.status()
    want = [to_bits(chain.output(i)).copy() for i in idx["down"] + idx["qkv"]]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            chain.launch()
    torch.cuda.synchronize()
    for rep in range(4):
        for i in idx["down"]:
            chain.output(i).fill_(0)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [to_bits(chain.output(i)) for i in idx["down"] + idx["qkv"]]
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b)
    chain.status()


def test_chain_many_launches_and_stage_times(cuda):
    h, _, q, _ = SHAPES["0.6B"]
    layers = make_layers("0.6B", 2, 900, cuda)
    hidden = seeded((1, h), 9, device=cuda)
    attn = seeded((1, q), 10, device=cuda)
    chain, idx = CH.decode_layers(layers, hidden, attn, EPS)
    chain.prepare()
    chain.launch()
    first = to_bits(chain.output(idx["down"][-1])).copy()
    for _ in range(200):
        chain.launch()
    chain.status()
    np.testing.assert_array_equal(to_bits(chain.output(idx["down"][-1])), first)
    times = chain.stage_us()
    assert len(times) == len(chain) and all(t > 0 for t in times)
    assert sum(times) < 10_000
