"""Timed selection (kernels/linear.py: _candidates, _agrees, _choose, _choice, refine; kernels/tune.py
knobs), the reference's policy of engine/kernels/linear.py:317-486 and engine/decode.py:556-583.

- On first use with tuning on, a shape's candidates are timed on cold weights against the native
  GEMM; the frozen choice is registered as a knob with its fastest alternatives and the planner
  default, and the result passes oracle parity, for a Qwen3-8B M = 1 shape (C3) and an M = 8 shape
  with the RMSNorm prologue (C4).
- A first use during graph capture raises RuntimeError (linear.py:497-498).
- ``refine`` re-judges the knobs inside a captured step; the graph captured with its final choices
  replays bit for bit as the eager step.
- Selection is on by default: a fresh process without FTK_TUNE selects on first use and raises on a
  first use under capture. A fused operation whose knob is put on "native" runs torch's GEMM
  directly, so capturing it needs no further selection.
"""

import os
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import seeded, to_bits
from oracle import bf16, path

from kernels import _native
from kernels import linear as L
from kernels import swiglu as S
from kernels import tune

pytestmark = pytest.mark.gpu

EPS = 1e-6


def within(got_bits, want_bits):
    g, w = bf16.to_f32(got_bits).astype(np.float64), bf16.to_f32(want_bits).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= 2e-2 + 1e-2 * np.abs(w)))


@pytest.fixture
def tuning(monkeypatch):
    """Tuning on, with fresh choice tables and knob registry (restored afterwards)."""
    monkeypatch.setattr(L, "TUNE", True)
    monkeypatch.setattr(L, "SHAPE_SECONDS", 2.0)
    monkeypatch.setattr(L, "_CHOICES", {})
    monkeypatch.setattr(L, "_VALIDATED", {})
    monkeypatch.setattr(L, "_TUNING_DEADLINE", None)
    monkeypatch.setattr(L, "inherited", {})
    monkeypatch.setattr(tune, "_REGISTRY", {})
    yield


def _knob(key):
    return next(k for k in tune._REGISTRY.values() if k.name == key)


def test_choose_freezes_a_checked_choice_at_a_c3_shape(cuda, tuning):
    x = seeded((1, 4096), 11, device=cuda)
    w = seeded((4096, 4096), 12, scale=0.02, device=cuda)
    y = L.linear(x, w)
    key = (cuda, 1, 4096, 4096)
    assert key in L._CHOICES
    timed = L._VALIDATED[key]
    assert timed and any(c == "native" for _, c in timed) and any(c is None for _, c in timed)
    assert [t for t, _ in timed] == sorted(t for t, _ in timed)
    knob = _knob(key)
    assert knob.rows == 1 and knob.get() == L._CHOICES[key] and None in knob.options
    assert within(to_bits(y), path.project(to_bits(x), to_bits(w)))
    # frozen: a second call does not select again, and returns the same bits
    before = dict(L._VALIDATED)
    np.testing.assert_array_equal(to_bits(L.linear(x, w)), to_bits(y))
    assert L._VALIDATED == before
    # a first use during capture raises (selection must finish during eager warmup)
    x2 = seeded((1, 4096), 13, device=cuda)
    w2 = seeded((2048, 4096), 14, scale=0.02, device=cuda)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="eager warmup"):
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                L.linear(x2, w2)
    torch.cuda.synchronize()


def test_choose_with_the_norm_prologue_at_a_c4_shape(cuda, tuning):
    x = seeded((8, 4096), 21, device=cuda)
    g = seeded((4096,), 22, scale=0.1, shift=1.0, device=cuda)
    w = seeded((6144, 4096), 23, scale=0.02, device=cuda)
    y = L.rms_norm_linear(x, g, EPS, w)
    key = ("norm", cuda, 8, 6144, 4096)
    assert key in L._CHOICES and L._VALIDATED[key]
    assert _knob(key).rows == 8
    assert within(to_bits(y), path.norm_project(to_bits(x), to_bits(g), EPS, to_bits(w)))
    # every option the knob offers gives the oracle's result too
    for option in _knob(key).options:
        _knob(key).select(option)
        assert within(to_bits(L.rms_norm_linear(x, g, EPS, w)),
                      path.norm_project(to_bits(x), to_bits(g), EPS, to_bits(w))), option


def test_refine_keeps_a_graph_identical_to_eager(cuda, tuning):
    h, i = 1024, 3072
    x = seeded((1, h), 31, device=cuda)
    g = seeded((h,), 32, scale=0.1, shift=1.0, device=cuda)
    layers = [(seeded((4096, h), 33 + 3 * j, scale=0.02, device=cuda),
               seeded((2 * i, h), 34 + 3 * j, scale=0.02, device=cuda),
               seeded((h, i), 35 + 3 * j, scale=0.02, device=cuda)) for j in range(4)]

    def step():
        hidden = x
        outs = []
        for w_qkv, w_gu, w_down in layers:
            outs.append(L.rms_norm_linear(hidden, g, EPS, w_qkv))
            hidden = L.linear(S.gate_up_swiglu(hidden, w_gu, g, EPS), w_down)
        return outs + [hidden]

    step()  # eager warmup: selects every shape
    assert len(tune.knobs(1)) == 3
    stream = torch.cuda.Stream()

    def capture():
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            step()
            with torch.cuda.graph(graph, stream=stream):
                outs = step()
        torch.cuda.synchronize()
        return graph, outs

    def step_seconds():
        graph, _ = capture()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        graph.replay()
        start.record()
        for _ in range(5):
            graph.replay()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / 5e3

    best = L.refine(step_seconds, rows=1, seconds=5.0)
    assert best > 0
    graph, outs = capture()
    eager = [to_bits(t).copy() for t in step()]
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, eager):
            np.testing.assert_array_equal(to_bits(got), want)


def test_past_the_process_budget_a_verify_block_inherits(cuda, tuning, monkeypatch):
    """Past the process budget (linear.py:441-443) a 5..32-row shape takes a launch choice frozen for
    the same weight at another row count above 4 once it agrees with the planner default
    (_inherit, linear.py:412-433); a shape of 4 or fewer rows takes its untuned default."""
    w = seeded((4096, 4096), 41, scale=0.02, device=cuda)
    ring = (_native.KIND_RING, 16, 2, 1, 8)
    L._CHOICES[(cuda, 8, 4096, 4096)] = ring  # as if selected at 8 rows before the budget ran out
    monkeypatch.setattr(L, "_TUNING_DEADLINE", 0.0)
    x5 = seeded((5, 4096), 42, device=cuda)
    y5 = L.linear(x5, w)
    assert L._CHOICES[(cuda, 5, 4096, 4096)] == ring
    assert L.inherited[(cuda, 5, 4096, 4096)] == ring
    assert _knob((cuda, 5, 4096, 4096)).get() == ring
    assert within(to_bits(y5), path.project(to_bits(x5), to_bits(w)))
    x3 = seeded((3, 4096), 43, device=cuda)
    y3 = L.linear(x3, w)
    assert L._CHOICES[(cuda, 3, 4096, 4096)] is None and L.inherited[(cuda, 3, 4096, 4096)] is None
    assert within(to_bits(y3), path.project(to_bits(x3), to_bits(w)))


DEFAULT_POLICY = textwrap.dedent("""
    import sys, torch
    sys.path.insert(0, sys.argv[1])
    from kernels import linear as L, tune
    assert L.TUNE, "selection must be on by default"
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    x = torch.randn((1, 1024), generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn((512, 1024), generator=g) * 0.02).to(torch.bfloat16).to(dev)
    y = L.linear(x, w)
    key = (dev, 1, 512, 1024)
    assert key in L._CHOICES and L._VALIDATED[key], "first use did not select"
    assert any(k.name == key for k in tune.knobs(1)), "no knob registered"
    ref = torch.nn.functional.linear(x, w).float()
    assert bool(((y.float() - ref).abs() <= ref.abs() * 0.016 + 0.001).all())
    x2 = torch.randn((1, 1024), generator=g).to(torch.bfloat16).to(dev)
    w2 = (torch.randn((256, 1024), generator=g) * 0.02).to(torch.bfloat16).to(dev)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                L.linear(x2, w2)
    except RuntimeError as e:
        assert "eager warmup" in str(e), e
        print("default policy ok", flush=True)
    else:
        raise AssertionError("a first use under capture did not raise")
    torch.cuda.synchronize()
""")


def test_selection_is_on_by_default_in_a_fresh_process(cuda):
    env = {k: v for k, v in os.environ.items() if k != "FTK_TUNE"}
    env["FTK_TUNE_SECONDS"] = "10"
    pkg = str(Path(__file__).resolve().parents[1] / "fast-transformer_amd")
    print("test_selection_is_on_by_default_in_a_fresh_process: child process starts", flush=True)
    proc = subprocess.run([sys.executable, "-c", DEFAULT_POLICY, pkg], env=env, capture_output=True, text=True,
                          timeout=100)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "default policy ok" in proc.stdout


@pytest.mark.parametrize("op", ["norm", "swiglu", "argmax"])
def test_a_fused_knob_on_native_captures_without_eager_warmup(cuda, tuning, op):
    """A fused operation whose frozen choice is "native" runs torch's GEMM itself (the form its
    selection timed): capturing it needs no selection of a plain projection key."""
    h = 1024
    x = seeded((1, h), 51, device=cuda)
    g = seeded((h,), 52, scale=0.1, shift=1.0, device=cuda)
    n = {"norm": 2048, "swiglu": 2 * 3072, "argmax": 8192}[op]
    w = seeded((n, h), 53, scale=0.02, device=cuda)
    from kernels import argmax as A
    from kernels.rmsnorm import rms_norm

    def call():
        if op == "norm":
            return L.rms_norm_linear(x, g, EPS, w)
        if op == "swiglu":
            return S.gate_up_swiglu(x, w, g, EPS)
        return A.lm_head_argmax(x, w, g, EPS, logits=True)[1]

    call()  # eager first use: selects under the fused key
    key = (op, cuda, 1, n, h)
    assert key in L._CHOICES
    L._CHOICES[key] = "native"  # what refine does when it keeps the native option
    plain = [k for k in L._CHOICES if not isinstance(k[0], str)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = call()
    torch.cuda.synchronize()
    assert [k for k in L._CHOICES if not isinstance(k[0], str)] == plain, "a plain projection was selected"
    logits = torch.nn.functional.linear(rms_norm(x, g, EPS), w)
    want = {"norm": logits, "swiglu": S.swiglu(logits), "argmax": logits}[op]
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_bits(out), to_bits(want))
