"""Benchmark of the decode-time skinny BF16 projection path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-shapes]

One step = one M=1 decode step's projections at Qwen3-8B shapes (BASELINE.json
config 3): 36 layers, each RMSNorm-prologue QKV 4096->6144, O 4096->4096,
RMSNorm-prologue gate/up 4096->2x12288 with the SwiGLU epilogue, down
12288->4096, every layer with its own weights (13.9 GB resident in HBM), then
the final RMSNorm + lm_head 4096->151936 + greedy argmax (1.24 GB). Weights and
inputs are synthetic (seed 0; W ~ N(0, 0.02), x ~ N(0, 1), gamma ~ 1 + N(0, 0.1)).
The step is captured once into a graph and replayed; the timed region is K
replays bracketed by device synchronizations.

value = algorithmic bytes of the step / step time (GB/s). Rank 0 prints one
JSON line with the contract fields plus ``roofline`` (dominant kernel: the
fused gate/up + SwiGLU GEMV), ``cpu_baseline`` (the reference's torch CPU path on
a bounded sample of the same workload) and ``per_shape`` (µs, GB/s and fraction
of the 8 TB/s HBM roofline for every BASELINE.json configuration, plus the split-KV
decode attention at Qwen3-8B heads, a whole decode layer and a whole greedy decode
step of a Qwen3-8B-shape transformers model through decode.py).
"""

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "fast-transformer_amd"))

from kernels import _native  # noqa: E402
from kernels import argmax as A  # noqa: E402
from kernels import decode_attention as DA  # noqa: E402
from kernels import linear as L  # noqa: E402
from kernels import qk_rope as R  # noqa: E402
from kernels import swiglu as S  # noqa: E402
from kernels.tune import knobs  # noqa: E402

METRIC = "M=1 bf16 GEMV HBM GB/s (% of peak) + µs/decode-layer, Qwen3-8B shapes"
PEAK_GBS = 8000.0          # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0  # dense BF16 MFMA
EPS = 1e-6

QWEN3_8B = dict(hidden=4096, inter=12288, q_heads=32, kv_heads=8, head_dim=128, layers=36, vocab=151936)
QWEN3_06B = dict(hidden=1024, inter=3072, q_heads=16, kv_heads=8, head_dim=128, layers=28, vocab=151936)


def layer_bytes(cfg, m):
    """Algorithmic bytes of one layer's projection set (2NK + 2MK + 2MN_out, + 2K per norm gain)."""
    h, i = cfg["hidden"], cfg["inter"]
    q = cfg["q_heads"] * cfg["head_dim"]
    qkv_n = q + 2 * cfg["kv_heads"] * cfg["head_dim"]
    qkv = 2 * qkv_n * h + 2 * m * h + 2 * m * qkv_n + 2 * h
    o = 2 * h * q + 2 * m * q + 2 * m * h
    gate_up = 2 * 2 * i * h + 2 * m * h + 2 * m * i + 2 * h
    down = 2 * h * i + 2 * m * i + 2 * m * h
    return {"qkv": qkv, "o": o, "gate_up": gate_up, "down": down}


def head_bytes(cfg, m):
    h, v = cfg["hidden"], cfg["vocab"]
    return 2 * v * h + 2 * m * h + 2 * m * v + 2 * h + 4 * m


class Model:
    """Synthetic random-init weights of one model's projection path, resident on the GPU."""

    def __init__(self, cfg, device, layers=None, head=True, seed=0):
        self.cfg = cfg
        g = torch.Generator(device=device).manual_seed(seed)
        h, i = cfg["hidden"], cfg["inter"]
        q = cfg["q_heads"] * cfg["head_dim"]
        qkv_n = q + 2 * cfg["kv_heads"] * cfg["head_dim"]

        def w(n, k):
            return (torch.randn((n, k), generator=g, device=device) * 0.02).to(torch.bfloat16)

        def gamma(k):
            return (1 + 0.1 * torch.randn((k,), generator=g, device=device)).to(torch.bfloat16)

        self.layers = []
        for _ in range(cfg["layers"] if layers is None else layers):
            self.layers.append(dict(qkv=w(qkv_n, h), o=w(h, q), gate_up=w(2 * i, h), down=w(h, i)))
        for layer in self.layers:
            layer["ln1"], layer["ln2"] = gamma(h), gamma(h)
        self.head = w(cfg["vocab"], h) if head else None
        self.final_norm = gamma(h)
        self.q = q


class Step:
    """The decode step's projection path at M rows, with its input/output buffers preallocated."""

    def __init__(self, model, m, device, seed=1):
        self.model, self.m = model, m
        cfg = model.cfg
        g = torch.Generator(device=device).manual_seed(seed)
        self.h = torch.randn((m, cfg["hidden"]), generator=g, device=device).to(torch.bfloat16)
        # attention output feeding O: attention itself is outside the path
        self.attn = torch.randn((m, model.q), generator=g, device=device).to(torch.bfloat16)
        self.resid = torch.randn((m, cfg["hidden"]), generator=g, device=device).to(torch.bfloat16)
        self.top = torch.empty(m, dtype=torch.float32, device=device)
        # the norms' sums of squares, handed from each producer to the norm that reads its rows
        # (RING launches, 5..16 rows; elsewhere each norm reads its rows)
        self.sums = L.SumSq()

    def layer(self, lw, h):
        qkv = L.rms_norm_linear(h, lw["ln1"], EPS, lw["qkv"], sumsq=self.sums)
        o = L.linear_sumsq(self.attn, lw["o"], self.sums)
        act = S.gate_up_swiglu(o, lw["gate_up"], lw["ln2"], EPS, sumsq=self.sums)
        return qkv, L.linear_sumsq(act, lw["down"], self.sums)

    def layers(self):
        h = self.h
        for lw in self.model.layers:
            _, h = self.layer(lw, h)
        return h

    def layers_residual(self):
        """The same projections in the decode data flow of engine/decode.py:229-261: each input
        norm also adds the residual stream and stores the new one (add_rms_norm folded in)."""
        hidden, resid = self.h, self.resid
        for lw in self.model.layers:
            _, resid = L.add_rms_norm_linear(hidden, resid, lw["ln1"], EPS, lw["qkv"])
            o = L.linear(self.attn, lw["o"])
            act, resid = S.gate_up_swiglu(o, lw["gate_up"], lw["ln2"], EPS, residual=resid)
            hidden = L.linear(act, lw["down"])
        return hidden, resid

    def layers_residual_epilogue(self):
        """The same data flow with the residual add in the O and down epilogues (decode.py's form):
        each norm then reads the stored stream as a plain x."""
        resid = self.resid
        for lw in self.model.layers:
            L.rms_norm_linear(resid, lw["ln1"], EPS, lw["qkv"], sumsq=self.sums)
            resid = L.linear_residual(self.attn, lw["o"], resid, sumsq=self.sums)
            act = S.gate_up_swiglu(resid, lw["gate_up"], lw["ln2"], EPS, sumsq=self.sums)
            resid = L.linear_residual(act, lw["down"], resid, sumsq=self.sums)
        return resid

    def run(self):
        h = self.layers()
        return A.lm_head_argmax(h, self.model.head, self.model.final_norm, EPS, logits=True, top=self.top,
                                ids_dtype=torch.int32, sumsq=self.sums)


def capture(fn, warm=2):
    """Warm ``fn`` eagerly (selection, workspaces), then capture it into a graph on a side stream.

    ``warm=0`` captures without running anything first (for calls that need no workspace or
    selection), so that every launch of the kernels a profiler sees comes from graph replays."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warm):
            fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            fn()
    torch.cuda.synchronize()
    return graph


def tuned_graph(fn, rows, seconds, label):
    """Warm ``fn`` with selection on (each new shape is timed once, kernels/linear.py _choose), re-judge
    the frozen choices of batch ``rows`` inside the captured step (linear.refine, engine/decode.py:556-583),
    then capture the final graph."""
    if not L.TUNE:
        return capture(fn)
    for _ in range(2):
        fn()
    torch.cuda.synchronize()

    def step_seconds():
        return time_graph(capture(fn, warm=0), reps=5) * 1e-6

    us = L.refine(step_seconds, rows, seconds) * 1e6
    stage(f"{label}: {len(knobs(rows))} shapes selected and re-judged in the captured step ({us:.1f} us)")
    return capture(fn)


def time_graph(graph, reps=10, inner=1, warm_s=None):
    """Median wall time of one replay, from HIP events on the replay stream (µs). ``warm_s``: replay
    untimed for that long first (default LAYER_WARM_S), so that every timing sees the clocks of a GPU
    that is already busy, wherever it falls in the run."""
    if warm_s is None:
        warm_s = LAYER_WARM_S
    graph.replay()
    torch.cuda.synchronize()
    t_end = time.monotonic() + warm_s
    while time.monotonic() < t_end:
        for _ in range(10):
            graph.replay()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(reps):
        start.record()
        for _ in range(inner):
            graph.replay()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3 / inner)
    return statistics.median(times)


def selection_summary():
    """The frozen launch choice of every shape the run selected (kernels/linear.py _CHOICES)."""
    names = {_native.KIND_GEMV: "gemv", _native.KIND_MFMA: "mfma", _native.KIND_STREAM: "stream",
             _native.KIND_MFMA_STREAM: "mfma_stream", _native.KIND_QUAD: "quad", _native.KIND_STAGE: "stage",
             _native.KIND_RING: "ring"}
    out = {}
    for key, choice in L._CHOICES.items():
        op, rest = (key[0], key[2:]) if isinstance(key[0], str) else ("linear", key[1:])
        label = f"{op} M={rest[0]} N={rest[1]} K={rest[2]}"
        if choice is None:
            out[label] = "planner default"
        elif choice == "native":
            out[label] = "native (hipBLASLt via F.linear)"
        else:
            out[label] = names.get(choice[0], str(choice[0])) + str(list(choice[1:]))
    past = {}
    for key, choice in L.inherited.items():
        op, rest = (key[0], key[2:]) if isinstance(key[0], str) else ("linear", key[1:])
        past[f"{op} M={rest[0]} N={rest[1]} K={rest[2]}"] = "untuned default" if choice in (None, "native") \
            else "inherited " + names.get(choice[0], str(choice[0])) + str(list(choice[1:]))
    return {"tuned": L.TUNE, "tuning_s": round(L.tuning_seconds, 1), "budget_s": L.PROCESS_SECONDS,
            "past_budget": past, "choices": out}


def shape_entry(us, byts, flops=None):
    e = {"us": round(us, 3), "GB_s": round(byts / us / 1e3, 1), "frac_hbm": round(byts / us / 1e3 / PEAK_GBS, 4),
         "bytes": int(byts)}
    if flops is not None:
        e["mfma_util"] = round(flops / us / 1e6 / PEAK_BF16_TFLOPS, 5)
    return e


#: Launch shapes of the pure streaming read (ftk_stream_read) tried for each floor: persistent
#: workgroups per CU (0: one-shot workgroups, the form of the projections that walk one tile per
#: workgroup) and 16-byte loads in flight per lane.
FLOOR_SHAPES = tuple((gpc, loads) for gpc in (1, 2, 4, 8) for loads in (2, 4, 8)) + \
    tuple((0, loads) for loads in (2, 4, 8, 16))


def read_floor(tensors, reps=5):
    """The fastest pure streaming read of ``tensors`` (ftk_stream_read: the projections' load path and
    nothing else), one launch per tensor in one graph, the same bytes and the same graph form as the
    projections that read them: (µs per launch, (workgroups per CU, loads per lane) that gave it)."""
    dev = tensors[0].device
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    most = max(t.numel() * t.element_size() for t in tensors)
    sink = torch.empty(max(8 * cus, -(-most // (4096 * 2))), dtype=torch.int32, device=dev)
    best = None
    for gpc, loads in FLOOR_SHAPES:
        def fn():
            for t in tensors:
                _native.call("ftk_stream_read", _native.ptr(t), t.numel() * t.element_size(), _native.ptr(sink),
                             gpc * cus, loads, _native.stream_of(t))
        us = time_graph(capture(fn, warm=1), reps=reps, warm_s=0.1) / len(tensors)
        if best is None or us < best[0]:
            best = (us, (gpc, loads))
    return best


def floor_entry(entry, floor):
    """A per_shape entry with the read floor of its bytes beside it."""
    us, (gpc, loads) = floor
    shape = f"{gpc} workgroups per CU" if gpc else "one-shot workgroups"
    return {**entry, "read_floor_us": round(us, 3), "over_floor_us": round(entry["us"] - us, 3),
            "floor_shape": f"{shape}, {loads} loads per lane"}


def planner_config(m, n, k, epilogue, prologue):
    """The planner's default launch for a shape as an explicit config (no selection involved)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    p = L.plan(m, n, k, epilogue, cus, None, prologue)
    gpc = -(-p.grid // cus)
    cfg = _native.Config(p.kind, p.rows_per_wave, p.unroll, gpc, p.waves)
    again = L.plan(m, n, k, epilogue, cus, cfg, prologue)
    assert (again.kind, again.grid, again.rows_per_wave, again.waves) == (p.kind, p.grid, p.rows_per_wave, p.waves)
    return cfg


def per_kind(step, kind, warm=2, config=None, warm_s=None):
    """One graph of the 36 (or 28) launches of one projection kind, distinct weights each; µs per launch.
    ``config`` pins the gate/up launch (otherwise each call takes its frozen choice)."""
    def fn():
        for lw in step.model.layers:
            if kind == "qkv":
                L.rms_norm_linear(step.h, lw["ln1"], EPS, lw["qkv"])
            elif kind == "o":
                L.linear(step.attn, lw["o"])
            elif kind == "gate_up":
                S.gate_up_swiglu(step.h, lw["gate_up"], lw["ln2"], EPS, config=config)
            else:
                L.linear(step.act_in, lw["down"])
    if kind == "down":
        step.act_in = torch.randn((step.m, step.model.cfg["inter"]), device=step.h.device).to(torch.bfloat16)
    if warm == 0:
        # no eager call before capture: size the shared workspace here (an allocation, no launch)
        cfg = step.model.cfg
        _native.project_workspace(step.h.device, step.m, 2 * cfg["inter"], cfg["hidden"], _native.EPI_SWIGLU,
                                  prologue=True)
    graph = capture(fn, warm)
    return time_graph(graph, warm_s=warm_s) / len(step.model.layers)


#: Untimed replays before the roofline kernel's timed ones (seconds).
ROOFLINE_WARM_S = 0.5
#: Untimed replays before each graph is timed (seconds): every timing then sees the clocks of a GPU
#: that is already busy, wherever it falls in the run.
LAYER_WARM_S = 0.3


def roofline(step):
    """The ``roofline`` object: the dominant kernel, the fused gate/up + SwiGLU GEMV (201 MB per launch
    at M=1), timed over graph replays of its 36 launches (distinct weights). The graph is captured
    without eager launches, so a kernel trace of ``bench.py --roofline-only`` holds replays only."""
    cfg = step.model.cfg
    # the planner's default launch, pinned, so that --roofline-only (whose kernel trace backs this
    # figure) launches exactly the same kernel and grid whether or not this run selected shapes
    pinned = planner_config(1, 2 * cfg["inter"], cfg["hidden"], _native.EPI_SWIGLU, True)
    # half a second of untimed replays first: the timed replays then see the clocks of a busy GPU,
    # in the default run (after the step) and in --roofline-only alike; the last 10 replays (360
    # launches) are the timed ones
    gu_us = per_kind(step, "gate_up", warm=0, config=pinned, warm_s=ROOFLINE_WARM_S)
    gu_bytes = layer_bytes(cfg, 1)["gate_up"]
    return {"bound": "hbm", "achieved": round(gu_bytes / gu_us / 1e3, 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(gu_bytes / gu_us / 1e3 / PEAK_GBS, 4), "traffic": load_traffic(),
            "kernel": kernel_name(L.plan(1, 2 * cfg["inter"], cfg["hidden"], _native.EPI_SWIGLU), True,
                                  "SWIGLU") + " (Qwen3-8B gate/up 4096->2x12288, M=1)",
            "avg_launch_us": round(gu_us, 3)}


def cpu_share():
    """(threads, how they were counted) for the CPU baseline: the cgroup CPU quota when one is set
    (the box's share of the host), else the CPUs this process may run on, else os.cpu_count()."""
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if quota != "max":
            return max(1, int(quota) // int(period)), "cgroup cpu.max quota"
    except (OSError, ValueError):
        pass
    try:
        return len(os.sched_getaffinity(0)), "sched_getaffinity"
    except (AttributeError, OSError):
        return os.cpu_count() or 1, "os.cpu_count()"


def _cpu_median(fn, seconds, max_reps=200):
    """Median wall time (µs) of ``fn`` after one warm call, repeated for about ``seconds``."""
    fn()
    times, t_end = [], time.monotonic() + seconds
    while (time.monotonic() < t_end or len(times) < 5) and len(times) < max_reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e6, len(times)


def cpu_baseline(model8, dev, budget_s):
    """The reference's torch-CPU path (BF16 F.linear + native-cast norm / SwiGLU + torch.argmax,
    oracle/torch_cpu.py) on the same seeded weights and inputs as the GPU run, for every BASELINE.json
    configuration, on a bounded sample: C1 per call; C2 per layer over 4 of the 28 Qwen3-0.6B-shape
    layers; C3 and C4 (M = 5, 8, 16) per layer over 2 of the 36 Qwen3-8B-shape layers; C5 per call.
    Each figure is the median of repeated passes over about budget_s / 8 seconds."""
    from oracle import torch_cpu

    threads, how = cpu_share()
    torch.set_num_threads(threads)
    each = budget_s / 8
    out = {}

    def layers_fn(layers, m, cfg, seed):
        g = torch.Generator().manual_seed(seed)
        h = torch.randn((m, cfg["hidden"]), generator=g).to(torch.bfloat16)
        attn = torch.randn((m, cfg["q_heads"] * cfg["head_dim"]), generator=g).to(torch.bfloat16)
        return lambda: [torch_cpu.layer_projections(h, attn, lw, EPS) for lw in layers]

    cfg8 = model8.cfg
    layers8 = [{k: v.cpu() for k, v in model8.layers[i].items()} for i in range(2)]
    for m in (1, 5, 8, 16):
        us, reps = _cpu_median(layers_fn(layers8, m, cfg8, m), each)
        us /= len(layers8)
        byts = sum(layer_bytes(cfg8, m).values())
        label = "C3 8B layer M=1" if m == 1 else f"C4 8B layer M={m}"
        out[label] = {"us_per_layer": round(us, 1), "GB_s": round(byts / us / 1e3, 2), "passes": reps,
                      "sample": "2 of 36 layers"}
    del layers8
    head, gamma = model8.head.cpu(), model8.final_norm.cpu()
    for m in (1, 5):
        x = torch.randn((m, cfg8["hidden"]), generator=torch.Generator().manual_seed(50 + m)).to(torch.bfloat16)
        us, reps = _cpu_median(lambda: torch_cpu.lm_head_argmax(x, head, gamma, EPS), each)
        out[f"C5 lm_head+argmax M={m}"] = {"us_per_call": round(us, 1),
                                           "GB_s": round(head_bytes(cfg8, m) / us / 1e3, 2), "passes": reps}
    del head
    model06 = Model(QWEN3_06B, dev, head=False, seed=2)
    layers06 = [{k: v.cpu() for k, v in model06.layers[i].items()} for i in range(4)]
    del model06
    us, reps = _cpu_median(layers_fn(layers06, 1, QWEN3_06B, 3), each)
    us /= len(layers06)
    out["C2 0.6B layer M=1"] = {"us_per_layer": round(us, 1),
                                "GB_s": round(sum(layer_bytes(QWEN3_06B, 1).values()) / us / 1e3, 2),
                                "passes": reps, "sample": "4 of 28 layers"}
    x = torch.randn((1, 1024), generator=torch.Generator().manual_seed(60)).to(torch.bfloat16)
    w = layers06[0]["qkv"]
    us, reps = _cpu_median(lambda: torch_cpu.linear(x, w), each, max_reps=5000)
    out["C1 0.6B qkv M=1 (no prologue)"] = {"us_per_call": round(us, 1),
                                            "GB_s": round((2 * 4096 * 1024 + 2 * 1024 + 2 * 4096) / us / 1e3, 2),
                                            "passes": reps}
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    c3 = out["C3 8B layer M=1"]
    return {"value": c3["GB_s"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"C3: 2 of the 36 Qwen3-8B-shape layers at M=1 (QKV+O+gate/up+SwiGLU+down, torch CPU BF16), "
                      f"median of {c3['passes']} passes, {c3['us_per_layer']:.0f} us/layer; every configuration in "
                      f"per_config; {threads} threads ({how}; os.cpu_count() = {os.cpu_count()}); CPU: {cpu_model}",
            "us_per_layer": c3["us_per_layer"], "per_config": out}


def kernel_name(plan, prologue, epilogue):
    """The device function a plan launches, as rocprofv3 lists it (template arguments in order)."""
    kinds = {_native.KIND_STREAM: "stream_kernel<MR=1, RPW={p.rows_per_wave}, C={p.unroll}, KW={p.waves}",
             _native.KIND_GEMV: "gemv_kernel<MR=1, RPW={p.rows_per_wave}, U={p.unroll}, KW={p.waves}"}
    head = kinds.get(plan.kind, "kind {p.kind}<").format(p=plan)
    return f"ftk::{head}, PRO={int(prologue)}, {epilogue}> grid {plan.grid}"


_T0 = time.monotonic()


def stage(msg):
    """One progress line per finished stage, with the seconds since start (stderr; the JSON result
    stays the only stdout line)."""
    print(f"[bench] {msg} [{time.monotonic() - _T0:.0f} s]", file=sys.stderr, flush=True)


def load_traffic():
    f = ROOT / "profiles" / "traffic_gate_up_swiglu_8b_m1.json"
    if f.exists():
        return json.loads(f.read_text()).get("traffic_bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-shapes", action="store_true", help="skip the per-configuration table")
    ap.add_argument("--cpu-seconds", type=float, default=24.0, help="CPU work of the CPU baseline, all configs")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the roofline measurement (graph replays of the 36 gate/up + SwiGLU launches): the "
                         "command whose rocprofv3 kernel trace backs roofline.avg_launch_us")
    ap.add_argument("--no-tune", action="store_true",
                    help="use the planner's launch defaults: skip the timed selection of each shape at warmup "
                         "and its refinement inside the captured step")
    ap.add_argument("--extras", action="store_true",
                    help="also time a whole decode layer with attention and a whole transformers decode step")
    ap.add_argument("--profile-gate-up", type=int, default=0, metavar="PASSES",
                    help="profiling mode: only PASSES eager passes of the 36 gate/up + SwiGLU launches, "
                         "then one 1 GiB device copy as the counter reference")
    ap.add_argument("--profile-attention", type=int, default=0, metavar="PASSES",
                    help="profiling mode: PASSES eager passes of decode attention, then of rope_attend, over each "
                         "ATTN_CASES cache set (distinct caches), then one 1 GiB device copy as the counter reference")
    ap.add_argument("--profile-kernels", type=int, default=0, metavar="PASSES",
                    help="profiling mode: PASSES eager passes of each bandwidth-bound configuration's kernels "
                         "(C3 layers, C5 at M=1 and 5, C2 layers, C1) on the planner's defaults, then one 1 GiB "
                         "device copy as the counter reference")
    ap.add_argument("--profile-rows", type=str, default="", metavar="M[,M...]",
                    help="profiling mode: two eager passes of the 36-layer projection set at each M rows "
                         "(the C4 workload), then one 1 GiB device copy as the counter reference")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this path has no multi-GPU form in this build "
              "(each GPU would run the same kernels on its shard of the weights); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    props = torch.cuda.get_device_properties(dev)
    _native.lib()

    cfg = QWEN3_8B
    if args.profile_kernels:
        profile_kernels(dev, args.profile_kernels)
        return
    if args.profile_gate_up:
        profile_gate_up(cfg, dev, args.profile_gate_up)
        return
    if args.profile_rows:
        profile_rows(cfg, dev, [int(m) for m in args.profile_rows.split(",")])
        return
    if args.profile_attention:
        profile_attention(cfg, dev, args.profile_attention)
        return
    if args.roofline_only:
        model = Model(cfg, dev, head=False)
        roof = roofline(Step(model, 1, dev))
        print(json.dumps({"mode": "roofline-only", "roofline": roof, "warm_s": ROOFLINE_WARM_S,
                          "timed_launches": 10 * cfg["layers"], "note": "the timed launches are the last ones"}),
              flush=True)
        return
    model = Model(cfg, dev)
    stage("Qwen3-8B weights resident")
    L.TUNE = not args.no_tune
    step = Step(model, 1, dev)
    graph = tuned_graph(step.run, 1, 20.0, "M=1 step")
    layer_graph = capture(step.layers)
    stage("decode step captured")

    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps

    lb = layer_bytes(cfg, 1)
    step_bytes = cfg["layers"] * sum(lb.values()) + head_bytes(cfg, 1)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    us_layers = time_graph(layer_graph, reps=10)
    us_per_layer = us_layers / cfg["layers"]
    layer_lb_us = sum(lb.values()) / (PEAK_GBS * 1e3)

    roof = roofline(step)

    per_shape = {}
    stage(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step")
    if not args.no_shapes:
        per_shape = shapes_table(model, step, dev, layer_graph)
        per_shape.update(shard_table(cfg, dev))
        per_shape.update(attention_table(cfg, dev))
        if args.extras:
            per_shape.update(full_layer_table(model, dev))
            per_shape.update(decode_model_table(cfg, dev))

    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "Qwen3-8B-shape decode projections, M=1: 36 layers (RMSNorm-prologue QKV, O, "
                               "RMSNorm-prologue gate/up + SwiGLU, down) + final RMSNorm + lm_head + argmax",
                   "rows": 1, "layers": cfg["layers"], "hidden": cfg["hidden"], "intermediate": cfg["inter"],
                   "vocab": cfg["vocab"], "weights_gb": round(step_bytes / 1e9, 2), "graph": True,
                   "parallelism": "single GPU"},
        "frac_peak": round(value / PEAK_GBS, 4),
        "us_per_layer": round(us_per_layer, 2), "layer_lower_bound_us": round(layer_lb_us, 2),
        "layer_vs_bound": round(us_per_layer / layer_lb_us, 3),
        "roofline": roof,
        "device": {"name": props.name, "cus": props.multi_processor_count},
        "selection": selection_summary(),
    }
    if per_shape:
        result["layer_read_floor_us"] = per_shape["C3 8B layer M=1"]["read_floor_us"]
        result["per_shape"] = per_shape
    if not args.no_cpu:
        stage("CPU baseline")
        result["cpu_baseline"] = cpu_baseline(model, dev, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    # Leave nothing to the exit handlers: the captured graphs and the cached blocks are released
    # here, while the HIP runtime (and a profiler's hooks into it) is still fully up.
    del graph, layer_graph
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def profile_gate_up(cfg, dev, passes):
    """Eager launches of the dominant kernel only, on the planner's default (for rocprofv3 counter runs),
    plus a copy of known size."""
    L.TUNE = False
    g = torch.Generator(device=dev).manual_seed(0)
    h, i = cfg["hidden"], cfg["inter"]
    weights = [(torch.randn((2 * i, h), generator=g, device=dev) * 0.02).to(torch.bfloat16)
               for _ in range(cfg["layers"])]
    gamma = (1 + 0.1 * torch.randn((h,), generator=g, device=dev)).to(torch.bfloat16)
    x = torch.randn((1, h), generator=g, device=dev).to(torch.bfloat16)
    for p in range(passes):
        for w in weights:
            S.gate_up_swiglu(x, w, gamma, EPS)
        torch.cuda.synchronize()
        print(f"profile pass {p + 1}/{passes} done", flush=True)
    src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)  # reference kernel: reads and writes exactly 1 GiB
    torch.cuda.synchronize()
    print(json.dumps({"mode": "profile-gate-up", "passes": passes, "launches": passes * cfg["layers"],
                      "bytes_per_launch": layer_bytes(cfg, 1)["gate_up"], "copy_bytes": 1 << 30}), flush=True)


def profile_rows(cfg, dev, rows):
    """Eager passes of the 36-layer projection set at M rows (for rocprofv3 counter runs), plus a
    copy of known size. Each layer is RMSNorm-prologue QKV, O, RMSNorm-prologue gate/up + SwiGLU, down,
    on the planner's defaults."""
    L.TUNE = False
    model = Model(cfg, dev, head=False)
    for m in rows:
        step = Step(model, m, dev, seed=m)
        for p in range(2):
            step.layers()
            torch.cuda.synchronize()
        print(f"profile M={m} done", flush=True)
    src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)  # reference kernel: reads and writes exactly 1 GiB
    torch.cuda.synchronize()
    print(json.dumps({"mode": "profile-rows", "rows": rows, "passes": 2, "layers": cfg["layers"],
                      "bytes_per_layer": {str(m): layer_bytes(cfg, m) for m in rows}, "copy_bytes": 1 << 30}),
          flush=True)


#: Distinct lm_head weight copies timed in one graph for C5 (1.24 GB each).
C5_COPIES = 4

#: Dispatch order of --profile-kernels: (label, projections per layer or call, layers or copies).
PROFILE_KERNELS = (("C3 8B M=1", ("qkv", "o", "gate_up", "down"), 36),
                   ("C5 M=1", ("lm_head",), C5_COPIES),
                   ("C5 M=5", ("lm_head",), C5_COPIES),
                   ("C2 0.6B M=1", ("qkv", "o", "gate_up", "down"), 28),
                   ("C1 0.6B qkv M=1 (no prologue)", ("qkv",), 64))


def profile_kernels(dev, passes=2):
    """Eager passes of every bandwidth-bound BASELINE configuration's kernels on the planner's
    defaults (for rocprofv3 counter runs), in the order of PROFILE_KERNELS, then a 1 GiB copy as the
    counter reference. All weights are made first, so the projection launches are the only ftk
    dispatches, ``passes`` times each: C3's 36 layers (QKV, O, gate/up + SwiGLU, down), C5's lm_head
    + argmax at M = 1 and 5 over C5_COPIES weight copies (at both the RING projection, whose walks
    end in claimed tiles, then the argmax finalize),
    C2's 28 layers, C1's QKV projection without the norm over 64 weight copies."""
    L.TUNE = False
    model8 = Model(QWEN3_8B, dev, head=True)
    step8 = Step(model8, 1, dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    heads = [model8.head] + [(torch.randn((QWEN3_8B["vocab"], QWEN3_8B["hidden"]), generator=gen, device=dev) * 0.02)
                             .to(torch.bfloat16) for _ in range(C5_COPIES - 1)]
    h_rows = {m: torch.randn((m, QWEN3_8B["hidden"]), generator=gen, device=dev).to(torch.bfloat16) for m in (1, 5)}
    top = torch.empty(5, dtype=torch.float32, device=dev)
    model06 = Model(QWEN3_06B, dev, head=False, seed=2)
    step06 = Step(model06, 1, dev, seed=3)
    x = torch.randn((1, 1024), generator=gen, device=dev).to(torch.bfloat16)
    copies = [(torch.randn((4096, 1024), generator=gen, device=dev) * 0.02).to(torch.bfloat16) for _ in range(64)]
    ys = [torch.empty((1, 4096), device=dev, dtype=torch.bfloat16) for _ in range(64)]
    src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    runs = {"C3 8B M=1": step8.layers,
            "C5 M=1": lambda: [A.lm_head_argmax(h_rows[1], w, model8.final_norm, EPS, logits=True, top=top[:1],
                                                ids_dtype=torch.int32) for w in heads],
            "C5 M=5": lambda: [A.lm_head_argmax(h_rows[5], w, model8.final_norm, EPS, logits=True, top=top,
                                                ids_dtype=torch.int32) for w in heads],
            "C2 0.6B M=1": step06.layers,
            "C1 0.6B qkv M=1 (no prologue)": lambda: [L.project(x, w, out=y) for w, y in zip(copies, ys)]}
    for label, _, _ in PROFILE_KERNELS:
        for _ in range(passes):
            runs[label]()
        torch.cuda.synchronize()
        stage(f"profile {label}: {passes} passes")
    dst.copy_(src)  # reference kernel: reads and writes exactly 1 GiB
    torch.cuda.synchronize()
    print(json.dumps({"mode": "profile-kernels", "passes": passes, "order": PROFILE_KERNELS, "copy_bytes": 1 << 30,
                      "bytes": {"C3": layer_bytes(QWEN3_8B, 1), "C2": layer_bytes(QWEN3_06B, 1),
                                "C5 M=1": head_bytes(QWEN3_8B, 1), "C5 M=5": head_bytes(QWEN3_8B, 5),
                                "C1": 2 * 4096 * 1024 + 2 * 1024 + 2 * 4096}}), flush=True)


def shapes_table(model8, step8, dev, layer_graph):
    """µs / GB/s / fraction of the HBM roofline for every BASELINE.json configuration (C1-C5), each
    M = 1 projection with the pure-read floor of its bytes (``read_floor``) beside it."""
    out = {}
    cfg = model8.cfg
    lb = layer_bytes(cfg, 1)
    floors = {}
    for kind in ("qkv", "o", "gate_up", "down"):
        us = per_kind(step8, kind)
        floors[kind] = read_floor([lw[kind] for lw in model8.layers])
        out[f"C3 8B {kind} M=1"] = floor_entry(shape_entry(us, lb[kind]), floors[kind])
    stage("C3 per-projection timings and read floors done")
    # C5: lm_head + argmax at M=1 and M=5, over C5_COPIES distinct weight copies per graph (5 GB:
    # nothing is served from the MALL, and a graph launch is not charged to a single call)
    gen = torch.Generator(device=dev).manual_seed(7)
    heads = [model8.head] + [(torch.randn((cfg["vocab"], cfg["hidden"]), generator=gen, device=dev) * 0.02)
                             .to(torch.bfloat16) for _ in range(C5_COPIES - 1)]
    for m in (1, 5):
        st = step8 if m == 1 else Step(model8, m, dev, seed=5)
        h = torch.randn((m, cfg["hidden"]), device=dev).to(torch.bfloat16)
        g = capture(lambda: [A.lm_head_argmax(h, w, model8.final_norm, EPS, logits=True, top=st.top,
                                              ids_dtype=torch.int32) for w in heads])
        us = time_graph(g) / len(heads)
        out[f"C5 lm_head+argmax M={m}"] = shape_entry(us, head_bytes(cfg, m), 2 * m * cfg["vocab"] * cfg["hidden"])
        stage(f"C5 M={m} done")
    head_floor = read_floor(heads, reps=3)
    for m in (1, 5):
        out[f"C5 lm_head+argmax M={m}"] = floor_entry(out[f"C5 lm_head+argmax M={m}"], head_floor)
    del heads
    # C4: 8B layer set at M = 5, 8, 16
    for m in (5, 8, 16):
        st = Step(model8, m, dev, seed=m)
        g = tuned_graph(st.layers, m, 20.0, f"C4 M={m}")
        us = time_graph(g, reps=5) / cfg["layers"]
        byts = sum(layer_bytes(cfg, m).values())
        flops = 2 * m * sum(n * k for n, k in ((6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288)))
        out[f"C4 8B layer M={m}"] = shape_entry(us, byts, flops)
        stage(f"C4 M={m} done")
    out.update(vendor_table(model8, dev))
    stage("C4 projections against hipBLASLt done")
    # C3 per layer (M=1): the headline's own layer graph, timed again late in the run
    us = time_graph(layer_graph, reps=10) / cfg["layers"]
    floor_us = sum(f[0] for f in floors.values())
    out["C3 8B layer M=1"] = {**shape_entry(us, sum(lb.values())), "read_floor_us": round(floor_us, 3),
                              "over_floor_us": round(us - floor_us, 3)}
    # ... and in the decode data flow: both norms also add the residual and store the new stream
    g = capture(step8.layers_residual)
    us = time_graph(g, reps=5) / cfg["layers"]
    out["C3 8B layer M=1, residual-add prologues"] = shape_entry(us, sum(lb.values()) + 4 * 2 * cfg["hidden"])
    g = capture(step8.layers_residual_epilogue)
    us = time_graph(g, reps=5) / cfg["layers"]
    out["C3 8B layer M=1, residual add in the O / down epilogues"] = shape_entry(
        us, sum(lb.values()) + 4 * 2 * cfg["hidden"])
    del g
    # C1 / C2: Qwen3-0.6B shapes
    model06 = Model(QWEN3_06B, dev, head=False, seed=2)
    st06 = Step(model06, 1, dev, seed=3)
    g = capture(st06.layers)
    us = time_graph(g, reps=10) / QWEN3_06B["layers"]
    floor_us = sum(read_floor([lw[kind] for lw in model06.layers])[0] for kind in ("qkv", "o", "gate_up", "down"))
    out["C2 0.6B layer M=1"] = {**shape_entry(us, sum(layer_bytes(QWEN3_06B, 1).values())),
                                "read_floor_us": round(floor_us, 3), "over_floor_us": round(us - floor_us, 3)}
    x = torch.randn((1, 1024), device=dev).to(torch.bfloat16)
    copies = [torch.randn((4096, 1024), device=dev).mul_(0.02).to(torch.bfloat16) for _ in range(64)]
    ys = [torch.empty((1, 4096), device=dev, dtype=torch.bfloat16) for _ in range(64)]
    g = capture(lambda: [L.project(x, w, out=y) for w, y in zip(copies, ys)])
    us = time_graph(g) / 64
    out["C1 0.6B qkv M=1 (no prologue)"] = floor_entry(shape_entry(us, 2 * 4096 * 1024 + 2 * 1024 + 2 * 4096),
                                                       read_floor(copies))
    del model06, copies
    return out


def vendor_table(model8, dev):
    """Each C4 weight shape as a plain projection (no norm, no SwiGLU) at M = 5, 8, 16: this library's
    planner default against torch's native GEMM (hipBLASLt), each a graph over the 36 layers' distinct
    weights, same process. µs per launch; the entry's figures are this library's."""
    out = {}
    cfg = model8.cfg
    for m in (5, 8, 16):
        gen = torch.Generator(device=dev).manual_seed(100 + m)
        for kind in ("qkv", "o", "gate_up", "down"):
            k = cfg["inter"] if kind == "down" else cfg["hidden"]
            x = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
            ws = [lw[kind] for lw in model8.layers]
            ys = [torch.empty((m, w.shape[0]), device=dev, dtype=torch.bfloat16) for w in ws]
            ours = time_graph(capture(lambda: [L.project(x, w, out=y) for w, y in zip(ws, ys)]), reps=5) / len(ws)
            native = time_graph(capture(lambda: [torch.nn.functional.linear(x, w) for w in ws]), reps=5) / len(ws)
            n = ws[0].shape[0]
            e = shape_entry(ours, 2 * n * k + 2 * m * k + 2 * m * n, 2 * m * n * k)
            e["hipblaslt_us"] = round(native, 3)
            e["speedup_vs_hipblaslt"] = round(native / ours, 3)
            out[f"C4 8B {kind} GEMM M={m} vs hipBLASLt"] = e
    return out


#: Decode attention next to the projections (Qwen3-8B heads: 32 query, 8 KV, D = 128):
#: (rows, cache slots, distinct caches timed in one graph: together over the 256 MB MALL).
ATTN_CASES = ((1, 4096, 36), (1, 32768, 8), (16, 4096, 4))


def profile_attention(cfg, dev, passes):
    """Eager decode-attention launches over every ATTN_CASES cache set (for rocprofv3): per case,
    ``passes`` passes of decode_attention, then as many of rope_attend (the QK norm + RoPE prologue);
    then a 1 GiB copy."""
    hq, hkv, d = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    for b, c, copies in ATTN_CASES:
        g = torch.Generator(device=dev).manual_seed(11)
        ks = [torch.randn((b, hkv, c, d), generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
        vs = [torch.randn((b, hkv, c, d), generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
        q = torch.randn((b, hq, 1, d), generator=g, device=dev).to(torch.bfloat16)
        pos = torch.tensor([c - 1], device=dev, dtype=torch.int64)
        for _ in range(passes):
            for k, v in zip(ks, vs):
                DA.decode_attention(q, k, v, pos, d ** -0.5)
        packed = torch.randn((b, (hq + 2 * hkv) * d), generator=g, device=dev).to(torch.bfloat16)
        gain = _Norm((1 + 0.1 * torch.randn((d,), generator=g, device=dev)).to(torch.bfloat16), EPS)
        table = torch.randn((c, d), generator=g, device=dev).to(torch.bfloat16)
        for _ in range(passes):
            for k, v in zip(ks, vs):
                DA.rope_attend(packed, gain, gain, table, table, pos, k, v, hq, d ** -0.5)
        torch.cuda.synchronize()
        stage(f"attention B={b} C={c}: {passes} passes over {copies} caches")
        del ks, vs
    src = torch.empty(1 << 29, dtype=torch.int16, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    stage("1 GiB reference copy done")


class _Norm:
    """The q_norm / k_norm interface qk_rope_cache reads: .weight and .variance_epsilon."""

    def __init__(self, weight, eps):
        self.weight, self.variance_epsilon = weight, eps


#: Cache slots of the full decode layer (every layer's cache distinct; 604 MB for 36 layers).
FULL_LAYER_CONTEXT = 4096


def full_layer_table(model, dev):
    """One whole M=1 decode layer on this library, per layer of the 36, at a 4K-slot cache:
    norm + QKV, QK norm + RoPE + cache write in the decode attention's prologue, O with the
    residual add in its epilogue, norm + gate/up + SwiGLU, down with the residual add in its
    epilogue (engine/decode.py:229-261, engine/layers.py:32-90; decode.py's data flow); and the
    same layer with QK norm + RoPE + cache write as a launch of its own."""
    cfg = model.cfg
    hq, hkv, d, c = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"], FULL_LAYER_CONTEXT
    g = torch.Generator(device=dev).manual_seed(13)
    caches = [(torch.randn((1, hkv, c, d), generator=g, device=dev).to(torch.bfloat16),
               torch.randn((1, hkv, c, d), generator=g, device=dev).to(torch.bfloat16)) for _ in model.layers]
    norms = [(_Norm((1 + 0.1 * torch.randn((d,), generator=g, device=dev)).to(torch.bfloat16), EPS),
              _Norm((1 + 0.1 * torch.randn((d,), generator=g, device=dev)).to(torch.bfloat16), EPS))
             for _ in model.layers]
    angle = torch.arange(c, device=dev, dtype=torch.float64)[:, None] / \
        1_000_000.0 ** (torch.arange(0, d, 2, device=dev, dtype=torch.float64) / d)
    cos = torch.cat([angle, angle], dim=1).cos().to(torch.bfloat16)  # whole [C, D] tables, as decode.py's
    sin = torch.cat([angle, angle], dim=1).sin().to(torch.bfloat16)
    pos = torch.tensor([c - 1], device=dev, dtype=torch.int64)
    phases = torch.zeros((1, 1), device=dev, dtype=torch.int64)
    resid = torch.randn((1, cfg["hidden"]), generator=g, device=dev).to(torch.bfloat16)

    def layers(fused):
        r = resid
        for lw, (k, v), (qn, kn) in zip(model.layers, caches, norms):
            qkv = L.rms_norm_linear(r, lw["ln1"], EPS, lw["qkv"])
            if fused:
                attn = DA.rope_attend(qkv, qn, kn, cos, sin, pos, k, v, hq, d ** -0.5, phases=phases)
            else:
                q = R.qk_rope_cache(qkv.view(1, 1, -1), qn, kn, cos, sin, pos, k, v, hq, rows=True, phases=phases)
                attn = DA.decode_attention(q, k, v, pos, d ** -0.5)
            r = L.linear_residual(attn.reshape(1, hq * d), lw["o"], r)
            act = S.gate_up_swiglu(r, lw["gate_up"], lw["ln2"], EPS)
            r = L.linear_residual(act, lw["down"], r)
        return r

    lb = layer_bytes(cfg, 1)
    byts = sum(lb.values()) + 4 * 2 * cfg["hidden"] + 2 * hkv * c * d * 2
    out = {}
    for fused, name in ((True, ""), (False, ", QK norm + RoPE launched apart")):
        graph = capture(lambda: layers(fused))
        us = time_graph(graph, reps=5) / len(model.layers)
        out[f"C3 8B full decode layer M=1 (attention over {c} slots{name})"] = shape_entry(us, byts)
        del graph
    del caches
    stage("full decode layer done")
    return out


def decode_model_table(cfg, dev, context=FULL_LAYER_CONTEXT):
    """One whole greedy decode step of a Qwen3-8B-shape transformers model (random weights) through
    fast-transformer_amd/decode.py at B = 1, attending over ``context`` cached slots: embedding
    gather + 36 layers + final norm + lm_head + argmax, one graph (engine/decode.py:215-297)."""
    from transformers import Qwen3Config, Qwen3ForCausalLM

    import decode as D

    hf = Qwen3Config(vocab_size=cfg["vocab"], hidden_size=cfg["hidden"], intermediate_size=cfg["inter"],
                     num_hidden_layers=cfg["layers"], num_attention_heads=cfg["q_heads"],
                     num_key_value_heads=cfg["kv_heads"], head_dim=cfg["head_dim"], rms_norm_eps=EPS,
                     rope_theta=1_000_000.0, tie_word_embeddings=False, max_position_embeddings=context)
    default = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev), torch.no_grad():
            hf_model = Qwen3ForCausalLM(hf).eval()
    finally:
        torch.set_default_dtype(default)
    dec = D.Decoder(hf_model, 1, context)
    g = torch.Generator(device=dev).manual_seed(17)
    dec.cache.store.copy_(torch.randn(dec.cache.store.shape, generator=g, device=dev).to(torch.bfloat16))
    dec.position.fill_(context - 1)
    dec.token_ids.fill_(1234)
    with torch.no_grad():
        graph = capture(dec.step)
    us = time_graph(graph, reps=10)
    lb = layer_bytes(cfg, 1)
    kv = 2 * cfg["layers"] * cfg["kv_heads"] * context * cfg["head_dim"] * 2
    byts = cfg["layers"] * sum(lb.values()) + head_bytes(cfg, 1) + kv + 2 * cfg["hidden"]
    del dec, hf_model, graph
    stage("whole decode step done")
    return {f"Qwen3-8B greedy decode step B=1 (transformers model through decode.py, attention over {context} "
            f"slots)": {**shape_entry(us, byts), "tokens_per_s": round(1e6 / us, 1)}}


#: One GPU's share of a Qwen3-8B layer under eight-way tensor parallelism: QKV by heads, O by its
#: input, gate/up by the intermediate rows, down by its input (the collectives are not part of this
#: build; each projection runs at its shard's real shape).
TP = 8


def shard_table(cfg, dev):
    """µs per layer of the TP = 8 shard projections (36 layers of distinct weights, one graph), at
    M = 1, 5 and 16, with the M = 1 pure-read floor of the same launches."""
    h, i = cfg["hidden"], cfg["inter"]
    qkv_n = (cfg["q_heads"] + 2 * cfg["kv_heads"]) * cfg["head_dim"] // TP
    q_in, i_s = cfg["q_heads"] * cfg["head_dim"] // TP, i // TP
    g = torch.Generator(device=dev).manual_seed(13)

    def mk(n, k):
        return (torch.randn((n, k), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    layers = [{"qkv": mk(qkv_n, h), "o": mk(h, q_in), "gate_up": mk(2 * i_s, h), "down": mk(h, i_s)}
              for _ in range(cfg["layers"])]
    gain = (1 + 0.1 * torch.randn((h,), generator=g, device=dev)).to(torch.bfloat16)
    out = {}
    for m in (1, 5, 16):
        x = torch.randn((m, h), generator=g, device=dev).to(torch.bfloat16)
        attn = torch.randn((m, q_in), generator=g, device=dev).to(torch.bfloat16)
        act = torch.randn((m, i_s), generator=g, device=dev).to(torch.bfloat16)

        def layer_set(x=x, attn=attn, act=act):
            for lw in layers:
                L.rms_norm_linear(x, gain, EPS, lw["qkv"])
                L.linear(attn, lw["o"])
                S.gate_up_swiglu(x, lw["gate_up"], gain, EPS)
                L.linear(act, lw["down"])
        graph = capture(layer_set)  # a new shape's first eager call selects its launch; no knob re-judging here
        us = time_graph(graph, reps=5) / cfg["layers"]
        del graph
        byts = ((2 * qkv_n * h + 2 * m * h + 2 * m * qkv_n + 2 * h) + (2 * h * q_in + 2 * m * q_in + 2 * m * h) +
                (2 * 2 * i_s * h + 2 * m * h + 2 * m * i_s + 2 * h) + (2 * h * i_s + 2 * m * i_s + 2 * m * h))
        entry = shape_entry(us, byts)
        if m == 1:
            floor_us = sum(read_floor([lw[key] for lw in layers], reps=3)[0] for key in ("qkv", "o", "gate_up", "down"))
            entry = {**entry, "read_floor_us": round(floor_us, 3), "over_floor_us": round(us - floor_us, 3)}
        out[f"TP{TP} shard 8B layer M={m} (QKV {qkv_n}x{h}, O {h}x{q_in}, gate/up 2x{i_s}x{h}, down {h}x{i_s})"] = entry
        stage(f"TP{TP} shard M={m} done")
    del layers
    return out


def attention_table(cfg, dev):
    """µs / GB/s / fraction of the HBM roofline of decode_attention over full caches (all slots valid),
    and of rope_attend (QK norm + RoPE + the cache write of the last slot in the attention's prologue)."""
    out = {}
    hq, hkv, d = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    for b, c, copies in ATTN_CASES:
        g = torch.Generator(device=dev).manual_seed(11)
        ks = [torch.randn((b, hkv, c, d), generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
        vs = [torch.randn((b, hkv, c, d), generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
        q = torch.randn((b, hq, 1, d), generator=g, device=dev).to(torch.bfloat16)
        pos = torch.tensor([c - 1], device=dev, dtype=torch.int64)
        graph = capture(lambda: [DA.decode_attention(q, k, v, pos, d ** -0.5) for k, v in zip(ks, vs)])
        us = time_graph(graph) / copies
        byts = 2 * b * hkv * c * d * 2 + 2 * 2 * b * hq * d
        out[f"attention 8B decode B={b} C={c}"] = shape_entry(us, byts)
        del graph
        packed = torch.randn((b, (hq + 2 * hkv) * d), generator=g, device=dev).to(torch.bfloat16)
        gain = _Norm((1 + 0.1 * torch.randn((d,), generator=g, device=dev)).to(torch.bfloat16), EPS)
        table = torch.randn((c, d), generator=g, device=dev).to(torch.bfloat16)
        graph = capture(lambda: [DA.rope_attend(packed, gain, gain, table, table, pos, k, v, hq, d ** -0.5)
                                 for k, v in zip(ks, vs)])
        us = time_graph(graph) / copies
        byts = 2 * b * hkv * (c - 1) * d * 2 + b * (hq + 2 * hkv) * d * 2 + 2 * b * hkv * d * 2 + 2 * b * hq * d
        out[f"attention 8B decode B={b} C={c}, QK norm + RoPE + cache write in the prologue"] = \
            shape_entry(us, byts)
        del ks, vs, graph
        stage(f"attention B={b} C={c} done")
    return out


if __name__ == "__main__":
    main()
