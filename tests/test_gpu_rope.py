"""GPU parity of the Q/K head norm + RoPE + KV-cache update (kernels/qk_rope.py, ftk_qk_rope_cache_bf16).

Against the CPU oracle (oracle/rope.py) on the same seeded inputs: the query
and the written key slots within one BF16 ulp and >= 99.9 % bit-equal (the sum
of squares associates differently, which can move inv_std by an ulp); the value
slots bit-exact; every other cache slot untouched, bit for bit.
"""

import numpy as np
import pytest
import torch

from conftest import to_bits
from oracle import rope
from test_oracle_rope import _tables

from kernels import qk_rope as R
from kernels.merged import Split

pytestmark = pytest.mark.gpu


class Norm:
    def __init__(self, weight, eps):
        self.weight, self.variance_epsilon = weight, eps


def _case(b, t, hq, hkv, d, cap, seed, device):
    g = torch.Generator().manual_seed(seed)
    packed = (torch.randn(b, t, (hq + 2 * hkv) * d, generator=g) * 2).to(torch.bfloat16)
    qg = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kg = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    keys = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16)
    values = torch.randn(b, hkv, cap, d, generator=g).to(torch.bfloat16)
    return [x.to(device) for x in (packed, qg, kg, keys, values)]


def _close(got_bits, want_bits):
    diff = np.abs(got_bits.astype(np.int32) - want_bits.astype(np.int32))
    return diff.max() <= 1 and np.mean(diff == 0) >= 0.999


def _check(q, keys, values, want):
    wq, wk, wv = want
    assert _close(to_bits(q.transpose(1, 2)), wq)
    assert _close(to_bits(keys), wk)
    np.testing.assert_array_equal(to_bits(values), wv)


@pytest.mark.parametrize("b,t,hq,hkv,d", [(1, 1, 32, 8, 128), (4, 1, 32, 8, 128), (1, 1, 16, 8, 128),
                                          (2, 3, 8, 2, 64), (3, 2, 40, 8, 128)])
def test_decode_matches_oracle(cuda, b, t, hq, hkv, d):
    cap, pos = 64, 29
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=hq + d + b, device=cuda)
    cos, sin = (x[None].to(cuda) for x in _tables([pos + i for i in range(t)], d))
    want = rope.qk_rope_cache(to_bits(packed), 1, to_bits(qg), to_bits(kg), 1e-6, 1e-6, to_bits(cos), to_bits(sin),
                              [pos], to_bits(keys), to_bits(values), hq)
    position = torch.tensor([pos], device=cuda, dtype=torch.int64)
    q = R.qk_rope_cache(packed, Norm(qg, 1e-6), Norm(kg, 1e-6), cos, sin, position, keys, values, hq)
    assert q.shape == (b, hq, t, d)
    _check(q, keys, values, want)


def test_rows_and_table_modes(cuda):
    b, t, hq, hkv, d, cap = 3, 2, 32, 8, 128, 48
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=3, device=cuda)
    pos = [4, 30, 17]
    full_cos, full_sin = (x.to(cuda) for x in _tables(list(range(cap)), d))
    idx = [p + i for p in pos for i in range(t)]
    cos, sin = full_cos[idx].reshape(b, t, d).contiguous(), full_sin[idx].reshape(b, t, d).contiguous()
    want = rope.qk_rope_cache(to_bits(packed), 1, to_bits(qg), to_bits(kg), 1e-6, 2e-6, to_bits(cos), to_bits(sin),
                              pos, to_bits(keys), to_bits(values), hq, rows=True)
    position = torch.tensor(pos, device=cuda, dtype=torch.int64)
    k1, v1 = keys.clone(), values.clone()
    q = R.qk_rope_cache(packed, Norm(qg, 1e-6), Norm(kg, 2e-6), cos, sin, position, k1, v1, hq, rows=True)
    _check(q, k1, v1, want)
    phases = torch.arange(t, device=cuda, dtype=torch.int64).repeat(b, 1).contiguous()
    k2, v2 = keys.clone(), values.clone()
    q2 = R.qk_rope_cache(packed, Norm(qg, 1e-6), Norm(kg, 2e-6), full_cos, full_sin, position, k2, v2, hq,
                         rows=True, phases=phases)
    assert torch.equal(q2, q) and torch.equal(k2, k1) and torch.equal(v2, v1)


def test_prefill_writes_the_first_slots(cuda):
    b, t, hq, hkv, d, cap = 2, 5, 16, 8, 128, 12
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=4, device=cuda)
    cos, sin = (x[None].to(cuda) for x in _tables(list(range(t)), d))
    want = rope.qk_rope_cache(to_bits(packed), 1, to_bits(qg), to_bits(kg), 1e-6, 1e-6, to_bits(cos), to_bits(sin),
                              list(range(t)), to_bits(keys), to_bits(values), hq, prefill=True)
    position = torch.arange(t, device=cuda, dtype=torch.int64)
    q = R.qk_rope_cache(packed, Norm(qg, 1e-6), Norm(kg, 1e-6), cos, sin, position, keys, values, hq, prefill=True)
    _check(q, keys, values, want)


def test_split_partials(cuda):
    b, t, hq, hkv, d, cap = 2, 1, 32, 8, 128, 16
    _, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=5, device=cuda)
    g = torch.Generator().manual_seed(6)
    n = (hq + 2 * hkv) * d
    partial = torch.randn(3, b * t, n, generator=g).to(cuda)
    cos, sin = (x[None].to(cuda) for x in _tables([7], d))
    want = rope.qk_rope_cache(partial.cpu().numpy().reshape(3, b, t, n), 3, to_bits(qg), to_bits(kg), 1e-6, 1e-6,
                              to_bits(cos), to_bits(sin), [7], to_bits(keys), to_bits(values), hq)
    position = torch.tensor([7], device=cuda, dtype=torch.int64)
    q = R.qk_rope_cache(Split(partial, (b, t, n)), Norm(qg, 1e-6), Norm(kg, 1e-6), cos, sin, position, keys, values,
                        hq)
    _check(q, keys, values, want)


def test_slot_past_the_cache_is_skipped(cuda):
    b, t, hq, hkv, d, cap = 1, 1, 32, 8, 128, 16
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=7, device=cuda)
    cos, sin = (x[None].to(cuda) for x in _tables([16], d))
    k0, v0 = keys.clone(), values.clone()
    position = torch.tensor([cap], device=cuda, dtype=torch.int64)  # one past the last slot
    R.qk_rope_cache(packed, Norm(qg, 1e-6), Norm(kg, 1e-6), cos, sin, position, keys, values, hq)
    assert torch.equal(keys, k0) and torch.equal(values, v0)


def test_graph_replays_follow_the_device_position(cuda):
    b, t, hq, hkv, d, cap = 1, 1, 32, 8, 128, 40
    packed, qg, kg, keys, values = _case(b, t, hq, hkv, d, cap, seed=8, device=cuda)
    cos, sin = (x[None].to(cuda).contiguous() for x in _tables([0], d))
    position = torch.tensor([0], device=cuda, dtype=torch.int64)
    norms = (Norm(qg, 1e-6), Norm(kg, 1e-6))
    R.qk_rope_cache(packed, *norms, cos, sin, position, keys, values, hq)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            q = R.qk_rope_cache(packed, *norms, cos, sin, position, keys, values, hq)
    torch.cuda.synchronize()
    for pos in (3, 39, 11):
        before = keys.clone()
        position.fill_(pos)
        graph.replay()
        torch.cuda.synchronize()
        want = rope.qk_rope_cache(to_bits(packed), 1, to_bits(qg), to_bits(kg), 1e-6, 1e-6, to_bits(cos),
                                  to_bits(sin), [pos], to_bits(before), to_bits(values), hq)
        assert _close(to_bits(q.transpose(1, 2)), want[0])
        assert _close(to_bits(keys), want[1])
