"""GPU parity of decode attention with the Q/K head norm + RoPE + cache update in its prologue
(kernels/decode_attention.py ``rope_attend``, ftk_rope_decode_attention_bf16).

Against the CPU oracle composed as the reference composes the two launches
(engine/layers.py:51-55 then :76): oracle/rope.py ``qk_rope_cache`` (decode
form, whole tables, per-row phases), then oracle/attention.py
``decode_attention`` for each row:
- the output within |y - ref| <= 2e-2 + 1e-2|ref|;
- the written key slot within one BF16 ulp of the oracle's and >= 99 %
  bit-equal (the head's sum of squares associates differently), the value
  slot bit-exact, every other cache slot untouched, bit for bit.
Against this library's own two launches (qk_rope_cache, then attend) on the
same inputs: outputs within one BF16 ulp (or 2^-8), caches as above.
Positions cover the first slot, load-unit and split boundaries, the last slot
and one past the cache (nothing written, every slot read); stale NaN sits in
every slot from the position on, the step's own slot included.
"""

import numpy as np
import pytest
import torch

from conftest import to_bits
from oracle import attention, rope
from test_gpu_attention import cfg, one_ulp, within
from test_oracle_rope import _tables

from kernels import _native
from kernels import decode_attention as A
from kernels import qk_rope as R

pytestmark = pytest.mark.gpu

D, EPS = 128, 1e-6


class Norm:
    def __init__(self, weight, eps):
        self.weight, self.variance_epsilon = weight, eps


def _case(b, hq, hkv, cap, positions, seed, device, table_rows=None, shifts=None):
    g = torch.Generator().manual_seed(seed)
    packed = (torch.randn(b, (hq + 2 * hkv) * D, generator=g) * 2).to(torch.bfloat16)
    qg = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kg = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    keys = torch.randn(b, hkv, cap, D, generator=g).to(torch.bfloat16)
    values = torch.randn(b, hkv, cap, D, generator=g).to(torch.bfloat16)
    rows = positions if len(positions) == b else positions * b
    for i, p in enumerate(rows):  # stale slots from the position on, the step's own slot too
        keys[i, :, p:] = float("nan")
        values[i, :, p:] = float("nan")
    cos, sin = _tables(list(range(table_rows or cap + 8)), D)
    phases = torch.tensor(shifts if shifts is not None else [0] * b, dtype=torch.int64).reshape(b, 1)
    position = torch.tensor(positions, dtype=torch.int64)
    return {k: v.to(device) for k, v in dict(packed=packed, qg=qg, kg=kg, keys=keys, values=values, cos=cos,
                                              sin=sin, phases=phases, position=position).items()}


def _oracle(c, hq, scale):
    """(output bits [B, Hq, D], key bits, value bits) of the two steps the fused launch replaces."""
    packed, keys, values = to_bits(c["packed"]), to_bits(c["keys"]), to_bits(c["values"])
    b, hkv, cap, _ = keys.shape
    rows = np.broadcast_to(c["position"].cpu().numpy(), (b,)).copy()
    reach = max(cap, int(rows.max()) + 1)  # a position past the cache writes into padding, cut off below
    pad = np.zeros((b, hkv, reach, D), np.uint16)
    kp, vp = pad.copy(), pad.copy()
    kp[:, :, :cap], vp[:, :, :cap] = keys, values
    q, kp, vp = rope.qk_rope_cache(packed.reshape(b, 1, -1), 1, to_bits(c["qg"]), to_bits(c["kg"]), EPS, EPS,
                                   to_bits(c["cos"]), to_bits(c["sin"]), rows, kp, vp, hq, rows=True,
                                   phases=c["phases"].cpu().numpy())
    kk, vv = kp[:, :, :cap], vp[:, :, :cap]
    out = np.stack([attention.decode_attention(q[i:i + 1, 0], kk[i:i + 1], vv[i:i + 1], min(int(rows[i]), cap - 1),
                                               scale)[0] for i in range(b)])
    return out, kk, vv


def _fused(c, hq, scale, config=None):
    return A.rope_attend(c["packed"], Norm(c["qg"], EPS), Norm(c["kg"], EPS), c["cos"], c["sin"], c["position"],
                         c["keys"], c["values"], hq, scale, phases=c["phases"], config=config)


def _two_launches(c, hq, scale, config=None):
    b = c["packed"].shape[0]
    q = R.qk_rope_cache(c["packed"].view(b, 1, -1), Norm(c["qg"], EPS), Norm(c["kg"], EPS), c["cos"], c["sin"],
                        c["position"].expand(b).contiguous(), c["keys"], c["values"], hq, rows=True,
                        phases=c["phases"])
    return A.attend(q.reshape(b, hq, D), c["keys"], c["values"], c["position"], scale, config)


def _key_close(got_bits, want_bits):
    diff = np.abs(got_bits.astype(np.int32) - want_bits.astype(np.int32))
    return diff.max() <= 1 and np.mean(diff == 0) >= 0.99


def _check_caches(c, before_k, before_v, want_k, want_v):
    got_k, got_v = to_bits(c["keys"]), to_bits(c["values"])
    b, _, cap, _ = got_k.shape
    pos = np.broadcast_to(c["position"].cpu().numpy(), (b,))
    for i in range(b):
        p = int(pos[i])
        others = [s for s in range(cap) if s != p]
        np.testing.assert_array_equal(got_k[i][:, others], before_k[i][:, others])
        np.testing.assert_array_equal(got_v[i][:, others], before_v[i][:, others])
        if p < cap:
            assert _key_close(got_k[i][:, p], want_k[i][:, p])
            np.testing.assert_array_equal(got_v[i][:, p], want_v[i][:, p])


#: (batch, Hq, Hkv, capacity, positions [1] or [B], RoPE phase shifts or None)
CASES = [
    (1, 32, 8, 4096, [0], None),
    (1, 32, 8, 4096, [1], None),
    (1, 32, 8, 4096, [15], None),
    (1, 32, 8, 4096, [16], None),
    (1, 32, 8, 4096, [127], None),
    (1, 32, 8, 4096, [128], None),
    (1, 32, 8, 4096, [129], None),
    (1, 32, 8, 4096, [2050], None),
    (1, 32, 8, 4096, [4095], None),
    (1, 32, 8, 4096, [4096], None),
    (3, 32, 8, 1000, [0, 517, 999], [0, 3, 1]),
    (3, 32, 8, 1000, [400], None),
    (2, 8, 8, 300, [5, 299], None),
    (1, 16, 8, 1000, [517], [5]),
    (3, 24, 8, 700, [0, 350, 699], None),
    (2, 8, 4, 64, [63, 64], None),
]


def _ids():
    return [f"b{b}-h{hq}x{hkv}-c{cap}-p{'_'.join(map(str, pos))}" + ("-ph" if sh else "")
            for b, hq, hkv, cap, pos, sh in CASES]


@pytest.mark.parametrize("b,hq,hkv,cap,positions,shifts", CASES, ids=_ids())
def test_matches_the_oracle(cuda, b, hq, hkv, cap, positions, shifts):
    scale = D ** -0.5
    c = _case(b, hq, hkv, cap, positions, seed=31 * cap + hq + positions[0], device=cuda, shifts=shifts)
    before_k, before_v = to_bits(c["keys"]), to_bits(c["values"])
    want, want_k, want_v = _oracle(c, hq, scale)
    got = _fused(c, hq, scale)
    torch.cuda.synchronize()
    assert got.shape == (b, 1, hq, D)
    g = to_bits(got).reshape(b, hq, D)
    assert not np.isnan(got.float().cpu().numpy()).any()
    assert within(g, want)
    _check_caches(c, before_k, before_v, want_k, want_v)


@pytest.mark.parametrize("config", [None, cfg(splits=1), cfg(splits=7), cfg(splits=64), cfg(waves=8),
                                    cfg(unroll=2), cfg(waves=8, unroll=2, splits=3)],
                         ids=["default", "s1", "s7", "s64", "w8", "u2", "w8u2s3"])
@pytest.mark.parametrize("positions", [[0], [33], [1999]])
def test_matches_the_two_launches(cuda, config, positions):
    """Same inputs through qk_rope_cache + attend: one BF16 ulp apart at most, caches alike."""
    b, hq, hkv, cap, scale = 2, 32, 8, 2000, D ** -0.5
    cf = _case(b, hq, hkv, cap, positions, seed=900 + positions[0], device=cuda)
    c2 = {k: v.clone() for k, v in cf.items()}
    got = _fused(cf, hq, scale, config)
    want = _two_launches(c2, hq, scale, config)
    torch.cuda.synchronize()
    assert one_ulp(to_bits(got), to_bits(want))
    assert _key_close(to_bits(cf["keys"]), to_bits(c2["keys"]))
    np.testing.assert_array_equal(to_bits(cf["values"]), to_bits(c2["values"]))


def test_phase_outside_the_table_writes_nothing(cuda):
    b, hq, hkv, cap = 2, 32, 8, 256
    c = _case(b, hq, hkv, cap, [10, 200], seed=77, device=cuda, table_rows=cap, shifts=[0, 60])
    before_k, before_v = to_bits(c["keys"]), to_bits(c["values"])
    want, want_k, want_v = _oracle({**c, "packed": c["packed"][:1], "keys": c["keys"][:1], "values": c["values"][:1],
                                    "position": c["position"][:1], "phases": c["phases"][:1]}, hq, D ** -0.5)
    got = _fused(c, hq, D ** -0.5)
    torch.cuda.synchronize()
    assert within(to_bits(got)[0, 0], want[0])  # row 0 is whole
    k, v = to_bits(c["keys"]), to_bits(c["values"])
    np.testing.assert_array_equal(k[1], before_k[1])  # row 1 rotates at 260 > 255: no slot written
    np.testing.assert_array_equal(v[1], before_v[1])
    assert _key_close(k[0][:, 10], want_k[0][:, 10])


def test_graph_replays_match_eager(cuda):
    b, hq, hkv, cap, scale = 2, 32, 8, 512, D ** -0.5
    c = _case(b, hq, hkv, cap, [100, 300], seed=5, device=cuda)
    ce = {k: v.clone() for k, v in c.items()}
    eager = _fused(ce, hq, scale)
    first_k = to_bits(c["keys"])  # bits: the stale slots hold NaN
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = _fused(c, hq, scale)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_bits(c["keys"]), first_k)  # capture launches nothing
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        np.testing.assert_array_equal(to_bits(c["keys"]), to_bits(ce["keys"]))
        np.testing.assert_array_equal(to_bits(c["values"]), to_bits(ce["values"]))
        torch.cuda.synchronize()


def test_rejects_what_it_does_not_take(cuda):
    scale = D ** -0.5
    with pytest.raises(ValueError):  # five query heads per KV head
        _fused(_case(1, 40, 8, 64, [3], seed=2, device=cuda), 40, scale)
    c = _case(1, 32, 8, 64, [3], seed=1, device=cuda)
    with pytest.raises(ValueError):  # the ROWS kind has no RoPE prologue
        _fused(c, 32, scale, config=cfg(kind=_native.ATTN_ROWS))
    big = torch.empty(c["packed"].numel() + 1, device=cuda, dtype=torch.bfloat16)
    odd = big[1:].view_as(c["packed"])
    odd.copy_(c["packed"])
    with pytest.raises(ValueError):  # 2-byte aligned rows
        _fused({**c, "packed": odd}, 32, scale)
