"""CPU-side checks of the decode attention: the planner's intervals cover every cache slot
once, the workspace matches the partials it holds, the C ABI rejects what the kernels do
not take before any launch, and the Python wrapper keeps the reference's assertions
(engine/kernels/decode_attention.py:229-237). No kernel runs here."""

import ctypes

import pytest
import torch

from kernels import _native
from kernels import decode_attention as A


def plan(b, hq, hkv, c, d, cfg=None, cus=256):
    return A.plan(b, hq, hkv, c, d, cfg, compute_units=cus)


@pytest.mark.parametrize("b,hq,hkv,c,d", [(1, 32, 8, 4096, 128), (1, 16, 8, 4096, 128), (16, 32, 8, 4096, 128),
                                          (1, 32, 8, 65, 128), (2, 8, 2, 65, 64), (1, 32, 8, 1, 128),
                                          (4, 32, 8, 2080, 128), (1, 32, 8, 32768, 128), (3, 40, 8, 777, 128)])
@pytest.mark.parametrize("splits", [0, 1, 3, 64, 1024])
def test_intervals_cover_every_slot_once(b, hq, hkv, c, d, splits):
    p = plan(b, hq, hkv, c, d, _native.AttnConfig(0, splits, 0, 0))
    assert p.splits >= 1 and p.chunk >= 1
    assert p.splits * p.chunk >= c > (p.splits - 1) * p.chunk  # no interval lies wholly past the cache
    assert p.grid == b * hkv * p.splits
    g = hq // hkv
    assert p.workspace_bytes == (b * hkv * p.splits * g * (d + 2) * 4 if p.splits > 1 else 0)
    if splits:
        assert p.chunk == -(-c // min(splits, c))  # the asked-for count, trimmed of intervals past the cache


def test_default_plan_for_qwen3_8b_decode():
    """About one workgroup per CU, and at least one load step per wave in every interval."""
    p = plan(1, 32, 8, 4096, 128)
    assert (p.kind, p.splits, p.chunk, p.waves, p.unroll, p.grid) == (_native.ATTN_QUAD, 32, 128, 4, 1, 256)
    p = plan(16, 32, 8, 4096, 128)
    assert (p.splits, p.chunk, p.grid) == (2, 2048, 256)
    for c in (1, 63, 64, 65, 100, 1000):  # short contexts: no more intervals than steps of 4 waves x 16 rows
        assert plan(1, 32, 8, c, 128).splits == min(32, -(-c // 64))


def test_kind_by_head_dim_and_group_size():
    """QUAD takes D = 128 with up to 4 query heads per KV head; ROWS the rest (D = 64, 5..8 heads)."""
    for g in range(1, 9):
        p = plan(1, 8 * g, 8, 1000, 128)
        assert p.kind == (_native.ATTN_QUAD if g <= 4 else _native.ATTN_ROWS)
        assert p.unroll == (1 if g <= 4 else 4 if g <= 6 else 2)
        assert plan(1, 8 * g, 8, 1000, 64).kind == _native.ATTN_ROWS
    assert plan(1, 64, 8, 1000, 128).unroll == 2  # 8 heads per KV head: fewer rows in flight


def test_unsupported_shapes_rejected():
    lib = _native.lib()
    out = _native.AttnPlan()
    st = lib.ftk_plan_decode_attention
    assert st(1, 32, 8, 100, 96, 256, None, ctypes.byref(out)) == _native.FTK_ERR_UNSUPPORTED  # dim
    assert st(1, 72, 8, 100, 128, 256, None, ctypes.byref(out)) == _native.FTK_ERR_UNSUPPORTED  # 9 per KV head
    assert st(1, 30, 8, 100, 128, 256, None, ctypes.byref(out)) == _native.FTK_ERR_INVALID  # Hq % Hkv
    assert st(0, 32, 8, 100, 128, 256, None, ctypes.byref(out)) == _native.FTK_ERR_INVALID
    assert st(1, 32, 8, 0, 128, 256, None, ctypes.byref(out)) == _native.FTK_ERR_INVALID
    def rejects(cfg, hq=32, d=128):
        return st(1, hq, 8, 4096, d, 256, ctypes.byref(cfg), ctypes.byref(out)) == _native.FTK_ERR_INVALID

    assert rejects(_native.AttnConfig(0, 1025, 0, 0))  # more intervals than the merge kernel takes
    assert rejects(_native.AttnConfig(0, 0, 3, 0))  # waves
    assert rejects(_native.AttnConfig(_native.ATTN_ROWS, 0, 4, 8))  # 8 rows in flight, 4 heads: too many registers
    assert rejects(_native.AttnConfig(_native.ATTN_QUAD, 0, 4, 3))  # QUAD: 1 or 2 units in flight ahead
    assert rejects(_native.AttnConfig(_native.ATTN_QUAD, 0, 0, 0), d=64)  # QUAD: D = 128 only
    assert rejects(_native.AttnConfig(_native.ATTN_QUAD, 0, 0, 0), hq=40)  # QUAD: up to 4 heads per KV head
    assert rejects(_native.AttnConfig(3, 0, 0, 0))  # no such kind
    fake = ctypes.c_void_p(16)
    call = lib.ftk_decode_attention_bf16
    assert call(None, fake, fake, fake, 1, fake, 1, 32, 8, 100, 128, 0.1, None, 0, None, None) == \
        _native.FTK_ERR_INVALID
    assert call(fake, fake, fake, fake, 3, fake, 2, 32, 8, 100, 128, 0.1, None, 0, None, None) == \
        _native.FTK_ERR_INVALID  # positions must be 1 or the batch
    odd = ctypes.c_void_p(18)
    assert call(odd, fake, fake, fake, 1, fake, 1, 32, 8, 100, 128, 0.1, None, 0, None, None) == \
        _native.FTK_ERR_UNSUPPORTED  # 16-byte alignment


def test_quad_needs_32_bit_cache_offsets():
    """QUAD addresses one (row, KV head) cache in 32-bit bytes: longer caches take ROWS."""
    out = _native.AttnPlan()
    assert plan(1, 32, 8, 16_000_000, 128).kind == _native.ATTN_QUAD
    assert plan(1, 32, 8, 1 << 24, 128).kind == _native.ATTN_ROWS
    quad = _native.AttnConfig(_native.ATTN_QUAD, 0, 0, 0)
    assert _native.lib().ftk_plan_decode_attention(1, 32, 8, 1 << 24, 128, 256, ctypes.byref(quad),
                                                   ctypes.byref(out)) == _native.FTK_ERR_UNSUPPORTED


def test_rope_entry_rejects_before_any_launch():
    call = _native.lib().ftk_rope_decode_attention_bf16
    f = ctypes.c_void_p(256)

    def run(packed=f, gain=f, cos=f, table=64, pos=f, positions=1, keys=f, out=f, b=1, hq=32, d=128, cfg=None):
        return call(packed, gain, gain, 1e-6, 1e-6, cos, cos, table, pos, positions, None, keys, keys, out, b, hq,
                    8, 64, d, 0.1, None, 0, cfg, None)

    assert run(packed=None) == _native.FTK_ERR_INVALID
    assert run(gain=None) == _native.FTK_ERR_INVALID
    assert run(table=0) == _native.FTK_ERR_INVALID
    assert run(pos=None) == _native.FTK_ERR_INVALID
    assert run(positions=2) == _native.FTK_ERR_INVALID  # 1 or the batch
    assert run(packed=ctypes.c_void_p(258)) == _native.FTK_ERR_UNSUPPORTED  # 16-byte alignment
    assert run(cos=ctypes.c_void_p(264)) == _native.FTK_ERR_UNSUPPORTED
    assert run(d=64) == _native.FTK_ERR_UNSUPPORTED  # QUAD only
    rows = _native.AttnConfig(_native.ATTN_ROWS, 0, 0, 0)
    assert run(cfg=ctypes.byref(rows)) == _native.FTK_ERR_UNSUPPORTED


def test_rope_wrapper_support_and_no_cpu_path():
    assert A.rope_attention_supported(32, 8, 128) and A.rope_attention_supported(8, 8, 128)
    assert not A.rope_attention_supported(40, 8, 128)  # five query heads per KV head
    assert not A.rope_attention_supported(32, 8, 64)
    assert not A.rope_attention_supported(32, 8, 128, _native.AttnConfig(_native.ATTN_ROWS, 0, 0, 0))
    assert A.rope_attention_supported(32, 8, 128, capacity=16_000_000)
    assert not A.rope_attention_supported(32, 8, 128, capacity=1 << 24)  # QUAD's 32-bit offsets

    class Norm:
        weight, variance_epsilon = torch.ones(128, dtype=torch.bfloat16), 1e-6

    k = torch.zeros(1, 8, 16, 128, dtype=torch.bfloat16)
    table = torch.zeros(16, 128, dtype=torch.bfloat16)
    packed = torch.zeros(1, 48 * 128, dtype=torch.bfloat16)
    pos = torch.zeros(1, dtype=torch.int64)
    with pytest.raises(ValueError, match="GPU"):
        A.rope_attend(packed, Norm, Norm, table, table, pos, k, k.clone(), 32, 0.1)
    with pytest.raises(AssertionError):
        A.rope_attend(packed[:, :-128], Norm, Norm, table, table, pos, k, k.clone(), 32, 0.1)  # width


def _args(b=1, hq=8, hkv=2, c=16, d=64, t=1):
    q = torch.zeros(b, hq, t, d, dtype=torch.bfloat16)
    k = torch.zeros(b, hkv, c, d, dtype=torch.bfloat16)
    return q, k, k.clone(), torch.zeros(1, dtype=torch.int64)


def test_wrapper_keeps_the_reference_assertions():
    q, k, v, pos = _args()
    with pytest.raises(AssertionError):
        A.decode_attention(torch.zeros(1, 8, 2, 64, dtype=torch.bfloat16), k, v, pos, 0.125)  # two tokens
    with pytest.raises(AssertionError):
        A.decode_attention(q.float(), k, v, pos, 0.125)
    with pytest.raises(AssertionError):
        A.decode_attention(q, k.transpose(2, 3), v, pos, 0.125)  # non-contiguous
    with pytest.raises(AssertionError):
        A.decode_attention(q, k, v, pos.int(), 0.125)
    with pytest.raises(AssertionError):
        A.decode_attention(*_args(d=96), 0.125)
    with pytest.raises(ValueError, match="per KV head"):
        A.decode_attention(*_args(hq=18, hkv=2), 0.125)
    with pytest.raises(ValueError, match="GPU"):
        A.decode_attention(q, k, v, pos, 0.125)  # CPU tensors: no fallback
