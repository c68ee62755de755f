"""CPU checks of the projection-chain planner (ftk_chain_plan / ftk_chain_shape): every stage of
the Qwen3-0.6B and Qwen3-8B layer stacks gets a built shape whose K split matches the stage's K,
the tile walk writes every output exactly once, and malformed stage lists are rejected before
anything touches a device."""

import ctypes

import pytest

from kernels import _native

CUS = 256
FAKE = 1 << 20  # a 256-byte-aligned stand-in address: the planner never dereferences it


def stage(n, k, epilogue=_native.EPI_STORE, source=-1, add_source=-1, after=-1, gamma=True, add=False):
    x = None if source >= 0 else FAKE
    return _native.ChainStage(FAKE, FAKE if gamma else None, x, FAKE if add else None, FAKE, n, k, epilogue,
                              source, add_source, after)


def layer_stack(hidden, inter, attn, qkv, layers, residual):
    out = []
    for i in range(layers):
        base = len(out)
        prev = base - 1 if i else -1
        out.append(stage(qkv, hidden, source=prev))
        out.append(stage(hidden, attn, gamma=False, after=base, add_source=prev if residual and i else -1,
                         add=residual and i == 0))
        out.append(stage(2 * inter, hidden, _native.EPI_SWIGLU, source=base + 1))
        out.append(stage(hidden, inter, gamma=False, source=base + 2, add_source=base + 1 if residual else -1))
    return out


def plan(stages, cus=CUS):
    n = len(stages)
    arr = (_native.ChainStage * n)(*stages)
    shapes, tiles = (ctypes.c_int * n)(), (ctypes.c_int * n)()
    status = _native.lib().ftk_chain_plan(arr, n, cus, shapes, tiles)
    return status, list(shapes), list(tiles)


def shape_of(sid):
    c, kw, rpw, epi = (ctypes.c_int() for _ in range(4))
    assert _native.lib().ftk_chain_shape(sid, ctypes.byref(c), ctypes.byref(kw), ctypes.byref(rpw),
                                         ctypes.byref(epi)) == _native.FTK_OK
    return c.value, kw.value, rpw.value, epi.value


@pytest.mark.parametrize("model", ["0.6B", "8B"])
@pytest.mark.parametrize("residual", [False, True])
def test_layer_stacks_plan_and_cover_every_output_once(model, residual):
    hidden, inter, attn, qkv = {"0.6B": (1024, 3072, 2048, 4096), "8B": (4096, 12288, 4096, 6144)}[model]
    stages = layer_stack(hidden, inter, attn, qkv, 3, residual)
    status, shapes, tiles = plan(stages)
    assert status == _native.FTK_OK
    for st, sid, t in zip(stages, shapes, tiles):
        c, kw, rpw, epi = shape_of(sid)
        assert epi == st.epilogue and st.K == 512 * c * kw
        groups = 16 // kw
        per_group = rpw // 2 if epi == _native.EPI_SWIGLU else rpw
        outputs = st.N // 2 if epi == _native.EPI_SWIGLU else st.N
        assert t == -(-outputs // (groups * per_group))
        assert -(-t // CUS) <= 8  # tiles per workgroup: their totals wait in LDS
        # the kernel's walk: workgroup b takes tiles b, b + grid, ...; output (tile, group, slot)
        counts = [0] * outputs
        for wg in range(CUS):
            for tile in range(wg, t, CUS):
                for g in range(groups):
                    for p in range(per_group):
                        col = (tile * groups + g) * per_group + p
                        if col < outputs:
                            counts[col] += 1
        assert all(v == 1 for v in counts)


def test_malformed_stage_lists_are_rejected():
    ok = [stage(4096, 1024), stage(1024, 2048, gamma=False, after=0)]
    assert plan(ok)[0] == _native.FTK_OK
    bad = {
        "source not earlier": [stage(4096, 1024, source=0)],
        "after not earlier": [stage(4096, 1024, after=1), stage(1024, 2048, gamma=False)],
        "K differs from the source's outputs": [stage(4096, 1024), stage(1024, 2048, source=0)],
        "odd SwiGLU rows": [stage(4095, 1024, _native.EPI_SWIGLU)],
        "residual with SwiGLU": [stage(4096, 1024, _native.EPI_SWIGLU, add=True)],
        "both x and source": [stage(4096, 1024), _native.ChainStage(FAKE, None, FAKE, None, None, 1024, 4096, 0, 0,
                                                                   -1, -1)],
        "neither x nor source": [_native.ChainStage(FAKE, None, None, None, None, 1024, 4096, 0, -1, -1, -1)],
        "residual width": [stage(4096, 1024), stage(1024, 2048, gamma=False, add_source=0)],
    }
    for why, stages in bad.items():
        assert plan(stages)[0] == _native.FTK_ERR_INVALID, why
    # K without a built shape, or past the LDS row
    assert plan([stage(1024, 1000)])[0] == _native.FTK_ERR_UNSUPPORTED
    assert plan([stage(1024, 16384)])[0] == _native.FTK_ERR_UNSUPPORTED
    assert plan([])[0] == _native.FTK_ERR_INVALID
    assert plan(ok, cus=0)[0] == _native.FTK_ERR_INVALID
