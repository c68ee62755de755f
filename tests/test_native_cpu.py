"""CPU-side checks of libftk.so: it loads, exports every entry point of include/ftk.h,
validates arguments before touching a device, and its launch plans cover every
output exactly once with in-bounds weight rows (replayed with the kernels' own
index functions). No kernel runs here."""

import ctypes
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT

from kernels import _native

HEADER = ROOT / "include" / "ftk.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(ftk_\w+)\(", text, re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    names = declared()
    assert len(names) >= 15
    lib = _native.lib()
    for name in names:
        assert hasattr(lib, name), name
    # and nm agrees: every declared name is a dynamic text symbol
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (ftk_\w+)", out))
    assert set(names) <= exported


def test_binding_signatures_cover_header():
    assert set(declared()) == set(_native.SIGNATURES)


def test_version_and_status_strings():
    lib = _native.lib()
    assert b"gfx950" in lib.ftk_version()
    for code in range(6):
        assert lib.ftk_status_string(code) != b"unknown status"
    assert lib.ftk_argmax_workspace_bytes(1, 8192) == 8
    assert lib.ftk_argmax_workspace_bytes(32, 151936) == 8 * 32 * 19


def test_persistent_programs_in_the_library_known_answers():
    """The planner's own persistent_programs (csrc/ftk_plan.h, exported as ftk_persistent_programs)
    against the reference's known answers (engine/kernels/gemm.py:333-335, 132 SMs) and the oracle."""
    from oracle import helpers

    lib = _native.lib()
    assert lib.ftk_persistent_programs(304, 132) == 102
    assert lib.ftk_persistent_programs(2374, 132) == 132
    for tiles in (1, 17, 131, 132):
        assert lib.ftk_persistent_programs(tiles, 132) == tiles
    assert lib.ftk_persistent_programs(0, 132) == 0 and lib.ftk_persistent_programs(5, 0) == 0
    for tiles in range(1, 3000, 37):
        for units in (132, 256, 304):
            assert lib.ftk_persistent_programs(tiles, units) == helpers.persistent_programs(tiles, units)


def test_ring_tile_mapping_covers_every_tile_once():
    """The RING kernels' tile of each (workgroup, step) (csrc/ftk_plan.h ring_tile): every tile
    exactly once; in a full round of a grid that is a multiple of 8, the workgroups of one XCD
    (wg % 8) hold one contiguous run of grid / 8 tiles, in workgroup order; otherwise wg + step grid."""
    lib = _native.lib()
    for tiles, grid in ((1536, 256), (512, 256), (256, 256), (9496, 500), (9496, 504), (1000, 256), (300, 192), (77, 40),
                        (263, 256), (10, 3), (384, 192)):
        seen = []
        for wg in range(grid):
            steps = (tiles - wg + grid - 1) // grid
            for step in range(steps):
                t = lib.ftk_ring_tile(wg, step, grid, tiles)
                seen.append(t)
                full = (step + 1) * grid <= tiles
                if grid % 8 == 0 and full:
                    per = grid // 8
                    assert t == step * grid + per * (wg % 8) + wg // 8, (tiles, grid, wg, step)
                else:
                    assert t == wg + step * grid, (tiles, grid, wg, step)
            assert lib.ftk_ring_tile(wg, steps, grid, tiles) == -1
        assert sorted(seen) == list(range(tiles)), (tiles, grid)
    assert lib.ftk_ring_tile(0, 0, 0, 10) == -1 and lib.ftk_ring_tile(5, 0, 4, 10) == -1


def test_invalid_arguments_rejected_before_any_launch():
    lib = _native.lib()
    assert lib.ftk_linear_bf16(None, None, None, 1, 8, 8, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_rms_norm_linear_bf16(None, None, 1e-6, None, None, 1, 8, 8, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_rms_norm_bf16(None, 8, None, None, 1, 8, 1e-6, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_swiglu_bf16(None, 0, 0, None, 1, 8, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_merge_splits_bf16(None, 1, 8, None, None) == _native.FTK_ERR_INVALID
    fake = ctypes.c_void_p(16)
    # argmax without a workspace
    assert lib.ftk_argmax_bf16(fake, 1, 8, fake, 8, None, None, 0, None) == _native.FTK_ERR_WORKSPACE
    # a fused argmax projection without its key workspace
    assert lib.ftk_project_bf16(fake, None, 0.0, fake, None, 1, 64, 64, _native.EPI_ARGMAX, fake, 8, None, None, 0,
                                None, None) in (_native.FTK_ERR_WORKSPACE, _native.FTK_ERR_HIP)
    assert lib.ftk_argmax_bf16(fake, 1, 8, fake, 3, None, fake, 64, None) == _native.FTK_ERR_INVALID
    # the epilogue's residual add needs a residual, and y may overlap only the residual itself
    x, w, r, y = (ctypes.c_void_p(a) for a in (1 << 16, 1 << 18, 1 << 20, 1 << 22))
    assert lib.ftk_project_add_bf16(x, w, None, y, 1, 64, 64, None, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_project_add_bf16(x, w, r, None, 1, 64, 64, None, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_project_add_bf16(x, w, r, ctypes.c_void_p((1 << 20) + 2), 1, 64, 64, None, None) \
        == _native.FTK_ERR_INVALID
    assert lib.ftk_project_add_bf16(x, w, r, ctypes.c_void_p((1 << 16) + 64), 1, 64, 64, None, None) \
        == _native.FTK_ERR_INVALID
    # the prologue's stored rows may not alias its inputs or outputs, and need the norm
    buf = ctypes.c_void_p(4096)
    rows = _native.Rows(buf, buf, None, 0)
    assert lib.ftk_project_rows_bf16(fake, ctypes.byref(rows), fake, 1e-6, fake, ctypes.c_void_p(1 << 20), 1, 64, 64,
                                     0, None, 0, None, None, 0, None, None) == _native.FTK_ERR_INVALID
    rows = _native.Rows(buf, ctypes.c_void_p(8192), None, 0)
    assert lib.ftk_project_rows_bf16(fake, ctypes.byref(rows), None, 1e-6, fake, ctypes.c_void_p(1 << 20), 1, 64, 64,
                                     0, None, 0, None, None, 0, None, None) == _native.FTK_ERR_INVALID
    rows = _native.Rows(None, None, fake, 3, 16)
    assert lib.ftk_project_rows_bf16(fake, ctypes.byref(rows), fake, 1e-6, fake, ctypes.c_void_p(1 << 20), 1, 64, 64,
                                     0, None, 0, None, None, 0, None, None) == _native.FTK_ERR_INVALID
    # gathered rows need the table's row count (the device clamps ids into it)
    for table_rows in (0, -1):
        rows = _native.Rows(None, None, fake, 8, table_rows)
        assert lib.ftk_project_rows_bf16(fake, ctypes.byref(rows), fake, 1e-6, fake, ctypes.c_void_p(1 << 20), 1, 64,
                                         64, 0, None, 0, None, None, 0, None, None) == _native.FTK_ERR_INVALID
    # the norm's sums of squares: sumsq feeds a norm (gamma) that reads x as it is; sumsq_out is
    # written by the STORE epilogue, 4-byte aligned, clear of the call's other buffers
    sq, y = ctypes.c_void_p(1 << 24), ctypes.c_void_p(1 << 20)

    def rows_call(rows, gamma, epi=0):
        return lib.ftk_project_rows_bf16(fake, ctypes.byref(rows), gamma, 1e-6, fake, y, 8, 64, 64, epi, None, 0,
                                         None, None, 0, None, None)

    assert rows_call(_native.Rows(None, None, None, 0, 0, sq, None), None) == _native.FTK_ERR_INVALID
    assert rows_call(_native.Rows(buf, None, None, 0, 0, sq, None), fake) == _native.FTK_ERR_INVALID
    assert rows_call(_native.Rows(None, None, fake, 8, 16, sq, None), fake) == _native.FTK_ERR_INVALID
    assert rows_call(_native.Rows(None, None, None, 0, 0, ctypes.c_void_p((1 << 24) + 8), None), fake) \
        == _native.FTK_ERR_UNSUPPORTED  # sums read in 16-byte pieces
    assert rows_call(_native.Rows(None, None, None, 0, 0, None, sq), None, _native.EPI_SWIGLU) \
        == _native.FTK_ERR_UNSUPPORTED
    assert rows_call(_native.Rows(None, None, None, 0, 0, None, ctypes.c_void_p((1 << 24) + 2)), None) \
        == _native.FTK_ERR_INVALID
    assert rows_call(_native.Rows(None, None, None, 0, 0, None, ctypes.c_void_p((1 << 20) + 64)), None) \
        == _native.FTK_ERR_INVALID  # inside y
    # the residual-add form takes sumsq_out only
    for rows in (_native.Rows(buf, None, None, 0, 0, None, sq), _native.Rows(None, None, None, 0, 0, sq, None)):
        assert lib.ftk_project_add_rows_bf16(x, ctypes.byref(rows), w, r, y, 1, 64, 64, None, None) \
            == _native.FTK_ERR_INVALID
    assert lib.ftk_embed_rms_norm_bf16(fake, 3, fake, fake, fake, fake, 1, 8, 1e-6, None) == _native.FTK_ERR_INVALID
    # the streaming-read reference: whole 16-byte chunks, an aligned source, a sink, a built window
    assert lib.ftk_stream_read(fake, 24, fake, 1, 4, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_stream_read(ctypes.c_void_p(18), 32, fake, 1, 4, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_stream_read(fake, 32, None, 1, 4, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_stream_read(fake, 32, fake, -1, 4, None) == _native.FTK_ERR_INVALID
    assert lib.ftk_stream_read(fake, 32, fake, 1, 3, None) == _native.FTK_ERR_INVALID


@pytest.mark.parametrize("m", [0, 33])
def test_rows_outside_one_to_max_rows_rejected(m):
    p = _native.Plan()
    assert _native.lib().ftk_plan_project(m, 64, 64, 0, 256, None, p) == _native.FTK_ERR_INVALID


SHAPES = [
    # Qwen3-0.6B and Qwen3-8B projections (N, K) plus lm_head, and the reference's ragged test shapes
    (4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072),
    (6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288), (151936, 4096),
    (200, 300), (130, 517), (173, 259), (257, 512), (127, 256), (70, 264),
]


def _coverage(plan, n, epilogue):
    outputs = n // 2 if epilogue == _native.EPI_SWIGLU else n
    counts = (ctypes.c_int32 * outputs)()
    max_row = ctypes.c_int64()
    _native.call("ftk_plan_coverage", plan, n, epilogue, counts, outputs, ctypes.byref(max_row))
    return np.frombuffer(counts, dtype=np.int32), max_row.value


#: (rows per group, chunks per lane C, KW) the STREAM kind instantiates (K = 512 C KW), for
#: M <= 4 and for the 8-row kernel (M = 5..8).
STREAM_SHAPES = ((2, 1, 2), (4, 1, 2), (8, 1, 2), (2, 1, 4), (4, 1, 4), (2, 3, 2), (4, 3, 2), (2, 2, 4), (4, 2, 4),
                 (8, 2, 4), (2, 6, 4), (4, 6, 4), (2, 3, 8))
STREAM_SHAPES_8 = ((2, 2, 4), (4, 2, 4), (2, 3, 8), (4, 3, 8))


def _stream_status(m, k, rpw, kw):
    if m > 8 or k % (512 * kw):
        return _native.FTK_ERR_UNSUPPORTED
    shapes = STREAM_SHAPES if m <= 4 else STREAM_SHAPES_8
    return _native.FTK_OK if (rpw, k // (512 * kw), kw) in shapes else _native.FTK_ERR_INVALID


#: (T, S, KW, U) the MFMA_STREAM kind instantiates (K = 32 S KW), by epilogue, without the prologue.
MSTREAM_EVEN = ((2, 8, 16, 4), (2, 16, 8, 4), (2, 16, 8, 8), (2, 16, 8, 16), (2, 8, 16, 8))
MSTREAM_ONE = ((1, 8, 16, 4), (1, 8, 16, 8), (1, 16, 8, 4), (1, 16, 8, 8), (1, 16, 8, 16), (1, 24, 16, 2),
               (1, 24, 16, 6), (1, 48, 8, 16))


def _mstream_shapes(epilogue):
    return MSTREAM_EVEN + (() if epilogue == _native.EPI_SWIGLU else MSTREAM_ONE)


def _mstream_status(m, k, epilogue, t, kw, u):
    if m > 16 or k % (32 * kw):
        return _native.FTK_ERR_UNSUPPORTED
    return _native.FTK_OK if (t, k // (32 * kw), kw, u) in _mstream_shapes(epilogue) else _native.FTK_ERR_INVALID


#: (row sets RS, segments per lane C, KW) the QUAD kind may build (K = 128 C KW); single row sets
#: only for store / argmax. A shape is built for a row count only where it fits the registers.
QUAD_SHAPES = ((2, 8, 4), (4, 8, 4), (2, 4, 8), (4, 4, 8), (6, 4, 8), (2, 12, 8), (2, 6, 16), (2, 2, 4), (2, 4, 4),
               (2, 6, 4))
QUAD_ONE = ((1, 8, 4), (1, 4, 8), (1, 12, 8))


def _quad_fits(mq, rs, c, kw, pro):
    """The register estimate of the QUAD kind (x slice, weight window, accumulators, prologue inputs)."""
    cap = 128 if kw >= 16 else 248
    main_loop = 4 * mq * c + 4 * rs * c + 4 * rs * mq + 32
    if not pro:
        return main_loop <= cap
    first_tile = main_loop + 4 * c + 24  # the gain lives through the first tile (normalised there)
    late = main_loop + 6 * mq * c + 4 * c > cap  # the window waits for the prologue
    prologue = 10 * mq * c + 4 * c + 32 if late else main_loop + 6 * mq * c + 4 * c
    return max(first_tile, prologue) <= cap


def _quad_status(m, k, epilogue, rows, kw, pro=False):
    if m > 16 or k % (128 * kw):
        return _native.FTK_ERR_UNSUPPORTED
    mq = 1 if m <= 4 else 2 if m <= 8 else 4
    c, rs = k // (128 * kw), rows // 4
    shapes = QUAD_SHAPES + (() if epilogue == _native.EPI_SWIGLU else QUAD_ONE)
    ok = rows % 4 == 0 and (rs, c, kw) in shapes and _quad_fits(mq, rs, c, kw, pro)
    return _native.FTK_OK if ok else _native.FTK_ERR_INVALID


#: (T, C, KW, U) the STAGE kind instantiates (K = 128 C KW): every epilogue, both prologue settings ...
STAGE_EVEN = ((2, 4, 8, 2), (2, 4, 8, 4))
#: ... store / argmax only, and the long K without the prologue.
STAGE_ONE = ((1, 4, 8, 2), (1, 4, 8, 4))
STAGE_LONG = ((1, 12, 8, 3), (1, 12, 8, 4))


def _stage_status(m, k, epilogue, t, kw, u, pro=False):
    if m > 16 or k % (128 * kw):
        return _native.FTK_ERR_UNSUPPORTED
    shapes = STAGE_EVEN + (() if epilogue == _native.EPI_SWIGLU else STAGE_ONE + (() if pro else STAGE_LONG))
    return _native.FTK_OK if (t, k // (128 * kw), kw, u) in shapes else _native.FTK_ERR_INVALID


#: (C, KW, D, pro) the RING kind is built for (NX follows M: 8 x rows up to M = 8, else 16)
RING_SHAPES = ((4, 8, 2),)
RING_LONG = ((12, 8, 2), (12, 8, 3))


def _ring_status(m, k, epilogue, kw, d, pro=False, rows=16):
    if not 1 <= m <= 16 or k % (128 * kw):
        return _native.FTK_ERR_UNSUPPORTED
    c = k // (128 * kw)
    if rows == 24:  # 24-row tiles: STORE, up to 8 x rows, C = 4
        ok = epilogue == _native.EPI_STORE and m <= 8 and (c, kw, d) == (4, 8, 2)
        return _native.FTK_OK if ok else _native.FTK_ERR_INVALID
    if rows == 12:  # 12-row tiles: STORE, any row count, C = 4
        ok = epilogue == _native.EPI_STORE and (c, kw, d) == (4, 8, 2)
        return _native.FTK_OK if ok else _native.FTK_ERR_INVALID
    shapes = RING_SHAPES + (RING_LONG if not pro and epilogue == _native.EPI_STORE else ())
    if (c, kw, d) == (12, 8, 3) and m > 8:
        return _native.FTK_ERR_INVALID  # three units of 16 x rows would not fit the LDS
    return _native.FTK_OK if (c, kw, d) in shapes else _native.FTK_ERR_INVALID


def _configs(m):
    gemv = []
    if m <= 4:
        gemv = [_native.Config(_native.KIND_GEMV, rpw, u, gpc, kw)
                for rpw, u, kw in ((2, 4, 1), (4, 2, 1), (8, 1, 1), (1, 2, 2), (2, 2, 2), (1, 1, 4), (2, 2, 4))
                for gpc in (1, 8)]
    if m <= 8:
        gemv += [_native.Config(_native.KIND_STREAM, rpw, 0, gpc, kw)
                 for rpw, _, kw in (STREAM_SHAPES if m <= 4 else STREAM_SHAPES_8) for gpc in (1, 8, 16)]
    if m <= 16:
        gemv += [_native.Config(_native.KIND_MFMA_STREAM, 16 * t, u, gpc, kw)
                 for t, _, kw, u in MSTREAM_EVEN + MSTREAM_ONE for gpc in (1, 4)]
        gemv += [_native.Config(_native.KIND_QUAD, 4 * rs, 0, gpc, kw)
                 for rs, _, kw in QUAD_SHAPES + QUAD_ONE for gpc in (1, 8)]
        gemv += [_native.Config(_native.KIND_STAGE, 16 * t, u, gpc, kw)
                 for t, _, kw, u in STAGE_EVEN + STAGE_ONE + STAGE_LONG for gpc in (1, 4)]
    if m <= 16:
        gemv += [_native.Config(_native.KIND_RING, rows, d, gpc, kw) for _, kw, d in RING_SHAPES + RING_LONG
                 for gpc in (1, 4) for rows in (12, 16, 24)]
    mfma = [_native.Config(_native.KIND_MFMA, rows, u, 0, w)
            for rows, u, w in ((16, 4, 4), (16, 8, 8), (16, 4, 16), (32, 8, 4), (32, 4, 16), (64, 2, 8), (64, 4, 4))]
    return [None] + gemv + mfma


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 16, 17, 32])
def test_plan_writes_every_output_once(m, n, k):
    for epilogue in (_native.EPI_STORE, _native.EPI_SWIGLU, _native.EPI_ARGMAX):
        if epilogue == _native.EPI_SWIGLU and n % 2:
            continue
        for cfg in _configs(m):
            if cfg is not None and k % 8:
                continue
            if (cfg is not None and epilogue == _native.EPI_SWIGLU
                    and cfg.rows_per_wave in ((16,) if cfg.kind in (_native.KIND_MFMA, _native.KIND_STAGE)
                                              else (4,) if cfg.kind == _native.KIND_QUAD else (1,))):
                continue  # a SwiGLU workgroup / row group needs a gate row and its up row
            p = _native.Plan()
            status = _native.lib().ftk_plan_project(m, n, k, epilogue, 256, cfg, p)
            if k % 8 and epilogue != _native.EPI_STORE:
                assert status == _native.FTK_ERR_UNSUPPORTED
                continue
            if cfg is not None and cfg.kind == _native.KIND_STREAM:
                want = _stream_status(m, k, cfg.rows_per_wave, cfg.waves)
                assert status == want, (m, n, k, epilogue, cfg)
                if want != _native.FTK_OK:
                    continue
            if cfg is not None and cfg.kind == _native.KIND_MFMA_STREAM:
                want = _mstream_status(m, k, epilogue, cfg.rows_per_wave // 16, cfg.waves, cfg.unroll)
                assert status == want, (m, n, k, epilogue, cfg)
                if want != _native.FTK_OK:
                    continue
            if cfg is not None and cfg.kind == _native.KIND_STAGE:
                want = _stage_status(m, k, epilogue, cfg.rows_per_wave // 16, cfg.waves, cfg.unroll)
                assert status == want, (m, n, k, epilogue, cfg)
                if want != _native.FTK_OK:
                    continue
            if cfg is not None and cfg.kind == _native.KIND_QUAD:
                want = _quad_status(m, k, epilogue, cfg.rows_per_wave, cfg.waves)
                assert status == want, (m, n, k, epilogue, cfg)
                if want != _native.FTK_OK:
                    continue
            if cfg is not None and cfg.kind == _native.KIND_RING:
                want = _ring_status(m, k, epilogue, cfg.waves, cfg.unroll, rows=cfg.rows_per_wave)
                assert status == want, (m, n, k, epilogue, cfg)
                if want != _native.FTK_OK:
                    continue
            assert status == _native.FTK_OK, (m, n, k, epilogue, cfg)
            counts, max_row = _coverage(p, n, epilogue)
            assert np.all(counts == 1), (m, n, k, epilogue, cfg)
            assert max_row == n - 1
            if p.kind == _native.KIND_GEMV:
                assert 1 <= p.grid <= p.tiles
                assert p.lds_bytes == m * k * 2
            if p.kind == _native.KIND_STREAM:
                # every walk equally deep (within one tile) and at most 8 tiles: their totals wait in LDS
                assert 1 <= p.grid <= p.tiles and -(-p.tiles // p.grid) <= 8
                assert p.unroll * 512 * p.waves == k and p.lds_bytes == 0
                assert p.threads == 64 * max(4, p.waves)
            if p.kind == _native.KIND_MFMA_STREAM:
                t = p.rows_per_wave // 16
                assert 1 <= p.grid <= p.tiles and -(-p.tiles // p.grid) <= 64 // (t * p.waves)
                assert p.threads == 64 * p.waves and k % (32 * p.waves) == 0
            if p.kind == _native.KIND_STAGE:
                # any walk depth (the epilogue runs every 64 // (T KW) tiles); groups_per_cu workgroups per CU
                gpc = cfg.groups_per_cu if cfg is not None and cfg.groups_per_cu else 1
                assert 1 <= p.grid <= min(p.tiles, 256 * gpc)
                assert p.threads == 64 * p.waves and k % (128 * p.waves) == 0
            if p.kind == _native.KIND_RING:
                # one workgroup per CU (groups_per_cu of them), 12, 16 or 24 weight rows per tile, any walk depth
                gpc = cfg.groups_per_cu if cfg is not None and cfg.groups_per_cu else 1
                assert 1 <= p.grid <= min(p.tiles, 256 * gpc) and p.rows_per_wave in (12, 16, 24)
                assert p.tiles == -(-(n // 2 if epilogue == _native.EPI_SWIGLU else n) //
                                    (8 if epilogue == _native.EPI_SWIGLU else p.rows_per_wave))
                assert p.threads == 64 * p.waves and k % (128 * p.waves) == 0
            if p.kind == _native.KIND_QUAD:
                assert 1 <= p.grid <= p.tiles and -(-p.tiles // p.grid) <= 8
                assert p.unroll * 128 * p.waves == k and p.threads == 64 * max(4, p.waves)
            if p.kind == _native.KIND_MFMA:
                # one workgroup per tile over all of K: no split-K, nothing shared between workgroups
                assert p.grid == p.tiles and p.splits == 1 and p.k_slice == k
            if epilogue == _native.EPI_ARGMAX and p.kind != _native.KIND_GENERIC:
                assert p.workspace_bytes >= 256 + 8 * m * p.grid  # one key per workgroup and row


def test_plan_kinds():
    p = _native.Plan()
    _native.call("ftk_plan_project", 1, 4096, 4096, 0, 256, None, p)
    assert p.kind == _native.KIND_STREAM and p.threads == 256 and p.unroll * 512 * p.waves == 4096
    _native.call("ftk_plan_project", 1, 4096, 4104, 0, 256, None, p)  # K % 512 != 0: the LDS-staged GEMV
    assert p.kind == _native.KIND_GEMV and p.threads == 256
    # lm_head + argmax without the norm prologue (no claimed-tail build): QUAD from 2 rows, STREAM at 1
    _native.call("ftk_plan_project", 4, 151936, 4096, _native.EPI_ARGMAX, 256, None, p)
    assert p.kind == _native.KIND_QUAD and -(-p.tiles // p.grid) <= 8
    _native.call("ftk_plan_project", 1, 151936, 4096, _native.EPI_ARGMAX, 256, None, p)
    assert p.kind == _native.KIND_STREAM and -(-p.tiles // p.grid) <= 8
    # with the prologue: RING from one row, one round of workgroups whose walks end in claimed tiles
    for m in (1, 2, 4):
        _native.call("ftk_plan_project", m, 151936, 4096, _native.EPI_ARGMAX | _native.PLAN_PROLOGUE, 256, None, p)
        assert p.kind == _native.KIND_RING and p.grid == 256 and p.tiles == 9496, m
        assert p.workspace_bytes >= 256 + 256 * m * 8
    # a vocabulary too short for 16 tiles per CU, or a K without a claimed-tail build: STREAM at one row
    _native.call("ftk_plan_project", 1, 16 * 16 * 256 - 16, 4096, _native.EPI_ARGMAX | _native.PLAN_PROLOGUE, 256,
                 None, p)
    assert p.kind == _native.KIND_STREAM
    _native.call("ftk_plan_project", 1, 151936, 2048, _native.EPI_ARGMAX | _native.PLAN_PROLOGUE, 256, None, p)
    assert p.kind == _native.KIND_STREAM
    _native.call("ftk_plan_project", 1, 173, 259, 0, 256, None, p)
    assert p.kind == _native.KIND_GENERIC
    # rows of <= 3072 elements at one x row: one wave per row group (KW = 1), one tile per workgroup
    # without the norm (C1), two with it (C2); two rows per wave at K = 1024, one at 2048 and 3072
    _native.call("ftk_plan_project", 1, 4096, 1024, 0, 256, None, p)
    assert p.kind == _native.KIND_STREAM and p.waves == 1 and p.rows_per_wave == 2 and p.grid == p.tiles == 512
    _native.call("ftk_plan_project", 1, 4096, 1024, _native.PLAN_PROLOGUE, 256, None, p)
    assert p.kind == _native.KIND_STREAM and p.waves == 1 and p.grid == 256 and p.tiles == 512
    _native.call("ftk_plan_project", 1, 1024, 3072, 0, 256, None, p)
    assert p.kind == _native.KIND_STREAM and p.waves == 1 and p.rows_per_wave == 1 and p.grid == p.tiles == 256
    _native.call("ftk_plan_project", 1, 6144, 1024, _native.EPI_SWIGLU | _native.PLAN_PROLOGUE, 256, None, p)
    assert p.kind == _native.KIND_STREAM and p.waves == 1 and p.rows_per_wave == 2 and p.grid == 384
    _native.call("ftk_plan_project", 1, 151936, 1024, _native.EPI_ARGMAX, 256, None, p)  # argmax: unchanged
    assert p.kind == _native.KIND_STREAM and p.waves != 1
    _native.call("ftk_plan_project", 1, 4096, 4096, 0, 256, None, p)  # the 8B shapes keep KW = 4
    assert p.waves == 4
    # 5..16 rows: weight and x segments loaded straight into LDS (RING), one workgroup per CU
    _native.call("ftk_plan_project", 5, 4096, 4096, 0, 256, None, p)
    assert p.kind == _native.KIND_RING and p.threads == 512 and p.unroll == 2 and p.grid == 256
    # N = 6144: 12-row tiles, two per CU on every CU, where 16-row ones leave half a round (192
    # workgroups walking two) -- with or without the norm, at any row count
    for m, flags in ((5, 0), (5, _native.PLAN_PROLOGUE), (8, _native.PLAN_PROLOGUE), (16, 0)):
        _native.call("ftk_plan_project", m, 6144, 4096, flags, 256, None, p)
        assert p.kind == _native.KIND_RING and p.rows_per_wave == 12 and p.waves == 8 and p.grid == 256, (m, flags)
    _native.call("ftk_plan_project", 5, 4096, 4096, 0, 256, None, p)  # N = 4096: one 16-row tile per CU
    assert p.kind == _native.KIND_RING and p.rows_per_wave == 16 and p.grid == 256
    _native.call("ftk_plan_project", 8, 4096, 12288, 0, 256, None, p)  # long K: three units in flight
    assert p.kind == _native.KIND_RING and p.waves == 8 and p.unroll == 3
    _native.call("ftk_plan_project", 8, 24576, 4096, _native.EPI_SWIGLU | _native.PLAN_PROLOGUE, 256, None, p)
    assert p.kind == _native.KIND_RING and p.tiles == 12288 // 8 and p.grid == 256
    assert p.workspace_bytes == 0  # six tiles per walk: the static order, no claims
    _native.call("ftk_plan_project", 16, 4096, 12288, 0, 256, None, p)  # 16 x rows: two units fit
    assert p.kind == _native.KIND_RING and p.unroll == 2
    _native.call("ftk_plan_project", 5, 151936, 4096, _native.EPI_ARGMAX | _native.PLAN_PROLOGUE, 256, None, p)
    # lm_head: one round (8 | grid), 37 tiles per walk, the last eighth claimed from the workspace
    assert p.kind == _native.KIND_RING and p.tiles == 9496 and p.grid == 256 and p.workspace_bytes >= 256 + 256 * 5 * 8
    # the prologue's residual add is not a RING form: such calls plan as before
    _native.call("ftk_plan_project", 5, 6144, 4096, _native.PLAN_PROLOGUE | _native.PLAN_RESIDUAL, 256, None, p)
    assert p.kind == _native.KIND_QUAD
    _native.call("ftk_plan_project", 16, 6144, 4096, _native.PLAN_PROLOGUE | _native.PLAN_RESIDUAL, 256, None, p)
    assert p.kind == _native.KIND_STAGE
    ring = _native.Config(_native.KIND_RING, 16, 2, 0, 8)
    assert _native.lib().ftk_plan_project(5, 6144, 4096, _native.PLAN_PROLOGUE | _native.PLAN_RESIDUAL, 256, ring,
                                          p) == _native.FTK_OK  # an explicit RING plan is accepted; the call refuses
    c = _native.Config(_native.KIND_MFMA_STREAM, 0, 0, 0, 0)  # x streamed beside the weights
    _native.call("ftk_plan_project", 16, 4096, 12288, 0, 256, c, p)
    assert p.kind == _native.KIND_MFMA_STREAM and p.waves == 8 and p.unroll == 16
    # K = 12288 with the prologue has no MFMA_STREAM kernel: the 8-row STREAM kernel (8 waves split K)
    _native.call("ftk_plan_project", 8, 4096, 12288, _native.PLAN_PROLOGUE, 256, None, p)
    assert p.kind == _native.KIND_STREAM and p.waves == 8 and p.threads == 512
    _native.call("ftk_plan_project", 12, 4096, 2048, 0, 256, None, p)  # no STREAM-schedule kind has this K
    assert p.kind == _native.KIND_MFMA and p.grid == 256 and p.splits == 1
    _native.call("ftk_plan_project", 17, 4096, 4096, 0, 256, None, p)
    assert p.kind == _native.KIND_MFMA
    _native.call("ftk_plan_project", 20, 24576, 4096, _native.EPI_SWIGLU, 256, None, p)
    assert p.kind == _native.KIND_MFMA and p.rows_per_wave == 32 and p.grid == 12288 // 16


def test_default_kind_for_8b_shapes():
    """The planner's choice at the Qwen3-8B shapes (from the MI355X sweeps): STREAM at M = 1 and,
    to M = 4, except gate/up from 3 and QKV at 4 (QUAD); RING for every projection and SwiGLU at
    5..16 (the 8-row STREAM kernel where K = 12288 has the prologue) and for lm_head + argmax
    (with the norm prologue) at every row count, its long walks ending in claimed tiles."""
    shapes = {"qkv": (6144, 4096, _native.EPI_STORE, True), "o": (4096, 4096, _native.EPI_STORE, False),
              "gate_up": (24576, 4096, _native.EPI_SWIGLU, True), "down": (4096, 12288, _native.EPI_STORE, False),
              "lm_head": (151936, 4096, _native.EPI_ARGMAX, True)}
    for m in range(1, 17):
        for name, (n, k, epi, pro) in shapes.items():
            p = _native.Plan()
            flags = epi | (_native.PLAN_PROLOGUE if pro else 0)
            _native.call("ftk_plan_project", m, n, k, flags, 256, None, p)
            quad_early = {"gate_up": 3, "qkv": 4}.get(name, 5)
            if name == "lm_head":
                want = _native.KIND_RING
            elif m < quad_early:
                want = _native.KIND_STREAM
            elif m <= 4:
                want = _native.KIND_QUAD
            else:
                want = _native.KIND_RING
            assert p.kind == want, (m, name, p.kind)
    # the prologue at K = 12288 has no QUAD or RING shape: the 8-row STREAM kernel
    p = _native.Plan()
    _native.call("ftk_plan_project", 8, 4096, 12288, _native.PLAN_PROLOGUE, 256, None, p)
    assert p.kind == _native.KIND_STREAM and p.waves == 8 and p.threads == 512


def test_native_gemm_from_seventeen_rows_without_a_config():
    from kernels import linear as L
    assert L.NATIVE_FROM_ROWS == 17
    assert not L.prefer_native(16) and L.prefer_native(17) and L.prefer_native(32)
    assert not L.prefer_native(32, _native.Config(_native.KIND_MFMA, 0, 0, 0, 0))


@pytest.mark.parametrize("m", [5, 8, 16])
def test_residual_calls_size_the_workspace_of_their_own_plan(m):
    """A call whose prologue adds a residual is planned on another kind and grid than the same call
    without it (RING does not take the add); the workspace is sized from that plan, so its argmax
    keys (one per workgroup and row) always fit."""
    flags = _native.EPI_ARGMAX | _native.PLAN_PROLOGUE
    plain = _native.lib().ftk_project_workspace_bytes(m, 151936, 4096, flags, None)
    with_residual = _native.lib().ftk_project_workspace_bytes(m, 151936, 4096, flags | _native.PLAN_RESIDUAL, None)
    p = _native.Plan()
    _native.call("ftk_plan_project", m, 151936, 4096, flags | _native.PLAN_RESIDUAL, 256, None, p)
    assert p.kind != _native.KIND_RING
    assert with_residual == p.workspace_bytes >= 256 + 8 * m * p.grid
    _native.call("ftk_plan_project", m, 151936, 4096, flags, 256, None, p)
    assert p.kind == _native.KIND_RING and plain == p.workspace_bytes


@pytest.mark.parametrize("cus", [64, 80, 100, 104, 228, 256, 304])
@pytest.mark.parametrize("m", [1, 2, 4, 5, 16])
def test_lm_head_plans_on_other_cu_counts(cus, m):
    """lm_head + argmax with the norm on devices of other CU counts (partitions, other parts): the
    plan writes every logit once, its argmax keys fit the workspace, and a RING plan whose walks are
    long enough for the claimed tail (at least 16 tiles per workgroup, as the kernel decides) has
    room for the claim counter; below 5 rows RING is chosen only where those walks are that long."""
    v, k = 151936, 4096
    flags = _native.EPI_ARGMAX | _native.PLAN_PROLOGUE
    p = _native.Plan()
    assert _native.lib().ftk_plan_project(m, v, k, flags, cus, None, p) == _native.FTK_OK
    counts, max_row = _coverage(p, v, _native.EPI_ARGMAX)
    assert np.all(counts == 1) and max_row == v - 1
    assert p.workspace_bytes >= 256 + 8 * m * p.grid
    if p.kind == _native.KIND_RING:
        assert 1 <= p.grid <= p.tiles
        if p.tiles >= 16 * p.grid:
            assert p.workspace_bytes >= 128 + 4
        if m < 5:
            assert p.tiles >= 16 * cus
