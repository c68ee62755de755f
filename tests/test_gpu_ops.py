"""GPU parity of the standalone operators (rms_norm, add_rms_norm, swiglu, argmax,
Split merge) against the golden fixtures (torch / transformers outputs) and the oracle."""

import numpy as np
import pytest
import torch

from conftest import GOLDEN, from_bits, seeded, to_bits
from oracle import bf16, path

from kernels import argmax as A
from kernels import merged as M
from kernels import rmsnorm as R
from kernels import swiglu as S

pytestmark = pytest.mark.gpu

NORM_SHAPES = [(3, 2560), (5, 128), (1, 100), (4, 1024), (2, 4096)]


def ulps(a, b):
    return np.abs(a.astype(np.int32) - b.astype(np.int32))


@pytest.mark.parametrize("shape", NORM_SHAPES)
def test_rms_norm_matches_qwen3_module(cuda, shape):
    data = np.load(GOLDEN / "rmsnorm.npz")
    key = "_".join(map(str, shape))
    x, w = from_bits(data[f"x_{key}"], cuda), from_bits(data[f"w_{key}"], cuda)
    x0 = x.clone()
    got = to_bits(R.rms_norm(x, w, 1e-6))
    assert torch.equal(x, x0)
    want = data[f"y_{key}"]
    assert np.mean(got == want) >= 0.999 and ulps(got, want).max() <= 2
    assert np.mean(got == path.rms_norm(data[f"x_{key}"], data[f"w_{key}"], 1e-6)) >= 0.999


@pytest.mark.parametrize("shape", NORM_SHAPES)
def test_add_rms_norm(cuda, shape):
    data = np.load(GOLDEN / "rmsnorm.npz")
    key = "_".join(map(str, shape))
    x, r, w = (from_bits(data[f"{p}_{key}"], cuda) for p in ("x", "r", "w"))
    x0, r0 = x.clone(), r.clone()
    y, s = R.add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(x, x0) and torch.equal(r, r0)
    assert np.array_equal(to_bits(s), data[f"sum_{key}"])
    got, want = to_bits(y), data[f"ysum_{key}"]
    assert np.mean(got == want) >= 0.999 and ulps(got, want).max() <= 2


def test_add_rms_norm_accepts_split(cuda):
    m, n = 6, 256
    partial = torch.randn(3, m, n, device=cuda) * 2
    split = M.Split(partial, (m, n))
    r = seeded((m, n), seed=1, device=cuda)
    w = seeded((n,), seed=2, scale=0.1, shift=1.0, device=cuda)
    merged = M.materialize(split)
    assert np.array_equal(to_bits(merged), path.merge_splits(partial.cpu().numpy()))
    a, b = R.add_rms_norm(split, r, w, 1e-6), R.add_rms_norm(merged, r, w, 1e-6)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("rows,width", [(4, 1500), (3, 64), (2, 3072), (1, 9728)])
def test_swiglu_matches_torch_silu(cuda, rows, width):
    data = np.load(GOLDEN / "swiglu.npz")
    p = from_bits(data[f"p_{rows}_{width}"], cuda)
    got, want = to_bits(S.swiglu(p)), data[f"y_{rows}_{width}"]
    assert np.mean(got == want) >= 0.999 and ulps(got, want).max() <= 1
    assert np.array_equal(got[:, :8], want[:, :8])
    assert np.mean(got == path.swiglu(data[f"p_{rows}_{width}"])) >= 0.999


def test_swiglu_accepts_split_and_batch_dims(cuda):
    partial = torch.randn(2, 5, 128, device=cuda)
    split = M.Split(partial, (1, 5, 128))
    got = S.swiglu(split)
    assert got.shape == (1, 5, 64)
    assert torch.equal(got.reshape(5, 64), S.swiglu(M.materialize(M.Split(partial, (5, 128)))))


ARGMAX_SHAPES = [(3, 1000), (4, 777), (5, 4096), (1, 300), (2, 151936)]


@pytest.mark.parametrize("shape", ARGMAX_SHAPES)
@pytest.mark.parametrize("kind", ["rand", "ties", "last", "equal"])
def test_argmax_fixture_suites(cuda, shape, kind):
    data = np.load(GOLDEN / "argmax.npz")
    key = f"{kind}_{'_'.join(map(str, shape))}"
    logits = from_bits(data[key], cuda)
    top = torch.empty(shape[0], dtype=torch.float32, device=cuda)
    ids = A.argmax(logits, top=top)
    assert ids.dtype == torch.int64
    assert np.array_equal(ids.cpu().numpy(), data[f"{key}_ids"])
    assert np.array_equal(top.cpu().numpy(), bf16.to_f32(data[key]).max(-1))


def test_argmax_batch_dims_and_nan(cuda):
    logits = seeded((2, 2, 777), seed=3, scale=4, device=cuda)
    assert torch.equal(A.argmax(logits), logits.float().argmax(-1))
    logits[0, 1, 500] = float("nan")
    assert A.argmax(logits)[0, 1].item() == 500


def test_merge_splits(cuda):
    partial = torch.randn(4, 3, 1000, device=cuda) * 100
    got = M.materialize(M.Split(partial, (3, 1000)))
    assert np.array_equal(to_bits(got), path.merge_splits(partial.cpu().numpy()))


@pytest.mark.parametrize("grid,loads", [(1, 2), (7, 4), (256, 8), (2048, 16), (0, 2), (0, 4), (0, 16)])
def test_stream_read_reads_every_chunk_into_its_owner(cuda, grid, loads):
    """The bandwidth reference (ftk_stream_read) really reads the bytes: a buffer of zeros with one
    chunk equal to the kernel's store constant makes exactly the workgroup that owns that chunk store
    the constant into its sink word. Persistent form: chunk c belongs to workgroup (c mod 256 grid) //
    256; one-shot form (grid 0): to workgroup c // (256 loads)."""
    from kernels import _native
    chunks = 3 * 256 * max(grid, 5) + 77              # a partial last round
    for c in (0, chunks // 2 + 3, chunks - 2):        # not the last chunk: it is re-read past the end
        buf = torch.zeros(chunks * 4, dtype=torch.int32, device=cuda)
        buf[4 * c] = int(np.int32(np.uint32(0x9E3779B9)))
        words = grid if grid else -(-chunks // (256 * loads))
        sink = torch.zeros(words, dtype=torch.int32, device=cuda)
        _native.call("ftk_stream_read", _native.ptr(buf), chunks * 16, _native.ptr(sink), grid, loads,
                     _native.stream_of(buf))
        torch.cuda.synchronize()
        want = np.zeros(words, dtype=np.uint32)
        want[(c % (256 * grid)) // 256 if grid else c // (256 * loads)] = 0x9E3779B9
        np.testing.assert_array_equal(sink.cpu().numpy().view(np.uint32), want)
