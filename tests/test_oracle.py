"""Pin the CPU oracle (oracle/) against implementations independent of it.

Each check is chosen so that a plausible mistake in the oracle fails it: a
dropped rounding, a moved rounding (the wrong-cast detector), a transposed
operand, a wrong tie rule, a wrong split order.
"""

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from conftest import GOLDEN, from_bits, to_bits
from oracle import bf16, helpers, path


def _load(name):
    return np.load(GOLDEN / name)


# ---- bf16 rounding ------------------------------------------------------------

def test_round_bits_matches_torch_fixture():
    data = _load("bf16_round.npz")
    got = bf16.round_bits(data["values"])
    want = data["expected"]
    # NaN payloads differ between torch's scalar (0x7FC0) and vectorized (0xFFFF) conversions:
    # compare NaN-ness there, bits everywhere else.
    nan_got = (got & 0x7F80) == 0x7F80
    nan_want = (want & 0x7F80) == 0x7F80
    is_nan = np.isnan(data["values"])
    assert np.array_equal(got[~is_nan], want[~is_nan])
    assert np.all((got[is_nan] & 0x7F) != 0) and np.all((want[is_nan] & 0x7F) != 0)
    assert np.array_equal(nan_got & ((got & 0x7F) != 0), nan_want & ((want & 0x7F) != 0))


def test_round_bits_ties_to_even():
    # 1 + 2^-8 is exactly halfway between BF16 1.0 and 1.0078125: even mantissa (1.0) wins.
    assert bf16.round_bits(np.float32(1 + 2 ** -8)) == 0x3F80
    # 1 + 3 * 2^-8 is halfway between 1.0078125 (odd) and 1.015625 (even).
    assert bf16.round_bits(np.float32(1 + 3 * 2 ** -8)) == 0x3F82
    assert bf16.round_bits(np.float32(np.nan)) == 0x7FC0


def test_to_f32_is_exact_inverse():
    b = np.arange(0, 1 << 16, dtype=np.uint16)
    finite = (b & 0x7F80) != 0x7F80
    assert np.array_equal(bf16.round_bits(bf16.to_f32(b))[finite], b[finite])


# ---- projection -------------------------------------------------------------------

LINEAR_SHAPES = [(1, 200, 300), (5, 200, 300), (16, 130, 517), (20, 70, 260), (1, 173, 259), (4, 257, 513),
                 (16, 127, 256), (3, 64, 1024)]


@pytest.mark.parametrize("m,n,k", LINEAR_SHAPES)
def test_project_within_three_quarter_ulp_of_fp64(m, n, k):
    """The reference's bar: <= 0.75 BF16 ulp of the exact product (run_numeric.py:59-61)."""
    data = _load("linear.npz")
    key = f"{m}_{n}_{k}"
    got = bf16.to_f32(path.project(data[f"x_{key}"], data[f"w_{key}"])).astype(np.float64)
    exact = data[f"exact_{key}"]
    assert np.all(np.abs(got - exact) / bf16.ulp(exact) <= 0.75)
    # and against torch CPU F.linear within 2e-2 + 1e-2|ref|
    ref = bf16.to_f32(data[f"torch_{key}"]).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2e-2 + 1e-2 * np.abs(ref))


def test_project_exact_on_integers():
    """Small integers: every FP32 partial sum is exact, so the result is bit-exact and order-free."""
    rng = np.random.default_rng(5)
    x = rng.integers(-4, 5, size=(3, 96)).astype(np.float32)
    w = rng.integers(-4, 5, size=(40, 96)).astype(np.float32)
    got = path.project(bf16.round_bits(x), bf16.round_bits(w))
    assert np.array_equal(bf16.to_f32(got), (x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32))


def test_project_orientation():
    """y[m, n] uses row n of W: a transposed operand would fail this (one-hot inputs)."""
    x = np.zeros((2, 8), np.float32)
    x[0, 3] = 1.0
    x[1, 5] = 2.0
    w = np.arange(6 * 8, dtype=np.float32).reshape(6, 8)
    got = bf16.to_f32(path.project(bf16.round_bits(x), bf16.round_bits(w)))
    assert np.array_equal(got[0], bf16.round_f32(w[:, 3]))
    assert np.array_equal(got[1], bf16.round_f32(2 * w[:, 5]))


def test_merge_splits_order_and_rounding():
    # Sequential FP32 adds in split order, then one rounding (merged.py:37-45).
    p = np.array([[1e8, 1.0], [1.0, 2.0], [-1e8, 3.0]], dtype=np.float32)
    got = bf16.to_f32(path.merge_splits(p))
    # (1e8 + 1) rounds back to 1e8 in FP32, so the first column is 0, not 1.
    assert got[0] == 0.0 and got[1] == 6.0


# ---- RMSNorm ----------------------------------------------------------------------

NORM_SHAPES = [(3, 2560), (5, 128), (1, 100), (4, 1024), (2, 4096)]


def _ulps(a, b):
    return np.abs(a.astype(np.int32) - b.astype(np.int32))


@pytest.mark.parametrize("shape", NORM_SHAPES)
def test_rms_norm_matches_qwen3_module(shape):
    """transformers' Qwen3RMSNorm outputs (fixture): >= 99.9% bit-equal, <= 2 ulp (verify_gpu.py:62-66)."""
    data = _load("rmsnorm.npz")
    key = "_".join(map(str, shape))
    got = path.rms_norm(data[f"x_{key}"], data[f"w_{key}"], 1e-6)
    want = data[f"y_{key}"]
    assert np.mean(got == want) >= 0.999
    assert _ulps(got, want).max() <= 2


@pytest.mark.parametrize("shape", NORM_SHAPES)
def test_add_rms_norm_matches_module_on_bf16_sum(shape):
    data = _load("rmsnorm.npz")
    key = "_".join(map(str, shape))
    y, s = path.add_rms_norm(data[f"x_{key}"], data[f"r_{key}"], data[f"w_{key}"], 1e-6)
    assert np.array_equal(s, data[f"sum_{key}"])
    assert np.mean(y == data[f"ysum_{key}"]) >= 0.999
    assert _ulps(y, data[f"ysum_{key}"]).max() <= 2


def test_embed_rms_norm_gathers_like_torch_embedding():
    """hidden = torch's embedding lookup of the same table (an independent gather); the norm is rms_norm's."""
    rng = np.random.default_rng(11)
    table = bf16.round_bits(rng.standard_normal((50, 96)).astype(np.float32))
    gamma = bf16.round_bits(1 + 0.1 * rng.standard_normal(96).astype(np.float32))
    ids = np.array([[3, 49, 0], [7, 7, 12]], dtype=np.int64)
    y, hidden = path.embed_rms_norm(ids, table, gamma, 1e-6)
    want = F.embedding(torch.from_numpy(ids), from_bits(table)).contiguous()
    assert np.array_equal(hidden, to_bits(want))
    assert np.array_equal(y, path.rms_norm(hidden, gamma, 1e-6))
    # consecutive ids reproduce the table itself
    assert np.array_equal(path.embed_rms_norm(np.arange(50), table, gamma, 1e-6)[1], table)


def test_rms_norm_wrong_cast_detector():
    """Keeping x_hat * gamma in FP32 is a different function (verify_gpu.py:56-61): >5% of outputs differ."""
    data = _load("rmsnorm.npz")
    x, w = data["x_3_2560"], data["w_3_2560"]
    v = bf16.to_f32(x).astype(np.float32)
    scale = (1 / np.sqrt((np.mean(v.astype(np.float64) ** 2, -1, keepdims=True) + 1e-6))).astype(np.float32)
    wrong = bf16.round_bits(v * scale * bf16.to_f32(w))
    assert np.mean(wrong != path.rms_norm(x, w, 1e-6)) > 0.05


# ---- SwiGLU ------------------------------------------------------------------------

@pytest.mark.parametrize("rows,width", [(4, 1500), (3, 64), (2, 3072), (1, 9728)])
def test_swiglu_matches_torch_silu(rows, width):
    data = _load("swiglu.npz")
    got = path.swiglu(data[f"p_{rows}_{width}"])
    want = data[f"y_{rows}_{width}"]
    assert np.mean(got == want) >= 0.999
    assert _ulps(got, want).max() <= 1
    # the special inputs [-100, -20, -1, 0, 1, 20, 100, 0.125] agree exactly
    assert np.array_equal(got[:, :8], want[:, :8])


def test_swiglu_rounds_silu_before_up():
    """Without the BF16 rounding of SiLU's output the results differ on some elements."""
    data = _load("swiglu.npz")
    p = data["p_2_3072"]
    g, u = bf16.to_f32(p[:, :3072]), bf16.to_f32(p[:, 3072:])
    unrounded = bf16.round_bits((g / (1 + np.exp(-g.astype(np.float64)))).astype(np.float32) * u)
    assert np.mean(unrounded != path.swiglu(p)) > 0.01


# ---- argmax -------------------------------------------------------------------------

ARGMAX_SHAPES = [(3, 1000), (4, 777), (5, 4096), (1, 300), (2, 151936)]


@pytest.mark.parametrize("shape", ARGMAX_SHAPES)
@pytest.mark.parametrize("kind", ["rand", "ties", "last", "equal"])
def test_argmax_first_matches_torch(shape, kind):
    data = _load("argmax.npz")
    key = f"{kind}_{'_'.join(map(str, shape))}"
    assert np.array_equal(path.argmax_first(data[key]), data[f"{key}_ids"])


def test_argmax_first_brute_force_ties():
    rng = np.random.default_rng(3)
    logits = bf16.round_bits(rng.integers(-2, 3, size=(6, 50)).astype(np.float32))
    vals = bf16.to_f32(logits)
    for row in range(6):
        best = 0
        for j in range(1, 50):
            if vals[row, j] > vals[row, best]:
                best = j
        assert path.argmax_first(logits)[row] == best


def test_lm_head_argmax_top_is_winning_logit():
    rng = np.random.default_rng(4)
    x = bf16.round_bits(rng.standard_normal((2, 64)).astype(np.float32))
    w = bf16.round_bits(rng.standard_normal((300, 64)).astype(np.float32) * 0.05)
    logits, ids, top = path.lm_head_argmax(x, w)
    assert np.array_equal(top, bf16.to_f32(logits).max(-1))
    assert np.array_equal(ids, path.argmax_first(logits))


def test_fused_forms_compose():
    rng = np.random.default_rng(6)
    x = bf16.round_bits(rng.standard_normal((2, 64)).astype(np.float32))
    gamma = bf16.round_bits(1 + 0.1 * rng.standard_normal(64).astype(np.float32))
    w = bf16.round_bits(rng.standard_normal((40, 64)).astype(np.float32) * 0.05)
    xn = path.rms_norm(x, gamma, 1e-6)
    assert np.array_equal(path.gate_up_swiglu(x, w, gamma, 1e-6), path.swiglu(path.project(xn, w)))
    assert np.array_equal(path.norm_project(x, gamma, 1e-6, w), path.project(xn, w))
    r = bf16.round_bits(rng.standard_normal((2, 64)).astype(np.float32))
    y, s = path.add_norm_project(x, r, gamma, 1e-6, w)
    normed, summed = path.add_rms_norm(x, r, gamma, 1e-6)
    assert np.array_equal(s, summed) and np.array_equal(y, path.project(normed, w))


def test_oracle_matches_torch_cpu_path():
    """The numpy oracle and the torch-CPU restatement agree within 2e-2 + 1e-2|ref| end to end."""
    from oracle import torch_cpu

    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 256, generator=g).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(256, generator=g)).to(torch.bfloat16)
    w = (torch.randn(512, 256, generator=g) * 0.02).to(torch.bfloat16)
    ref = torch_cpu.gate_up_swiglu(x, w, gamma, 1e-6).float().numpy()
    got = bf16.to_f32(path.gate_up_swiglu(to_bits(x), to_bits(w), to_bits(gamma), 1e-6))
    assert np.all(np.abs(got - ref) <= 2e-2 + 1e-2 * np.abs(ref))
    assert from_bits(path.rms_norm(to_bits(x), to_bits(gamma), 1e-6)).shape == (1, 256)
    ref_lin = F.linear(x, w).float().numpy()
    assert np.all(np.abs(bf16.to_f32(path.project(to_bits(x), to_bits(w))) - ref_lin) <= 2e-2 + 1e-2 * np.abs(ref_lin))


# ---- integer helpers (known answers of the reference) -----------------------------------

def test_persistent_programs_known_answers():
    # engine/kernels/gemm.py:333-335 on the H100's 132 SMs
    assert helpers.persistent_programs(304, 132) == 102
    assert helpers.persistent_programs(2374, 132) == 132
    for tiles in (1, 17, 132):
        assert helpers.persistent_programs(tiles, 132) == tiles


def test_exact_splits_known_answers():
    # engine/kernels/linear.py:359-361: 128-wide K blocks, the power-of-two split count 8
    assert helpers.exact_splits(2560, 128, 8) == 5
    assert helpers.exact_splits(9728, 128, 8) == 4
    assert helpers.exact_splits(4096, 128, 8) == 8
    assert helpers.exact_splits(4100, 128, 8) == 8  # not whole blocks: the wanted count stays


def test_exact_splits_against_a_simulated_split_layout():
    """Brute force: lay the K blocks out over s split programs of ceil(blocks / s) contiguous blocks
    each; the rule's answer is the largest s <= wanted whose programs all get the same, non-zero
    number of blocks (no partial and no dead split program)."""
    for blocks in range(1, 97):
        for wanted in range(1, 17):
            exact = []
            for s in range(1, wanted + 1):
                chunk = -(-blocks // s)
                counts = [max(0, min((i + 1) * chunk, blocks) - i * chunk) for i in range(s)]
                if all(c == chunk for c in counts):
                    exact.append(s)
            assert helpers.exact_splits(blocks * 64, 64, wanted) == max(exact), (blocks, wanted)


def test_tile_owners_each_once():
    for tiles, units in ((304, 132), (2374, 132), (9496, 256), (17, 256)):
        programs = helpers.persistent_programs(tiles, units)
        assert all(o == 1 for o in helpers.tile_owners(tiles, programs))
