"""The selection policy on the host (kernels/linear.py, engine/kernels/linear.py:412-449): the
process budget and the inheritance of a choice across row counts. ``run`` stands in for the
kernels with a CPU computation, so the policy is checked without a GPU."""

import pytest
import torch

from kernels import _native
from kernels import linear as L

DEV = torch.device("cpu")
RING = (_native.KIND_RING, 16, 2, 1, 8)
QUAD = (_native.KIND_QUAD, 8, 0, 1, 8)


@pytest.fixture
def fresh(monkeypatch):
    monkeypatch.setattr(L, "_CHOICES", {})
    monkeypatch.setattr(L, "_VALIDATED", {})
    monkeypatch.setattr(L, "inherited", {})
    monkeypatch.setattr(L, "_TUNING_DEADLINE", 0.0)  # the budget is spent
    yield


def _run(bad=(), missing=()):
    """A stand-in for one projection launch: exact for good choices, off by 5 % for ``bad`` ones,
    raising the planner's error for ``missing`` ones (no such launch at this row count)."""
    def run(choice, w, inp):
        if choice in missing:
            raise _native.FtkError("ftk_project_rows_bf16", _native.FTK_ERR_INVALID)
        y = inp.float() @ w.float().T
        return y * 1.05 if choice in bad else y
    return run


def _native_gemm(w, inp):
    """The native GEMM's output, the reference every inherited choice must agree with."""
    return inp.float() @ w.float().T


def _operands(m, n=64, k=32):
    g = torch.Generator().manual_seed(m)
    return torch.randn((m, k), generator=g).to(torch.bfloat16), torch.randn((n, k), generator=g).to(torch.bfloat16)


def test_past_the_budget_a_verify_block_inherits_an_agreeing_choice(fresh):
    x, w = _operands(5)
    L._CHOICES[(DEV, 8, 64, 32)] = RING
    assert L._choose("linear", x, w, _run(), _native_gemm) == RING
    assert L.inherited[(DEV, 5, 64, 32)] == RING
    assert L._VALIDATED[(DEV, 5, 64, 32)][0] == (0.0, RING)


def test_a_choice_that_disagrees_or_does_not_exist_is_not_inherited(fresh):
    x, w = _operands(5)
    L._CHOICES[(DEV, 8, 64, 32)] = RING
    L._CHOICES[(DEV, 16, 64, 32)] = QUAD
    assert L._choose("linear", x, w, _run(bad=(RING,), missing=(QUAD,)), _native_gemm) is None
    assert L.inherited[(DEV, 5, 64, 32)] is None


def test_only_the_same_operation_and_weight_shape_at_more_than_4_rows(fresh):
    x, w = _operands(5)
    L._CHOICES[(DEV, 4, 64, 32)] = RING              # 4 rows: not a verify block
    L._CHOICES[(DEV, 8, 128, 32)] = RING             # another weight shape
    L._CHOICES[("norm", DEV, 8, 64, 32)] = RING      # another operation
    L._CHOICES[(DEV, 12, 64, 32)] = "native"          # native is not a launch choice
    assert L._choose("linear", x, w, _run(), _native_gemm) is None
    L._CHOICES[("norm", DEV, 8, 64, 32)] = QUAD
    assert L._choose("norm", x, w, _run(), _native_gemm) == QUAD


@pytest.mark.parametrize("m,default,missing", [(3, None, ()), (1, None, ()), (40, "native", ()),
                                               (20, "native", (RING,))])
def test_other_row_counts_take_their_untuned_default(fresh, m, default, missing):
    """4 rows or fewer, or more than MAX_ROWS, never inherit; 17..32 rows inherit only a launch
    that exists there (RING stops at 16 rows), else take the native GEMM."""
    x, w = _operands(m)
    L._CHOICES[(DEV, 8, 64, 32)] = RING
    assert L._choose("linear", x, w, _run(missing=missing), _native_gemm) == default
    assert L._VALIDATED[(DEV, m, 64, 32)] == [(0.0, default)]
