"""GPU: the torch custom ops (torch.ops.ftk.*) give exactly the results of the package functions they
wrap (same C entry points), pass torch.library.opcheck's schema and fake-tensor checks, and one compiles
under torch.compile into a graph that calls the op."""

import pytest
import torch

import kernels.ops  # noqa: F401
from conftest import seeded
from kernels import argmax as A
from kernels import decode_attention as DA
from kernels import linear as L
from kernels import swiglu as S

pytestmark = pytest.mark.gpu


def test_ops_equal_the_functions(cuda):
    x = seeded((3, 1024), seed=1, device=cuda)
    w = seeded((4096, 1024), seed=2, scale=0.02, device=cuda)
    g = seeded((1024,), seed=3, scale=0.1, shift=1.0, device=cuda)
    r = seeded((3, 1024), seed=4, device=cuda)
    assert torch.equal(torch.ops.ftk.linear(x, w), L.linear(x, w))
    r4 = seeded((3, 4096), seed=11, device=cuda)
    assert torch.equal(torch.ops.ftk.linear_residual(x, w, r4), L.linear_residual(x, w, r4))
    assert torch.equal(torch.ops.ftk.rms_norm_linear(x, g, 1e-6, w), L.rms_norm_linear(x, g, 1e-6, w))
    for got, want in zip(torch.ops.ftk.add_rms_norm_linear(x, r, g, 1e-6, w), L.add_rms_norm_linear(x, r, g, 1e-6, w)):
        assert torch.equal(got, want)
    assert torch.equal(torch.ops.ftk.gate_up_swiglu(x, w, g, 1e-6), S.gate_up_swiglu(x, w, g, 1e-6))
    ids, logits = torch.ops.ftk.lm_head_argmax(x, w, g, 1e-6)
    want_ids, want_logits = A.lm_head_argmax(x, w, g, 1e-6, logits=True)
    assert torch.equal(ids, want_ids) and torch.equal(logits, want_logits)
    q = seeded((1, 16, 1, 128), seed=5, device=cuda)
    k, v = seeded((1, 8, 96, 128), seed=6, device=cuda), seeded((1, 8, 96, 128), seed=7, device=cuda)
    pos = torch.tensor([80], device=cuda, dtype=torch.int64)
    assert torch.equal(torch.ops.ftk.decode_attention(q, k, v, pos, 128 ** -0.5),
                       DA.decode_attention(q, k, v, pos, 128 ** -0.5))
    packed = seeded((1, 32 * 128), seed=8, device=cuda)
    gq, gk = seeded((128,), seed=9, scale=0.1, shift=1.0, device=cuda), seeded((128,), seed=10, device=cuda)
    cos, sin = seeded((96, 128), seed=11, device=cuda), seeded((96, 128), seed=12, device=cuda)
    k2, v2 = k.clone(), v.clone()
    got = torch.ops.ftk.rope_attend(packed, gq, gk, 1e-6, 1e-6, cos, sin, pos, k, v, 16, 128 ** -0.5)

    class Norm:
        def __init__(self, weight):
            self.weight, self.variance_epsilon = weight, 1e-6

    want = DA.rope_attend(packed, Norm(gq), Norm(gk), cos, sin, pos, k2, v2, 16, 128 ** -0.5)
    assert torch.equal(got, want) and torch.equal(k, k2) and torch.equal(v, v2)


def test_opcheck_schema_and_fake(cuda):
    x = seeded((2, 512), seed=8, device=cuda)
    w = seeded((256, 512), seed=9, scale=0.02, device=cuda)
    g = seeded((512,), seed=10, scale=0.1, shift=1.0, device=cuda)
    r = seeded((2, 256), seed=12, device=cuda)
    for op, args in ((torch.ops.ftk.linear.default, (x, w)), (torch.ops.ftk.rms_norm_linear.default, (x, g, 1e-6, w)),
                     (torch.ops.ftk.linear_residual.default, (x, w, r)),
                     (torch.ops.ftk.swiglu.default, (x,))):
        torch.library.opcheck(op, args, test_utils=("test_schema", "test_faketensor"))


def test_compiles_into_a_graph(cuda):
    x = seeded((1, 1024), seed=11, device=cuda)
    w = seeded((2048, 1024), seed=12, scale=0.02, device=cuda)
    g = seeded((1024,), seed=13, scale=0.1, shift=1.0, device=cuda)

    def step(h):
        return torch.ops.ftk.rms_norm_linear(h, g, 1e-6, w) * 2

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    assert torch.equal(compiled(x), step(x))
