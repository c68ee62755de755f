"""The torch custom ops (kernels/ops.py) register, and their fake implementations give the output
shapes under FakeTensorMode without touching a device. No kernel runs here."""

import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import kernels.ops  # noqa: F401  (registers torch.ops.ftk.*)

NAMES = ("linear", "linear_residual", "rms_norm_linear", "add_rms_norm_linear", "gate_up_swiglu", "lm_head_argmax", "rms_norm",
         "add_rms_norm", "swiglu", "argmax", "decode_attention", "qk_rope_cache", "rope_attend")


def test_every_op_is_registered():
    for name in NAMES:
        assert hasattr(torch.ops.ftk, name), name


def test_fake_shapes():
    bf = torch.bfloat16
    with FakeTensorMode():
        x = torch.empty(5, 4096, dtype=bf)
        w = torch.empty(6144, 4096, dtype=bf)
        g = torch.empty(4096, dtype=bf)
        assert torch.ops.ftk.linear(x, w).shape == (5, 6144)
        assert torch.ops.ftk.linear_residual(x, w, torch.empty(5, 6144, dtype=bf)).shape == (5, 6144)
        assert torch.ops.ftk.rms_norm_linear(x, g, 1e-6, w).shape == (5, 6144)
        y, s = torch.ops.ftk.add_rms_norm_linear(x, x, g, 1e-6, w)
        assert y.shape == (5, 6144) and s.shape == (5, 4096)
        assert torch.ops.ftk.gate_up_swiglu(x, torch.empty(24576, 4096, dtype=bf), g, 1e-6).shape == (5, 12288)
        ids, logits = torch.ops.ftk.lm_head_argmax(x, torch.empty(1000, 4096, dtype=bf), g, 1e-6)
        assert ids.shape == (5,) and ids.dtype == torch.int64 and logits.shape == (5, 1000)
        assert torch.ops.ftk.rms_norm(x, g, 1e-6).shape == (5, 4096)
        n, s = torch.ops.ftk.add_rms_norm(x, x, g, 1e-6)
        assert n.shape == s.shape == (5, 4096)
        assert torch.ops.ftk.swiglu(torch.empty(5, 2 * 3072, dtype=bf)).shape == (5, 3072)
        assert torch.ops.ftk.argmax(torch.empty(5, 1000, dtype=bf)).shape == (5,)
        q = torch.empty(2, 32, 1, 128, dtype=bf)
        cache = torch.empty(2, 8, 64, 128, dtype=bf)
        pos = torch.empty(1, dtype=torch.int64)
        assert torch.ops.ftk.decode_attention(q, cache, cache, pos, 0.088).shape == (2, 1, 32, 128)
        packed = torch.empty(2, 1, (32 + 16) * 128, dtype=bf)
        rope_q = torch.ops.ftk.qk_rope_cache(packed, torch.empty(128, dtype=bf), torch.empty(128, dtype=bf), 1e-6,
                                             1e-6, torch.empty(1, 1, 128, dtype=bf), torch.empty(1, 1, 128, dtype=bf),
                                             pos, cache, torch.empty_like(cache), 32)
        assert rope_q.shape == (2, 1, 32, 128)
        table = torch.empty(64, 128, dtype=bf)
        out = torch.ops.ftk.rope_attend(packed.view(2, -1), torch.empty(128, dtype=bf), torch.empty(128, dtype=bf),
                                        1e-6, 1e-6, table, table, pos, cache, torch.empty_like(cache), 32, 0.088)
        assert out.shape == (2, 1, 32, 128)
