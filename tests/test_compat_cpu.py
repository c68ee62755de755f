"""The reference's engine imports load against this package (engine/layers.py:7-11,
engine/decode.py:12-20, engine/engine.py:9), and the out-of-scope names fail loudly."""

import pytest

from kernels import pdl, spec
from kernels.argmax import argmax, fused_argmax, greedy_tokens  # noqa: F401
from kernels.decode_attention import block_attention, decode_attention  # noqa: F401
from kernels.linear import MAX_ROWS, keep_native, linear  # noqa: F401
from kernels.qk_rope import qk_rope_cache  # noqa: F401
from kernels.rmsnorm import add_rms_norm, embed_rms_norm, rms_norm  # noqa: F401
from kernels.swiglu import swiglu  # noqa: F401
from kernels.tune import knobs  # noqa: F401


def test_pdl_reports_off_as_the_reference_does_without_it():
    assert pdl.ENABLED is False and pdl.install() is False
    assert pdl.self_test("cuda:0") is False
    pdl.uninstall()
    pdl.wait()


def test_speculation_names_raise():
    for fn, args in ((spec.propose, (None,) * 8), (spec.within_margin, (None,) * 4), (spec.settle, (None,) * 10),
                     (spec.relocate, (None,) * 3), (block_attention, (None,) * 6)):
        with pytest.raises(NotImplementedError):
            fn(*args)
