"""The in-scope names the reference's engine imports load from this package
(engine/layers.py:7-11, engine/decode.py:12-20), with the reference's call signatures."""

import inspect

from kernels.argmax import argmax, fused_argmax, greedy_tokens
from kernels.decode_attention import decode_attention
from kernels.linear import MAX_ROWS, keep_native, linear
from kernels.merged import Split, source
from kernels.rmsnorm import add_rms_norm, embed_rms_norm, rms_norm
from kernels.swiglu import swiglu
from kernels.tune import Knob, knobs, pick, register


def test_signatures_match_the_reference_call_sites():
    params = lambda fn: list(inspect.signature(fn).parameters)  # noqa: E731
    assert params(linear) == ["x", "weight", "split_ok"]
    assert params(keep_native) == ["rows", "weight"]
    assert MAX_ROWS == 32
    assert params(rms_norm) == ["x", "weight", "eps"]
    assert params(add_rms_norm) == ["x", "residual", "weight", "eps"]
    assert params(embed_rms_norm) == ["token_ids", "table", "weight", "eps"]
    assert params(swiglu) == ["packed"]
    assert params(argmax)[:1] == ["logits"] and "top" in params(argmax)
    assert params(fused_argmax)[:2] == ["x", "weight"]
    assert params(greedy_tokens)[:3] == ["x", "weight", "linear"]
    assert params(decode_attention) == ["query", "key", "value", "position", "scale"]
    assert params(register) == ["name", "rows", "weight", "options", "get", "select"]
    assert params(pick) == ["key", "default", "options", "launch"]
    assert callable(knobs) and callable(source)
    assert set(Knob.__slots__) == {"name", "rows", "weight", "options", "get", "select"}
    assert set(Split.__slots__) == {"partial", "shape"}
