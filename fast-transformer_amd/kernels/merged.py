"""A projection's FP32 split partials standing for a BF16 tensor (engine/kernels/merged.py:1-45).

This library's projections finish their split-K inside the workgroup and
always return a BF16 tensor, so they never create a ``Split``. The type and
``source`` are kept so callers and consumers written against the reference's
protocol work unchanged: ``swiglu`` and ``add_rms_norm`` here accept a
``Split`` and sum its partials in split order before rounding once, as
``load_merged`` does (merged.py:37-45).
"""

import torch

from kernels import _native


class Split:
    """A BF16 result handed over unmerged: ``partial`` holds S FP32 planes of M x N partial sums
    whose split-order sum, rounded once, is the tensor of logical ``shape`` (..., N).

    ``splits`` is S and ``count`` the elements of one plane (M N); the slot layout and the two
    properties are the protocol of engine/kernels/merged.py:13-27.
    """

    __slots__ = ("partial", "shape")

    def __init__(self, partial, shape):
        self.partial, self.shape = partial, tuple(shape)

    @property
    def splits(self):
        return self.partial.shape[0]

    @property
    def count(self):
        return self.partial.shape[1] * self.partial.shape[2]


def source(x):
    """What a consumer reads for ``x``: ``(data, S, plane elements, logical shape)``.

    A plain tensor reads as one split of plane size 1; a ``Split`` as its partials
    (the 4-tuple of engine/kernels/merged.py:30-34).
    """
    if isinstance(x, Split):
        return x.partial, x.splits, x.count, x.shape
    return x, 1, 1, tuple(x.shape)


def materialize(x):
    """The BF16 tensor a Split stands for: bf16(sum of partials in split order) (linear.py:81-93)."""
    if not isinstance(x, Split):
        return x
    partial = x.partial.contiguous()
    _native.require_gpu(partial)
    if partial.dtype != torch.float32:
        raise ValueError("Split partials are FP32")
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=partial.device)
    _native.call("ftk_merge_splits_bf16", _native.ptr(partial), x.splits, x.count, _native.ptr(out),
                 _native.stream_of(partial))
    return out
