"""MI355X (gfx950) kernels for the decode-time skinny BF16 projection path.

A drop-in for the reference's ``kernels`` package (engine/kernels/__init__.py:1-6):
put this directory's parent on ``sys.path`` and ``from kernels.linear import
linear``, ``from kernels.swiglu import swiglu`` ... resolve here, with the
reference's names and signatures. Under them, every operator is a hand-written
HIP kernel in libftk.so (C ABI: include/ftk.h), loaded by ``kernels._native``.
"""
