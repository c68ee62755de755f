"""Write the small golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference stores no golden vectors (every reference test draws seeded
inputs at run time), so these fixtures hold seeded inputs together with the
outputs of implementations independent of our oracle:
  * torch's own float -> bfloat16 conversion,
  * fp64 products (numpy) for the projection,
  * transformers' Qwen3RMSNorm (the module the reference's norm must match),
  * torch CPU F.silu(g) * u on BF16 (what run_numeric.py:30 compares with),
  * torch.argmax (first index on ties).
The shapes and special cases are the reference's own test cases:
agent/local_cpu/interp/run_numeric.py:19, :28, :48-49, :137-145, :150-155 and
agent/verify_gpu.py:52, :70, :85-89, :175.
"""

from pathlib import Path

import numpy as np
import torch
from torch.nn import functional as F

OUT = Path(__file__).resolve().parent


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def bf16_round():
    g = gen(11)
    rnd = torch.randn(4096, generator=g) * torch.exp2(torch.randint(-30, 30, (4096,), generator=g).float())
    one = 1.0
    specials = torch.tensor([
        0.0, -0.0, 1.0, -1.0, one + 2 ** -8, one + 3 * 2 ** -8, one + 2 ** -8 + 2 ** -20, -(one + 2 ** -8),
        3.0e38, -3.0e38, 3.4e38, float("inf"), float("-inf"), float("nan"), 1e-40, -1e-40, 1.17e-38, 2 ** -133,
        65504.0, 0.1, 1 / 3, 255.5, 256.5, 257.5,
    ], dtype=torch.float32)
    values = torch.cat([specials, rnd])
    expected = bits(values.to(torch.bfloat16))
    np.savez_compressed(OUT / "bf16_round.npz", values=values.numpy(), expected=expected)


def linear():
    cases = {}
    shapes = [(1, 200, 300), (5, 200, 300), (16, 130, 517), (20, 70, 260), (1, 173, 259), (4, 257, 513),
              (16, 127, 256), (3, 64, 1024)]
    for i, (m, n, k) in enumerate(shapes):
        g = gen(100 + i)
        x = torch.randn(m, k, generator=g).to(torch.bfloat16)
        w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
        exact = x.double() @ w.double().T
        cases[f"x_{m}_{n}_{k}"] = bits(x)
        cases[f"w_{m}_{n}_{k}"] = bits(w)
        cases[f"exact_{m}_{n}_{k}"] = exact.numpy()
        cases[f"torch_{m}_{n}_{k}"] = bits(F.linear(x, w))
    np.savez_compressed(OUT / "linear.npz", **cases)


def rmsnorm():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    cases = {}
    for i, shape in enumerate([(3, 2560), (5, 128), (1, 100), (4, 1024), (2, 4096)]):
        g = gen(200 + i)
        x = (torch.randn(shape, generator=g) * 3).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(shape[-1], generator=g)).to(torch.bfloat16)
        r = torch.randn(shape, generator=g).to(torch.bfloat16)
        norm = Qwen3RMSNorm(shape[-1], eps=1e-6).to(torch.bfloat16)
        with torch.no_grad():
            norm.weight.copy_(w)
            y = norm(x)
            s = x + r
            ys = norm(s)
        key = "_".join(map(str, shape))
        cases[f"x_{key}"], cases[f"w_{key}"], cases[f"r_{key}"] = bits(x), bits(w), bits(r)
        cases[f"y_{key}"], cases[f"sum_{key}"], cases[f"ysum_{key}"] = bits(y), bits(s), bits(ys)
    np.savez_compressed(OUT / "rmsnorm.npz", **cases)


def swiglu():
    cases = {}
    for i, (rows, width) in enumerate([(4, 1500), (3, 64), (2, 3072), (1, 9728)]):
        g = gen(300 + i)
        p = (torch.randn(rows, 2 * width, generator=g) * 2).to(torch.bfloat16)
        p[:, :8] = torch.tensor([-100, -20, -1, 0, 1, 20, 100, 0.125], dtype=torch.bfloat16)
        gate, up = p.chunk(2, -1)
        cases[f"p_{rows}_{width}"] = bits(p)
        cases[f"y_{rows}_{width}"] = bits(F.silu(gate) * up)
    np.savez_compressed(OUT / "swiglu.npz", **cases)


def argmax():
    cases = {}
    for i, shape in enumerate([(3, 1000), (4, 777), (5, 4096), (1, 300), (2, 151936)]):
        g = gen(400 + i)
        key = "_".join(map(str, shape))
        logits = (torch.randn(shape, generator=g) * 4).to(torch.bfloat16)
        coarse = torch.randint(-3, 4, shape, generator=g).to(torch.bfloat16)       # many exact ties
        last = torch.zeros(shape, dtype=torch.bfloat16)
        last[..., -1] = 1.0                                                        # maximum at the very end
        equal = torch.full(shape, -7.0, dtype=torch.bfloat16)                      # all equal
        for name, t in (("rand", logits), ("ties", coarse), ("last", last), ("equal", equal)):
            cases[f"{name}_{key}"] = bits(t)
            cases[f"{name}_{key}_ids"] = t.float().argmax(-1).numpy()
    np.savez_compressed(OUT / "argmax.npz", **cases)


if __name__ == "__main__":
    bf16_round()
    linear()
    rmsnorm()
    swiglu()
    argmax()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
