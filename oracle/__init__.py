"""CPU oracle for the decode-time skinny BF16 projection path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the `kernels` package, the
HIP library) imports, links or calls anything here. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may use it,
and only as the checker or the timed CPU baseline.

Modules:
  bf16     -- bit-level BF16 round-to-nearest-even in numpy (torch's rule).
  path     -- numpy restatement of the path: projection, RMSNorm prologue,
              SwiGLU epilogue, greedy argmax, split merge.
  torch_cpu -- the reference's own torch-CPU formulation of the same path
              (BF16 F.linear + native-cast-placement norm / SwiGLU / argmax),
              used as the timed CPU baseline and as a second opinion.
  helpers  -- the reference's integer tiling helpers, restated.

How each function is pinned (independent checks, in tests/test_oracle.py):
  bf16.round_bits        -- torch's float->bfloat16 conversion on random,
                            tie, overflow, subnormal and NaN inputs.
  path.project           -- fp64 exact product: <= 0.75 BF16 ulp (the
                            reference's bar, agent/local_cpu/interp/
                            run_numeric.py:59-61); torch CPU F.linear within
                            the 2e-2 + 1e-2|ref| bar; integer-valued inputs whose
                            product is exact must match bit for bit.
  path.rms_norm          -- transformers' Qwen3RMSNorm (library routine):
                            >= 99.9% bit-equal, <= 2 ulp; the wrong-cast
                            detector (reference agent/verify_gpu.py:56-66).
  path.add_rms_norm      -- sum equals torch BF16 addition bit for bit; norm
                            as rms_norm.
  path.swiglu            -- torch F.silu(g) * u on BF16, special inputs
                            [-100, -20, -1, 0, 1, 20, 100, 0.125]
                            (verify_gpu.py:87-89).
  path.argmax_first      -- torch.argmax and brute-force Python loop on tie
                            suites (run_numeric.py:134-145).
  path.merge_splits      -- exact small-integer partials.
  helpers.*              -- the reference's own known answers
                            (gemm.py:333-335, linear.py:359-361).
No oracle function is left "parity unpinned".
"""
