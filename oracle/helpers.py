"""The reference's integer tiling helpers, restated (test infrastructure only).

``persistent_programs`` fixes how a persistent launch spreads tiles over
compute units; the C library's planner runs the same rule
(``ftk_persistent_programs``, csrc/ftk_plan.h) and tests/test_oracle.py checks
the library's function against this one and the reference's known answers.
``exact_splits`` is the reference's split-K count rule; nothing in this build
splits K across workgroups, so it has no counterpart in the library and is kept
here, pinned to the reference's known answers, for the record of the rule.
"""


def persistent_programs(tiles, units):
    """Programs of a persistent launch over ``tiles`` tiles on ``units`` compute units.

    Every program walks at most depth = ceil(tiles / units) tiles; the fewest
    programs that still reach that depth keep every program busy to the end.
    (engine/kernels/gemm.py:330-338; known answers at gemm.py:333-335 for 132 units:
    304 tiles -> 102 programs, 2374 -> 132, <= 132 -> one each.)
    """
    if tiles <= 0:
        return 0
    depth = -(-tiles // units)
    return -(-tiles // depth)


def tile_owners(tiles, programs):
    """How many programs own each tile when program p walks p, p + programs, ... (each must be 1).

    The write-exactly-once property of agent/local_cpu/shim/references.py:331-347.
    """
    owners = [0] * tiles
    for p in range(programs):
        for t in range(p, tiles, programs):
            owners[t] += 1
    return owners


def exact_splits(k, block_k, wanted):
    """Split count for K in whole BLOCK_K blocks: the largest count <= ``wanted`` that divides the
    block count, so that no split program is left without a block (engine/kernels/gemm.py:428-433;
    known answers at engine/kernels/linear.py:359-361 with 128-wide blocks and 8 wanted: K = 2560 ->
    5, K = 9728 -> 4). A K that is not a whole number of blocks keeps ``wanted``.
    """
    if k % block_k:
        return wanted
    blocks = k // block_k
    splits = wanted
    while blocks % splits:
        splits -= 1
    return splits
