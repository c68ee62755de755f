"""The reference's integer tiling helpers, restated (test infrastructure only).

These fix how a persistent launch spreads tiles over compute units and how a
split-K count is made to tile K exactly. The host planner in the product
(kernels/plan.py and the C library's planner) is checked against them.
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


def exact_splits(k, block_k, wanted):
    """Largest split count <= wanted whose chunks tile K with whole BLOCK_K blocks.

    (engine/kernels/gemm.py:428-433; known answers at engine/kernels/linear.py:359-361:
    K = 2560, BLOCK_K = 128, wanted 8 -> 5; K = 9728 -> 4.) A ragged K keeps ``wanted``.
    """
    if k % block_k:
        return wanted
    blocks = k // block_k
    return max(s for s in range(1, wanted + 1) if blocks % s == 0)


def tile_owners(tiles, programs):
    """How many programs own each tile when program p walks p, p + programs, ... (each must be 1).

    The write-exactly-once property of agent/local_cpu/shim/references.py:331-347.
    """
    owners = [0] * tiles
    for p in range(programs):
        for t in range(p, tiles, programs):
            owners[t] += 1
    return owners
