"""Programmatic dependent launch: off on MI355X (engine/kernels/pdl.py, for import compatibility).

The reference's pdl module patches Triton's CUDA launcher so that a kernel may
launch while its predecessor drains (a Hopper launch attribute), and keeps it
only if ``self_test`` passes. HIP on gfx950 has no such launch attribute, and
the reference ships with it disabled anyway (``ENABLED = False``,
engine/kernels/pdl.py:27-32: it measured batch-1 passes 13 % slower with it).
So this module keeps the reference's names and reports PDL as off: ``self_test``
returns False, exactly what the reference returns when PDL is unavailable, and
engine code that calls it runs on.
"""

FLAG = "FASTY_PDL"
ENABLED = False


def wait():
    """No-op: there is no dependent launch to wait for (the reference's is a Triton device function)."""


def install():
    """The launcher patch: nothing to install on HIP. Returns False (not installed)."""
    return False


def uninstall():
    """Nothing was installed."""


def self_test(device, count=1024):
    """PDL stays off (engine/kernels/pdl.py:120-160 returns False whenever it cannot be used)."""
    print("PDL: off (no programmatic dependent launch on this device)", flush=True)
    return False
