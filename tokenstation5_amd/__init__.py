"""ts5's token loop on MI355X (gfx950): libts5hip.so and its Python binding.

The product is the HIP library built from tokenstation5_amd/csrc behind the C
ABI in include/ts5hip.h; ts5hip.py binds it for tests and benchmarks.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build(jobs: int = 8) -> str:
    """Compiles libts5hip.so for gfx950 in-tree; returns its path."""
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "csrc"), f"-j{jobs}"], check=True)
    return os.path.join(HERE, "libts5hip.so")
