"""Builds libllmdot_hip.so in-tree for gfx950 (hipcc via dotllm_amd/csrc/Makefile)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(jobs: int = 8, arch: str = "gfx950", force: bool = True) -> str:
    """Compiles every HIP source; returns the path of the shared library."""
    env = dict(os.environ)
    args = ["make", "-C", CSRC, f"-j{jobs}", f"ARCH={arch}"]
    if force:
        subprocess.run(["make", "-C", CSRC, "clean"], check=True, env=env, stdout=subprocess.DEVNULL)
    subprocess.run(args, check=True, env=env)
    return os.path.join(HERE, "libllmdot_hip.so")


if __name__ == "__main__":
    print(build())
