"""Compile libkernrelay.so for gfx950 with hipcc (kernrelay_amd/csrc/Makefile)."""

import os
import subprocess
from pathlib import Path

CSRC = Path(__file__).resolve().parent / "csrc"
LIB = Path(__file__).resolve().parent / "lib" / "libkernrelay.so"


def build(force=True, jobs=None):
    """Run make in csrc/ (always recompiling when force=True); returns the .so path."""
    jobs = jobs or min(8, os.cpu_count() or 1)
    cmd = ["make", "-C", str(CSRC), "-j%d" % jobs]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)
    if not LIB.exists():
        raise RuntimeError("build finished without producing %s" % LIB)
    return LIB


if __name__ == "__main__":
    print(build())
