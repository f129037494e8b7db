"""Build the CPU oracle ``oracle/libqf_oracle.so`` (test infrastructure only).

``gcc -O2 -ffp-contract=off -fno-fast-math``: every f32 operation of the
restatement is rounded exactly where the source says, with no FMA contraction.
The reference (jadenpxrk/starter) is Python/Triton with no C or C++ sources,
so there is no ``oracle/_ref`` build: nothing of the reference compiles here.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

ORACLE = Path(__file__).resolve().parent
SOURCE = ORACLE / "qf_oracle.c"
LIBRARY = ORACLE / "libqf_oracle.so"
FLAGS = ["-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
         "-fvisibility=hidden", "-Wall", "-Wextra"]


def build(verbose: bool = False) -> Path:
    cc = os.environ.get("CC") or shutil.which("gcc") or "gcc"
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [cc, *FLAGS, "-o", str(tmp), str(SOURCE), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
