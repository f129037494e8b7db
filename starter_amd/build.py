"""Build ``starter_amd/kernels/libqwen_fused.so`` from ``starter_amd/csrc/*.hip``.

Every source is compiled for gfx950 only, with:

* ``-ffp-contract=off`` - no silent multiply-add fusion; the kernels round to
  bf16 at exactly the points the reference does, and an FMA would change the
  f32 value being rounded;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` - no packed-f32 VALU
  instructions (the host pass warns that it does not know the feature; that
  warning is harmless);
* HIP's default correctly rounded f32 divide and sqrt.

A second library, ``starter_amd/kernels/libqwen_fused_phases.so``, holds only
the decode attention built with ``-DQF_PHASE_STAMPS``: the same kernels plus
an instrumented entry point that records per-workgroup phase timestamps
(``starter_amd.attention_phases`` reads them).  Nothing in the product loads
it.

Run ``python -m starter_amd.build`` or call :func:`build`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
OBJ_DIR = PACKAGE / "_build"
LIBRARY = PACKAGE / "kernels" / "libqwen_fused.so"
PHASES_LIBRARY = PACKAGE / "kernels" / "libqwen_fused_phases.so"
PHASES_SOURCE = "decode_attention.hip"
SOURCES = ("rmsnorm.hip", "silu_mul.hip", "qk_norm_rope.hip", "embedding.hip", "skinny_gemm.hip",
           "decode_attention.hip", "prefill_attention.hip", "row_gemv.hip")
ARCH = "gfx950"

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-I", str(ROOT / "include"),
]
# Per-source additions.  The attention kernels rescale their f32
# accumulators between matrix-core products; with the accumulators in
# ordinary VGPRs (instead of AGPRs) no copies are needed between the two
# register files (prefill 1.3x, decode 2% faster, same occupancy).
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
EXTRA_FLAGS = {
    "decode_attention.hip": _VGPR_MFMA,
    "prefill_attention.hip": _VGPR_MFMA,
}


def hipcc() -> str:
    path = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError(f"hipcc not found (looked for {path})")
    return path


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass always warns about the device-only packed-fp32 feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library (and the phase
    timing library); return the product library's path."""
    cc = hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    jobs = []
    for name in SOURCES:
        obj = OBJ_DIR / (Path(name).stem + ".o")
        jobs.append((obj, [cc, *COMPILE_FLAGS, *EXTRA_FLAGS.get(name, ()), "-c", str(CSRC / name),
                           "-o", str(obj)]))
    phases_obj = OBJ_DIR / (Path(PHASES_SOURCE).stem + "_phases.o")
    phases_job = (phases_obj, [cc, *COMPILE_FLAGS, *EXTRA_FLAGS.get(PHASES_SOURCE, ()),
                               "-DQF_PHASE_STAMPS", "-c", str(CSRC / PHASES_SOURCE),
                               "-o", str(phases_obj)])
    workers = min(len(jobs) + 1, max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        for fut in [pool.submit(_run, cmd, verbose) for _, cmd in (*jobs, phases_job)]:
            fut.result()
    for library, objects in ((LIBRARY, [obj for obj, _ in jobs]), (PHASES_LIBRARY, [phases_obj])):
        tmp = library.with_suffix(".so.tmp")
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
              *[str(obj) for obj in objects]], verbose)
        os.replace(tmp, library)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
