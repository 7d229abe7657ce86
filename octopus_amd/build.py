"""Build libocto_head.so (the gfx950 HIP kernels and their C ABI) in-tree with hipcc.

    python -m octopus_amd.build [--verbose]

The library lands next to this file, so it travels with the source tree; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libocto_head.so")
SOURCES = ["head_abi.hip", "head_gemm.hip", "head_aux.hip"]
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 generation (the host pass warns it does not know the
# feature; that warning is harmless). -munsafe-fp-atomics: hardware fp32 atomic add.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-munsafe-fp-atomics", "-Wno-unused-result"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def build(verbose: bool = False, extra: list[str] | None = None) -> str:
    """Compile every source into LIB (always recompiles) and return its path."""
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *FLAGS, *(extra or []), "-o", tmp, *[os.path.join(CSRC, s) for s in SOURCES]]
    t0 = time.time()
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{out}")
    os.replace(tmp, LIB)
    if verbose:
        print(out)
        print(f"built {LIB} in {time.time() - t0:.1f} s")
    return LIB


if __name__ == "__main__":
    build(verbose="--verbose" in sys.argv,
          extra=["-Rpass-analysis=kernel-resource-usage"] if "--resources" in sys.argv else None)
