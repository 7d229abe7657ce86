"""Build libocto_head.so (the gfx950 HIP kernels and their C ABI) in-tree with hipcc.

    python -m octopus_amd.build [--verbose] [--resources]

Each translation unit compiles to its own object in parallel, then one link. The library lands next to this
file, so it travels with the source tree; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
import time
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libocto_head.so")
SOURCES = ["head_abi.hip", "head_gemm.hip", "head_aux.hip", "tree_pairs.hip"]
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 generation (the host pass warns it does not know the
# feature; that warning is harmless). -munsafe-fp-atomics: hardware fp32 atomic add.
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-munsafe-fp-atomics", "-Wno-unused-result"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False, extra: list[str] | None = None, out: str = LIB) -> str:
    """Compile every source and link `out` (always recompiles). Returns its path."""
    t0 = time.time()
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="octo_build_") as tmp:
        objs = [os.path.join(tmp, s.replace(".hip", ".o")) for s in SOURCES]
        cmds = [[cc, *FLAGS, *(extra or []), "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(len(cmds)) as pool:
            logs = list(pool.map(_run, cmds))
        linked = os.path.join(tmp, "lib.so")
        logs.append(_run([cc, *FLAGS, "-shared", *objs, "-o", linked]))
        shutil.copyfile(linked, out + ".tmp")
        os.chmod(out + ".tmp", 0o755)
        os.replace(out + ".tmp", out)
    if verbose:
        text = "\n".join(x for x in logs if x.strip())
        if text:
            print(text)
        print(f"built {out} in {time.time() - t0:.1f} s")
    return out


if __name__ == "__main__":
    build(verbose="--verbose" in sys.argv,
          extra=["-Rpass-analysis=kernel-resource-usage"] if "--resources" in sys.argv else None)
