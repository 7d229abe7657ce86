"""The workspace planners and the GEMMs' tile order under AddressSanitizer and UndefinedBehaviorSanitizer on the CPU:
tests/plan_check.cpp, built with g++ from octopus_amd/csrc/plan.h and tile_order.h (the code libocto_head.so is built
from), sweeps row counts, widths, vocabulary sizes, weight types, gradient sets, gathers, budgets and workspace sizes
and checks every region of each plan against the workspace total and the others, each K-major read extent against its
buffer, and the tile order's coverage of every grid. A planted mistake in a copy of the planner must fail it."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "tests", "plan_check.cpp")
SAN = ["-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
       "-fno-sanitize-recover=all"]

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")


def _build_and_run(src_root, tmp_path):
    exe = str(tmp_path / "plan_check")
    subprocess.run(["g++", *SAN, os.path.join(src_root, "tests", "plan_check.cpp"), "-o", exe], check=True,
                   capture_output=True, text=True, timeout=300)
    return subprocess.run([exe], capture_output=True, text=True, timeout=300)


def test_planners_and_tile_order_pass_the_sanitized_sweep(tmp_path):
    r = _build_and_run(ROOT, tmp_path)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr


def test_a_planted_overlap_fails_the_sweep(tmp_path):
    """A copy of the planner whose staging region is one row short (so the next region overlaps its last row)."""
    copy = tmp_path / "src"
    for rel in ("include/octo_head.h", "octopus_amd/csrc/plan.h", "octopus_amd/csrc/tile_order.h",
                "tests/plan_check.cpp"):
        (copy / rel).parent.mkdir(parents=True, exist_ok=True)
        shutil.copy(os.path.join(ROOT, rel), copy / rel)
    plan = copy / "octopus_amd/csrc/plan.h"
    text = plan.read_text()
    good = "off += align_up((size_t)L.P * L.V_pad * L.esz);"
    assert text.count(good) == 1
    plan.write_text(text.replace(good, "off += align_up((size_t)(L.P - 1) * L.V_pad * L.esz);"))
    r = _build_and_run(str(copy), tmp_path)
    assert r.returncode != 0 and "FAIL" in r.stderr
