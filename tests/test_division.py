"""The 16-bit FP8 row quantiser forms x / s without a division (flide_amd/csrc/rowwise.hip,
div_markstein). This CPU test compiles tests/csrc/division_check.c with gcc and checks that claim over
every (x, row maximum) pair of bfloat16 and of float16: the same float32 bits as the correctly rounded
division wherever they can change an e4m3 byte. The kernel itself is compared with the division kernel
byte for byte on the GPU (test_gpu_parity.py::test_quantize_rows_vec_matches_division)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "csrc" / "division_check.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    exe = tmp_path_factory.mktemp("division") / "division_check"
    # no contraction: the check must see exactly the roundings the kernel performs (its fmas are explicit)
    cmd = [gcc, "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", str(SRC), "-o", str(exe), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


@pytest.mark.parametrize("fmt,pairs", [("bf16", 1_065_402_240), ("f16", 1_007_713_280)])
def test_corrected_quotient_matches_division(checker, fmt, pairs):
    r = subprocess.run([str(checker), fmt], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    n, bad, tiny = map(int, r.stdout.split()[-3:])
    assert n == pairs and bad == 0
