"""Host build of the kernels' bit-plane transforms (csrc/kvszp_bits.h),
checked against the reference's stream word layout by naive bit gathers."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import PKG, REPO


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_bit_transforms_match_word_layout(tmp_path):
    exe = tmp_path / "bits_host_test"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-I", os.path.join(PKG, "csrc"),
         os.path.join(REPO, "tests", "host", "bits_host_test.cpp"), "-o",
         str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches=0" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None,
                    reason="needs gcc and g++")
def test_whole_field_quantizer_matches_oracle(tmp_path):
    """The encoder's fast quantizer (field from t alone) against the oracle's
    quantizer over every BF16 value, both variants, boundary reciprocals."""
    obj = tmp_path / "oracle.o"
    subprocess.run(
        ["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
         "-fopenmp", "-c", os.path.join(REPO, "oracle", "kvszp_oracle.c"),
         "-o", str(obj)], check=True)
    exe = tmp_path / "quant_field_test"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I",
         os.path.join(PKG, "csrc"), "-I", os.path.join(REPO, "oracle"),
         os.path.join(REPO, "tests", "host", "quant_field_test.cpp"), str(obj),
         "-fopenmp", "-lm", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches=0" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_tile_plan_walk(tmp_path):
    """Every tile of random calls placed by the kernels' lookup, with bounds
    checks, on plans built by the C-ABI's own functions (csrc/kvszp_plan.h);
    the launch check accepts them and rejects plans that do not add up."""
    exe = tmp_path / "tile_plan_test"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-I", os.path.join(PKG, "csrc"),
         os.path.join(REPO, "tests", "host", "tile_plan_test.cpp"), "-o", str(exe)],
        check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches=0" in out.stdout
