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
