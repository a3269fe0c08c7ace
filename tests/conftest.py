"""Shared test setup.

* ``gpu`` marks tests that need an MI355X (run with ``-m gpu``).
* The codec package directory and ``oracle/`` are put on ``sys.path`` the way
  the reference's connector puts its module directory there before
  ``import cuszp_wrapper_cpp`` (vllm_v1_compressed_offload.py:41-45).
"""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(
    REPO,
    "reducing-pcie-bottlenecks-for-llm-serving-with-cuszp-compressed-kv-cache-transfer_amd")
ORACLE = os.path.join(REPO, "oracle")
GOLDEN = os.path.join(REPO, "tests", "golden")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o
