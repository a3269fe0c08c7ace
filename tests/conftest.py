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


@pytest.fixture(scope="session")
def c1(oracle):
    """Benchmark configuration 1 on the device (256 Qwen2.5-1.5B pages of
    [2, 28, 16, 2, 128] BF16, seed 0) and the oracle's (stream, bound) of every
    segment request of its mixed-bound store (group by group, page by page:
    layers {0,1,2,5,19,20,21} at REL 1e-5, the other 21 at 1e-4)."""
    import numpy as np
    import torch

    import kv_synth

    shape = kv_synth.QWEN25_1P5B_4K
    pages = kv_synth.paged_kv(shape, seed=0, device="cuda")
    host = pages.view(torch.int16).cpu().numpy().view(np.uint16)
    groups = kv_synth.mixed_bound_groups()
    want = []
    for bound, layers in groups:
        streams, sizes, bounds = oracle.compress_batch(
            host, [bound] * host.shape[0], relative=True, threads=8,
            layer_indices=list(layers), source_layers=shape.layers,
            elements_per_layer=shape.elements_per_layer)
        want += list(zip(streams, bounds))
    return dict(shape=shape, pages=pages, groups=groups, want=want)


def fixed_wrapper():
    """A drop-in CuSZpWrapper in the connector's fixed-mode configuration
    (vllm_v1_compressed_offload.py:540-553)."""
    import cuszp_wrapper_cpp as cpp

    cfg = cpp.CompressionConfig(1e-4, True, cpp.DIM_1D, cpp.MODE_FIXED, cpp.TYPE_FLOAT)
    return cpp.CuSZpWrapper(cfg, 0)


def c1_requests(c1):
    """The grouped store's requests for config 1: (inputs, buffers, eps,
    layer index tensors, group sizes); buffers are 8N slices of one slab."""
    import torch

    shape, pages = c1["shape"], c1["pages"]
    inputs, caps, eps, idx, counts = [], [], [], [], []
    for bound, layers in c1["groups"]:
        n = 2 * len(layers) * shape.elements_per_layer
        idx.append(torch.tensor(layers, dtype=torch.long, device="cuda"))
        counts.append(pages.shape[0])
        for p in range(pages.shape[0]):
            inputs.append(pages[p])
            caps.append(8 * n)
            eps.append(bound)
    slab = torch.empty(sum(caps), dtype=torch.uint8, device="cuda")
    bufs, off = [], 0
    for cap in caps:
        bufs.append(slab[off:off + cap])
        off += cap
    return inputs, bufs, eps, idx, counts


def c1_compress(w, c1, req):
    inputs, bufs, eps, idx, counts = req
    shape = c1["shape"]
    return w.compress_batch_fixed_bf16_indexed_groups(
        inputs, bufs, idx, counts, 2, shape.layers, shape.elements_per_layer, eps)
