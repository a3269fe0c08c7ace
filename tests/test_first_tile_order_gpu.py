"""GPU parity: the persistent encoder's two first-tile orders.

Workgroup b of a persistent encoder launch walks tiles f, f + G, f + 2G, ...
from a first tile f.  Launches of at least 16 rounds of the grid take the
unit-major order (each compute unit holds consecutive tiles,
`persistent_first_tile` in csrc/kvszp_plan.h), shorter ones f = b.  The
order changes which workgroup encodes a tile, never the stream: the same
pages are stored under KVSZP_SLOT_MIX=0 (always f = b), 1 (the default rule)
and 2 (the unit-major order whenever the grid allows), on a launch of ~5.5
rounds (the rule keeps f = b) and one of ~17 rounds (the rule mixes), and
every stream is compared with the oracle byte for byte and the restored
values bit for bit.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
N = 229376  # one Qwen2.5-1.5B 4K page: 28 tiles


@pytest.fixture(scope="module")
def cpp():
    import cuszp_wrapper_cpp

    return cuszp_wrapper_cpp


def make(cpp, mode: str):
    old = os.environ.get("KVSZP_SLOT_MIX")
    os.environ["KVSZP_SLOT_MIX"] = mode
    try:
        cfg = cpp.CompressionConfig(1e-4, True, cpp.DIM_1D, cpp.MODE_FIXED,
                                    cpp.TYPE_FLOAT)
        w = cpp.CuSZpWrapper(cfg, 0)
    finally:
        if old is None:
            del os.environ["KVSZP_SLOT_MIX"]
        else:
            os.environ["KVSZP_SLOT_MIX"] = old
    return w


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def pages(batch, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    scales = torch.exp(torch.randn(batch, 1, generator=g))
    return (torch.randn(batch, N, generator=g) * scales).to(torch.bfloat16).to(DEV)


def store_restore(cpp, w, x, eps):
    batch = x.shape[0]
    cap = cpp.CuSZpWrapper.estimate_compressed_buffer_size(4 * N)
    slab = torch.full((batch, cap), 0xAB, dtype=torch.uint8, device=DEV)
    bufs = list(slab)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(x), bufs, eps)
    assert ok
    out = torch.full((batch * N,), 1.75, dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, N, bounds)
    assert w.synchronize()
    return ([bufs[i][:sizes[i]].cpu().numpy() for i in range(batch)], list(bounds),
            u16(out))


# 300 pages: 8400 tiles, ~5.5 rounds of a 1536-workgroup grid; 920 pages:
# 25760 tiles, ~16.8 rounds.
@pytest.mark.parametrize("batch", [300, 920])
def test_first_tile_orders_give_the_oracle_streams(cpp, oracle, batch):
    x = pages(batch, seed=batch)
    eps = [1e-4 if i % 3 else 1e-5 for i in range(batch)]
    runs = {m: store_restore(cpp, make(cpp, m), x, eps) for m in ("0", "1", "2")}
    bits = u16(x)
    pre = np.full(N, 0x3FE0, dtype=np.uint16)  # 1.75
    ref = runs["0"]
    for i in range(batch):
        eb = oracle.relative_bound(bits[i], N, eps[i])
        assert np.float32(ref[1][i]) == np.float32(eb), (i, ref[1][i], eb)
        want = oracle.compress_page(bits[i], N, float(eb))
        for m, got in runs.items():
            assert np.array_equal(got[0][i], want), f"mode {m}, page {i}: stream differs"
            assert np.float32(got[1][i]) == np.float32(eb), (m, i)
        if i % 16 == 0:
            restored = oracle.decompress_contiguous(want, N, float(eb), 1, pre.copy())
            assert np.array_equal(ref[2][i * N:(i + 1) * N], restored), f"page {i} restored"
    for m in ("1", "2"):
        assert np.array_equal(runs[m][2], ref[2]), f"mode {m}: restored pages differ"
