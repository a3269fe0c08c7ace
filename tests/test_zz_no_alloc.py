"""The no-allocation encoder entry point against the allocating one.

kvszp_compress_batch_fixed_bf16_noalloc keeps its device state in the
library's per-GPU scratch array instead of the context's workspaces; on the
same inputs it must return the same sizes and bounds and write the same
bytes as kvszp_compress_batch_fixed_bf16, call after call (the array keeps
the previous call's words), from any context on the GPU, and refuse calls
beyond its limits before touching the device.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ctx(relative=True, slot_mix=None):
    import os

    import kvszp

    cfg = kvszp.Config(1e-4, 1 if relative else 0, kvszp.DIM_1D,
                       kvszp.MODE_FIXED, kvszp.TYPE_FLOAT)
    old = os.environ.get("KVSZP_SLOT_MIX")
    if slot_mix is not None:
        os.environ["KVSZP_SLOT_MIX"] = slot_mix
    try:
        return kvszp.Context(cfg, 0)
    finally:
        if slot_mix is not None:
            if old is None:
                del os.environ["KVSZP_SLOT_MIX"]
            else:
                os.environ["KVSZP_SLOT_MIX"] = old


def _pages(batch, n, seed):
    g = torch.Generator().manual_seed(seed)
    scale = torch.exp(torch.randn(batch, 1, generator=g))
    x = (torch.randn(batch, n, generator=g) * scale).to(torch.bfloat16)
    x[-1] = 0.8125  # a constant page: every block at rate 31 under REL
    return x.to(DEV)


def _run(kvszp, ctx, noalloc, pages, eps):
    batch, n = pages.shape
    cap = 8 * n + 2048
    slab = torch.full((batch * cap,), 0xAB, dtype=torch.uint8, device=DEV)
    sizes = (ctypes.c_uint64 * batch)()
    bounds = (ctypes.c_float * batch)()
    fn = ctx.compress_noalloc if noalloc else ctx.compress
    rc = fn(kvszp.ptr_array([p.data_ptr() for p in pages]),
            kvszp.ptr_array([slab.data_ptr() + i * cap for i in range(batch)]),
            kvszp.u64_array([cap] * batch), kvszp.f32_array(eps), batch, n,
            torch.cuda.current_stream().cuda_stream, sizes, bounds)
    assert rc == kvszp.OK, kvszp.last_error()
    host = slab.cpu().numpy().reshape(batch, cap)
    return list(sizes), list(bounds), [host[i, :sizes[i]].copy() for i in range(batch)]


@pytest.mark.parametrize("relative", [True, False])
def test_noalloc_matches_allocating_entry_point(relative):
    import kvszp

    ctx = _ctx(relative)
    other = _ctx(relative)   # a second context shares the GPU's scratch array
    # the persistent encoder in unit-major tile order (1024 tiles on a grid
    # of 4 workgroups per compute unit)
    mixed = _ctx(relative, slot_mix="2")
    # two calls in a row, the second smaller; then a long page (min/max
    # pre-pass mode), a call from the other context and one in unit-major order
    for c, (batch, n, seed) in ((ctx, (6, 229376, 1)), (ctx, (3, 36864, 2)),
                                (ctx, (2, 2_500_032, 3)), (other, (5, 8192 * 3 + 64, 4)),
                                (mixed, (128, 65536, 5))):
        pages = _pages(batch, n, seed)
        eps = ([1e-4, 1e-5, 3e-4, 1e-4, 2e-4, 1e-4] * 22)[:batch] if relative else \
              ([1e-3, 2e-2, 5e-4, 1e-3, 1e-3, 1e-3] * 22)[:batch]
        s1, b1, d1 = _run(kvszp, c, True, pages, eps)
        s2, b2, d2 = _run(kvszp, c, False, pages, eps)
        assert s1 == s2, (batch, n)
        assert [np.float32(v) for v in b1] == [np.float32(v) for v in b2]
        for i in range(batch):
            assert np.array_equal(d1[i], d2[i]), (batch, n, i)


def test_noalloc_rejects_calls_beyond_its_limits():
    import kvszp

    ctx = _ctx()
    page = torch.zeros(8192, dtype=torch.bfloat16, device=DEV)
    buf = torch.empty(8 * 8192 + 2048, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    for batch, n in ((4097, 8192), (9, 8192 * 8192)):  # too many pages / tiles
        sizes = (ctypes.c_uint64 * batch)()
        bounds = (ctypes.c_float * batch)()
        rc = ctx.compress_noalloc(
            kvszp.ptr_array([page.data_ptr()] * batch),
            kvszp.ptr_array([buf.data_ptr()] * batch), None,
            kvszp.f32_array([1e-4] * batch), batch, n, stream, sizes, bounds)
        assert rc == kvszp.EINVAL
        assert "no-allocation compress takes at most" in kvszp.last_error()
    # the context still works afterwards
    s, _, d = _run(kvszp, ctx, True, _pages(2, 8192, 7), [1e-4, 1e-4])
    assert all(v > 0 for v in s)


_CTXS = {}


def _cached_ctx(relative):
    if relative not in _CTXS:
        _CTXS[relative] = _ctx(relative)
    return _CTXS[relative]


def _random_pages(rng, batch, n):
    rows = []
    for _ in range(batch):
        kind = rng.choice(["gauss", "gauss", "gauss", "zero", "constant", "wide"])
        if kind == "zero":
            rows.append(np.zeros(n, np.float32))
        elif kind == "constant":
            rows.append(np.full(n, rng.choice([0.8125, -3.5, 1e-3]), np.float32))
        elif kind == "wide":
            rows.append((rng.standard_normal(n) * 10.0 ** rng.integers(-3, 4)).astype(np.float32))
        else:
            rows.append((rng.standard_normal(n) * np.exp(rng.standard_normal())).astype(np.float32))
    return torch.from_numpy(np.stack(rows)).to(torch.bfloat16).to(DEV)


# KVSZP_NOALLOC_SEEDS=n widens the sweep below to seeds 0 .. n-1 (16 by default)
_NOALLOC_SEEDS = range(int(__import__("os").environ.get("KVSZP_NOALLOC_SEEDS", "16")))


@pytest.mark.parametrize("seed", _NOALLOC_SEEDS)
def test_noalloc_random_shapes_match_allocating_entry_point(seed):
    """Seeded shapes, two calls in a row on the same scratch array: segment
    lengths off the block and tile sizes, 1-24 pages, relative and absolute
    bounds (eps 0 and negative fall back to the configured bound), zero and
    constant pages."""
    import kvszp

    rng = np.random.default_rng(1000 + seed)
    relative = bool(rng.integers(2))
    ctx = _cached_ctx(relative)
    for _ in range(2):
        n = int(rng.choice([1, 31, 32, 33, 8191, 8192, 8193, 36864, 65553, 229376]))
        batch = int(rng.integers(1, 25 if n <= 65553 else 9))
        pages = _random_pages(rng, batch, n)
        pool = [1e-4, 1e-5, 3e-3, 0.0, -1.0] if relative else [1e-3, 1e-2, 5e-5, 0.5, 0.0]
        eps = [float(rng.choice(pool)) for _ in range(batch)]
        s1, b1, d1 = _run(kvszp, ctx, True, pages, eps)
        s2, b2, d2 = _run(kvszp, ctx, False, pages, eps)
        assert s1 == s2, (seed, batch, n)
        assert [np.float32(v) for v in b1] == [np.float32(v) for v in b2], (seed, batch, n)
        for i in range(batch):
            assert np.array_equal(d1[i], d2[i]), (seed, batch, n, i)
