"""Epoch tags across their wrap-around.

The encoders' cross-workgroup words (look-back, min/max, job flags) carry the
epoch of the launch that wrote them, so no call clears them; when a context's
tags run out (2^30 - 2 launches; for the no-allocation entry point, launches
on the GPU), every tagged word is cleared and the tags start again.  One of
those words is the abort mark: the epoch of the last launch whose
time-bounded waits gave up.  A mark left standing across the wrap would make
every wait of the later launch with the same epoch give up without telling
the host, and that call would return without having written its streams.

KVSZP_EPOCH_LIMIT lowers the limit to a few launches, so that the test
crosses the wrap several times.  Launches before each wrap are made to give
up from the host (a wait bound of zero; every kernel still exits normally),
the launches after it run with the normal bound (KVSZP_SAFE_CALLS=0: no call
skips the persistent encoder because an earlier one gave up).  Output buffers are filled
with 0xAB before every call, so that a call which wrote nothing cannot pass
on the previous call's bytes.  Every stream is checked against the oracle.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import c1_compress, c1_requests, fixed_wrapper

pytestmark = pytest.mark.gpu

DEV = "cuda"
LIMIT = 5          # epochs per cycle of the test contexts
FORCED = 3         # calls with a zero wait bound before each stretch of normal calls
NORMAL = 2 * LIMIT  # normal calls: every epoch value of the next cycle at least once


def _check_c1(c1, bufs, sizes, bounds):
    host = [b.cpu().numpy() for b in bufs]
    for k, (stream, eb) in enumerate(c1["want"]):
        assert np.float32(bounds[k]) == np.float32(eb), k
        assert sizes[k] == stream.size, k
        assert np.array_equal(host[k][:sizes[k]], stream), k


def test_grouped_store_across_epoch_wraps(c1, monkeypatch):
    """The full configuration-1 store (512 segments, persistent encoder with
    the fused bound exchange) through two wraps of a 5-epoch context."""
    monkeypatch.setenv("KVSZP_EPOCH_LIMIT", str(LIMIT))
    monkeypatch.setenv("KVSZP_SAFE_CALLS", "0")  # every call tries the persistent encoder
    w = fixed_wrapper()
    ctx = w._ctx
    req = c1_requests(c1)
    slab = req[1][0]._base  # the buffers are slices of one slab
    assert slab is not None
    redone = ctx.reencode_count()
    for cycle in range(2):
        for wait_us, calls in ((0.0, FORCED), (200.0, NORMAL)):
            ctx.set_wait_bound(wait_us)
            for call in range(calls):
                slab.fill_(0xAB)
                ok, sizes, bounds = c1_compress(w, c1, req)
                assert ok, (cycle, wait_us, call)
                _check_c1(c1, req[1], sizes, bounds)
    # the forced calls did give up and were encoded again
    assert ctx.reencode_count() > redone


def test_noalloc_across_epoch_wraps(oracle, monkeypatch):
    """The no-allocation entry point, whose tags come from one counter per
    GPU, through two wraps of a 5-epoch limit."""
    import kvszp

    import kv_synth

    monkeypatch.setenv("KVSZP_EPOCH_LIMIT", str(LIMIT))
    monkeypatch.setenv("KVSZP_SAFE_CALLS", "0")
    cfg = kvszp.Config(1e-4, 1, kvszp.DIM_1D, kvszp.MODE_FIXED, kvszp.TYPE_FLOAT)
    ctx = kvszp.Context(cfg, 0)
    pages = kv_synth.paged_kv(kv_synth.QWEN25_1P5B_4K, seed=5, device=DEV, tokens=16 * 64)
    batch, n = pages.shape
    host = pages.view(torch.int16).cpu().numpy().view(np.uint16)
    eps = [1e-4 if i % 3 else 1e-5 for i in range(batch)]
    streams, _, want_bounds = oracle.compress_batch(host, eps, relative=True, threads=8)
    cap = 8 * n
    slab = torch.empty(batch * cap, dtype=torch.uint8, device=DEV)
    sizes = (ctypes.c_uint64 * batch)()
    bounds = (ctypes.c_float * batch)()
    stream = torch.cuda.current_stream().cuda_stream
    args = (kvszp.ptr_array([p.data_ptr() for p in pages]),
            kvszp.ptr_array([slab.data_ptr() + i * cap for i in range(batch)]),
            kvszp.u64_array([cap] * batch), kvszp.f32_array(eps), batch, n, stream,
            sizes, bounds)
    redone = ctx.reencode_count()
    for cycle in range(2):
        for wait_us, calls in ((0.0, FORCED), (200.0, NORMAL)):
            ctx.set_wait_bound(wait_us)
            for call in range(calls):
                slab.fill_(0xAB)
                rc = ctx.compress_noalloc(*args)
                assert rc == kvszp.OK, kvszp.last_error()
                got = slab.cpu().numpy().reshape(batch, cap)
                for i in range(batch):
                    assert np.float32(bounds[i]) == np.float32(want_bounds[i]), (cycle, call, i)
                    assert sizes[i] == streams[i].size, (cycle, call, i)
                    assert np.array_equal(got[i, :sizes[i]], streams[i]), (cycle, call, i)
    assert ctx.reencode_count() > redone


def test_wait_bound_setter_rejects_bad_values():
    import kvszp

    cfg = kvszp.Config(1e-4, 1, kvszp.DIM_1D, kvszp.MODE_FIXED, kvszp.TYPE_FLOAT)
    ctx = kvszp.Context(cfg, 0)
    for bad in (-1.0, float("nan"), 2e6):
        with pytest.raises(kvszp.KvszpError):
            ctx.set_wait_bound(bad)
    ctx.set_wait_bound(0.0)
    ctx.set_wait_bound(1e6)
