"""GPU parity: job tables carried in the persistent kernels' arguments.

Persistent launches whose job table fits an ArgTable (14 336 bytes: up to
597 records of 24 bytes) take it in the kernel arguments instead of a table
copy on the stream; 16 jobs or fewer use the parameter block's own inline
records, larger tables the uploaded copy.  Batches on either side of each
limit are stored and restored with the tables carried in the arguments and,
in a second context (KVSZP_ARG_TABLES=0), with every table uploaded: every
stream is compared byte for byte with the oracle and between the two
contexts, every restored value bit for bit with the oracle.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
N = 32768  # four tiles per job: 597 jobs make a persistent restore (> 2048 tiles)


@pytest.fixture(scope="module")
def cpp():
    import cuszp_wrapper_cpp

    return cuszp_wrapper_cpp


def make(cpp, arg_tables: bool):
    old = os.environ.get("KVSZP_ARG_TABLES")
    os.environ["KVSZP_ARG_TABLES"] = "3" if arg_tables else "0"
    try:
        cfg = cpp.CompressionConfig(1e-4, True, cpp.DIM_1D, cpp.MODE_FIXED,
                                    cpp.TYPE_FLOAT)
        w = cpp.CuSZpWrapper(cfg, 0)
    finally:
        if old is None:
            del os.environ["KVSZP_ARG_TABLES"]
        else:
            os.environ["KVSZP_ARG_TABLES"] = old
    return w


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def pages(batch, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    scales = torch.exp(torch.randn(batch, 1, generator=g))
    return (torch.randn(batch, N, generator=g) * scales).to(torch.bfloat16).to(DEV)


def store_restore(cpp, w, x, eps):
    batch = x.shape[0]
    cap = max(cpp.CuSZpWrapper.estimate_compressed_buffer_size(4 * N),
              1024 + 128 * (N // 32))
    bufs = [torch.full((cap,), 0xAB, dtype=torch.uint8, device=DEV) for _ in range(batch)]
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(x), bufs, eps)
    assert ok
    out = torch.full((batch * N,), 1.75, dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, N, bounds)
    assert w.synchronize()
    streams = [bufs[i][:sizes[i]].cpu().numpy() for i in range(batch)]
    return streams, list(bounds), u16(out)


# 16 and 17 jobs: inline records / ArgTable for the store; 597 and 598
# jobs: the largest ArgTable and the first uploaded table, for the store
# and for the persistent restore
@pytest.mark.parametrize("batch", [16, 17, 597, 598])
def test_arg_tables_match_oracle_and_uploaded_tables(cpp, oracle, batch):
    x = pages(batch, seed=batch)
    eps = [1e-4 if i % 4 else 1e-5 for i in range(batch)]
    got = store_restore(cpp, make(cpp, True), x, eps)
    ref = store_restore(cpp, make(cpp, False), x, eps)
    bits = u16(x)
    pre = np.full(N, 0x3FE0, dtype=np.uint16)  # 1.75
    for i in range(batch):
        eb = oracle.relative_bound(bits[i], N, eps[i])
        assert np.float32(got[1][i]) == np.float32(eb), (i, got[1][i], eb)
        want = oracle.compress_page(bits[i], N, float(eb))
        assert np.array_equal(got[0][i], want), f"page {i}: stream differs from the oracle"
        assert np.array_equal(ref[0][i], want), f"page {i}: uploaded-table stream differs"
        restored = oracle.decompress_contiguous(want, N, float(eb), 1, pre.copy())
        assert np.array_equal(got[2][i * N:(i + 1) * N], restored), f"page {i} restored"
    assert np.array_equal(got[2], ref[2])
