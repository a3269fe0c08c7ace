"""GPU parity: waves whose blocks all hold one value and whose payload does
not fit the persistent encoder's staging words.

Such a wave (a constant page under a relative bound saturates every value:
rate 31, 128 bytes per 32 values) has a payload that is one block repeated,
the sign word and planes 0 .. rate - 1 of |q|, each word all ones or all
zeros (cuszp_batched_fixed.cu:302-358).  The persistent encoder writes it
from q alone; a wave that overflows with differing blocks (a NaN, another
value, absent blocks past the end of the segment) marks its job for the
one-workgroup-per-tile re-encode.  Every stream is compared byte for byte
with the oracle, every restored value bit for bit, and the context's
re-encode count tells which of the two ways each call took.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def cpp():
    import cuszp_wrapper_cpp

    return cuszp_wrapper_cpp


def make(cpp, relative, quantizer=0):
    cfg = cpp.CompressionConfig(1e-4, relative, cpp.DIM_1D, cpp.MODE_FIXED,
                                cpp.TYPE_FLOAT)
    w = cpp.CuSZpWrapper(cfg, 0)
    w.set_codec_options(quantizer, 1)
    return w


def bf16_bits(v: float) -> int:
    return int((np.array([v], dtype=np.float32).view(np.uint32)[0] >> 16))


def from_bits(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)


def buffers(cpp, batch, n):
    cap = max(cpp.CuSZpWrapper.estimate_compressed_buffer_size(4 * n),
              1024 * ((n + 32767) // 32768) + 128 * ((n + 31) // 32))
    return [torch.full((cap,), 0xAB, dtype=torch.uint8, device=DEV)
            for _ in range(batch)]


def round_trip(cpp, oracle, w, bits, eps, relative, quantizer):
    """Store the rows of `bits`, compare streams and bounds with the oracle,
    restore them and compare the values; returns the re-encodes it took."""
    batch, n = bits.shape
    before = w._ctx.reencode_count()
    bufs = buffers(cpp, batch, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(from_bits(bits)), bufs, eps)
    assert ok
    redone = w._ctx.reencode_count() - before
    for i in range(batch):
        eb = (oracle.relative_bound(bits[i], n, eps[i]) if relative
              else np.float32(eps[i]))
        assert np.float32(bounds[i]) == np.float32(eb), (i, bounds[i], eb)
        want = oracle.compress_page(bits[i], n, float(eb), None, 0, 0, quantizer)
        got = bufs[i][:sizes[i]].cpu().numpy()
        assert sizes[i] == len(want), (i, sizes[i], len(want))
        if not np.array_equal(got, want):
            bad = np.nonzero(got != want)[0]
            pytest.fail(f"page {i}: {bad.size} bytes differ, first at {bad[0]} "
                        f"(got {got[bad[0]]}, want {want[bad[0]]})")
    out = torch.full((batch * n,), 1.75, dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
    assert w.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    pre = np.full(n, bf16_bits(1.75), dtype=np.uint16)
    for i in range(batch):
        stream = bufs[i][:sizes[i]].cpu().numpy()
        want = oracle.decompress_contiguous(stream, n, bounds[i], 1, pre.copy())
        assert np.array_equal(got[i * n:(i + 1) * n], want), f"page {i} restored"
    return redone


# (value, bound): the rate of every block, hence the period of the repeated
# block in words (rate + 1), and the sign word.
ABSOLUTE_CASES = [
    (1.0, 1e-5),       # |q| = 50000: rate 16, 17 words per block
    (-3.0, 1e-6),      # |q| = 1500000: rate 21, 22 words, sign word all ones
    (-0.8125, 1e-9),   # |q| = 406250000: rate 29, 30 words
    (2.5, 1e-12),      # saturated: q = INT_MAX, rate 31, 32 words
    (float("inf"), 1e-3),
    (float("-inf"), 1e-3),
]


# 40960 and 229376 elements: jobs of 5 and 28 tiles, which the persistent
# encoder runs with the look-back beside the bound exchange and after the
# tile scan respectively
@pytest.mark.parametrize("n", [40960, 229376])
@pytest.mark.parametrize("quantizer", [0, 1])
def test_uniform_waves_absolute(cpp, oracle, n, quantizer):
    bits = np.stack([np.full(n, bf16_bits(v), dtype=np.uint16)
                     for v, _ in ABSOLUTE_CASES])
    eps = [eb for _, eb in ABSOLUTE_CASES]
    w = make(cpp, relative=False, quantizer=quantizer)
    assert round_trip(cpp, oracle, w, bits, eps, False, quantizer) == 0


@pytest.mark.parametrize("n", [40960, 229376])
@pytest.mark.parametrize("quantizer", [0, 1])
def test_uniform_waves_relative(cpp, oracle, n, quantizer):
    """Constant pages under a relative bound (eb = eps * 1e-6: every value
    saturates, except on the zero and the tiny page, which stay at rate 0)
    beside random pages in the same launch."""
    rng = np.random.default_rng(n + quantizer)
    rows = []
    for k, v in enumerate([0.8125, -2.5, 1e30, -1e-30, 0.0]):
        rows.append(np.full(n, bf16_bits(v), dtype=np.uint16))
        x = (rng.standard_normal(n) * (k + 1)).astype(np.float32)
        rows.append((x.view(np.uint32) >> 16).astype(np.uint16))
    bits = np.stack(rows)
    eps = [1e-4, 1e-5] * 5
    w = make(cpp, relative=True, quantizer=quantizer)
    assert round_trip(cpp, oracle, w, bits, eps, True, quantizer) == 0


@pytest.mark.parametrize("n", [40960, 229376])
def test_mixed_waves_fall_back(cpp, oracle, n):
    """Overflowing waves whose blocks differ: a NaN in a constant page, one
    other value in a constant page (its block at a higher rate), and a
    segment whose last wave holds fewer blocks than a full one.  Their jobs
    are encoded again; the uniform waves of the same tiles were written by
    the persistent launch first."""
    rows = []
    nan = np.full(n, bf16_bits(0.8125), dtype=np.uint16)
    nan[3 * 8192 + 4096 + 77] = 0x7FC0
    rows.append(nan)
    other = np.full(n, bf16_bits(1.0), dtype=np.uint16)
    other[8192 + 100] = bf16_bits(1.5)
    rows.append(other)
    bits = np.stack(rows)
    w = make(cpp, relative=False)
    assert round_trip(cpp, oracle, w, bits, [1e-12, 1e-5], False, 0) >= 1
    # the NaN page alone under a relative bound
    w = make(cpp, relative=True)
    assert round_trip(cpp, oracle, w, bits[:1], [1e-4], True, 0) >= 1
    # a partial last tile: 8192 + 4096 + 640 values, whose second tile has a
    # full uniform wave 0 and a wave 1 of 20 blocks (no overflow)
    m = 8192 + 4096 + 640
    part = np.full((2, m), bf16_bits(-0.8125), dtype=np.uint16)
    w = make(cpp, relative=True)
    assert round_trip(cpp, oracle, w, part, [1e-4, 1e-5], True, 0) == 0
