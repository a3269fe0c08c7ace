"""CPU oracle: the plain and outlier (Lorenzo) modes of the fp32 single-page
API.

The reference hands these modes to upstream cuSZp (cuszp_wrapper.cpp:302-313,
922-933), whose sources are not vendored, so the oracle states this build's
own specification of them (kvszp_oracle.c, "Lorenzo modes"): fixed-mode
quantization, residuals against the previous value inside each 32-value
block, the fixed-length block code over the residuals, and in outlier mode
the block's first value kept aside as a 4-byte word.  Byte parity with
upstream cuSZp is unpinned.  What pins the oracle here:
  * hand-computed streams;
  * the decoded values equal the fixed mode's decoded values of the same page
    bit for bit (the residual code reconstructs every q exactly);
  * header bytes and stream size against a numpy restatement of the residual
    arithmetic (32-bit wrap-around, |INT_MIN| = 2^31 at rate 32);
  * malformed streams are rejected.
"""

from __future__ import annotations

import numpy as np
import pytest

PLAIN, OUTLIER = 1, 2


def _residual_headers(oracle, x, eb, mode, variant=0):
    """Header bytes and stream size from numpy: q by the quantizer, residuals
    per block with 32-bit wrap-around, rates of their magnitudes."""
    n = x.size
    recip = np.float32(0.5) / np.float32(eb)
    q = oracle.quantize(x, float(recip), variant).astype(np.int64)
    nb = (n + 31) // 32
    pad = nb * 32 - n
    if pad:
        q = np.concatenate([q, np.full(pad, q[-1], dtype=np.int64)])
    qb = q.reshape(nb, 32)
    prev = np.concatenate([np.zeros((nb, 1), dtype=np.int64), qb[:, :-1]], axis=1)
    d = (qb - prev) & 0xFFFFFFFF
    o = np.zeros(nb, dtype=np.int64)
    if mode == OUTLIER:
        o = d[:, 0].copy()
        d[:, 0] = 0
    mag = np.where(d >= 2**31, (2**32 - d) & 0xFFFFFFFF, d)
    top = mag.max(axis=1)
    rate = np.array([int(v).bit_length() for v in top], dtype=np.int64)
    hdr = rate | np.where(o != 0, 0x80, 0)
    size = oracle.header_bytes(n) + int(np.sum(np.where(o != 0, 4, 0) +
                                               np.where(rate > 0, 4 + 4 * rate, 0)))
    return hdr.astype(np.uint8), size


def test_hand_examples(oracle):
    # eb = 0.5 -> recip = 1; x = [1, -1, 3, 3] quantizes to q = [1, -1, 3, 3]
    # (1.5 -> 1; -1 < -0.5 so s = 1 and -0.5 truncates to 0, q = -1; 3.5 -> 3).
    x = np.array([1.0, -1.0, 3.0, 3.0], dtype=np.float32)
    # plain: residuals [1, -2, 4, 0]: rate 3, element 1 negative
    s = oracle.compress_page_f32_mode(x, 0.5, PLAIN)
    assert s.size == 1024 + 16
    assert s[0] == 3 and not s[1:1024].any()
    assert list(s[1024:1040]) == [0x40, 0, 0, 0,    # sign word: element 1
                                  0x80, 0, 0, 0,    # plane 0: element 0 (|1|)
                                  0x40, 0, 0, 0,    # plane 1: element 1 (|-2|)
                                  0x20, 0, 0, 0]    # plane 2: element 2 (|4|)
    # outlier: q_0 = 1 kept aside, residuals [0, -2, 4, 0] coded at rate 3
    s = oracle.compress_page_f32_mode(x, 0.5, OUTLIER)
    assert s.size == 1024 + 4 + 16
    assert s[0] == 0x83
    assert list(s[1024:1044]) == [1, 0, 0, 0,       # outlier word, LSB first
                                  0x40, 0, 0, 0, 0, 0, 0, 0, 0x40, 0, 0, 0, 0x20, 0, 0, 0]
    for mode in (PLAIN, OUTLIER):
        y = oracle.decompress_f32_mode(oracle.compress_page_f32_mode(x, 0.5, mode), 4,
                                       0.5, mode)
        assert list(y) == [1.0, -1.0, 3.0, 3.0]
    # a constant block: plain codes one nonzero residual, outlier none
    ones = np.ones(32, dtype=np.float32)
    s = oracle.compress_page_f32_mode(ones, 0.5, PLAIN)
    assert s.size == 1024 + 8 and s[0] == 1
    assert list(s[1024:1032]) == [0, 0, 0, 0, 0x80, 0, 0, 0]
    s = oracle.compress_page_f32_mode(ones, 0.5, OUTLIER)
    assert s.size == 1024 + 4 and s[0] == 0x80
    assert list(s[1024:1028]) == [1, 0, 0, 0]
    # a ramp q_v = v: residuals [0, 1, ..., 1], no outlier
    ramp = np.arange(32, dtype=np.float32)
    for mode in (PLAIN, OUTLIER):
        s = oracle.compress_page_f32_mode(ramp, 0.5, mode)
        assert s.size == 1024 + 8 and s[0] == 1
        assert list(s[1024:1032]) == [0, 0, 0, 0, 0x7F, 0xFF, 0xFF, 0xFF]


def test_rate_32_residual(oracle):
    """q = [-1, INT_MAX]: the residual wraps to INT_MIN, whose magnitude 2^31
    needs 32 planes."""
    x = np.array([-1.0, 3e38], dtype=np.float32)
    q = oracle.quantize(x, 1.0)
    assert list(q) == [-1, 2**31 - 1]
    s = oracle.compress_page_f32_mode(x, 0.5, PLAIN)
    assert s[0] == 32 and s.size == 1024 + 4 + 4 * 32
    # residuals [-1, INT_MIN]: both negative; only the second has bit 31
    assert list(s[1024:1028]) == [0xC0, 0, 0, 0]
    assert list(s[1024 + 4 * 32:1024 + 4 * 33]) == [0x40, 0, 0, 0]  # plane 31
    s = oracle.compress_page_f32_mode(x, 0.5, OUTLIER)
    assert s[0] == 0x80 | 32 and s.size == 1024 + 4 + 4 + 4 * 32
    assert list(s[1024:1032]) == [0xFF, 0xFF, 0xFF, 0xFF, 0x40, 0, 0, 0]
    for mode in (PLAIN, OUTLIER):
        y = oracle.decompress_f32_mode(oracle.compress_page_f32_mode(x, 0.5, mode), 2,
                                       0.5, mode)
        assert np.array_equal(y.view(np.uint32), oracle.decompress_f32(
            oracle.compress_page_f32(x, 0.5), 2, 0.5).view(np.uint32))


def _pages():
    rng = np.random.default_rng(11)
    yield "randn", (rng.standard_normal(36864) * 3).astype(np.float32)
    yield "tail", (rng.standard_normal(1000) * 0.01).astype(np.float32)
    smooth = np.cumsum(rng.standard_normal(40000) * 0.01).astype(np.float32)
    yield "smooth", smooth
    yield "zeros", np.zeros(100, dtype=np.float32)
    special = (rng.standard_normal(3000) * 10).astype(np.float32)
    special[::97] = np.nan
    special[5::211] = np.inf
    special[7::223] = -np.inf
    special[11::53] = 3e38
    special[13::59] = -3e38
    special[17::61] = 1e-40                              # denormals
    yield "special", special
    yield "one", np.array([2.5], dtype=np.float32)


@pytest.mark.parametrize("mode", [PLAIN, OUTLIER])
@pytest.mark.parametrize("variant", [0, 1])
def test_decodes_equal_fixed_mode_decodes(oracle, mode, variant):
    for name, x in _pages():
        for eb in (3e-6, 1e-3, 0.5):
            s = oracle.compress_page_f32_mode(x, eb, mode, variant)
            for policy in (0, 1):
                got = np.full(x.size, 7.0, dtype=np.float32)
                want = np.full(x.size, 7.0, dtype=np.float32)
                oracle.decompress_f32_mode(s, x.size, eb, mode, policy, out=got)
                fixed = oracle.compress_page_f32(x, eb, variant)
                oracle.decompress_f32(fixed, x.size, eb, policy, out=want)
                # header byte 0 <=> every q of the block is 0 <=> fixed rate 0,
                # so both rate-0 policies leave the same blocks untouched
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


@pytest.mark.parametrize("mode", [PLAIN, OUTLIER])
def test_headers_and_size_match_numpy_residuals(oracle, mode):
    for name, x in _pages():
        for eb in (1e-4, 0.05):
            s = oracle.compress_page_f32_mode(x, eb, mode)
            hdr, size = _residual_headers(oracle, x, eb, mode)
            nb = hdr.size
            assert s.size == size, name
            assert np.array_equal(s[:nb], hdr), name
            assert not s[nb:oracle.header_bytes(x.size)].any()
            assert s.size <= oracle.max_stream_bytes_lorenzo(x.size)


def test_malformed_streams_are_rejected(oracle):
    x = np.linspace(-3, 3, 64, dtype=np.float32)
    for mode in (PLAIN, OUTLIER):
        s = oracle.compress_page_f32_mode(x, 1e-3, mode)
        with pytest.raises(ValueError):
            oracle.decompress_f32_mode(s[:-4], 64, 1e-3, mode)       # truncated
        bad = s.copy()
        bad[0] = 33 if mode == PLAIN else 0x80 | 33                 # rate > 32
        with pytest.raises(ValueError):
            oracle.decompress_f32_mode(bad, 64, 1e-3, mode)
    bad = oracle.compress_page_f32_mode(x, 1e-3, PLAIN)
    bad[0] |= 0x80                                                  # outlier bit in plain
    with pytest.raises(ValueError):
        oracle.decompress_f32_mode(bad, 64, 1e-3, PLAIN)


def test_worst_case_stream(oracle):
    """Alternating extremes: every residual wraps, rate 32 in every block
    (outlier mode adds the outlier word): R + 136 bytes per block."""
    n = 96
    x = np.where(np.arange(n) % 2 == 0, np.float32(-1.0), np.float32(3e38)).astype(np.float32)
    s = oracle.compress_page_f32_mode(x, 0.5, OUTLIER)
    assert list(s[:3]) == [0x80 | 32] * 3
    assert s.size == oracle.max_stream_bytes_lorenzo(n) == 1024 + 136 * 3


def _naive_lorenzo_stream(q, n, mode) -> bytes:
    """A second, per-bit restatement of the residual codes (pure Python,
    independent of kvszp_oracle.c): 32-bit wrap-around residuals, header
    byte, outlier word, then the fixed mode's sign word and planes with
    element v at bit 7 - (v & 7) of byte v >> 3."""
    nb = (n + 31) // 32
    header = bytearray(1024 * ((n + 32767) // 32768))
    payload = bytearray()
    for b in range(nb):
        blk = [int(v) for v in q[32 * b:32 * b + 32]]
        blk += [blk[-1]] * (32 - len(blk))
        prev, codes = 0, []
        for v in range(32):
            codes.append(((blk[v] - prev + 2**31) % 2**32) - 2**31)
            prev = blk[v]
        o = 0
        if mode == OUTLIER:
            o, codes[0] = codes[0], 0
        mags = [abs(c) for c in codes]
        rate = max(mags).bit_length()
        header[b] = rate | (0x80 if o else 0)
        if o:
            payload += (o & 0xFFFFFFFF).to_bytes(4, "little")
        if rate == 0:
            continue
        words = [bytearray(4) for _ in range(rate + 1)]
        for v in range(32):
            bit = 1 << (7 - (v & 7))
            if codes[v] < 0:
                words[0][v >> 3] |= bit
            for p in range(rate):
                if (mags[v] >> p) & 1:
                    words[1 + p][v >> 3] |= bit
        for w in words:
            payload += w
    return bytes(header) + bytes(payload)


@pytest.mark.parametrize("mode", [PLAIN, OUTLIER])
@pytest.mark.parametrize("fused", [False, True])
def test_streams_equal_naive_restatement(oracle, mode, fused):
    """Whole streams, byte for byte, against the per-bit restatement fed by
    the golden generator's own quantizer (tests/golden/make_golden.py)."""
    import importlib.util
    import os

    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(__file__), "golden", "make_golden.py"))
    golden = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(golden)
    rng = np.random.default_rng(21)
    pages = [
        (rng.standard_normal(1000) * 3).astype(np.float32),
        np.cumsum(rng.standard_normal(2500) * 0.02).astype(np.float32),
        np.where(np.arange(70) % 2 == 0, np.float32(-1.0), np.float32(3e38)).astype(np.float32),
        np.array([0.0, -0.0, 1e-40, -7.5, 7.5, 2.5, 2.5, 2.5, -3e38], dtype=np.float32),
    ]
    special = (rng.standard_normal(700) * 50).astype(np.float32)
    special[::31] = np.nan
    special[3::37] = np.inf
    pages.append(special)
    for x in pages:
        for eb in (np.float32(1e-3), np.float32(0.25), np.float32(7.0)):
            recip = np.float32(np.float32(0.5) / eb)
            q = golden.quantize(x, recip, fused)
            want = _naive_lorenzo_stream(q, x.size, mode)
            got = oracle.compress_page_f32_mode(x, float(eb), mode, 1 if fused else 0)
            assert got.tobytes() == want, (x.size, float(eb))
