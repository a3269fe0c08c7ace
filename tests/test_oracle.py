"""Pins the CPU oracle (oracle/kvszp_oracle.c) without running the reference.

The reference holds no golden vectors for this path, so every oracle
function is checked against facts fixed independently of its own code:
hand-computed streams, exact rational arithmetic, Python/numpy/torch
built-ins, brute force over small index spaces, and closed-form invariants.
Each check is chosen so that a plausible slip (dropped term, wrong sign,
swapped bit order, off-by-one block) fails.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

INT_MAX = 2**31 - 1


def bf16_bits(values) -> np.ndarray:
    """float -> BF16 bit patterns through torch's CPU conversion (RNE)."""
    t = torch.tensor(np.asarray(values, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def bits_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- quantizer (cuszp_batched_fixed.cu:10-25) -------------------------------

KNOWN_QUANT = [  # (x, recip, q) computed by hand from the PTX text
    (0.0, 1.0, 0), (0.49, 1.0, 0), (0.5, 1.0, 1), (-0.5, 1.0, 0),
    (-0.51, 1.0, -1), (1.5, 1.0, 2), (-1.5, 1.0, -2), (2.5, 1.0, 3),
    (-2.5, 1.0, -3), (-0.0, 1.0, 0), (7.0, 0.25, 2), (-7.0, 0.25, -2),
    (float("nan"), 1.0, -1), (float("inf"), 1.0, INT_MAX),
    (float("-inf"), 1.0, INT_MAX),          # saturates to INT_MIN, minus 1 wraps
    (3e9, 1.0, INT_MAX), (-3e9, 1.0, INT_MAX),
    (2.0**31, 1.0, INT_MAX), (-(2.0**31), 1.0, INT_MAX),
    (2.0**23 + 1, 1.0, 2**23 + 2),          # v+0.5 ties to even
    (-(2.0**23 + 1), 1.0, -(2**23 + 1)),    # t = -2^23 (even), c - 1
    (2.0**24, 1.0, 2**24), (1.0, 0.0, 0),
]


@pytest.mark.parametrize("x,recip,q", KNOWN_QUANT)
@pytest.mark.parametrize("variant", [0, 1])
def test_quantizer_known_answers(oracle, x, recip, q, variant):
    assert int(oracle.quantize([x], recip, variant)[0]) == q


def _exact_quant(x: float, r: float, fused: bool) -> int:
    """The PTX sequence in exact rational arithmetic + one f32 rounding per
    rounded operation (numpy provides the correctly-rounded f32 casts)."""
    v = np.float32(np.float32(x) * np.float32(r))  # mul.f32 rounds once
    s = 0 if v >= -0.5 else 1
    if fused:
        if not (np.isfinite(x) and np.isfinite(r)):
            t = np.float32(np.float32(x) * np.float32(r) + np.float32(0.5))
        else:  # one rounding of the exact x*r + 1/2
            t = _round_f32(Fraction(float(np.float32(x))) *
                           Fraction(float(np.float32(r))) + Fraction(1, 2))
    else:
        t = np.float32(v + np.float32(0.5))
    if t != t:
        c = 0
    elif t >= 2.0**31:
        c = INT_MAX
    elif t <= -(2.0**31):
        c = -(2**31)
    else:
        c = int(t)
    return ((c - s + 2**31) % 2**32) - 2**31


def _round_f32(q: Fraction) -> np.float32:
    """Round an exact rational to the nearest f32 (ties to even)."""
    if q == 0:
        return np.float32(0.0)
    lo = np.float32(float(q))
    # walk to the bracketing f32 pair around q
    while Fraction(float(lo)) > q:
        lo = np.nextafter(lo, np.float32(-np.inf), dtype=np.float32)
    while Fraction(float(np.nextafter(lo, np.float32(np.inf), dtype=np.float32))) <= q:
        lo = np.nextafter(lo, np.float32(np.inf), dtype=np.float32)
    hi = np.nextafter(lo, np.float32(np.inf), dtype=np.float32)
    dl, dh = q - Fraction(float(lo)), Fraction(float(hi)) - q
    if dl < dh:
        return lo
    if dh < dl:
        return hi
    return lo if (lo.view(np.uint32) & 1) == 0 else hi


def test_quantizer_matches_exact_arithmetic(oracle):
    rng = np.random.default_rng(7)
    xs = bits_to_f32(bf16_bits(rng.standard_normal(3000) * 40.0))
    for r in (np.float32(1.0) / np.float32(3.0), np.float32(0.5) / np.float32(1.7e-3),
              np.float32(12345.678), np.float32(0.1)):
        for fused in (False, True):
            got = oracle.quantize(xs, float(r), int(fused))
            want = [_exact_quant(float(x), float(r), fused) for x in xs]
            assert list(got) == want


def test_quantizer_variants_differ_where_double_rounding_crosses(oracle):
    """Find inputs where x*recip lies within half an ulp below k+0.5 so that
    rounding the product first lands on the tie: the two readings of the PTX
    must then disagree, each as exact arithmetic says."""
    rng = np.random.default_rng(11)
    found = 0
    for _ in range(400):
        # |x*recip| in [2^23, 2^25): the product rounds to an integer-spaced
        # float, so fl(v + 0.5) ties to even while fma rounds p + 0.5 once
        # (what a constant page under a relative bound hits).
        x = np.float32(bits_to_f32(bf16_bits([rng.uniform(1.0, 2.0) *
                                              rng.choice([-1.0, 1.0])]))[0])
        r = np.float32(rng.uniform(2.0**23, 2.0**24))
        a = _exact_quant(float(x), float(r), False)
        b = _exact_quant(float(x), float(r), True)
        if a != b:
            found += 1
            assert int(oracle.quantize([x], float(r), 0)[0]) == a
            assert int(oracle.quantize([x], float(r), 1)[0]) == b
    assert found > 0


def test_bit_count(oracle):
    for v in [0, 1, 2, 3, 4, 255, 256, 5000, INT_MAX, 2**31, 2**32 - 1]:
        assert oracle.bit_count(v) == int(v).bit_length()


# ---- BF16 rounding ----------------------------------------------------------

def test_f32_to_bf16_matches_torch(oracle):
    rng = np.random.default_rng(3)
    u = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    u = u[((u >> 23) & 0xFF) != 0xFF]  # finite only (NaN pattern is unpinned)
    edge = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7FFFFF, 0x00000001,
                     0x80000001, 0x7F800000, 0xFF800000, 0, 0x80000000,
                     0x3F7FFFFF, 0x007FFFFF], dtype=np.uint32)
    vals = np.concatenate([u, edge]).view(np.float32)
    want = bf16_bits(vals)
    got = oracle.f32_to_bf16(vals)
    assert np.array_equal(got, want)
    nan = oracle.f32_to_bf16([float("nan")])[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


# ---- layer map (cu:33-50) ---------------------------------------------------

@pytest.mark.parametrize("prefix,src,epl,idx", [
    (2, 8, 4096, [1, 3, 6]), (2, 28, 64, [0, 1, 2, 5, 19, 20, 21]),
    (1, 5, 7, [4, 0, 2]), (3, 4, 33, [3]), (2, 6, 10, [5, 4, 3, 2, 1, 0])])
def test_source_index_matches_index_select(oracle, prefix, src, epl, idx):
    """Same equivalence the reference's test relies on (tests :98-100)."""
    a = np.arange(prefix * src * epl).reshape(prefix, src, epl)
    want = a[:, idx, :].reshape(-1)
    stride = max(1, want.size // 997)
    for i in range(0, want.size, stride):
        assert oracle.source_index(i, idx, len(idx), src, epl) == want[i]


# ---- relative bound (cu:55-133) ----------------------------------------------

def test_relative_bound_closed_forms(oracle):
    x = bf16_bits([-3.0, 1.0, 2.5, 0.0])
    eb = oracle.relative_bound(x, 4, 1e-4)
    assert eb == np.float32(np.float32(1e-4) * np.float32(5.5))
    # NaN never wins the min/max
    x = bf16_bits([float("nan"), -1.0, 1.0])
    assert oracle.relative_bound(x, 3, 1e-3) == np.float32(np.float32(1e-3) * np.float32(2.0))
    # constant, all-NaN and single-element pages fall back to the 1e-6 floor
    for vals in ([4.0] * 9, [float("nan")] * 5, [7.0]):
        x = bf16_bits(vals)
        assert oracle.relative_bound(x, len(vals), 0.5) == np.float32(
            np.float32(0.5) * np.float32(1e-6))
    # an infinity makes the range infinite
    x = bf16_bits([float("inf"), 0.0])
    assert oracle.relative_bound(x, 2, 1e-4) == np.inf
    # only the first n values count
    x = bf16_bits([1.0, 2.0, 1000.0])
    assert oracle.relative_bound(x, 2, 1.0) == np.float32(1.0)


def test_relative_bound_indexed_uses_selected_layers(oracle):
    prefix, src, epl, idx = 2, 4, 8, [1, 3]
    page = np.zeros(prefix * src * epl, dtype=np.float32)
    view = page.reshape(prefix, src, epl)
    view[:, 0, :] = 100.0       # unselected layers hold the extremes
    view[:, 2, :] = -100.0
    view[0, 1, 3] = -2.0
    view[1, 3, 5] = 6.0
    eb = oracle.relative_bound(bf16_bits(page), prefix * 2 * epl, 1e-2, idx,
                               src, epl)
    assert eb == np.float32(np.float32(1e-2) * np.float32(8.0))


# ---- stream format (cu:135-359) -----------------------------------------------

def _page(values, n=None):
    v = np.zeros(n or len(values), dtype=np.float32)
    v[:len(values)] = values
    return bf16_bits(v)


def test_stream_hand_example_two_values(oracle):
    # x=[1,-1,0...], eb=0.5 -> recip=1, q=[1,-1,0...], rate 1
    s = oracle.compress_page(_page([1.0, -1.0], 32), 32, 0.5)
    assert len(s) == 1024 + 8
    assert s[0] == 1 and not s[1:1024].any()
    assert list(s[1024:]) == [0x40, 0, 0, 0, 0xC0, 0, 0, 0]


def test_stream_hand_example_rate3_and_byte_positions(oracle):
    # q = [5, -3, 0, 2, 0, 0, 0, 0, -1, 0 ... 0, 1]  (recip = 1)
    x = np.zeros(32, dtype=np.float32)
    x[[0, 1, 3, 8, 31]] = [5.0, -3.0, 2.0, -1.0, 1.0]
    s = oracle.compress_page(_page(x), 32, 0.5)
    assert s[0] == 3
    payload = list(s[1024:])
    assert payload == [
        0x40, 0x80, 0x00, 0x00,   # sign: element 1 (byte0 bit6), 8 (byte1 bit7)
        0xC0, 0x80, 0x00, 0x01,   # plane 0: elements 0,1,8,31
        0x50, 0x00, 0x00, 0x00,   # plane 1: elements 1,3
        0x80, 0x00, 0x00, 0x00,   # plane 2: element 0
    ]


def test_stream_tail_and_header_padding(oracle):
    # 33 elements: block 1 has one value; R stays 1024.
    x = np.zeros(33, dtype=np.float32)
    x[32] = -2.0
    s = oracle.compress_page(_page(x), 33, 0.5)
    assert s[0] == 0 and s[1] == 2 and not s[2:1024].any()
    assert list(s[1024:]) == [0x80, 0, 0, 0, 0x00, 0, 0, 0, 0x80, 0, 0, 0]
    # header bytes R = 1024 * ceil(n / 32768)
    for n, r in [(1, 1024), (32768, 1024), (32769, 2048), (36864, 2048),
                 (229376, 7168), (172032, 6144), (57344, 2048),
                 (1048576, 32768)]:
        assert oracle.header_bytes(n) == r


def test_all_zero_page_is_header_only(oracle):
    n = 1 << 20
    s = oracle.compress_page(np.zeros(n, dtype=np.uint16), n, 1e-4)
    assert len(s) == 32768 and not s.any()
    assert (2 * n) / len(s) == 64


def _rates_from_stream(s, n):
    return s[:(n + 31) // 32].astype(np.int64)


@pytest.mark.parametrize("n", [32, 100, 8192, 36864, 70000])
def test_size_formula_and_round_trip(oracle, n):
    rng = np.random.default_rng(n)
    x = bf16_bits(rng.standard_normal(n) * rng.uniform(0.01, 50))
    for eps, rel in ((1e-4, True), (1e-3, True), (0.05, False)):
        eb = oracle.relative_bound(x, n, eps) if rel else np.float32(eps)
        s = oracle.compress_page(x, n, float(eb))
        rates = _rates_from_stream(s, n)
        r_bytes = oracle.header_bytes(n)
        assert len(s) == r_bytes + int(np.sum(np.where(rates > 0, 4 + 4 * rates, 0)))
        # rates are the bit lengths of the per-block max |q| (numpy, no oracle)
        recip = np.float32(0.5) / np.float32(eb)
        q = oracle.quantize(bits_to_f32(x), float(recip), 0).astype(np.int64)
        qp = np.zeros(((n + 31) // 32) * 32, dtype=np.int64)
        qp[:n] = q
        mx = np.abs(qp).reshape(-1, 32).max(axis=1)
        assert np.array_equal(rates, [int(m).bit_length() for m in mx])
        # decode(encode(x)) == bf16((q * eb) * 2), with torch doing the bf16
        y = oracle.decompress_contiguous(s, n, float(eb))
        ref = (q.astype(np.float32) * np.float32(eb)) * np.float32(2.0)
        assert np.array_equal(y, bf16_bits(ref))
        # error bound: fp32 reconstruction within eb (+ fp32 slack), the
        # reference's own tolerances: 1.01*eb + 1e-7 (tests :45) and 2*eb
        # for BF16 output (tests :457)
        xf = bits_to_f32(x)
        assert np.max(np.abs(ref - xf)) <= float(eb) * 1.01 + 1e-7
        assert np.max(np.abs(bits_to_f32(y) - xf)) <= 2 * float(eb) + 1e-7


def test_decoder_rate0_policies(oracle):
    n = 64
    x = np.zeros(n, dtype=np.float32)
    x[40] = 3.0                     # block 0 rate 0, block 1 rate > 0
    s = oracle.compress_page(_page(x), n, 0.5)
    pre = np.full(n, 0x1234, dtype=np.uint16)
    skip = oracle.decompress_contiguous(s, n, 0.5, oracle.RATE0_SKIP, pre.copy())
    assert np.all(skip[:32] == 0x1234)          # reference: untouched
    zero = oracle.decompress_contiguous(s, n, 0.5, oracle.RATE0_ZERO, pre.copy())
    assert np.all(zero[:32] == 0)
    assert np.array_equal(skip[32:], zero[32:])
    assert zero[40] == bf16_bits([3.0])[0]


def test_decoder_rejects_malformed_streams(oracle):
    s = oracle.compress_page(_page([1.0, 2.0, 3.0], 32), 32, 0.5)
    bad = s.copy()
    bad[0] = 40
    with pytest.raises(ValueError):
        oracle.decompress_contiguous(bad, 32, 0.5)
    with pytest.raises(ValueError):
        oracle.decompress_contiguous(s[:-4], 32, 0.5)
    with pytest.raises(ValueError):
        oracle.decompress_contiguous(s[:1000], 32, 0.5)


def test_indexed_stream_equals_gathered_stream(oracle):
    """Encoding layer-selected segments in place equals encoding the
    index_select-ed copy (the reference's own equivalence, tests :98-100)."""
    prefix, src, epl, idx = 2, 8, 100, [1, 3, 6]
    rng = np.random.default_rng(5)
    page = bf16_bits(rng.standard_normal(prefix * src * epl))
    gathered = page.reshape(prefix, src, epl)[:, idx, :].reshape(-1).copy()
    n = gathered.size
    eb = oracle.relative_bound(page, n, 1e-3, idx, src, epl)
    assert eb == oracle.relative_bound(gathered, n, 1e-3)
    a = oracle.compress_page(page, n, eb, idx, src, epl)
    b = oracle.compress_page(gathered, n, eb)
    assert np.array_equal(a, b)
    # indexed decode writes exactly the selected layers of the full page
    out = np.full(prefix * src * epl, 0x7777, dtype=np.uint16)
    oracle.decompress_indexed(a, n, eb, out, idx, src, epl)
    flat = oracle.decompress_contiguous(b, n, eb)
    view = out.reshape(prefix, src, epl)
    assert np.array_equal(view[:, idx, :].reshape(-1), flat)
    others = [l for l in range(src) if l not in idx]
    assert np.all(view[:, others, :] == 0x7777)


def test_scatter_decode_splits_at_destination_boundaries(oracle):
    n, dpp = 300, 3
    epd = n // dpp
    rng = np.random.default_rng(9)
    x = bf16_bits(rng.standard_normal(n))
    s = oracle.compress_page(x, n, 0.01)
    flat = oracle.decompress_contiguous(s, n, 0.01)
    dests = [np.zeros(epd, dtype=np.uint16) for _ in range(dpp)]
    oracle.decompress_scatter(s, n, 0.01, dests, epd)
    assert np.array_equal(np.concatenate(dests), flat)


def test_batch_api_eps_resolution(oracle):
    rng = np.random.default_rng(1)
    pages = bf16_bits(rng.standard_normal((3, 4096)).astype(np.float32))
    pages = pages.reshape(3, 4096)
    streams, sizes, bounds = oracle.compress_batch(
        pages, [0.0, 2e-3, -1.0], default_eps=1e-3, relative=False)
    assert list(bounds) == [np.float32(1e-3), np.float32(2e-3), np.float32(1e-3)]
    for i in range(3):
        assert np.array_equal(streams[i],
                              oracle.compress_page(pages[i], 4096, float(bounds[i])))


# ---- INT8 host codec (vllm_v1_compressed_offload.py:711-724, 2090-2123) -----

def test_int8_codec_matches_torch_formula(oracle):
    rng = np.random.default_rng(2)
    x = torch.tensor(rng.standard_normal(5000).astype(np.float32) * 3).to(torch.bfloat16)
    scale_t = x.abs().max() / 127.0
    q_t = torch.clamp(torch.round(x / scale_t), -127, 127).to(torch.int8)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    q, scale = oracle.int8_encode(bits)
    assert scale == float(scale_t)
    assert np.array_equal(q, q_t.numpy())
    y_t = (q_t.to(torch.float32) * float(scale_t)).to(torch.bfloat16)
    y = oracle.int8_decode(q, scale)
    assert np.array_equal(y, y_t.view(torch.int16).numpy().view(np.uint16))


# ---- fp32 single-page path (CuSZpWrapper::compress / decompress) -------------

def _aminmax_bound(x: np.ndarray, eps: float) -> np.float32:
    """cuszp_wrapper.cpp:249-257 through torch's own aminmax (NaN propagates)."""
    mn, mx = torch.aminmax(torch.from_numpy(x))
    rng = np.float32(mx.item()) - np.float32(mn.item())
    if rng < np.float32(1e-6):
        rng = np.float32(1e-6)
    return np.float32(np.float32(eps) * rng)


@pytest.mark.parametrize("case", ["randn", "const", "nan", "infs", "pos_inf",
                                  "signed_zero", "tiny"])
def test_relative_bound_f32_matches_torch_aminmax(oracle, case):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(5000) * 3).astype(np.float32)
    if case == "const":
        x[:] = 2.5
    elif case == "nan":
        x[1234] = np.nan
    elif case == "infs":
        x[10], x[20] = np.inf, -np.inf
    elif case == "pos_inf":
        x[:] = np.inf
    elif case == "signed_zero":
        x[:] = 0.0
        x[::2] = -0.0
    elif case == "tiny":
        x = (x * 1e-9).astype(np.float32)
    want = _aminmax_bound(x, 1e-4)
    got = np.float32(oracle.relative_bound_f32(x, 1e-4))
    if np.isnan(want):
        assert np.isnan(got)
    else:
        assert got == want


def test_f32_stream_hand_example(oracle):
    # x = [0.75, -1.0000001, 3.0, 0...], eb = 0.5 -> recip = 1:
    # q = [1, -1, 3]: 0.75+0.5 -> 1; v = -1.0000001 < -0.5 gives s = 1 and
    # t = -0.5000001 truncates to 0, so q = -1; 3.5 -> 3.  Rate 2.
    x = np.zeros(40, dtype=np.float32)
    x[:3] = [0.75, np.float32(-1.0000001), 3.0]
    s = oracle.compress_page_f32(x, 0.5)
    assert s.size == 1024 + 4 + 4 * 2
    assert s[0] == 2 and s[1] == 0 and not s[2:1024].any()
    assert list(s[1024:1028]) == [0x40, 0, 0, 0]   # element 1 negative
    assert list(s[1028:1032]) == [0xE0, 0, 0, 0]   # plane 0: elements 0,1,2
    assert list(s[1032:1036]) == [0x20, 0, 0, 0]   # plane 1: element 2 (q=3)
    y = oracle.decompress_f32(s, 40, 0.5)
    assert list(y[:4]) == [1.0, -1.0, 3.0, 0.0] and not y[4:].any()


@pytest.mark.parametrize("n", [40, 36864, 70001])
def test_f32_encoder_on_widened_bf16_equals_bf16_encoder(oracle, n):
    """A BF16 page widened to fp32 has the same values, so with the same
    bound the fp32 path must write the BF16 path's stream."""
    rng = np.random.default_rng(n)
    bits = bf16_bits(rng.standard_normal(n) * 2)
    x = bits_to_f32(bits)
    eb = np.float32(oracle.relative_bound(bits, n, 1e-4))
    assert eb == np.float32(oracle.relative_bound_f32(x, 1e-4))
    assert np.array_equal(oracle.compress_page_f32(x, float(eb)),
                          oracle.compress_page(bits, n, float(eb)))


def test_f32_decoder_rounded_is_bf16_decoder(oracle):
    """torch's fp32 -> BF16 rounding of the fp32 decode is the BF16
    decoders' output (cu:535-538 differs only by that rounding)."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(50000) * 5).astype(np.float32)
    x[:3000] = 0.0                                  # rate-0 blocks
    eb = oracle.relative_bound_f32(x, 1e-5)
    s = oracle.compress_page_f32(x, eb)
    y = oracle.decompress_f32(s, x.size, eb)
    rounded = torch.from_numpy(y).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(rounded, oracle.decompress_contiguous(s, x.size, eb))
    assert np.abs(y - x).max() <= 1.01 * eb + 1e-7  # reference tolerance (tests :45)


def test_stream_capacity_covers_partial_blocks_at_rate_31(oracle):
    """One value on a constant page under a relative bound has rate 31: its
    block takes 4 + 124 bytes whatever the block's length."""
    for n in (1, 33, 100):
        x = np.full(n, 2.5, dtype=np.float32)
        s = oracle.compress_page_f32(x, oracle.relative_bound_f32(x, 1e-4))
        nb = (n + 31) // 32
        assert s.size == oracle.header_bytes(n) + 128 * nb == oracle.max_stream_bytes(n)
        assert list(s[:nb]) == [31] * nb


def test_threaded_indexed_batch_decode_equals_page_by_page(oracle):
    rng = np.random.default_rng(4)
    prefix, src, epl, layers = 2, 5, 640, [4, 1, 2]
    pages = bf16_bits(rng.standard_normal((6, prefix * src * epl)))
    n = prefix * len(layers) * epl
    streams, sizes, bounds = oracle.compress_batch(
        pages, [1e-4] * 6, threads=3, layer_indices=layers, source_layers=src,
        elements_per_layer=epl)
    got = np.full(pages.shape, 7, dtype=np.uint16)
    oracle.decompress_batch_indexed(streams, sizes, n, bounds, got, layers, src, epl,
                                    threads=4)
    for i in range(6):
        want = np.full(pages.shape[1], 7, dtype=np.uint16)
        oracle.decompress_indexed(streams[i], n, float(bounds[i]), want, layers, src, epl)
        assert np.array_equal(got[i], want)
