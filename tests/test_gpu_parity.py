"""GPU parity: the HIP codec behind ``cuszp_wrapper_cpp`` against the oracle.

Every stream the GPU writes is compared byte-for-byte with the scalar CPU
oracle on the same seeded pages, and every decoded BF16 value bit-for-bit.
Edge cases follow the reference's semantics (cuszp_batched_fixed.cu):
partial blocks and tiles, header padding, NaN/Inf/saturation, rate-0 blocks,
layer gathers that straddle layers, multi-destination splits.
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


def make(cpp, eb=1e-4, relative=True, quantizer=0, rate0=1):
    cfg = cpp.CompressionConfig(eb, relative, cpp.DIM_1D, cpp.MODE_FIXED,
                                cpp.TYPE_FLOAT)
    w = cpp.CuSZpWrapper(cfg, 0)
    w.set_codec_options(quantizer, rate0)
    return w


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def from_bits(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)


def rand_pages(batch, n, seed, scale=1.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    scales = torch.exp(torch.randn(batch, 1, generator=g)) * scale
    x = torch.randn(batch, n, generator=g) * scales
    return x.to(torch.bfloat16).to(DEV)


def buffers(cpp, batch, n):
    cap = max(cpp.CuSZpWrapper.estimate_compressed_buffer_size(4 * n),
              1024 * ((n + 32767) // 32768) + 128 * ((n + 31) // 32))
    return [torch.full((cap,), 0xAB, dtype=torch.uint8, device=DEV)
            for _ in range(batch)]


def assert_streams(oracle, pages_bits, n, eps, relative, bufs, sizes, bounds,
                   quantizer=0, layers=None, src=0, epl=0):
    for i in range(len(bufs)):
        if relative:
            eb = oracle.relative_bound(pages_bits[i], n, eps[i], layers, src, epl)
        else:
            eb = np.float32(eps[i])
        assert np.float32(bounds[i]) == np.float32(eb), (i, bounds[i], eb)
        want = oracle.compress_page(pages_bits[i], n, float(eb), layers, src,
                                    epl, quantizer)
        got = bufs[i][:sizes[i]].cpu().numpy()
        assert sizes[i] == len(want), (i, sizes[i], len(want))
        if not np.array_equal(got, want):
            bad = np.nonzero(got != want)[0]
            pytest.fail(f"page {i}: {bad.size} bytes differ, first at {bad[0]} "
                        f"(got {got[bad[0]]}, want {want[bad[0]]})")


# ---- compress: contiguous pages ----------------------------------------------

# 196608 and 204800 elements: jobs of 24 and 25 tiles, the longest that the
# persistent encoder runs with the look-back beside the bound exchange and
# the shortest that it runs with the look-back after the tile scan
@pytest.mark.parametrize("n", [32, 33, 1000, 8192, 8193, 32768, 36864, 100003,
                               196608, 204800, 229376])
@pytest.mark.parametrize("relative", [True, False])
def test_compress_bytes_match_oracle(cpp, oracle, n, relative):
    batch = 3
    pages = rand_pages(batch, n, seed=n)
    eps = [1e-4, 1e-3, 2e-5] if relative else [1e-3, 5e-2, 2e-4]
    w = make(cpp, relative=relative)
    bufs = buffers(cpp, batch, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs, eps)
    assert ok
    assert_streams(oracle, u16(pages), n, eps, relative, bufs, sizes, bounds)


# 40000 and 229376 elements: jobs of 5 and 28 tiles, which the persistent
# encoder runs with the look-back beside the bound exchange and after the
# tile scan respectively
@pytest.mark.parametrize("n", [40000, 229376])
@pytest.mark.parametrize("quantizer", [0, 1])
def test_quantizer_variants_match_oracle(cpp, oracle, quantizer, n):
    pages = rand_pages(2, n, seed=5)
    const = torch.full((n,), 1.3125, dtype=torch.bfloat16, device=DEV)
    pages = torch.stack([pages[0], pages[1], const])
    eps = [1e-4, 1e-5, 1e-4]
    w = make(cpp, quantizer=quantizer)
    bufs = buffers(cpp, 3, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs, eps)
    assert ok
    assert_streams(oracle, u16(pages), n, eps, True, bufs, sizes, bounds,
                   quantizer=quantizer)


def _special_page(n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32) * 3
    bits = (x.view(np.uint32) >> 16).astype(np.uint16)
    specials = np.array([0x7FC0, 0xFFC0, 0x7F80, 0xFF80, 0x8000, 0x0000, 0x0001,
                         0x8001, 0x7F7F, 0xFF7F, 0x3F80], dtype=np.uint16)
    idx = rng.choice(n, size=min(n, 200), replace=False)
    bits[idx] = specials[rng.integers(0, specials.size, idx.size)]
    return bits


@pytest.mark.parametrize("relative", [True, False])
def test_special_values_match_oracle(cpp, oracle, relative):
    n = 20000
    rows = [_special_page(n, s) for s in range(3)]
    rows.append(np.zeros(n, dtype=np.uint16))                 # all zero
    rows.append(np.full(n, 0x4049, dtype=np.uint16))          # constant 3.14
    nan = np.full(n, 0x7FC0, dtype=np.uint16)
    nan[::7] = 0x3F80
    rows.append(nan)                                          # mostly NaN
    rows.append(np.full(n, 0x7FC0, dtype=np.uint16))          # all NaN
    bits = np.stack(rows)
    pages = from_bits(bits)
    eps = [1e-4] * len(rows) if relative else [1e-2] * len(rows)
    w = make(cpp, relative=relative)
    bufs = buffers(cpp, len(rows), n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs, eps)
    assert ok
    assert_streams(oracle, bits, n, eps, relative, bufs, sizes, bounds)


@pytest.mark.parametrize("n", [192, 8192 + 64, 100000])
@pytest.mark.parametrize("relative", [True, False])
def test_bounds_that_make_recip_infinite(cpp, oracle, n, relative):
    """eb below 0.5 / FLT_MAX (a denormal absolute bound, or a relative one
    whose eps * range underflows) makes recip infinite: nonzero values
    saturate and zeros quantize to -1 (0 * Inf = NaN).  Blocks past the end
    of a page stay rate 0, so the streams match the oracle and no byte past
    a stream is written (the canary after it stays 0xAB)."""
    pages = rand_pages(4, n, seed=n)
    bits = u16(pages)
    eps = [1e-40, 1e-45, 2e-39, 1e-38] if not relative else [1e-40, 1e-45, 1e-44, 3e-39]
    w = make(cpp, relative=relative)
    bufs = [torch.cat([b, torch.full((4096,), 0xAB, dtype=torch.uint8, device=DEV)])
            for b in buffers(cpp, 4, n)]
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs, eps)
    assert ok
    assert_streams(oracle, bits, n, eps, relative, bufs, sizes, bounds)
    for i, b in enumerate(bufs):
        tail = b[sizes[i]:].cpu().numpy()
        assert (tail == 0xAB).all(), (i, int(np.nonzero(tail != 0xAB)[0][0]))


def test_eps_resolution_and_default_bound(cpp, oracle):
    n = 9000
    pages = rand_pages(3, n, seed=2)
    w = make(cpp, eb=3e-4)
    bufs = buffers(cpp, 3, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs,
                                                    [0.0, 1e-3, -5.0])
    assert ok
    eps = [np.float32(3e-4), np.float32(1e-3), np.float32(3e-4)]
    assert_streams(oracle, u16(pages), n, eps, True, bufs, sizes, bounds)
    ok2, sizes2, _ = w.compress_batch_fixed_bf16(list(pages), bufs, [])
    assert ok2 and sizes2[0] == sizes[0] and sizes2[2] == sizes[2]


# ---- decompress ---------------------------------------------------------------

def _encode(cpp, w, pages, eps):
    n = pages.shape[1]
    bufs = buffers(cpp, pages.shape[0], n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs, eps)
    assert ok
    return bufs, sizes, bounds


# 327683 and 1048576 elements: jobs of 40 and 128 tiles, so the persistent
# decoder's runs of consecutive tiles start and end inside a job
@pytest.mark.parametrize("n", [32, 77, 8192, 36864, 229376, 327683, 1048576])
@pytest.mark.parametrize("rate0", [0, 1])
def test_decompress_contiguous_matches_oracle(cpp, oracle, n, rate0):
    pages = rand_pages(3, n, seed=n + 1)
    pages[1, : min(n, 5000)] = 0  # rate-0 blocks
    w = make(cpp, rate0=rate0)
    bufs, sizes, bounds = _encode(cpp, w, pages, [1e-4, 1e-4, 1e-3])
    out = torch.full((3 * n + 5,), 1.75, dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
    assert w.synchronize()
    got = u16(out)
    pre = u16(torch.full((n,), 1.75, dtype=torch.bfloat16))
    for i in range(3):
        stream = bufs[i][:sizes[i]].cpu().numpy()
        want = oracle.decompress_contiguous(stream, n, bounds[i], rate0,
                                            pre.copy())
        assert np.array_equal(got[i * n:(i + 1) * n], want), f"page {i}"
    assert np.all(got[3 * n:] == pre[0])  # nothing written past the batch


@pytest.mark.parametrize("n", [8192, 229376])
def test_scatter_single_destination(cpp, oracle, n):
    pages = rand_pages(4, n, seed=3)
    w = make(cpp)
    bufs, sizes, bounds = _encode(cpp, w, pages, [1e-4] * 4)
    pool = torch.zeros(10, n, dtype=torch.bfloat16, device=DEV)
    slots = [7, 2, 9, 0]
    dests = [pool[s] for s in slots]
    assert w.decompress_batch_fixed_bf16_scatter(bufs, sizes, dests, n, 1, n,
                                                 bounds)
    assert w.synchronize()
    got = u16(pool)
    for i, s in enumerate(slots):
        stream = bufs[i][:sizes[i]].cpu().numpy()
        assert np.array_equal(got[s], oracle.decompress_contiguous(stream, n,
                                                                   bounds[i]))
    for s in set(range(10)) - set(slots):
        assert not got[s].any()


@pytest.mark.parametrize("dpp,epd", [(2, 4096), (3, 1000), (5, 77)])
def test_scatter_multi_destination(cpp, oracle, dpp, epd):
    n = dpp * epd
    pages = rand_pages(3, n, seed=dpp)
    w = make(cpp)
    bufs, sizes, bounds = _encode(cpp, w, pages, [1e-4] * 3)
    outs = [torch.zeros(epd + 3, dtype=torch.bfloat16, device=DEV)
            for _ in range(3 * dpp)]
    assert w.decompress_batch_fixed_bf16_scatter(bufs, sizes, outs, n, dpp,
                                                 epd, bounds)
    assert w.synchronize()
    for i in range(3):
        stream = bufs[i][:sizes[i]].cpu().numpy()
        want = oracle.decompress_contiguous(stream, n, bounds[i])
        got = np.concatenate([u16(outs[i * dpp + d])[:epd] for d in range(dpp)])
        assert np.array_equal(got, want)
        for d in range(dpp):
            assert not u16(outs[i * dpp + d])[epd:].any()


# ---- layer-indexed paths ---------------------------------------------------------

@pytest.mark.parametrize("prefix,src,epl,idx", [
    (2, 8, 4096, [1, 3, 6]),          # the reference's test shape (:60-72)
    (2, 28, 4096, [0, 1, 2, 5, 19, 20, 21]),
    (2, 6, 100, [5, 0, 3]),           # blocks straddle layers
    (3, 4, 8200, [2]),
])
def test_indexed_compress_and_scatter(cpp, oracle, prefix, src, epl, idx):
    batch = 3
    full = rand_pages(batch, prefix * src * epl, seed=epl)
    layer_idx = torch.tensor(idx, dtype=torch.long, device=DEV)
    n = prefix * len(idx) * epl
    w = make(cpp)
    bufs = buffers(cpp, batch, n)
    eps = [1e-4, 1e-5, 1e-3]
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed(
        list(full), bufs, layer_idx, prefix, src, epl, eps)
    assert ok
    bits = u16(full)
    assert_streams(oracle, bits, n, eps, True, bufs, sizes, bounds,
                   layers=idx, src=src, epl=epl)
    dest = torch.full_like(full, -2.0)
    assert w.decompress_batch_fixed_bf16_indexed_scatter(
        bufs, sizes, list(dest), layer_idx, prefix, src, epl, bounds)
    assert w.synchronize()
    got = u16(dest)
    for i in range(batch):
        want = u16(torch.full((prefix * src * epl,), -2.0, dtype=torch.bfloat16))
        stream = bufs[i][:sizes[i]].cpu().numpy()
        oracle.decompress_indexed(stream, n, bounds[i], want, idx, src, epl)
        assert np.array_equal(got[i], want), f"page {i}"


@pytest.mark.parametrize("prefix,src,epl,groups", [
    (2, 28, 4096, [[0, 1, 2, 5, 19, 20, 21],
                   [3, 4, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 22,
                    23, 24, 25, 26, 27]]),   # the mixed-bound restore
    (2, 6, 100, [[5, 0], [3], [1, 2, 4]]),   # blocks straddle layers
    (3, 4, 8200, [[2], [0, 3]]),             # partial tiles per job
])
def test_grouped_indexed_scatter_matches_oracle(cpp, oracle, prefix, src, epl,
                                                groups):
    """One grouped launch writes exactly what the per-group indexed scatter
    calls write: every group's layers decoded, all other values untouched."""
    per_group = [3, 2, 4][:len(groups)]
    full = rand_pages(max(per_group), prefix * src * epl, seed=epl + 7)
    w = make(cpp)
    bufs, sizes, bounds, idx_t, dests, jobs = [], [], [], [], [], []
    for g, layers in enumerate(groups):
        it = torch.tensor(layers, dtype=torch.long, device=DEV)
        n = prefix * len(layers) * epl
        b = buffers(cpp, per_group[g], n)
        eps = [1e-4, 1e-5, 1e-3, 2e-4][:per_group[g]]
        ok, s, e = w.compress_batch_fixed_bf16_indexed(
            list(full[:per_group[g]]), b, it, prefix, src, epl, eps)
        assert ok
        bufs += b
        sizes += list(s)
        bounds += list(e)
        idx_t.append(it)
        jobs += [(layers, n, i) for i in range(per_group[g])]
    dest = torch.full((len(jobs), prefix * src * epl), -2.0,
                      dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, list(dest), idx_t, per_group, prefix, src, epl, bounds)
    assert w.synchronize()
    got = u16(dest)
    for k, (layers, n, _) in enumerate(jobs):
        want = u16(torch.full((prefix * src * epl,), -2.0, dtype=torch.bfloat16))
        stream = bufs[k][:sizes[k]].cpu().numpy()
        oracle.decompress_indexed(stream, n, bounds[k], want, layers, src, epl)
        assert np.array_equal(got[k], want), f"job {k}"
    # the same jobs through the per-group calls give the same values
    ref = torch.full_like(dest, -2.0)
    k = 0
    for it, cnt in zip(idx_t, per_group):
        assert w.decompress_batch_fixed_bf16_indexed_scatter(
            bufs[k:k + cnt], sizes[k:k + cnt], list(ref[k:k + cnt]), it,
            prefix, src, epl, bounds[k:k + cnt])
        k += cnt
    assert w.synchronize()
    assert np.array_equal(u16(ref), got)


def test_grouped_indexed_scatter_skewed_groups(cpp, oracle):
    """Groups of very different payloads in one launch: all-zero pages
    (every block rate 0) beside random pages at REL 1e-6 (rates near 20,
    high plane words).  The decoder's runs are balanced by bytes, so its
    workgroups hold uneven tile counts, some none; every value must still
    come out as the oracle decodes it."""
    prefix, src, epl = 2, 6, 4096
    groups = [[0, 1, 2], [3, 4, 5]]
    counts = [3, 4]
    n = prefix * 3 * epl
    pages = [torch.zeros(counts[0], prefix * src * epl, dtype=torch.bfloat16, device=DEV),
             rand_pages(counts[1], prefix * src * epl, seed=11)]
    w = make(cpp)
    bufs, sizes, bounds, idx_t, jobs = [], [], [], [], []
    for g, layers in enumerate(groups):
        it = torch.tensor(layers, dtype=torch.long, device=DEV)
        b = buffers(cpp, counts[g], n)
        ok, s, e = w.compress_batch_fixed_bf16_indexed(
            list(pages[g]), b, it, prefix, src, epl, [1e-4 if g == 0 else 1e-6] * counts[g])
        assert ok
        bufs += b
        sizes += list(s)
        bounds += list(e)
        idx_t.append(it)
        jobs += [layers] * counts[g]
    assert max(sizes[counts[0]:]) > 4 * min(sizes[:counts[0]])
    dest = torch.full((len(jobs), prefix * src * epl), -2.0, dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, list(dest), idx_t, counts, prefix, src, epl, bounds)
    assert w.synchronize()
    got = u16(dest)
    for k, layers in enumerate(jobs):
        want = u16(torch.full((prefix * src * epl,), -2.0, dtype=torch.bfloat16))
        oracle.decompress_indexed(bufs[k][:sizes[k]].cpu().numpy(), n, bounds[k], want,
                                  layers, src, epl)
        assert np.array_equal(got[k], want), f"job {k}"


def test_grouped_indexed_scatter_rejects_bad_groups(cpp):
    full = rand_pages(2, 2 * 4 * 64, seed=3)
    w = make(cpp)
    it = torch.tensor([1, 2], dtype=torch.long, device=DEV)
    n = 2 * 2 * 64
    bufs = buffers(cpp, 2, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed(
        list(full), bufs, it, 2, 4, 64, [1e-4, 1e-4])
    assert ok
    dest = list(torch.zeros_like(full))
    # group sizes that do not cover the batch, an empty group, a group of
    # more layers than the source holds
    assert not w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, dest, [it], [1], 2, 4, 64, bounds)
    assert not w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, dest, [it, it], [2, 0], 2, 4, 64, bounds)
    big = torch.arange(5, dtype=torch.long, device=DEV) % 4
    assert not w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, dest, [big], [2], 2, 4, 64, bounds)
    assert w.synchronize()


def test_indexed_groups_match_oracle(cpp, oracle):
    import kv_synth

    shape = kv_synth.QWEN25_1P5B_4K
    pages = kv_synth.paged_kv(shape, seed=1, device=DEV, tokens=96)  # 6 pages
    groups = kv_synth.mixed_bound_groups()
    epl = shape.elements_per_layer
    bits = u16(pages)
    inputs, bufs, eps, idx_t, sizes_g = [], [], [], [], []
    for bound, layers in groups:
        n = 2 * len(layers) * epl
        for p in range(pages.shape[0]):
            inputs.append(pages[p])
            bufs.extend(buffers(cpp, 1, n))
            eps.append(bound)
        idx_t.append(torch.tensor(layers, dtype=torch.long, device=DEV))
        sizes_g.append(pages.shape[0])
    w = make(cpp)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed_groups(
        inputs, bufs, idx_t, sizes_g, 2, shape.layers, epl, eps)
    assert ok
    k = 0
    for (bound, layers), cnt in zip(groups, sizes_g):
        n = 2 * len(layers) * epl
        for p in range(cnt):
            eb = oracle.relative_bound(bits[p], n, bound, list(layers),
                                       shape.layers, epl)
            assert np.float32(bounds[k]) == eb
            want = oracle.compress_page(bits[p], n, float(eb), list(layers),
                                        shape.layers, epl)
            assert sizes[k] == len(want)
            assert np.array_equal(bufs[k][:sizes[k]].cpu().numpy(), want)
            k += 1
    # restore each group back into fresh pages, as the connector does
    dest = torch.zeros_like(pages)
    k = 0
    for (bound, layers), cnt, it in zip(groups, sizes_g, idx_t):
        assert w.decompress_batch_fixed_bf16_indexed_scatter(
            bufs[k:k + cnt], sizes[k:k + cnt], list(dest), it, 2, shape.layers,
            epl, bounds[k:k + cnt])
        k += cnt
    assert w.synchronize()
    err = (dest.float() - pages.float()).abs().view(pages.shape[0], 2,
                                                    shape.layers, epl)
    for (bound, layers), base in zip(groups, (0, sizes_g[0])):
        for p in range(pages.shape[0]):
            lim = 2 * bounds[base + p] + 1e-7
            assert float(err[p][:, list(layers)].max()) <= lim


def test_bad_layer_index_is_reported(cpp):
    full = rand_pages(2, 2 * 4 * 64, seed=1)
    idx = torch.tensor([1, 9], dtype=torch.long, device=DEV)  # 9 >= 4 layers
    w = make(cpp)
    bufs = buffers(cpp, 2, 2 * 2 * 64)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed(
        list(full), bufs, idx, 2, 4, 64, [1e-4, 1e-4])
    assert not ok and sizes == [] and bounds == []
    # the context stays usable
    idx_ok = torch.tensor([1, 3], dtype=torch.long, device=DEV)
    ok, _, _ = w.compress_batch_fixed_bf16_indexed(
        list(full), bufs, idx_ok, 2, 4, 64, [1e-4, 1e-4])
    assert ok


def test_malformed_streams_are_reported(cpp):
    n = 4096
    pages = rand_pages(2, n, seed=4)
    w = make(cpp)
    bufs, sizes, bounds = _encode(cpp, w, pages, [1e-4, 1e-4])
    out = torch.zeros(2 * n, dtype=torch.bfloat16, device=DEV)
    bad = bufs[0].clone()
    bad[3] = 40  # rate byte > 31
    assert w.decompress_batch_fixed_bf16([bad, bufs[1]], sizes, out, n, bounds)
    assert not w.synchronize()
    # a store enqueued behind a bad restore reports only its own launches;
    # the restore's error waits for synchronize()
    assert w.decompress_batch_fixed_bf16([bad, bufs[1]], sizes, out, n, bounds)
    ok, _, _ = w.compress_batch_fixed_bf16(list(pages), buffers(cpp, 2, n), [1e-4, 1e-4])
    assert ok
    assert not w.synchronize()
    short = [sizes[0] - 4, sizes[1]]
    assert w.decompress_batch_fixed_bf16(bufs, short, out, n, bounds)
    assert not w.synchronize()
    # shorter than the header: rejected before launch
    assert not w.decompress_batch_fixed_bf16(bufs, [100, sizes[1]], out, n, bounds)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
    assert w.synchronize()


# ---- long pages: relative bound from the pre-pass ----------------------------------

def test_long_page_uses_prepass_and_matches_oracle(cpp, oracle):
    n = 2_500_000 + 17  # > 256 tiles of 8192: min/max pre-pass
    pages = rand_pages(2, n, seed=8)
    w = make(cpp)
    bufs = buffers(cpp, 2, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs,
                                                    [1e-4, 1e-5])
    assert ok
    assert_streams(oracle, u16(pages), n, [1e-4, 1e-5], True, bufs, sizes,
                   bounds)
    out = torch.empty((2, n), dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
    assert w.synchronize()
    got = u16(out)
    for i in range(2):
        want = oracle.decompress_contiguous(bufs[i][:sizes[i]].cpu().numpy(), n,
                                            bounds[i])
        assert np.array_equal(got[i], want), f"page {i}"


# ---- repeated calls, workspace growth, shared state ------------------------------

def test_repeated_calls_and_growth(cpp, oracle):
    w = make(cpp)
    for batch, n, seed in [(2, 5000, 1), (40, 36864, 2), (1, 9000, 3),
                           (40, 36864, 4)]:
        pages = rand_pages(batch, n, seed)
        bufs, sizes, bounds = _encode(cpp, w, pages, [1e-4] * batch)
        out = torch.empty(batch * n, dtype=torch.bfloat16, device=DEV)
        assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
        assert w.synchronize()
        bits = u16(pages)
        for i in (0, batch - 1):
            eb = oracle.relative_bound(bits[i], n, 1e-4)
            want = oracle.compress_page(bits[i], n, float(eb))
            assert np.array_equal(bufs[i][:sizes[i]].cpu().numpy(), want)
            assert np.array_equal(u16(out)[i * n:(i + 1) * n],
                                  oracle.decompress_contiguous(want, n, eb))


def test_shim_rejects_invalid_arguments(cpp):
    w = make(cpp)
    n = 4096
    pages = rand_pages(2, n, seed=1)
    bufs = buffers(cpp, 2, n)
    assert w.compress_batch_fixed_bf16([], [], []) == (False, [], [])
    assert w.compress_batch_fixed_bf16(list(pages), bufs[:1], [1e-4]) == (False, [], [])
    assert w.compress_batch_fixed_bf16(list(pages.float()), bufs, [1e-4] * 2)[0] is False
    small = [torch.empty(100, dtype=torch.uint8, device=DEV)] * 2
    assert w.compress_batch_fixed_bf16(list(pages), small, [1e-4] * 2)[0] is False
    strided = torch.stack([pages, pages], dim=2)[:, :, 0]  # stride-2 rows
    assert not strided[0].is_contiguous()
    assert w.compress_batch_fixed_bf16(list(strided), bufs, [1e-4] * 2)[0] is False
    plain = cpp.CuSZpWrapper(cpp.CompressionConfig(), 0)  # MODE_PLAIN default
    assert plain.compress_batch_fixed_bf16(list(pages), bufs, [1e-4] * 2)[0] is False
    assert w.decompress_batch_fixed_bf16([], [], torch.empty(0, device=DEV), n, [])


# ---- both encoder schedules --------------------------------------------------
# Launches whose blocks are all whole, single-layer and 16-byte aligned use
# the persistent encoder; KVSZP_PERSISTENT=0 (read when a context is
# created) selects one workgroup per tile.  Both must write the same bytes.

@pytest.mark.parametrize("persistent", ["1", "0"])
def test_both_encoder_schedules_match_oracle(cpp, oracle, persistent, monkeypatch):
    monkeypatch.setenv("KVSZP_PERSISTENT", persistent)
    n = 36864                                   # 4.5 tiles: a partial last tile
    pages = rand_pages(4, n, seed=21)
    const = torch.full((n,), -2.75, dtype=torch.bfloat16, device=DEV)  # rate 31
    pages = torch.cat([pages, const[None]])
    for relative, eps in ((True, [1e-4, 1e-5, 2e-4, 1e-3, 1e-4]),
                          (False, [1e-3, 1e-2, 5e-4, 1e-3, 1e-3])):
        for quantizer in (0, 1):
            w = make(cpp, relative=relative, quantizer=quantizer)
            bufs = buffers(cpp, pages.shape[0], n)
            ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs, eps)
            assert ok
            assert_streams(oracle, u16(pages), n, eps, relative, bufs, sizes,
                           bounds, quantizer=quantizer)


@pytest.mark.parametrize("persistent", ["1", "0"])
@pytest.mark.parametrize("rate0", [0, 1])
def test_both_decoder_schedules_match_oracle(cpp, oracle, persistent, rate0,
                                            monkeypatch):
    monkeypatch.setenv("KVSZP_PERSISTENT", persistent)
    n = 36864 + 40                              # partial last block and tile
    pages = rand_pages(5, n, seed=31)
    pages[2, :9000] = 0                         # rate-0 blocks
    pages[3] = torch.full((n,), 7.0, dtype=torch.bfloat16, device=DEV)
    w = make(cpp, rate0=rate0)
    bufs, sizes, bounds = _encode(cpp, w, pages, [1e-4, 1e-5, 1e-4, 1e-4, 1e-3])
    pre = u16(torch.full((n,), 1.75, dtype=torch.bfloat16))
    out = torch.full((5 * n,), 1.75, dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
    assert w.synchronize()
    got = u16(out)
    for i in range(5):
        want = oracle.decompress_contiguous(bufs[i][:sizes[i]].cpu().numpy(), n,
                                            bounds[i], rate0, pre.copy())
        assert np.array_equal(got[i * n:(i + 1) * n], want), f"page {i}"


@pytest.mark.parametrize("persistent", ["1", "0"])
@pytest.mark.parametrize("target", ["contiguous", "scatter", "indexed"])
def test_malformed_streams_every_decoder(cpp, oracle, persistent, target, monkeypatch):
    """The checks above for every batched decoder and both schedules, with
    the bad byte in a later tile than the first: a header byte above 31 and
    a declared size shorter than the payload are reported at the next
    synchronize(), and the context then decodes valid streams exactly."""
    monkeypatch.setenv("KVSZP_PERSISTENT", persistent)
    prefix, src, epl, idx = 2, 6, 4096, [4, 1, 3]
    full = rand_pages(3, prefix * src * epl, seed=77)
    layer_idx = torch.tensor(idx, dtype=torch.long, device=DEV)
    n = prefix * len(idx) * epl                 # 24576: 3 tiles of 256 blocks
    w = make(cpp)
    bufs = buffers(cpp, 3, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed(
        list(full), bufs, layer_idx, prefix, src, epl, [1e-4] * 3)
    assert ok

    def decode(streams, stream_sizes):
        if target == "contiguous":
            out = torch.zeros(3 * n, dtype=torch.bfloat16, device=DEV)
            return out, w.decompress_batch_fixed_bf16(streams, stream_sizes, out, n, bounds)
        if target == "scatter":
            outs = [torch.zeros(n, dtype=torch.bfloat16, device=DEV) for _ in range(3)]
            return outs, w.decompress_batch_fixed_bf16_scatter(
                streams, stream_sizes, outs, n, 1, n, bounds)
        outs = torch.zeros_like(full)
        return outs, w.decompress_batch_fixed_bf16_indexed_scatter(
            streams, stream_sizes, list(outs), layer_idx, prefix, src, epl, bounds)

    bad = [b.clone() for b in bufs]
    bad[1][300] = 40                            # block 300 (second tile) of page 1
    _, ok = decode(bad, sizes)
    assert ok                                   # enqueue only
    assert w.synchronize() is False
    _, ok = decode(bufs, [sizes[0], sizes[1], sizes[2] - 4])
    assert ok
    assert w.synchronize() is False
    out, ok = decode(bufs, sizes)
    assert ok and w.synchronize()
    for i in range(3):
        stream = bufs[i][:sizes[i]].cpu().numpy()
        if target == "indexed":
            want = u16(torch.zeros(prefix * src * epl, dtype=torch.bfloat16))
            oracle.decompress_indexed(stream, n, bounds[i], want, idx, src, epl)
            got = u16(out[i])
        else:
            want = oracle.decompress_contiguous(stream, n, bounds[i], 1)
            got = u16(out)[i * n:(i + 1) * n] if target == "contiguous" else u16(out[i])
        assert np.array_equal(got, want), f"page {i}"


@pytest.mark.parametrize("rate0", [0, 1])
def test_large_batch_of_mixed_pages(cpp, oracle, rate0):
    """1100 requests in one call: the persistent decoder's runs are then
    balanced job by job (each job's output plus payload bytes).  Pages of
    very different rates side by side (all-zero, constant, heavy-tailed,
    Gaussian) and a partial last tile per page; every restored value is
    compared with the oracle, contiguous and single-destination scatter."""
    batch, n = 1100, 20000                      # 3 tiles per page, the last partial
    g = torch.Generator(device="cpu").manual_seed(99)
    x = torch.randn(batch, n, generator=g)
    kind = torch.randint(0, 4, (batch,), generator=g)
    x[kind == 0] = 0.0
    x[kind == 1] = 1.5
    heavy = kind == 2
    x[heavy] = x[heavy] / torch.rand(int(heavy.sum()), n, generator=g).clamp_min(1e-3)
    pages = x.to(torch.bfloat16).to(DEV)
    w = make(cpp, rate0=rate0)
    bufs, sizes, bounds = _encode(cpp, w, pages, [1e-4] * batch)
    pre = np.full(n, 0x3FE0, dtype=np.uint16)                # 1.75
    out = torch.from_numpy(np.tile(pre, batch).view(np.int16)).view(torch.bfloat16).to(DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
    dests = [torch.full((n,), 1.75, dtype=torch.bfloat16, device=DEV) for _ in range(batch)]
    assert w.decompress_batch_fixed_bf16_scatter(bufs, sizes, dests, n, 1, n, bounds)
    assert w.synchronize()
    got = u16(out).reshape(batch, n)
    got_s = u16(torch.stack(dests))
    for i in range(batch):
        want = oracle.decompress_contiguous(bufs[i][:sizes[i]].cpu().numpy(), n, bounds[i],
                                            rate0, pre.copy())
        assert np.array_equal(got[i], want), f"page {i} (class {int(kind[i])})"
        assert np.array_equal(got_s[i], want), f"scatter page {i}"


def test_indexed_groups_beyond_sixteen_groups(cpp, oracle):
    """One REL bound per Qwen2.5-1.5B layer: 28 layer groups of 8 pages in
    one compress_batch_fixed_bf16_indexed_groups call (the reference takes
    any number of groups, cuszp_wrapper.cpp:683-868) and one grouped
    restore; byte-exact against the oracle."""
    import kv_synth

    shape = kv_synth.QWEN25_1P5B_4K
    pages = kv_synth.paged_kv(shape, seed=4, device=DEV, tokens=128)  # 8 pages
    epl, layers = shape.elements_per_layer, shape.layers
    bits = u16(pages)
    eps_of = [1e-5 if l in kv_synth.QWEN15B_SENSITIVE_LAYERS else 1e-4 * (1 + l % 3)
              for l in range(layers)]
    inputs, bufs, eps, idx_t, counts, jobs = [], [], [], [], [], []
    n = 2 * epl
    for l in range(layers):
        idx_t.append(torch.tensor([l], dtype=torch.long, device=DEV))
        counts.append(pages.shape[0])
        for p in range(pages.shape[0]):
            inputs.append(pages[p])
            eps.append(eps_of[l])
            jobs.append((l, p))
        bufs.extend(buffers(cpp, pages.shape[0], n))
    w = make(cpp)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed_groups(
        inputs, bufs, idx_t, counts, 2, layers, epl, eps)
    assert ok and len(sizes) == layers * pages.shape[0]
    for k, (l, p) in enumerate(jobs):
        eb = oracle.relative_bound(bits[p], n, eps_of[l], [l], layers, epl)
        assert np.float32(bounds[k]) == np.float32(eb), (l, p)
        want = oracle.compress_page(bits[p], n, float(eb), [l], layers, epl)
        assert sizes[k] == want.size and np.array_equal(
            bufs[k][:sizes[k]].cpu().numpy(), want), (l, p)
    # restore every layer group of every page in one grouped call
    dest = torch.full((len(jobs), pages.shape[1]), -2.0, dtype=torch.bfloat16, device=DEV)
    assert w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, list(dest), idx_t, counts, 2, layers, epl, bounds)
    assert w.synchronize()
    got = u16(dest)
    for k, (l, p) in enumerate(jobs):
        want = u16(torch.full((pages.shape[1],), -2.0, dtype=torch.bfloat16))
        oracle.decompress_indexed(bufs[k][:sizes[k]].cpu().numpy(), n, bounds[k],
                                  want, [l], layers, epl)
        assert np.array_equal(got[k], want), (l, p)
    # into shared pages: all 28 groups of a page land in the same page
    shared = torch.zeros_like(pages)
    dests = [shared[p] for (_, p) in jobs]
    assert w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, dests, idx_t, counts, 2, layers, epl, bounds)
    assert w.synchronize()
    err = (shared.float() - pages.float()).abs().view(pages.shape[0], 2, layers, epl)
    for k, (l, p) in enumerate(jobs):
        assert float(err[p, :, l].max()) <= 2 * bounds[k] + 1e-7
