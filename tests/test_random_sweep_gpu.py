"""Seeded random sweep through the drop-in module on the GPU.

Each case draws its call shape and its values from its own seed: segments
from one element to several 8192-element tiles, batches of one to five
pages, pages that are only 2-byte aligned, relative and absolute bounds
(among them bounds that make 0.5 / eb overflow or underflow, and eps that
falls back to the configured bound: zero, negative, NaN), both quantizer
readings and both rate-0 policies, layer maps and layer groups,
multi-destination restores, packed publication and restore, and the fp32
API in all three modes.  Every stream is compared byte for byte with the
oracle, every returned bound with the oracle's fp32 bound, every restored
value bit for bit, and no byte past a stream may change (the buffers are
filled with 0xAB first).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
CONFIG_EB = 1e-4          # the wrappers' configured bound (eps <= 0 or NaN)
# KVSZP_SWEEP_SEEDS=n widens the sweep to seeds 0 .. n-1 (64 by default)
SEEDS = range(int(os.environ.get("KVSZP_SWEEP_SEEDS", "64")))

EXTREME_ABS = [1e-40, 1e-45, 2e-39, float("inf"), float("nan"), 0.0, -1.0, 3e38]
EXTREME_REL = [1e-40, 1e-45, 3e-39, float("inf"), float("nan"), 0.0, -1.0, 1e30]
KINDS = ["normal", "normal", "normal", "offset", "constant", "special", "tiny",
         "zeros", "huge"]


@pytest.fixture(scope="module")
def cpp():
    import cuszp_wrapper_cpp

    return cuszp_wrapper_cpp


def wrapper(cpp, relative, quantizer=0, rate0=1, mode="MODE_FIXED"):
    w = cpp.CuSZpWrapper(cpp.CompressionConfig(CONFIG_EB, relative, cpp.DIM_1D,
                                               getattr(cpp, mode), cpp.TYPE_FLOAT), 0)
    if mode == "MODE_FIXED":
        w.set_codec_options(quantizer, rate0)
    return w


def pick_eps(rng, relative, usual):
    if rng.random() < 0.15:
        return float(rng.choice(EXTREME_REL if relative else EXTREME_ABS))
    return float(rng.choice(usual))


def effective(eps):
    """cuszp_wrapper.cpp:473-479: eps_i > 0 ? eps_i : config.error_bound."""
    e = np.float32(eps)
    return e if e > 0 else np.float32(CONFIG_EB)


def values(rng, rows, n, kind):
    """fp32 values of one kind; the BF16 pages are their RNE roundings."""
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x *= np.exp(rng.standard_normal((rows, 1)) * 2).astype(np.float32)
    m = rng.random((rows, n))
    if kind == "offset":
        x += 50.0
    elif kind == "constant":
        x[:] = 3.25
    elif kind == "special":
        x[m < 0.01] = np.inf
        x[m > 0.995] = -np.inf
        x[(m > 0.5) & (m < 0.502)] = np.nan
    elif kind == "tiny":
        x *= np.float32(1e-30)
    elif kind == "zeros":
        x[:] = 0.0
    elif kind == "huge":
        x[m < 0.02] = 3.0e38
        x[m > 0.98] = -3.0e38
        x[(m > 0.5) & (m < 0.501)] = np.inf
    return x


def bf16_pages(rng, rows, n, kind):
    return torch.from_numpy(values(rng, rows, n, kind)).to(torch.bfloat16).to(DEV)


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def canary_buffers(oracle, count, n):
    cap = max(8 * n, oracle.max_stream_bytes(n))
    return [torch.full((cap,), 0xAB, dtype=torch.uint8, device=DEV) for _ in range(count)]


def check_streams(oracle, bits, n, bufs, sizes, bounds, eps, relative, quantizer,
                  layers=None, src=0, epl=0):
    for i, buf in enumerate(bufs):
        e = effective(eps[i])
        eb = oracle.relative_bound(bits[i], n, float(e), layers, src, epl) if relative else e
        same = np.float32(bounds[i]) == np.float32(eb) or (np.isnan(eb) and np.isnan(bounds[i]))
        assert same, ("bound", i, bounds[i], eb)
        want = oracle.compress_page(bits[i], n, float(eb), layers, src, epl, quantizer)
        host = buf.cpu().numpy()
        assert sizes[i] == want.size, ("size", i, sizes[i], want.size)
        got = host[:sizes[i]]
        if not np.array_equal(got, want):
            pytest.fail(f"stream {i}: first differing byte {int(np.nonzero(got != want)[0][0])}")
        assert (host[sizes[i]:] == 0xAB).all(), ("written past the stream", i)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_contiguous_pages(cpp, oracle, seed):
    """compress_batch_fixed_bf16 then decompress_batch_fixed_bf16."""
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.choice([rng.integers(1, 300), rng.integers(300, 20000),
                        rng.integers(20000, 70000)]))
    batch = int(rng.integers(1, 6))
    relative = bool(rng.random() < 0.7)
    quantizer, rate0 = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    kind = str(rng.choice(KINDS))
    usual = ([1e-2, 1e-3, 1e-4, 1e-5, 3e-6, 0.5, 2.0] if relative else
             [1e-1, 1e-2, 1e-3, 0.5, 1e-30, 1e30])
    eps = [pick_eps(rng, relative, usual) for _ in range(batch)]
    pages = bf16_pages(rng, batch, n, kind)
    bits = u16(pages)
    if rng.random() < 0.4:                      # element-offset views: 2-byte aligned
        off = int(rng.integers(1, 8))
        big = torch.zeros(batch, n + 8, dtype=torch.bfloat16, device=DEV)
        big[:, off:off + n] = pages
        inputs = [big[i, off:off + n] for i in range(batch)]
    else:
        inputs = list(pages)
    w = wrapper(cpp, relative, quantizer, rate0)
    bufs = canary_buffers(oracle, batch, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(inputs, bufs, eps)
    assert ok
    check_streams(oracle, bits, n, bufs, sizes, bounds, eps, relative, quantizer)
    before = np.full(n, 0x3FE0, dtype=np.uint16)          # 1.75
    out = torch.from_numpy(np.tile(before, batch).view(np.int16)).view(torch.bfloat16).to(DEV)
    assert w.decompress_batch_fixed_bf16(bufs, sizes, out, n, bounds)
    assert w.synchronize()
    got = u16(out)
    for i in range(batch):
        want = oracle.decompress_contiguous(bufs[i][:sizes[i]].cpu().numpy(), n,
                                            float(bounds[i]), rate0, before.copy())
        assert np.array_equal(got[i * n:(i + 1) * n], want), ("restore", i)


def random_layers(rng, src):
    sel = int(rng.integers(1, src + 1))
    return [int(v) for v in rng.permutation(src)[:sel]]


@pytest.mark.parametrize("seed", SEEDS)
def test_random_indexed_pages(cpp, oracle, seed):
    """compress_batch_fixed_bf16_indexed then the indexed scatter restore."""
    rng = np.random.default_rng(2000 + seed)
    prefix, src = int(rng.integers(1, 4)), int(rng.integers(1, 31))
    epl = int(rng.choice([32, 64, 100, 1000, 4096, 5000]))
    layers = random_layers(rng, src)
    batch = int(rng.integers(1, 5))
    relative = bool(rng.random() < 0.7)
    quantizer, rate0 = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    kind = str(rng.choice(KINDS))
    numel, n = prefix * src * epl, prefix * len(layers) * epl
    pages = bf16_pages(rng, batch, numel, kind)
    bits = u16(pages)
    eps = [pick_eps(rng, relative, [1e-3, 1e-4, 1e-5] if relative else [1e-2, 1e-3])
           for _ in range(batch)]
    idx = torch.tensor(layers, dtype=torch.long, device=DEV)
    w = wrapper(cpp, relative, quantizer, rate0)
    bufs = canary_buffers(oracle, batch, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed(list(pages), bufs, idx, prefix,
                                                            src, epl, eps)
    assert ok
    check_streams(oracle, bits, n, bufs, sizes, bounds, eps, relative, quantizer,
                  layers, src, epl)
    dest = torch.full_like(pages, -2.0)
    assert w.decompress_batch_fixed_bf16_indexed_scatter(bufs, sizes, list(dest), idx,
                                                         prefix, src, epl, bounds)
    assert w.synchronize()
    want = np.tile(u16(torch.full((numel,), -2.0, dtype=torch.bfloat16)), (batch, 1))
    for i in range(batch):
        oracle.decompress_indexed(bufs[i][:sizes[i]].cpu().numpy(), n, float(bounds[i]),
                                  want[i], layers, src, epl, rate0)
    assert np.array_equal(u16(dest), want)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_layer_groups(cpp, oracle, seed):
    """compress_batch_fixed_bf16_indexed_groups (one bound per group) then
    the grouped indexed scatter restore into the same pages."""
    rng = np.random.default_rng(3000 + seed)
    prefix, src = int(rng.integers(1, 4)), int(rng.integers(2, 41))
    epl = int(rng.choice([32, 64, 100, 1000, 1024, 4096, 5000]))
    order = [int(v) for v in rng.permutation(src)]
    cuts = sorted(int(v) for v in rng.choice(np.arange(1, src), size=min(src - 1, int(
        rng.integers(0, 20))), replace=False)) if src > 1 else []
    groups = [order[a:b] for a, b in zip([0] + cuts, cuts + [src])]
    groups = [sorted(g) if rng.random() < 0.5 else g for g in groups]
    pages_n = int(rng.integers(1, 5))
    relative = bool(rng.random() < 0.8)
    quantizer = int(rng.integers(0, 2))
    kind = str(rng.choice(["normal", "normal", "offset", "special", "tiny"]))
    numel = prefix * src * epl
    pages = bf16_pages(rng, pages_n, numel, kind)
    bits = u16(pages)
    inputs, eps, idx, counts, ns = [], [], [], [], []
    for layers in groups:
        e = pick_eps(rng, relative, [1e-3, 1e-4, 1e-5] if relative else [1e-2, 1e-3])
        inputs += list(pages)
        eps += [e] * pages_n
        idx.append(torch.tensor(layers, dtype=torch.long, device=DEV))
        counts.append(pages_n)
        ns.append(prefix * len(layers) * epl)
    bufs = [b for m in ns for b in canary_buffers(oracle, pages_n, m)]
    w = wrapper(cpp, relative, quantizer)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed_groups(inputs, bufs, idx, counts,
                                                                   prefix, src, epl, eps)
    assert ok
    for gi, layers in enumerate(groups):
        k = slice(gi * pages_n, (gi + 1) * pages_n)
        check_streams(oracle, bits, ns[gi], bufs[k], sizes[k], bounds[k], eps[k], relative,
                      quantizer, layers, src, epl)
    dest = torch.zeros_like(pages)
    assert w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, list(dest) * len(groups), idx, counts, prefix, src, epl, bounds)
    assert w.synchronize()
    want = np.zeros((pages_n, numel), dtype=np.uint16)
    for gi, layers in enumerate(groups):
        for p in range(pages_n):
            k = gi * pages_n + p
            oracle.decompress_indexed(bufs[k][:sizes[k]].cpu().numpy(), ns[gi],
                                      float(bounds[k]), want[p], layers, src, epl)
    assert np.array_equal(u16(dest), want)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_multi_destination_restore(cpp, oracle, seed):
    """decompress_batch_fixed_bf16_scatter over dpp destinations of epd
    values, each destination a little longer than epd (the tail untouched)."""
    rng = np.random.default_rng(4000 + seed)
    dpp = int(rng.integers(1, 9))
    epd = int(rng.choice([32, 64, 96, 1000, 4096, 5000, 8192]))
    n, batch = dpp * epd, int(rng.integers(1, 5))
    relative, rate0 = bool(rng.random() < 0.7), int(rng.integers(0, 2))
    eps = [pick_eps(rng, relative, [1e-3, 1e-4, 1e-5] if relative else [1e-2, 1e-3])
           for _ in range(batch)]
    pages = bf16_pages(rng, batch, n, str(rng.choice(["normal", "offset", "special"])))
    bits = u16(pages)
    w = wrapper(cpp, relative, 0, rate0)
    bufs = canary_buffers(oracle, batch, n)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(pages), bufs, eps)
    assert ok
    check_streams(oracle, bits, n, bufs, sizes, bounds, eps, relative, 0)
    dests = [torch.zeros(epd + int(rng.integers(0, 4)), dtype=torch.bfloat16, device=DEV)
             for _ in range(batch * dpp)]
    assert w.decompress_batch_fixed_bf16_scatter(bufs, sizes, dests, n, dpp, epd, bounds)
    assert w.synchronize()
    for i in range(batch):
        want = [np.zeros(d.numel(), dtype=np.uint16) for d in dests[i * dpp:(i + 1) * dpp]]
        oracle.decompress_scatter(bufs[i][:sizes[i]].cpu().numpy(), n, float(bounds[i]),
                                  want, epd, rate0)
        for j in range(dpp):
            assert np.array_equal(u16(dests[i * dpp + j]), want[j]), ("destination", i, j)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_fp32_pages(cpp, oracle, seed):
    """The single-page fp32 API (compress / decompress) in the fixed, plain
    and outlier modes."""
    rng = np.random.default_rng(5000 + seed)
    mode = str(rng.choice(["MODE_FIXED", "MODE_PLAIN", "MODE_OUTLIER"]))
    mode_id = {"MODE_FIXED": 0, "MODE_PLAIN": 1, "MODE_OUTLIER": 2}[mode]
    n = int(rng.choice([rng.integers(1, 100), rng.integers(100, 40000)]))
    relative = bool(rng.random() < 0.7)
    kind = str(rng.choice(["normal", "normal", "smooth", "special", "constant", "tiny"]))
    if kind == "smooth":
        x = np.cumsum(values(rng, 1, n, "normal")[0] * np.float32(0.01)).astype(np.float32)
    else:
        x = values(rng, 1, n, kind)[0]
    eps = pick_eps(rng, relative, [1e-2, 1e-3, 1e-4, 1e-5] if relative else
                   [1e-1, 1e-3, 0.5, 2.0])
    w = wrapper(cpp, relative, mode=mode)
    buf = torch.full((max(w.estimate_compressed_buffer_size(4 * n),
                          oracle.max_stream_bytes_lorenzo(n)),), 0xAB, dtype=torch.uint8,
                     device=DEV)
    ok, buf, size, bound = w.compress(torch.from_numpy(x).to(DEV), buf, eps)
    assert ok
    e = effective(eps)
    eb = oracle.relative_bound_f32(x, float(e)) if relative else e
    assert np.float32(bound) == np.float32(eb) or (np.isnan(eb) and np.isnan(bound))
    want = oracle.compress_page_f32_mode(x, float(eb), mode_id)
    host = buf.cpu().numpy()
    assert size == want.size and np.array_equal(host[:size], want)
    assert (host[size:] == 0xAB).all()
    out = torch.full((n,), 9.0, device=DEV)
    assert w.decompress(buf, size, out, bound)
    assert w.synchronize()
    ref = oracle.decompress_f32_mode(want, n, float(eb), mode_id)
    got = out.cpu().numpy()
    assert np.all((got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref)))


def packed_offsets(sizes):
    """8-byte-aligned exclusive scan of the payload sizes (the slab layout
    of vllm_v1_compressed_offload.py:371-447) and the slab's used length."""
    offs, end = [], 0
    for s in sizes:
        start = (end + 7) // 8 * 8
        offs.append(start)
        end = start + s
    return offs, end


@pytest.mark.parametrize("seed", SEEDS)
def test_random_packed_store_and_restore(cpp, oracle, seed):
    """Grouped indexed store, payloads packed into one slab (pinned host or
    device memory) and the packed grouped restore (from a device staging
    copy or straight from the pinned slab): slab bytes equal the streams at
    the scan offsets with zeroed gaps, and the restored pages equal the
    oracle's decode of every stream."""
    rng = np.random.default_rng(6000 + seed)
    prefix, src = 2, int(rng.integers(2, 29))
    epl = int(rng.choice([256, 1024, 4096]))
    order = [int(v) for v in rng.permutation(src)]
    ngroups = int(rng.integers(1, min(src, 4) + 1))
    cuts = sorted(int(v) for v in rng.choice(np.arange(1, src), size=ngroups - 1,
                                             replace=False))
    groups = [sorted(order[a:b]) for a, b in zip([0] + cuts, cuts + [src])]
    pages_n = int(rng.integers(1, 6))
    pages = bf16_pages(rng, pages_n, prefix * src * epl,
                       str(rng.choice(["normal", "normal", "offset", "special", "zeros"])))
    inputs, eps, idx, counts, ns = [], [], [], [], []
    for layers in groups:
        inputs += list(pages)
        eps += [float(rng.choice([1e-3, 1e-4, 1e-5]))] * pages_n
        idx.append(torch.tensor(layers, dtype=torch.long, device=DEV))
        counts.append(pages_n)
        ns.append(prefix * len(layers) * epl)
    bufs = [b for m in ns for b in canary_buffers(oracle, pages_n, m)]
    w = wrapper(cpp, True)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed_groups(inputs, bufs, idx, counts,
                                                                   prefix, src, epl, eps)
    assert ok
    streams = [bufs[k][:sizes[k]] for k in range(len(bufs))]
    want_offs, want_end = packed_offsets(sizes)
    on_host = bool(rng.random() < 0.7)
    slab = torch.full((want_end + 64,), 0xCD, dtype=torch.uint8)
    slab = slab.pin_memory() if on_host else slab.to(DEV)
    ok, offsets, packed = w.pack_payloads(streams, slab)
    assert ok and offsets == want_offs and packed == want_end
    host = slab.cpu().numpy()
    cursor = 0
    for k, s in enumerate(streams):
        assert not host[cursor:offsets[k]].any(), ("gap", k)
        assert np.array_equal(host[offsets[k]:offsets[k] + sizes[k]], s.cpu().numpy()), k
        cursor = offsets[k] + sizes[k]
    assert (host[packed:] == 0xCD).all()
    want = np.zeros((pages_n, prefix * src * epl), dtype=np.uint16)
    for gi, layers in enumerate(groups):
        for p in range(pages_n):
            k = gi * pages_n + p
            oracle.decompress_indexed(streams[k].cpu().numpy(), ns[gi], float(bounds[k]),
                                      want[p], layers, src, epl)
    if on_host:
        staging = (torch.empty(packed, dtype=torch.uint8, device=DEV)
                   if rng.random() < 0.5 else None)
        dest = torch.zeros_like(pages)
        assert w.decompress_batch_fixed_bf16_indexed_scatter_groups_packed(
            slab, packed, staging, offsets, sizes, list(dest) * len(groups), idx, counts,
            prefix, src, epl, bounds)
        assert w.synchronize()
        assert np.array_equal(u16(dest), want)


# KVSZP_SWEEP_LARGE_SEEDS=n widens the large grouped restore below (4 seeds by default)
LARGE_SEEDS = range(int(os.environ.get("KVSZP_SWEEP_LARGE_SEEDS", "4")))


@pytest.mark.parametrize("seed", LARGE_SEEDS)
def test_random_large_grouped_restore(cpp, oracle, seed):
    """Grouped indexed store, then one grouped indexed-scatter restore of
    2400-6000 tiles: more tiles than the persistent decoder's grid, so its
    workgroup runs start inside jobs of the groups' different tile counts
    (layer sizes off the block size); 60-600 requests, so job tables travel
    in the kernel arguments or, above 597 requests, are copied.  Every
    stream and bound equals the oracle's, and every restored value the
    oracle's decode of its stream."""
    rng = np.random.default_rng(9000 + seed)
    prefix, src = 2, int(rng.integers(8, 29))
    epl = int(rng.integers(6000, 20001))
    order = [int(v) for v in rng.permutation(src)]
    ngroups = int(rng.integers(1, 4))
    cuts = sorted(int(v) for v in rng.choice(np.arange(1, src), size=ngroups - 1,
                                             replace=False))
    groups = [sorted(order[a:b]) for a, b in zip([0] + cuts, cuts + [src])]
    tile = 8192
    tiles_per_page = sum(-(-prefix * len(g) * epl // tile) for g in groups)
    target = int(rng.integers(2500, 6001))
    pages_n = max(1, min(600 // ngroups, -(-target // tiles_per_page)))
    pages = bf16_pages(rng, pages_n, prefix * src * epl,
                       str(rng.choice(["normal", "offset", "special"])))
    inputs, eps, idx, counts, ns = [], [], [], [], []
    for layers in groups:
        inputs += list(pages)
        eps += [float(rng.choice([1e-3, 1e-4, 1e-5]))] * pages_n
        idx.append(torch.tensor(layers, dtype=torch.long, device=DEV))
        counts.append(pages_n)
        ns.append(prefix * len(layers) * epl)
    assert sum(pages_n * -(-m // tile) for m in ns) > 2048
    bufs = [b for m in ns for b in canary_buffers(oracle, pages_n, m)]
    w = wrapper(cpp, True)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed_groups(inputs, bufs, idx, counts,
                                                                   prefix, src, epl, eps)
    assert ok
    # the store: a persistent encoder launch of several rounds over the same jobs
    bits = u16(pages)
    for gi, layers in enumerate(groups):
        k = slice(gi * pages_n, (gi + 1) * pages_n)
        check_streams(oracle, bits, ns[gi], bufs[k], sizes[k], bounds[k], eps[k], True, 0,
                      layers, src, epl)
    dest = torch.zeros_like(pages)
    assert w.decompress_batch_fixed_bf16_indexed_scatter_groups(
        bufs, sizes, list(dest) * len(groups), idx, counts, prefix, src, epl, bounds)
    assert w.synchronize()
    want = np.zeros((pages_n, prefix * src * epl), dtype=np.uint16)
    for gi, layers in enumerate(groups):
        for p in range(pages_n):
            k = gi * pages_n + p
            oracle.decompress_indexed(bufs[k][:sizes[k]].cpu().numpy(), ns[gi],
                                      float(bounds[k]), want[p], layers, src, epl)
    assert np.array_equal(u16(dest), want)
