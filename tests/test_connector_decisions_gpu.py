"""The connector's decisions on what the codec returns, replayed through the
drop-in ``cuszp_wrapper_cpp`` and checked against the oracle.

tests/test_connector_calls_gpu.py replays every call shape the reference
connector (integration/compression_pipeline/vllm_v1_compressed_offload.py)
issues.  This module replays the places where the connector acts on the
results of those calls, with the rules restated from the cited lines:

* raw fallback: a segment whose returned size is at least its BF16 bytes is
  stored raw (:994-1005 uniform path, :1253-1266 gathered path, :726-738
  per-segment path);
* the indexed path gives up the whole job when any segment would expand
  (:1529-1534) and the job goes to the gathered path (:2245-2250,
  :1030-1284), which gathers each layer group with index_select and calls
  compress_batch_fixed_bf16 per segment length;
* jobs of one page skip every batched path (:853, :1041, :1296) and go
  through the per-segment path: BF16 widened to fp32 and compressed with the
  selected mode's single-page compress (:617, :716-738, :2251-2260); the
  restore decodes fp32 and converts to BF16 (:2141-2180);
* the packed store puts raw and compressed payloads side by side in one
  pinned slab at 8-byte-aligned offsets (:371-447); the restore copies raw
  full-page payloads straight into the pages (:1578-1615, :1627-1642),
  index_copy_s raw layer-group payloads (:2057-2079) and decodes the rest
  with the batched kernels (:1880-1938).

The saturating page is the one the reference's own decision exists for: a
constant BF16 page under a relative bound has eb = eps * 1e-6, every value
quantizes to INT_MAX and every block gets rate 31, 129 bytes per 64 bytes of
BF16.  Pages are Qwen2.5-1.5B vLLM blocks [2, 28, 16, 2, 128] (229 376 values).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
LAYERS, EPL = 28, 16 * 2 * 128
PAGE_N = 2 * LAYERS * EPL
SENSITIVE = (0, 1, 2, 5, 19, 20, 21)    # data/qwen2.5-1.5b_mixed_21x1e-4_7x1e-5.json
OTHERS = tuple(l for l in range(LAYERS) if l not in SENSITIVE)
CONSTANT = 0.8125                        # a BF16 value


@pytest.fixture(scope="module")
def cpp():
    import cuszp_wrapper_cpp

    return cuszp_wrapper_cpp


@pytest.fixture(scope="module")
def pages():
    import kv_synth

    return kv_synth.paged_kv(kv_synth.QWEN25_1P5B_4K, seed=11, device=DEV,
                             tokens=64)  # 4 pages


def wrapper(cpp, mode="MODE_FIXED"):
    cfg = cpp.CompressionConfig(1e-4, True, cpp.CuszpDim.DIM_1D,
                                getattr(cpp.CuszpMode, mode), cpp.CuszpType.TYPE_FLOAT)
    return cpp.CuSZpWrapper(cfg, 0)


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def slab_slices(caps):
    slab = torch.empty(sum(caps), dtype=torch.uint8, device=DEV)
    out, off = [], 0
    for c in caps:
        out.append(slab[off:off + c])
        off += c
    return out


def stored_as(size: int, original_bytes: int) -> str:
    """:994-1005 / :1253-1266 / :733-738: compressed only if smaller."""
    return "cuszp" if size < original_bytes else "raw"


def packed_layout(payload_sizes):
    """CompressedPageStore.put_many_packed (:386-393): payload i starts at
    the running end rounded up to 8 bytes."""
    starts, total = [], 0
    for size in payload_sizes:
        start = (total + 7) // 8 * 8
        starts.append(start)
        total = start + size
    return starts, total


def test_uniform_store_raw_fallback_packed_and_restored(cpp, oracle, pages):
    """Uniform flat store of four pages, one of them constant: that page's
    stream is larger than the page, so it is stored raw beside the three
    streams in one packed slab; the restore copies it back and decodes the
    others straight into their pages."""
    src = pages.clone()
    src[1] = CONSTANT
    batch = src.shape[0]
    w = wrapper(cpp)
    bufs = slab_slices([8 * PAGE_N] * batch)
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(src), bufs, [1e-4] * batch)
    assert ok
    bits = u16(src)
    original = 2 * PAGE_N
    kinds, payloads = [], []
    for i in range(batch):
        eb = oracle.relative_bound(bits[i], PAGE_N, 1e-4)
        assert np.float32(bounds[i]) == np.float32(eb)
        want = oracle.compress_page(bits[i], PAGE_N, float(eb))
        assert sizes[i] == want.size
        assert np.array_equal(bufs[i][:sizes[i]].cpu().numpy(), want)
        kinds.append(stored_as(sizes[i], original))
        payloads.append(bufs[i][:sizes[i]] if kinds[-1] == "cuszp"
                        else src[i].view(torch.uint8))
    assert kinds == ["cuszp", "raw", "cuszp", "cuszp"]
    # rate 31 in every block: header + 128 bytes per block
    assert sizes[1] == 7168 + 128 * (PAGE_N // 32) and sizes[1] >= original

    starts, total = packed_layout([int(p.numel()) for p in payloads])
    slab = torch.full((total + 64,), 0xCD, dtype=torch.uint8).pin_memory()
    ok, offsets, packed = w.pack_payloads(payloads, slab)
    assert ok and offsets == starts and packed == total
    host = slab.numpy()
    for p, start in zip(payloads, starts):
        assert np.array_equal(host[start:start + p.numel()], p.cpu().numpy())

    dest = torch.zeros_like(src)
    for i, start in enumerate(starts):      # raw full pages (:1578-1615)
        if kinds[i] == "raw":
            dest[i].view(torch.uint8).copy_(slab[start:start + original], non_blocking=True)
    comp = [i for i in range(batch) if kinds[i] == "cuszp"]
    staged = [slab[starts[i]:starts[i] + sizes[i]].to(DEV) for i in comp]
    assert w.decompress_batch_fixed_bf16_scatter(      # :1930-1938
        staged, [sizes[i] for i in comp], [dest[i] for i in comp], PAGE_N, 1, PAGE_N,
        [bounds[i] for i in comp])
    assert w.synchronize()
    got = u16(dest)
    assert np.array_equal(got[1], bits[1])
    for i in comp:
        want = oracle.decompress_contiguous(host[starts[i]:starts[i] + sizes[i]], PAGE_N,
                                            bounds[i])
        assert np.array_equal(got[i], want), i


def test_indexed_store_gives_way_to_the_gathered_path(cpp, oracle, pages):
    """Mixed-bound store with one constant page: the grouped indexed call
    returns expanding sizes for that page's two segments, so the connector
    drops the indexed result and runs the gathered path, whose per-length
    calls write the same streams; that page's segments go raw, the others
    compressed, and the restore puts every layer back."""
    src = pages.clone()
    src[2] = CONSTANT
    batch = src.shape[0]
    groups = sorted({1e-5: SENSITIVE, 1e-4: OTHERS}.items())   # :1312-1317
    w = wrapper(cpp)
    idx = [torch.tensor(ls, dtype=torch.long, device=DEV) for _, ls in groups]
    inputs, caps, eps, meta = [], [], [], []
    for g, (bound, layers) in enumerate(groups):
        n = 2 * len(layers) * EPL
        for p in range(batch):
            inputs.append(src[p])
            caps.append(8 * n)
            eps.append(bound)
            meta.append((p, g, n))
    bufs = slab_slices(caps)
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed_groups(
        inputs, bufs, idx, [batch] * len(groups), 2, LAYERS, EPL, eps)
    assert ok
    bits = u16(src)
    indexed_streams = []
    for k, (p, g, n) in enumerate(meta):
        layers = list(groups[g][1])
        eb = oracle.relative_bound(bits[p], n, eps[k], layers, LAYERS, EPL)
        assert np.float32(bounds[k]) == np.float32(eb)
        want = oracle.compress_page(bits[p], n, float(eb), layers, LAYERS, EPL)
        assert sizes[k] == want.size
        assert np.array_equal(bufs[k][:sizes[k]].cpu().numpy(), want)
        indexed_streams.append(want)
    expanding = [k for k, (_, _, n) in enumerate(meta) if sizes[k] >= 2 * n]
    assert [meta[k][0] for k in expanding] == [2, 2]   # :1529-1534: the job falls back

    # gathered path (:1030-1284): every (page, group) segment gathered, then
    # one compress_batch_fixed_bf16 call per segment length (:1211-1221)
    gathered = {}
    for p in range(batch):
        view = src[p].view(2, LAYERS, EPL)
        for g in range(len(groups)):
            gathered[(p, g)] = view.index_select(1, idx[g]).contiguous().view(-1)
    stored = {}
    for g, (bound, layers) in enumerate(groups):
        n = 2 * len(layers) * EPL
        keys = [(p, g) for p in range(batch)]
        gbufs = slab_slices([8 * n] * batch)
        ok, gsizes, gbounds = w.compress_batch_fixed_bf16(
            [gathered[key] for key in keys], gbufs, [bound] * batch)
        assert ok
        for key, buf, size, eb in zip(keys, gbufs, gsizes, gbounds):
            k = meta.index((key[0], key[1], n))
            assert size == sizes[k] and np.float32(eb) == np.float32(bounds[k])
            assert np.array_equal(buf[:size].cpu().numpy(), indexed_streams[k])
            kind = stored_as(size, 2 * n)
            assert kind == ("raw" if key[0] == 2 else "cuszp")
            stored[key] = (kind, buf[:size] if kind == "cuszp"
                           else gathered[key].view(torch.uint8), float(eb) if kind == "cuszp"
                           else 0.0)

    dest = torch.zeros_like(src)
    for g, (_, layers) in enumerate(groups):
        comp = [p for p in range(batch) if stored[(p, g)][0] == "cuszp"]
        # :1897-1908 with :1713-1760: one indexed scatter per layer group
        assert w.decompress_batch_fixed_bf16_indexed_scatter(
            [stored[(p, g)][1] for p in comp],
            [int(stored[(p, g)][1].numel()) for p in comp],
            [dest[p] for p in comp], idx[g], 2, LAYERS, EPL,
            [stored[(p, g)][2] for p in comp])
        for p in range(batch):              # raw layer groups: :2057-2079
            if stored[(p, g)][0] == "raw":
                restored = stored[(p, g)][1].view(torch.bfloat16).view(2, len(layers), EPL)
                dest[p].view(2, LAYERS, EPL).index_copy_(1, idx[g], restored)
    assert w.synchronize()
    got = u16(dest)
    assert np.array_equal(got[2], bits[2])
    for p in (0, 1, 3):
        want = np.zeros(PAGE_N, dtype=np.uint16)
        for g, (_, layers) in enumerate(groups):
            n = 2 * len(layers) * EPL
            k = meta.index((p, g, n))
            oracle.decompress_indexed(indexed_streams[k], n, bounds[k], want, list(layers),
                                      LAYERS, EPL)
        assert np.array_equal(got[p], want), p


@pytest.mark.parametrize("mode", ["MODE_FIXED", "MODE_PLAIN"])
def test_one_page_job_takes_the_per_segment_path(cpp, oracle, pages, mode):
    """A job of one page: the page widened to fp32 and compressed with the
    selected mode's single-page compress ("plain" is the connector's default
    mode, :498; the benchmarks select "fixed"), stored compressed when
    smaller; restored by the fp32 decode and converted to BF16.  A constant
    page expands in both modes (the plain code's first residual of every
    block is the saturated value itself) and is stored raw."""
    m = {"MODE_FIXED": 0, "MODE_PLAIN": 1}[mode]
    w = wrapper(cpp, mode)
    for page, expect in ((pages[0], "cuszp"), (torch.full_like(pages[0], CONSTANT), "raw")):
        x = page.to(torch.float32).contiguous()     # :617 (no MIN padding above 36 864)
        buf = torch.empty(w.estimate_compressed_buffer_size(4 * PAGE_N), dtype=torch.uint8,
                          device=DEV)
        ok, buf, size, bound = w.compress(x, buf, 1e-4)
        assert ok
        xs = x.cpu().numpy()
        eb = oracle.relative_bound_f32(xs, 1e-4)
        assert np.float32(bound) == np.float32(eb)
        want = oracle.compress_page_f32_mode(xs, eb, m)
        assert size == want.size and np.array_equal(buf[:size].cpu().numpy(), want)
        kind = stored_as(size, 2 * PAGE_N)
        assert kind == expect
        if kind == "raw":
            continue
        restored = torch.empty(PAGE_N, dtype=torch.float32, device=DEV)   # :2142-2150
        assert w.decompress(buf[:size].clone(), size, restored, bound)
        dest = torch.zeros_like(page)
        dest.copy_(restored.to(torch.bfloat16))                            # :2175-2178
        assert w.synchronize()
        want_f32 = oracle.decompress_f32_mode(want, PAGE_N, float(bound), m)
        assert np.array_equal(restored.cpu().numpy(), want_f32)
        # every mode decodes to the fixed mode's values, and their BF16
        # rounding is the batched BF16 decoder's output
        fixed_stream = oracle.compress_page_f32(xs, eb)
        assert np.array_equal(u16(dest), oracle.decompress_contiguous(
            fixed_stream, PAGE_N, float(bound)))
