"""The call shapes the reference connector issues, replayed through the
drop-in ``cuszp_wrapper_cpp`` and checked against the oracle.

The connector itself (integration/compression_pipeline/
vllm_v1_compressed_offload.py) stays the reference's own and needs vLLM, which
is absent; what the drop-in must satisfy is the set of calls it makes.  Each
entry of CALLS below writes one of them out: the method, batch, logical
length N, buffer capacity, layer sets and destination split, with the
connector line that issues it.  Pages are Qwen2.5-1.5B vLLM blocks
[2 (K/V), 28 layers, 16 tokens, 2 heads, 128] in BF16 (229 376 values),
either as one flat tensor per page or as 28 per-layer tensors of 8192 values
(the two layouts the connector's helpers accept, :874-886, :1713-1812).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
LAYERS, EPL = 28, 16 * 2 * 128          # elements per layer per K or V
PAGE_N = 2 * LAYERS * EPL               # 229 376
MIN_CUSZP_ELEMENTS = 36864              # :49
SENSITIVE = (0, 1, 2, 5, 19, 20, 21)    # data/qwen2.5-1.5b_mixed_21x1e-4_7x1e-5.json
OTHERS = tuple(l for l in range(LAYERS) if l not in SENSITIVE)

# name -> call shape (B = pages in the job)
CALLS = {
    # :540-553 -- one wrapper per mode, REL bound, 1D, TYPE_FLOAT
    "construct": dict(modes=("MODE_FIXED", "MODE_PLAIN", "MODE_OUTLIER")),
    # :855-963 -- uniform bound, flat pages, 8N slab slices
    "uniform_flat": dict(method="compress_batch_fixed_bf16", B=6, N=PAGE_N,
                         cap=8 * PAGE_N, eps=1e-4),
    # :909-913 -- a page below 36 864 values is zero-padded to it (one
    # per-layer tensor of 8192 values here), capacity 8 * 36 864
    "uniform_min_padded": dict(method="compress_batch_fixed_bf16", B=5,
                               unpadded=EPL * 2, N=MIN_CUSZP_ELEMENTS,
                               cap=8 * MIN_CUSZP_ELEMENTS, eps=1e-4),
    # :1405-1483 -- layers grouped by bound, one grouped call, request
    # capacity 8 * selected_numel
    "indexed_groups": dict(method="compress_batch_fixed_bf16_indexed_groups",
                           B=6, groups=((1e-5, SENSITIVE), (1e-4, OTHERS))),
    # :1499-1520 -- the per-group fallback, one indexed call per group
    "indexed_per_group": dict(method="compress_batch_fixed_bf16_indexed", B=6,
                              groups=((1e-5, SENSITIVE), (1e-4, OTHERS))),
    # :1899-1908 with :1713-1760 -- restore each group into the full flat
    # pages (prefix 2, 28 source layers)
    "indexed_scatter": dict(method="decompress_batch_fixed_bf16_indexed_scatter",
                            B=6, groups=((1e-5, SENSITIVE), (1e-4, OTHERS))),
    # :1930-1938 with :1762-1812 -- per-layer tensors: 28 destinations of
    # 8192 values per page; a flat page is one destination of 229 376
    "direct_scatter_per_layer": dict(method="decompress_batch_fixed_bf16_scatter",
                                     B=4, dpp=LAYERS, epd=2 * EPL),
    "direct_scatter_flat": dict(method="decompress_batch_fixed_bf16_scatter",
                                B=4, dpp=1, epd=PAGE_N),
    # :1948-1968 -- contiguous staging storage of B * N, then copied out
    "contiguous_staging": dict(method="decompress_batch_fixed_bf16", B=5,
                               N=PAGE_N),
    # :566-758 -- the per-segment path: BF16 widened to fp32, padded to
    # 36 864, single-page compress with the selected mode's wrapper (:726;
    # "plain" is the connector's default mode, :498); restored by decompress
    # (:2139-2144) or decompress_batch (:1970-1975), then .to(bfloat16)
    "fp32_segment": dict(method="compress", B=3, unpadded=EPL * 2,
                         N=MIN_CUSZP_ELEMENTS,
                         modes=("MODE_FIXED", "MODE_PLAIN", "MODE_OUTLIER")),
}


@pytest.fixture(scope="module")
def cpp():
    import cuszp_wrapper_cpp

    return cuszp_wrapper_cpp


@pytest.fixture(scope="module")
def pages():
    import kv_synth

    return kv_synth.paged_kv(kv_synth.QWEN25_1P5B_4K, seed=3, device=DEV,
                             tokens=96)  # 6 pages of 229 376


def fixed(cpp, eb=1e-4):
    cfg = cpp.CompressionConfig(eb, True, cpp.CuszpDim.DIM_1D,
                                cpp.CuszpMode.MODE_FIXED, cpp.CuszpType.TYPE_FLOAT)
    return cpp.CuSZpWrapper(cfg, 0)


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def slab_slices(total_caps):
    """One uint8 slab cut into consecutive request slices (:922-941)."""
    slab = torch.empty(sum(total_caps), dtype=torch.uint8, device=DEV)
    out, off = [], 0
    for c in total_caps:
        out.append(slab[off:off + c])
        off += c
    return out


def check(oracle, bits, n, eps, buf, size, bound, layers=None):
    src, epl = (LAYERS, EPL) if layers else (0, 0)
    eb = oracle.relative_bound(bits, n, eps, layers, src, epl)
    assert np.float32(bound) == np.float32(eb)
    want = oracle.compress_page(bits, n, float(eb), layers, src, epl)
    assert size == want.size
    assert np.array_equal(buf[:size].cpu().numpy(), want)
    return want, eb


def test_construct(cpp):
    call = CALLS["construct"]
    for mode in call["modes"]:
        cfg = cpp.CompressionConfig(
            error_bound=1e-4, use_relative_error=True,
            processing_dim=cpp.CuszpDim.DIM_1D,
            encoding_mode=getattr(cpp.CuszpMode, mode),
            data_type=cpp.CuszpType.TYPE_FLOAT)
        w = cpp.CuSZpWrapper(cfg, 0)
        got = w.get_config()
        assert got.encoding_mode == getattr(cpp, mode)
        assert got.use_relative_error and np.float32(got.error_bound) == np.float32(1e-4)


def test_uniform_flat(cpp, oracle, pages):
    c = CALLS["uniform_flat"]
    src = pages[:c["B"]]
    bufs = slab_slices([c["cap"]] * c["B"])
    w = fixed(cpp)
    ok, sizes, bounds = getattr(w, c["method"])(list(src), bufs, [c["eps"]] * c["B"])
    assert ok
    bits = u16(src)
    for i in range(c["B"]):
        check(oracle, bits[i], c["N"], c["eps"], bufs[i], sizes[i], bounds[i])


def test_uniform_min_padded(cpp, oracle, pages):
    c = CALLS["uniform_min_padded"]
    # one per-layer tensor of each page: layer 4 of K and V, 8192 values
    seg = pages[:c["B"]].view(c["B"], 2, LAYERS, EPL)[:, :, 4].reshape(c["B"], -1)
    padded = torch.nn.functional.pad(seg, (0, c["N"] - c["unpadded"])).contiguous()
    bufs = slab_slices([c["cap"]] * c["B"])
    w = fixed(cpp)
    ok, sizes, bounds = getattr(w, c["method"])(list(padded), bufs, [c["eps"]] * c["B"])
    assert ok
    bits = u16(padded)
    for i in range(c["B"]):
        check(oracle, bits[i], c["N"], c["eps"], bufs[i], sizes[i], bounds[i])


def _grouped(cpp, oracle, pages, per_group: bool):
    c = CALLS["indexed_per_group" if per_group else "indexed_groups"]
    src = pages[:c["B"]]
    w = fixed(cpp)
    inputs, caps, eps, idx, counts, meta = [], [], [], [], [], []
    for bound, layers in c["groups"]:
        n = 2 * len(layers) * EPL
        idx.append(torch.tensor(layers, dtype=torch.long, device=DEV))
        counts.append(c["B"])
        for p in range(c["B"]):
            inputs.append(src[p])
            caps.append(8 * n)
            eps.append(bound)
            meta.append((p, n, list(layers), bound))
    bufs = slab_slices(caps)
    if per_group:
        sizes, bounds, k = [], [], 0
        for it, cnt in zip(idx, counts):
            ok, s, b = getattr(w, c["method"])(
                inputs[k:k + cnt], bufs[k:k + cnt], it, 2, LAYERS, EPL, eps[k:k + cnt])
            assert ok
            sizes += s
            bounds += b
            k += cnt
    else:
        ok, sizes, bounds = getattr(w, c["method"])(inputs, bufs, idx, counts, 2,
                                                    LAYERS, EPL, eps)
        assert ok
    bits = u16(src)
    for k, (p, n, layers, bound) in enumerate(meta):
        check(oracle, bits[p], n, bound, bufs[k], sizes[k], bounds[k], layers)
    return w, bufs, sizes, bounds, idx, counts, meta


def test_indexed_groups(cpp, oracle, pages):
    _grouped(cpp, oracle, pages, per_group=False)


def test_indexed_per_group(cpp, oracle, pages):
    _grouped(cpp, oracle, pages, per_group=True)


def test_indexed_scatter(cpp, oracle, pages):
    c = CALLS["indexed_scatter"]
    w, bufs, sizes, bounds, idx, counts, meta = _grouped(cpp, oracle, pages, False)
    dest = torch.zeros(c["B"], PAGE_N, dtype=torch.bfloat16, device=DEV)
    k = 0
    for it, cnt in zip(idx, counts):
        assert getattr(w, c["method"])(bufs[k:k + cnt], sizes[k:k + cnt],
                                       list(dest), it, 2, LAYERS, EPL,
                                       bounds[k:k + cnt])
        k += cnt
    assert w.synchronize()
    want = np.zeros((c["B"], PAGE_N), dtype=np.uint16)
    for k, (p, n, layers, _) in enumerate(meta):
        oracle.decompress_indexed(bufs[k][:sizes[k]].cpu().numpy(), n, bounds[k],
                                  want[p], layers, LAYERS, EPL)
    assert np.array_equal(u16(dest), want)


def _uniform_streams(cpp, oracle, src, n):
    w = fixed(cpp)
    bufs = slab_slices([8 * n] * src.shape[0])
    ok, sizes, bounds = w.compress_batch_fixed_bf16(list(src), bufs,
                                                    [1e-4] * src.shape[0])
    assert ok
    bits = u16(src)
    streams = [check(oracle, bits[i], n, 1e-4, bufs[i], sizes[i], bounds[i])[0]
               for i in range(src.shape[0])]
    return w, bufs, sizes, bounds, streams


def test_direct_scatter_per_layer(cpp, oracle, pages):
    c = CALLS["direct_scatter_per_layer"]
    # per-layer KV tensors [layer][block] of 8192 values; a page's payload is
    # the 28 tensors' blocks concatenated (:874-886)
    src = pages[:c["B"]].view(c["B"], 2, LAYERS, EPL).permute(0, 2, 1, 3).reshape(c["B"], -1)
    w, bufs, sizes, bounds, streams = _uniform_streams(cpp, oracle, src.contiguous(), PAGE_N)
    kv = torch.zeros(LAYERS, 8, c["epd"], dtype=torch.bfloat16, device=DEV)
    blocks = [5, 1, 7, 2]
    outs = [kv[l, blocks[i]] for i in range(c["B"]) for l in range(c["dpp"])]
    assert getattr(w, c["method"])(bufs, sizes, outs, PAGE_N, c["dpp"], c["epd"], bounds)
    assert w.synchronize()
    got = u16(kv)
    for i in range(c["B"]):
        want = oracle.decompress_contiguous(streams[i], PAGE_N, bounds[i])
        assert np.array_equal(got[:, blocks[i]].reshape(-1), want)
    untouched = sorted(set(range(8)) - set(blocks))
    assert not got[:, untouched].any()


def test_direct_scatter_flat(cpp, oracle, pages):
    c = CALLS["direct_scatter_flat"]
    src = pages[:c["B"]]
    w, bufs, sizes, bounds, streams = _uniform_streams(cpp, oracle, src, PAGE_N)
    pool = torch.zeros(9, PAGE_N, dtype=torch.bfloat16, device=DEV)
    slots = [8, 0, 3, 6]
    assert getattr(w, c["method"])(bufs, sizes, [pool[s] for s in slots], PAGE_N,
                                   c["dpp"], c["epd"], bounds)
    assert w.synchronize()
    got = u16(pool)
    for i, s in enumerate(slots):
        assert np.array_equal(got[s], oracle.decompress_contiguous(streams[i], PAGE_N, bounds[i]))


def test_contiguous_staging(cpp, oracle, pages):
    c = CALLS["contiguous_staging"]
    src = pages[:c["B"]]
    w, bufs, sizes, bounds, streams = _uniform_streams(cpp, oracle, src, c["N"])
    storage = torch.empty(c["B"] * c["N"], dtype=torch.bfloat16, device=DEV)
    assert getattr(w, c["method"])(bufs, sizes, storage, c["N"], bounds)
    assert w.synchronize()
    got = u16(storage).reshape(c["B"], c["N"])
    for i in range(c["B"]):
        assert np.array_equal(got[i], oracle.decompress_contiguous(streams[i], c["N"], bounds[i]))


@pytest.mark.parametrize("mode", CALLS["fp32_segment"]["modes"])
def test_fp32_segment(cpp, oracle, pages, mode):
    c = CALLS["fp32_segment"]
    cfg = cpp.CompressionConfig(1e-4, True, cpp.CuszpDim.DIM_1D,
                                getattr(cpp.CuszpMode, mode), cpp.CuszpType.TYPE_FLOAT)
    w = cpp.CuSZpWrapper(cfg, 0)
    m = {"MODE_FIXED": 0, "MODE_PLAIN": 1, "MODE_OUTLIER": 2}[mode]
    seg = pages[:c["B"]].view(c["B"], 2, LAYERS, EPL)[:, :, 9].reshape(c["B"], -1)
    srcs = [torch.nn.functional.pad(s.to(torch.float32), (0, c["N"] - c["unpadded"])).contiguous()
            for s in seg]
    results = []
    for x in srcs:
        buf = torch.empty(w.estimate_compressed_buffer_size(4 * c["N"]),
                          dtype=torch.uint8, device=DEV)
        ok, buf, size, bound = getattr(w, c["method"])(x, buf, 1e-4)
        assert ok
        xs = x.cpu().numpy()
        eb = oracle.relative_bound_f32(xs, 1e-4)
        assert np.float32(bound) == np.float32(eb)
        stream = oracle.compress_page_f32_mode(xs, eb, m)
        assert size == stream.size and np.array_equal(buf[:size].cpu().numpy(), stream)
        results.append((buf, size, bound, stream, oracle.compress_page_f32(xs, eb)))
    # restore one by one (:2139-2144) and as a batch (:1970-1975)
    singles = [torch.empty(c["N"], device=DEV) for _ in srcs]
    for (buf, size, bound, _, _), out in zip(results, singles):
        assert w.decompress(buf, size, out, bound)
    batch = [torch.empty(c["N"], device=DEV) for _ in srcs]
    assert w.decompress_batch([r[0] for r in results], [r[1] for r in results], batch,
                              [r[2] for r in results])
    assert w.synchronize()
    for (_, _, bound, stream, fixed_stream), a, b in zip(results, singles, batch):
        want = oracle.decompress_f32_mode(stream, c["N"], float(bound), m)
        assert np.array_equal(a.cpu().numpy(), want) and np.array_equal(b.cpu().numpy(), want)
        # the connector's .to(bfloat16) of the unpadded part: every mode
        # decodes to the fixed mode's values, whose BF16 rounding is the BF16
        # decoder's output
        rb = a[:c["unpadded"]].to(torch.bfloat16)
        assert np.array_equal(u16(rb), oracle.decompress_contiguous(
            fixed_stream, c["N"], float(bound))[:c["unpadded"]])
