"""Host-side checks of compression_pipeline (the connector's codec-facing
logic, vllm_v1_compressed_offload.py:360-455, 825-1028, 1286-1569,
1578-2184) on CPU tensors.

The codec is replaced by a stand-in with the ``CuSZpWrapper`` method
signatures whose streams come from the CPU oracle, so these tests pin the
orchestration -- minimum-size padding, raw fallback, grouping by bound, slab
layout, the grouped call's argument order, the choice of restore path and
the packed host store -- independently of the GPU.  The same flows run on
the HIP codec in test_pipeline_gpu.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def as_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


class OracleCompressor:
    """CuSZpWrapper stand-in: relative bound, fixed-mode streams (oracle)."""

    def __init__(self, oracle, default_eps=1e-4):
        self.o = oracle
        self.default_eps = default_eps
        self.calls = []

    def _bound(self, page, n, eps, layers=None, src=0, epl=0):
        eps = eps if eps > 0 else self.default_eps
        return np.float32(self.o.relative_bound(page, n, eps, layers, src, epl))

    def _encode(self, inputs, outputs, eps, layers=None, src=0, epl=0, n=None):
        sizes, bounds = [], []
        for x, out, e in zip(inputs, outputs, eps):
            page = bits(x)
            nn = page.size if n is None else n
            eb = self._bound(page, nn, e, layers, src, epl)
            stream = self.o.compress_page(page, nn, float(eb), layers, src, epl)
            out[:stream.size] = torch.from_numpy(stream)
            sizes.append(int(stream.size))
            bounds.append(float(eb))
        return True, sizes, bounds

    def compress_batch_fixed_bf16(self, inputs, outputs, eps):
        self.calls.append(("batch", len(inputs)))
        return self._encode(inputs, outputs, eps)

    def compress_batch_fixed_bf16_indexed(self, inputs, outputs, layer_indices,
                                          prefix, src, epl, eps):
        layers = [int(v) for v in layer_indices]
        self.calls.append(("indexed", tuple(layers), len(inputs)))
        return self._encode(inputs, outputs, eps, layers, src, epl,
                            prefix * len(layers) * epl)

    def compress_batch_fixed_bf16_indexed_groups(self, inputs, outputs,
                                                 layer_indices, group_sizes,
                                                 prefix, src, epl, eps):
        self.calls.append(("groups", [tuple(int(v) for v in li) for li in layer_indices],
                           list(group_sizes)))
        sizes, bounds, at = [], [], 0
        for li, gs in zip(layer_indices, group_sizes):
            layers = [int(v) for v in li]
            _, s, b = self._encode(inputs[at:at + gs], outputs[at:at + gs],
                                   eps[at:at + gs], layers, src, epl,
                                   prefix * len(layers) * epl)
            sizes += s
            bounds += b
            at += gs
        return True, sizes, bounds

    def decompress_batch_fixed_bf16_indexed_scatter(self, bufs, sizes, outputs,
                                                    layer_indices, prefix, src,
                                                    epl, bounds):
        layers = [int(v) for v in layer_indices]
        self.calls.append(("indexed_scatter", tuple(layers), len(bufs)))
        n = prefix * len(layers) * epl
        for buf, size, out, eb in zip(bufs, sizes, outputs, bounds):
            dst = bits(out).copy()
            self.o.decompress_indexed(buf[:size].numpy(), n, eb, dst, layers, src, epl)
            out.copy_(as_bf16(dst))
        return True

    def decompress_batch_fixed_bf16_scatter(self, bufs, sizes, outputs, n, dpp,
                                            epd, bounds):
        self.calls.append(("scatter", len(bufs), dpp))
        for i, (buf, size, eb) in enumerate(zip(bufs, sizes, bounds)):
            dec = self.o.decompress_contiguous(buf[:size].numpy(), n, eb)
            for d in range(dpp):
                outputs[i * dpp + d].copy_(as_bf16(dec[d * epd:(d + 1) * epd]))
        return True

    def decompress_batch_fixed_bf16(self, bufs, sizes, output, n, bounds):
        self.calls.append(("contiguous", len(bufs)))
        for i, (buf, size, eb) in enumerate(zip(bufs, sizes, bounds)):
            output[i * n:(i + 1) * n].copy_(
                as_bf16(self.o.decompress_contiguous(buf[:size].numpy(), n, eb)))
        return True


@pytest.fixture(scope="module")
def pipeline():
    import compression_pipeline

    return compression_pipeline


def kv_pages(pages, layers, epl, seed, scale=1.0):
    """Gaussian pages with a few large outliers per layer, like K caches:
    the range is set by the outliers, so most values need few bits."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(pages, 2 * layers, epl, generator=g) * scale
    x[:, :, :4] = 40.0 * scale
    x[:, :, 4:8] = -40.0 * scale
    return x.reshape(pages, -1).to(torch.bfloat16)


def test_adaptive_indexed_groups_round_trip(pipeline, oracle):
    layers, epl = 6, 4096          # 2 * 5 * 4096 = 40960 >= 36864 per segment
    kv = kv_pages(4, layers, epl, seed=1, scale=3.0)
    bounds = {i: (1e-5 if i == 2 else 1e-4) for i in range(layers)}
    comp = OracleCompressor(oracle)
    codec = pipeline.KVPageCodec([kv], error_bound=1e-4,
                                 compressors={"fixed": comp}, flat_layer_prefix=2)
    ops = [((0,), b, 100 + b) for b in range(4)]
    # the 1-layer group has 2*1*4096 < 36864 elements: the reference gives up
    assert codec.compress_adaptive_fixed_bundles_indexed(ops, bounds) is None

    bounds = {i: (1e-5 if i in (0, 1, 3, 4, 5) else 0.0) for i in range(layers)}
    entries = codec.compress_adaptive_fixed_bundles_indexed(ops, {**bounds, 2: 0.0})
    assert entries is not None and len(entries) == 4
    # groups sorted by bound: (0.0 -> raw layer 2), (1e-5 -> 5 layers)
    for cpu_id, bundle in entries:
        raw, cz = bundle.segments
        assert raw.encoding == "raw" and raw.components[0].layer_indices == (2,)
        assert cz.encoding == "cuszp" and cz.components[0].layer_indices == (0, 1, 3, 4, 5)
        assert cz.cuszp_mode == "fixed" and cz.compressed_size < cz.original_bytes
    # one native call for the one compressed group
    assert [c[0] for c in comp.calls] == ["indexed"]

    store = pipeline.CompressedPageStore()
    store.put_many_packed(entries)
    original = kv.clone()
    kv.zero_()
    codec.decompress_bundles_batched([(b, store.get(100 + b)) for b in range(4)])
    assert comp.calls[-1][0] == "indexed_scatter"
    view_o = original.view(4, 2, layers, epl)
    view_r = kv.view(4, 2, layers, epl)
    assert torch.equal(view_r[:, :, 2], view_o[:, :, 2])           # raw layer exact
    for b in range(4):
        seg = store.get(100 + b).segments[1]
        err = (view_r[b][:, [0, 1, 3, 4, 5]].float() - view_o[b][:, [0, 1, 3, 4, 5]].float()).abs()
        assert err.max().item() <= 2 * seg.actual_error_bound


def test_adaptive_two_bounds_use_one_grouped_call(pipeline, oracle):
    layers, epl = 10, 4096          # groups of 5 layers: 40960 values each
    kv = kv_pages(3, layers, epl, seed=2)
    bounds = {i: (1e-5 if i < 5 else 1e-4) for i in range(layers)}
    comp = OracleCompressor(oracle)
    codec = pipeline.KVPageCodec([kv], compressors={"fixed": comp})
    entries = codec.compress_adaptive_fixed_bundles_indexed(
        [((0,), b, b) for b in range(3)], bounds)
    assert entries is not None
    kind, groups, sizes = comp.calls[0]
    assert kind == "groups" and groups == [(0, 1, 2, 3, 4), (5, 6, 7, 8, 9)] and sizes == [3, 3]
    # every stream equals the oracle's for its segment, bound included
    for b, (_, bundle) in enumerate(entries):
        for seg, eps, lay in zip(bundle.segments, (1e-5, 1e-4),
                                 ((0, 1, 2, 3, 4), (5, 6, 7, 8, 9))):
            page = bits(kv[b])
            n = 2 * 5 * epl
            eb = np.float32(oracle.relative_bound(page, n, eps, list(lay), layers, epl))
            assert np.float32(seg.actual_error_bound) == eb
            want = oracle.compress_page(page, n, float(eb), list(lay), layers, epl)
            assert np.array_equal(seg.payload.numpy(), want)


def test_uniform_batch_pads_small_pages_and_falls_back_to_raw(pipeline, oracle):
    # two KV tensors of 1024 elements each per page: 2048 < 36864 -> MIN-pad
    k = kv_pages(3, 1, 512, seed=3)
    v = kv_pages(3, 1, 512, seed=4)
    comp = OracleCompressor(oracle)
    codec = pipeline.KVPageCodec([k, v], error_bound=1e-4, compressors={"fixed": comp})
    ops = [((0, 1), b, b) for b in range(3)]
    entries = codec.compress_fixed_bundles_batched(ops)
    assert entries is not None
    for _, bundle in entries:
        (seg,) = bundle.segments
        assert seg.compressed_numel == pipeline.MIN_CUSZP_ELEMENTS
        assert seg.unpadded_numel == 2048
        # a padded 2048-value page compresses to more than its 4096 raw bytes
        # (the 36864-value header alone is 2048 bytes) -> raw
        assert seg.encoding == "raw" and seg.compressed_size == seg.original_bytes == 4096
    store = pipeline.CompressedPageStore()
    store.put_many_packed(entries)
    k0, v0 = k.clone(), v.clone()
    k.zero_()
    v.zero_()
    codec.decompress_bundles_batched([(b, store.get(b)) for b in range(3)])
    assert torch.equal(k, k0) and torch.equal(v, v0)


def test_uniform_batch_compressed_pages_restore_by_direct_scatter(pipeline, oracle):
    kv = kv_pages(3, 28, 4096, seed=5, scale=2.0)          # 229376 per page
    comp = OracleCompressor(oracle)
    codec = pipeline.KVPageCodec([kv], error_bound=1e-4, compressors={"fixed": comp})
    entries = codec.compress_fixed_bundles_batched([((0,), b, b) for b in range(3)])
    assert all(e[1].segments[0].encoding == "cuszp" for e in entries)
    store = pipeline.CompressedPageStore()
    store.put_many_packed(entries)
    # payloads are packed 8-byte aligned in one host slab
    segs = [store.get(b).segments[0] for b in range(3)]
    base = segs[0].payload.untyped_storage().data_ptr()
    assert all(s.payload.untyped_storage().data_ptr() == base for s in segs)
    assert all(s.payload.storage_offset() % 8 == 0 for s in segs)
    orig = kv.clone()
    kv.zero_()
    codec.decompress_bundles_batched([(b, store.get(b)) for b in range(3)])
    assert comp.calls[-1][:1] == ("scatter",)
    for b, s in enumerate(segs):
        want = oracle.decompress_contiguous(s.payload.numpy(), kv.shape[1],
                                            s.actual_error_bound)
        assert np.array_equal(bits(kv[b]), want)
    assert (kv.float() - orig.float()).abs().max().item() <= 2 * max(
        s.actual_error_bound for s in segs)


def test_uniform_batch_declines_like_the_reference(pipeline, oracle):
    kv = kv_pages(2, 2, 4096, seed=6)
    comp = OracleCompressor(oracle)
    codec = pipeline.KVPageCodec([kv], compressors={"fixed": comp})
    ops = [((0,), b, b) for b in range(2)]
    assert codec.compress_fixed_bundles_batched(ops[:1]) is None          # one page
    assert codec.compress_fixed_bundles_batched(ops, {0: 1e-4, 1: 1e-5}) is None
    assert codec.compress_fixed_bundles_batched(ops, {1: 1e-4}) is None   # not 0..L-1
    assert codec.compress_fixed_bundles_batched(ops, active_mode="plain") is None
    assert codec.compress_fixed_bundles_batched(ops, {0: 0.0, 1: 0.0}) is None
    assert comp.calls == []
