"""Packed publication and restore against the oracle.

The reference's store concatenates a job's payloads on the device at
8-byte-aligned offsets and copies the result into one pinned host slab
(CompressedPageStore.put_many_packed, vllm_v1_compressed_offload.py:371-447);
its restore copies the slab back in one piece and decodes from it
(:1618-1711).  Here kvszp_pack_streams writes the payloads straight into the
pinned slab with one gather kernel, and the packed restore copies the slab
to the device once and runs the grouped indexed scatter on it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import c1_compress, c1_requests, fixed_wrapper

pytestmark = pytest.mark.gpu

DEV = "cuda"


def expected_offsets(sizes):
    offs, end = [], 0
    for s in sizes:
        start = (end + 7) // 8 * 8
        offs.append(start)
        end = start + s
    return offs, end


def test_config1_packed_store_and_restore(c1, oracle):
    shape, pages = c1["shape"], c1["pages"]
    w = fixed_wrapper()
    req = c1_requests(c1)
    ok, sizes, bounds = c1_compress(w, c1, req)
    assert ok
    bufs = req[1]
    payloads = [b[:s] for b, s in zip(bufs, sizes)]
    total = sum(sizes) + 8 * len(sizes)
    slab = torch.full((total,), 0xCD, dtype=torch.uint8).pin_memory()
    ok, offsets, packed = w.pack_payloads(payloads, slab)
    assert ok
    want_offs, want_end = expected_offsets(sizes)
    assert offsets == want_offs and packed == want_end
    host = slab.numpy()
    cursor = 0
    for k, (stream, eb) in enumerate(c1["want"]):
        assert np.float32(bounds[k]) == np.float32(eb)
        o = offsets[k]
        assert not host[cursor:o].any(), f"gap before payload {k}"
        assert np.array_equal(host[o:o + sizes[k]], stream), f"payload {k}"
        cursor = o + sizes[k]
    assert (host[packed:] == 0xCD).all()  # nothing past the last payload
    # restore from the slab: one copy to the device and one grouped decode,
    # or the decoder reading the slab across the link itself
    staging = torch.empty(packed, dtype=torch.uint8, device=DEV)
    _, _, _, idx, counts = req
    dests = []
    for stage in (staging, None):
        dest = torch.zeros_like(pages)
        assert w.decompress_batch_fixed_bf16_indexed_scatter_groups_packed(
            slab, packed, stage, offsets, sizes,
            [dest[p] for p in range(pages.shape[0])] * len(counts), idx, counts, 2,
            shape.layers, shape.elements_per_layer, bounds)
        assert w.synchronize()
        dests.append(dest)
    want = np.zeros(tuple(pages.shape), dtype=np.uint16)
    k = 0
    for bound, layers in c1["groups"]:
        n = 2 * len(layers) * shape.elements_per_layer
        for p in range(pages.shape[0]):
            stream, eb = c1["want"][k]
            oracle.decompress_indexed(stream, n, float(eb), want[p], list(layers),
                                      shape.layers, shape.elements_per_layer)
            k += 1
    for dest in dests:
        assert np.array_equal(dest.view(torch.int16).cpu().numpy().view(np.uint16), want)


@pytest.mark.parametrize("where", ["pinned", "device"])
def test_pack_mixed_payloads(where):
    """Streams and raw BF16 pages (the raw fallback, :994-1005) of any
    length and alignment, packed like the reference's slab layout."""
    g = torch.Generator().manual_seed(5)
    base = torch.randint(0, 256, (1 << 20,), generator=g, dtype=torch.uint8).to(DEV)
    # payloads above 64 KiB are cut into pieces spread over the grid
    # (start, length): 8-, 4-, 2- and 1-byte aligned sources, odd lengths,
    # an empty payload and one that ends the slab unaligned
    spans = [(0, 4096), (4, 7), (2, 1002), (1, 33), (64, 0), (1000, 65537),
             (8, 8), (3, 5), (4096, 131072), (6, 3), (16, 0), (0, 0),
             (5, 300001), (24, 65536 * 3 + 8)]
    payloads = [base[s:s + n] for s, n in spans]
    sizes = [n for _, n in spans]
    offs, end = expected_offsets(sizes)
    cap = end + 64
    slab = (torch.full((cap,), 0xEE, dtype=torch.uint8).pin_memory() if where == "pinned"
            else torch.full((cap,), 0xEE, dtype=torch.uint8, device=DEV))
    w = fixed_wrapper()
    ok, offsets, packed = w.pack_payloads(payloads, slab)
    assert ok and offsets == offs and packed == end
    host = slab.cpu().numpy()
    src = base.cpu().numpy()
    cursor = 0
    for (s, n), o in zip(spans, offs):
        assert not host[cursor:o].any()
        assert np.array_equal(host[o:o + n], src[s:s + n])
        cursor = o + n
    assert (host[end:] == 0xEE).all()
    # a slab that is too small is refused before anything is written
    small = torch.zeros(end - 1, dtype=torch.uint8).pin_memory()
    assert w.pack_payloads(payloads, small)[0] is False
    assert not small.numpy().any()
