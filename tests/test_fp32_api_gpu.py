"""GPU parity of the single-page fp32 API (fixed mode) against the oracle.

The reference serves ``compress``, ``compress_batch_fixed``, ``decompress``
and ``decompress_batch`` (cuszp_wrapper.cpp:216-1033) with upstream cuSZp's
fp32 kernels, whose stream layout the batched BF16 codec shares
(cuszp_batched_fixed.cu:52-54).  The connector calls them for every segment
its batched paths decline (vllm_v1_compressed_offload.py:566-758, MIN-padded
to 36 864 values, and :2021-2182 for the restore); the reference's own tests
decode a batched BF16 stream with the fp32 ``decompress``
(tests/test_vllm_v1_compressed_offload.py:47-110).  Parity with upstream's
own kernels is unpinned (not vendored); parity here is byte-exact streams and
bit-exact values against the CPU oracle's fp32 path, whose fp32-vs-BF16
invariants are pinned on the CPU (tests/test_oracle.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
MIN_CUSZP_ELEMENTS = 36864  # vllm_v1_compressed_offload.py:49


@pytest.fixture(scope="module")
def cpp():
    import cuszp_wrapper_cpp

    return cuszp_wrapper_cpp


def make(cpp, eb=1e-4, relative=True, mode=None):
    mode = cpp.MODE_FIXED if mode is None else mode
    cfg = cpp.CompressionConfig(eb, relative, cpp.DIM_1D, mode, cpp.TYPE_FLOAT)
    return cpp.CuSZpWrapper(cfg, 0)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().astype(np.float32, copy=False)


def same_values(got: np.ndarray, want: np.ndarray) -> bool:
    """Bit-equal fp32 arrays, any NaN matching any NaN (0 * inf gives the
    default NaN, whose sign differs between x86 and the GPU)."""
    eq = got.view(np.uint32) == want.view(np.uint32)
    return bool(np.all(eq | (np.isnan(got) & np.isnan(want))))


def same_bound(got: float, want: float) -> bool:
    got, want = np.float32(got), np.float32(want)
    return (np.isnan(got) and np.isnan(want)) or got == want


def check_stream(oracle, x: np.ndarray, eps: float, relative: bool, buf,
                 size: int, bound: float):
    eb = oracle.relative_bound_f32(x, eps) if relative else np.float32(eps)
    assert same_bound(bound, eb), (bound, eb)
    want = oracle.compress_page_f32(x, float(eb))
    assert size == want.size, (size, want.size)
    got = buf[:size].cpu().numpy()
    if not np.array_equal(got, want):
        bad = np.nonzero(got != want)[0]
        pytest.fail(f"{bad.size} bytes differ, first at {bad[0]}")
    return want, eb


@pytest.mark.parametrize("n", [1, 100, 8192, 36864, 65536, 229377])
@pytest.mark.parametrize("relative", [True, False])
def test_compress_single_matches_oracle(cpp, oracle, n, relative):
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(n, generator=g) * 2.5).to(DEV)   # not BF16 values
    w = make(cpp, relative=relative)
    cap = w.estimate_compressed_buffer_size(4 * n)
    buf = torch.empty(max(cap, 1024 + 128), dtype=torch.uint8, device=DEV)
    eps = 1e-4 if relative else 3e-3
    ok, buf2, size, bound = w.compress(x, buf, eps)
    assert ok
    stream, eb = check_stream(oracle, f32(x), eps, relative, buf2, size, bound)
    out = torch.full((n,), 9.0, device=DEV)
    assert w.decompress(buf2, size, out, bound)
    assert w.synchronize()
    want = oracle.decompress_f32(stream, n, float(eb))
    assert np.array_equal(f32(out).view(np.uint32), want.view(np.uint32))


def test_compress_replaces_a_small_buffer(cpp, oracle):
    """cuszp_wrapper.cpp:229-237: a buffer below estimate(nbytes) is replaced
    by a new one of that size, returned in the tuple."""
    n = 5000
    x = torch.randn(n, device=DEV)
    w = make(cpp)
    small = torch.empty(16, dtype=torch.uint8, device=DEV)
    ok, buf, size, bound = w.compress(x, small)
    assert ok and buf.numel() == 8 * n and buf.data_ptr() != small.data_ptr()
    check_stream(oracle, f32(x), 1e-4, True, buf, size, bound)


def test_min_padded_bf16_segment(cpp, oracle):
    """The connector's per-segment path: a BF16 segment below 36 864 values
    widened to fp32 and zero-padded (vllm_v1_compressed_offload.py:616-622,
    693-731).  The stream equals the BF16 encoder's on the same padded page."""
    g = torch.Generator().manual_seed(7)
    seg = (torch.randn(2 * 16 * 2 * 128, generator=g) * 0.7).to(torch.bfloat16)
    src = torch.nn.functional.pad(seg.float(), (0, MIN_CUSZP_ELEMENTS - seg.numel()))
    x = src.to(DEV).contiguous()
    w = make(cpp)
    buf = torch.empty(w.estimate_compressed_buffer_size(4 * x.numel()),
                      dtype=torch.uint8, device=DEV)
    ok, buf, size, bound = w.compress(x, buf, 1e-4)
    assert ok
    stream, eb = check_stream(oracle, f32(x), 1e-4, True, buf, size, bound)
    bits = torch.nn.functional.pad(seg, (0, MIN_CUSZP_ELEMENTS - seg.numel()))
    bits = bits.view(torch.int16).numpy().view(np.uint16)
    assert np.float32(oracle.relative_bound(bits, bits.size, 1e-4)) == np.float32(bound)
    assert np.array_equal(stream, oracle.compress_page(bits, bits.size, float(eb)))
    # ... and the BF16 batched encoder writes it too, on the device
    bbuf = torch.empty_like(buf)
    okb, sizes, bounds = w.compress_batch_fixed_bf16(
        [torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(DEV)], [bbuf], [1e-4])
    assert okb and sizes[0] == size and np.float32(bounds[0]) == np.float32(bound)
    assert np.array_equal(bbuf[:size].cpu().numpy(), stream)
    # the restore: fp32 decode, then the connector's .to(bfloat16)
    out = torch.empty(MIN_CUSZP_ELEMENTS, device=DEV)
    assert w.decompress(buf, size, out, bound)
    restored = out[: seg.numel()].to(torch.bfloat16).view(torch.int16).cpu().numpy()
    want = oracle.decompress_contiguous(stream, MIN_CUSZP_ELEMENTS, float(eb))
    assert np.array_equal(restored.view(np.uint16), want[: seg.numel()])


def test_compress_batch_fixed_round_trip(cpp, oracle):
    """tests/test_vllm_v1_compressed_offload.py:8-45, with byte parity."""
    w = make(cpp, eb=1e-5)
    g = torch.Generator().manual_seed(1)
    inputs = [torch.randn(65536, generator=g).to(DEV),
              (torch.randn(65536, generator=g) * 3.0).to(DEV)]
    cap = w.estimate_compressed_buffer_size(inputs[0].numel() * 4)
    outputs = [torch.empty(cap, dtype=torch.uint8, device=DEV) for _ in inputs]
    ok, sizes, bounds = w.compress_batch_fixed(inputs, outputs, [1e-5, 1e-5])
    assert ok and len(sizes) == 2 and len(bounds) == 2
    for x, buf, size, bound in zip(inputs, outputs, sizes, bounds):
        stream, eb = check_stream(oracle, f32(x), 1e-5, True, buf, size, bound)
        restored = torch.empty_like(x)
        assert w.decompress(buf, size, restored, bound)
        assert float((restored - x).abs().max()) <= float(bound) * 1.01 + 1e-7
        assert np.array_equal(f32(restored), oracle.decompress_f32(stream, x.numel(), eb))


def test_bf16_indexed_stream_decoded_by_f32_decompress(cpp, oracle):
    """tests/test_vllm_v1_compressed_offload.py:47-110: a stream of the
    batched BF16 indexed encoder decoded by the fp32 single-page decoder."""
    w = make(cpp, eb=1e-5)
    prefix, src, epl = 2, 8, 4096
    idx = torch.tensor([1, 3, 6], dtype=torch.long, device=DEV)
    g = torch.Generator().manual_seed(2)
    inputs = [torch.randn(prefix * src * epl, generator=g).to(torch.bfloat16).to(DEV)
              for _ in range(2)]
    n = prefix * idx.numel() * epl
    cap = w.estimate_compressed_buffer_size(n * 4)
    outputs = [torch.empty(cap, dtype=torch.uint8, device=DEV) for _ in inputs]
    ok, sizes, bounds = w.compress_batch_fixed_bf16_indexed(
        inputs, outputs, idx, prefix, src, epl, [1e-5] * 2)
    assert ok
    for source, buf, size, bound in zip(inputs, outputs, sizes, bounds):
        expected = source.view(prefix, src, epl).index_select(1, idx).contiguous().view(-1)
        restored = torch.empty(n, dtype=torch.float32, device=DEV)
        assert w.decompress(buf, size, restored, bound)
        assert float((restored - expected.float()).abs().max()) <= float(bound) * 1.01 + 1e-7
        stream = buf[:size].cpu().numpy()
        assert np.array_equal(f32(restored), oracle.decompress_f32(stream, n, float(bound)))
        # rounded to BF16 it is what the BF16 decoders write
        rb = restored.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(rb, oracle.decompress_contiguous(stream, n, float(bound)))


def test_decompress_batch_mixed_lengths(cpp, oracle):
    """cuszp_wrapper.cpp:944-1033: each output keeps its own length."""
    w = make(cpp)
    lengths = [36864, 36864, 1000, 229376, 36864, 33]
    g = torch.Generator().manual_seed(3)
    xs = [(torch.randn(n, generator=g) * (i + 1)).to(DEV) for i, n in enumerate(lengths)]
    bufs, sizes, bounds, streams = [], [], [], []
    for x in xs:
        buf = torch.empty(max(8 * x.numel(), 2048), dtype=torch.uint8, device=DEV)
        ok, buf, size, bound = w.compress(x, buf, 2e-4)
        assert ok
        streams.append(check_stream(oracle, f32(x), 2e-4, True, buf, size, bound))
        bufs.append(buf)
        sizes.append(size)
        bounds.append(bound)
    outs = [torch.full((x.numel(),), -3.0, device=DEV) for x in xs]
    assert w.decompress_batch(bufs, sizes, outs, bounds)
    assert w.synchronize()
    for out, (stream, eb), x in zip(outs, streams, xs):
        assert np.array_equal(f32(out), oracle.decompress_f32(stream, x.numel(), float(eb)))
    assert w.decompress_batch([], [], [], [])


def test_special_values_f32(cpp, oracle):
    """NaN makes the aminmax bound NaN (cuszp_wrapper.cpp:253); infinities
    make it infinite; the streams follow the quantizer on those bounds."""
    n = 20000
    rng = np.random.default_rng(5)
    rows = []
    base = (rng.standard_normal(n) * 3).astype(np.float32)
    r = base.copy(); r[77] = np.nan; rows.append(r)
    r = base.copy(); r[5] = np.inf; r[6] = -np.inf; rows.append(r)
    rows.append(np.full(n, np.inf, dtype=np.float32))
    rows.append(np.zeros(n, dtype=np.float32))
    rows.append(np.full(n, 1.0e30, dtype=np.float32))
    r = base.copy(); r[::3] = 3.0e38; rows.append(r)
    w = make(cpp)
    for row in rows:
        x = torch.from_numpy(row).to(DEV)
        buf = torch.empty(8 * n, dtype=torch.uint8, device=DEV)
        ok, buf, size, bound = w.compress(x, buf, 1e-4)
        assert ok
        stream, eb = check_stream(oracle, row, 1e-4, True, buf, size, bound)
        out = torch.zeros(n, device=DEV)
        assert w.decompress(buf, size, out, bound)
        assert w.synchronize()
        want = oracle.decompress_f32(stream, n, float(eb))
        assert same_values(f32(out), want)


def test_fp32_api_rejects_what_it_cannot_serve(cpp):
    n = 4096
    x = torch.randn(n, device=DEV)
    buf = torch.empty(8 * n, dtype=torch.uint8, device=DEV)
    plain = make(cpp, mode=cpp.MODE_PLAIN)
    assert plain.compress_batch_fixed([x], [buf], [])[0] is False   # fixed only (cpp:339-342)
    cfg = cpp.CompressionConfig(1e-4, True, cpp.DIM_2D, cpp.MODE_PLAIN, cpp.TYPE_FLOAT)
    two_d = cpp.CuSZpWrapper(cfg, 0)
    assert two_d.compress(x, buf)[0] is False                        # 1D only
    w = make(cpp)
    assert w.compress(x.to(torch.bfloat16), buf)[0] is False   # not fp32
    assert w.compress(x.cpu(), buf)[0] is False
    assert w.compress_batch_fixed([x, x[:100]], [buf, buf], [])[0] is False
    assert w.compress_batch_fixed([x], [buf[:100]], [])[0] is False
    assert w.decompress_batch([buf], [0], [x], [1e-4]) is False
    assert w.decompress_batch([buf], [2000], [x, x], [1e-4]) is False
