"""Python bindings for the CPU oracle -- TEST INFRASTRUCTURE ONLY.

The oracle (``kvszp_oracle.c``) is a scalar restatement of the reference's
batched cuSZp fixed-mode BF16 codec
(``integration/cuszp_wrapper/cuszp_batched_fixed.cu``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this module, and only as the checker or the timed CPU baseline.  The product
path (the HIP library behind ``cuszp_wrapper_cpp``) never imports it.

BF16 data travels as ``numpy.uint16`` bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkvszp_oracle.so")

QUANT_TWO_ROUNDINGS = 0
QUANT_FUSED = 1
RATE0_SKIP = 0
RATE0_ZERO = 1
MODE_FIXED = 0
MODE_PLAIN = 1
MODE_OUTLIER = 2
BLOCK = 32
REF_TILE = 32768

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u64 = ctypes.c_uint64
_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc, no fast-math)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.kvo_quantize.restype = ctypes.c_int32
        L.kvo_quantize.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_int]
        L.kvo_quantize_array.restype = None
        L.kvo_quantize_array.argtypes = [
            ctypes.c_void_p, _u64, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
        L.kvo_bit_count.restype = ctypes.c_int
        L.kvo_bit_count.argtypes = [ctypes.c_uint32]
        L.kvo_f32_to_bf16_rne.restype = ctypes.c_uint16
        L.kvo_f32_to_bf16_rne.argtypes = [ctypes.c_float]
        L.kvo_bf16_to_f32.restype = ctypes.c_float
        L.kvo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.kvo_source_index.restype = _u64
        L.kvo_source_index.argtypes = [_u64, ctypes.c_void_p, _u64, _u64, _u64]
        L.kvo_header_bytes.restype = _u64
        L.kvo_header_bytes.argtypes = [_u64]
        L.kvo_relative_bound.restype = ctypes.c_float
        L.kvo_relative_bound.argtypes = [
            ctypes.c_void_p, _u64, ctypes.c_void_p, _u64, _u64, _u64,
            ctypes.c_float]
        L.kvo_compress_page.restype = _u64
        L.kvo_compress_page.argtypes = [
            ctypes.c_void_p, _u64, ctypes.c_void_p, _u64, _u64, _u64,
            ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
        L.kvo_decompress_contiguous.restype = ctypes.c_int
        L.kvo_decompress_contiguous.argtypes = [
            ctypes.c_void_p, _u64, _u64, ctypes.c_float, ctypes.c_int,
            ctypes.c_void_p]
        L.kvo_decompress_scatter.restype = ctypes.c_int
        L.kvo_decompress_scatter.argtypes = [
            ctypes.c_void_p, _u64, _u64, ctypes.c_float, ctypes.c_int,
            ctypes.c_void_p, _u64, _u64]
        L.kvo_decompress_indexed.restype = ctypes.c_int
        L.kvo_decompress_indexed.argtypes = [
            ctypes.c_void_p, _u64, _u64, ctypes.c_float, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_void_p, _u64, _u64, _u64]
        L.kvo_compress_batch.restype = ctypes.c_int
        L.kvo_compress_batch.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, _u64, _u64, ctypes.c_void_p,
            _u64, _u64, _u64, ctypes.c_void_p, ctypes.c_float, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        L.kvo_decompress_batch_contiguous.restype = ctypes.c_int
        L.kvo_decompress_batch_contiguous.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, _u64, _u64, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        L.kvo_relative_bound_f32.restype = ctypes.c_float
        L.kvo_relative_bound_f32.argtypes = [ctypes.c_void_p, _u64, ctypes.c_float]
        L.kvo_compress_page_f32.restype = _u64
        L.kvo_compress_page_f32.argtypes = [
            ctypes.c_void_p, _u64, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
        L.kvo_decompress_f32.restype = ctypes.c_int
        L.kvo_decompress_f32.argtypes = [
            ctypes.c_void_p, _u64, _u64, ctypes.c_float, ctypes.c_int,
            ctypes.c_void_p]
        L.kvo_compress_page_f32_mode.restype = _u64
        L.kvo_compress_page_f32_mode.argtypes = [
            ctypes.c_void_p, _u64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p]
        L.kvo_decompress_f32_mode.restype = ctypes.c_int
        L.kvo_decompress_f32_mode.argtypes = [
            ctypes.c_void_p, _u64, _u64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p]
        L.kvo_decompress_batch_indexed.restype = ctypes.c_int
        L.kvo_decompress_batch_indexed.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, _u64, _u64, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, _u64,
            _u64, _u64]
        L.kvo_int8_encode.restype = ctypes.c_float
        L.kvo_int8_encode.argtypes = [ctypes.c_void_p, _u64, ctypes.c_void_p]
        L.kvo_int8_decode.restype = None
        L.kvo_int8_decode.argtypes = [
            ctypes.c_void_p, _u64, ctypes.c_float, ctypes.c_void_p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _as_u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype != np.uint16:
        raise TypeError("BF16 data must be passed as uint16 bit patterns")
    return a


def _layer_args(layer_indices):
    if layer_indices is None:
        return None, None
    idx = np.ascontiguousarray(np.asarray(layer_indices, dtype=np.int64))
    return idx, idx.ctypes.data


# ---- scalar helpers --------------------------------------------------------

def quantize(x, recip: float, variant: int = QUANT_TWO_ROUNDINGS) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    q = np.empty(x.shape, dtype=np.int32)
    lib().kvo_quantize_array(x.ctypes.data, x.size, float(recip), variant,
                             q.ctypes.data)
    return q


def bit_count(v: int) -> int:
    return lib().kvo_bit_count(v)


def f32_to_bf16(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib().kvo_f32_to_bf16_rne(float(v)) for v in x],
                    dtype=np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    return (h.astype(np.uint32) << 16).view(np.float32)


def header_bytes(n: int) -> int:
    return int(lib().kvo_header_bytes(n))


def source_index(i: int, layer_indices, selected_layers: int,
                 source_layers: int, elements_per_layer: int) -> int:
    idx, p = _layer_args(layer_indices)
    return int(lib().kvo_source_index(i, p, selected_layers, source_layers,
                                      elements_per_layer))


# ---- page codec --------------------------------------------------------------

def relative_bound(page, n: int, eps: float, layer_indices=None,
                   source_layers: int = 0, elements_per_layer: int = 0) -> float:
    page = _as_u16(page)
    idx, p = _layer_args(layer_indices)
    sel = 0 if idx is None else idx.size
    return float(lib().kvo_relative_bound(
        page.ctypes.data, n, p, sel, source_layers, elements_per_layer, eps))


def max_stream_bytes(n: int) -> int:
    """Largest stream of n values: the header plus 4 + 4*31 bytes for every
    block, partial ones included (a block of one value can have rate 31)."""
    return header_bytes(n) + 128 * ((n + BLOCK - 1) // BLOCK)


def compress_page(page, n: int, eb: float, layer_indices=None,
                  source_layers: int = 0, elements_per_layer: int = 0,
                  variant: int = QUANT_TWO_ROUNDINGS) -> np.ndarray:
    """Encode one page; returns the S stream bytes (header padding zeroed)."""
    page = _as_u16(page)
    idx, p = _layer_args(layer_indices)
    sel = 0 if idx is None else idx.size
    out = np.zeros(max_stream_bytes(n), dtype=np.uint8)
    size = lib().kvo_compress_page(page.ctypes.data, n, p, sel, source_layers,
                                   elements_per_layer, eb, variant,
                                   out.ctypes.data)
    return out[:size].copy()


def decompress_contiguous(stream, n: int, eb: float,
                          rate0_policy: int = RATE0_ZERO,
                          out: np.ndarray | None = None) -> np.ndarray:
    stream = np.ascontiguousarray(np.asarray(stream, dtype=np.uint8))
    if out is None:
        out = np.zeros(n, dtype=np.uint16)
    rc = lib().kvo_decompress_contiguous(stream.ctypes.data, stream.size, n,
                                         eb, rate0_policy, out.ctypes.data)
    if rc != 0:
        raise ValueError("malformed fixed-mode stream")
    return out


def decompress_scatter(stream, n: int, eb: float, destinations: list,
                       elements_per_destination: int,
                       rate0_policy: int = RATE0_ZERO) -> None:
    stream = np.ascontiguousarray(np.asarray(stream, dtype=np.uint8))
    ptrs = (ctypes.c_void_p * len(destinations))(
        *[d.ctypes.data for d in destinations])
    rc = lib().kvo_decompress_scatter(stream.ctypes.data, stream.size, n, eb,
                                      rate0_policy, ptrs, len(destinations),
                                      elements_per_destination)
    if rc != 0:
        raise ValueError("malformed fixed-mode stream")


def decompress_indexed(stream, n: int, eb: float, destination: np.ndarray,
                       layer_indices, source_layers: int,
                       elements_per_layer: int,
                       rate0_policy: int = RATE0_ZERO) -> None:
    stream = np.ascontiguousarray(np.asarray(stream, dtype=np.uint8))
    idx, p = _layer_args(layer_indices)
    rc = lib().kvo_decompress_indexed(stream.ctypes.data, stream.size, n, eb,
                                      rate0_policy, destination.ctypes.data,
                                      p, idx.size, source_layers,
                                      elements_per_layer)
    if rc != 0:
        raise ValueError("malformed fixed-mode stream")


def compress_batch(pages: np.ndarray, eps, default_eps: float = 1e-4,
                   relative: bool = True, variant: int = QUANT_TWO_ROUNDINGS,
                   threads: int = 1, layer_indices=None, source_layers: int = 0,
                   elements_per_layer: int = 0, n: int | None = None,
                   return_elapsed: bool = False):
    """Encode ``pages`` (shape [B, page_numel], uint16) like the reference's
    batched call.  Returns (list of stream arrays, sizes, bounds), plus the
    seconds spent in the C encoder when ``return_elapsed``."""
    pages = _as_u16(pages)
    batch = pages.shape[0]
    idx, p = _layer_args(layer_indices)
    sel = 0 if idx is None else idx.size
    if n is None:
        n = pages.shape[1] if idx is None else (
            pages.shape[1] // source_layers * sel)
    cap = max_stream_bytes(n)
    outs = np.zeros((batch, cap), dtype=np.uint8)
    page_ptrs = (ctypes.c_void_p * batch)(
        *[pages.ctypes.data + i * pages.strides[0] for i in range(batch)])
    out_ptrs = (ctypes.c_void_p * batch)(
        *[outs.ctypes.data + i * cap for i in range(batch)])
    eps_arr = None if eps is None else np.ascontiguousarray(
        np.asarray(eps, dtype=np.float32))
    sizes = np.zeros(batch, dtype=np.uint64)
    bounds = np.zeros(batch, dtype=np.float32)
    t0 = time.perf_counter()
    lib().kvo_compress_batch(page_ptrs, out_ptrs, batch, n, p, sel,
                             source_layers, elements_per_layer, _ptr(eps_arr),
                             default_eps, int(relative), variant, threads,
                             sizes.ctypes.data, bounds.ctypes.data)
    elapsed = time.perf_counter() - t0
    streams = [outs[i, :int(sizes[i])].copy() for i in range(batch)]
    if return_elapsed:
        return streams, sizes, bounds, elapsed
    return streams, sizes, bounds


# ---- fp32 single-page path (CuSZpWrapper::compress / decompress) -----------

def _as_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype != np.float32:
        raise TypeError("fp32 pages must be float32 arrays")
    return a


def relative_bound_f32(x, eps: float) -> float:
    """at::aminmax bound of cuszp_wrapper.cpp:249-257 (NaN propagates)."""
    x = _as_f32(x)
    return float(lib().kvo_relative_bound_f32(x.ctypes.data, x.size, eps))


def compress_page_f32(x, eb: float,
                      variant: int = QUANT_TWO_ROUNDINGS) -> np.ndarray:
    """Encode a contiguous fp32 page; returns the S stream bytes."""
    x = _as_f32(x)
    out = np.zeros(max_stream_bytes(x.size), dtype=np.uint8)
    size = lib().kvo_compress_page_f32(x.ctypes.data, x.size, eb, variant,
                                       out.ctypes.data)
    return out[:size].copy()


def decompress_f32(stream, n: int, eb: float,
                   rate0_policy: int = RATE0_ZERO,
                   out: np.ndarray | None = None) -> np.ndarray:
    """fp32 decode y = fl(fl(q*eb)*2) of n values."""
    stream = np.ascontiguousarray(np.asarray(stream, dtype=np.uint8))
    if out is None:
        out = np.zeros(n, dtype=np.float32)
    rc = lib().kvo_decompress_f32(stream.ctypes.data, stream.size, n, eb,
                                  rate0_policy, out.ctypes.data)
    if rc != 0:
        raise ValueError("malformed fixed-mode stream")
    return out


def max_stream_bytes_lorenzo(n: int) -> int:
    """Worst-case plain/outlier stream: R + 136 bytes per block (a 4-byte
    outlier, the sign word and 32 planes)."""
    return int(lib().kvo_header_bytes(n)) + 136 * ((n + 31) // 32)


def compress_page_f32_mode(x, eb: float, mode: int,
                           variant: int = QUANT_TWO_ROUNDINGS) -> np.ndarray:
    """Encode a contiguous fp32 page in MODE_FIXED, MODE_PLAIN or
    MODE_OUTLIER (this build's specification of the last two, stated in
    kvszp_oracle.c); returns the S stream bytes."""
    x = _as_f32(x)
    out = np.zeros(max(max_stream_bytes(x.size), max_stream_bytes_lorenzo(x.size)),
                   dtype=np.uint8)
    size = lib().kvo_compress_page_f32_mode(x.ctypes.data, x.size, eb, variant, mode,
                                            out.ctypes.data)
    return out[:size].copy()


def decompress_f32_mode(stream, n: int, eb: float, mode: int,
                        rate0_policy: int = RATE0_ZERO,
                        out: np.ndarray | None = None) -> np.ndarray:
    """fp32 decode of a stream of the given mode."""
    stream = np.ascontiguousarray(np.asarray(stream, dtype=np.uint8))
    if out is None:
        out = np.zeros(n, dtype=np.float32)
    rc = lib().kvo_decompress_f32_mode(stream.ctypes.data, stream.size, n, eb, mode,
                                       rate0_policy, out.ctypes.data)
    if rc != 0:
        raise ValueError("malformed stream")
    return out


def decompress_batch_indexed(streams, sizes, n: int, bounds, out: np.ndarray,
                             layer_indices, source_layers: int,
                             elements_per_layer: int, threads: int = 1,
                             rate0_policy: int = RATE0_ZERO) -> None:
    """Decode stream p into the full page out[p] (uint16, [B, page_numel])
    through the layer map, pages split across `threads` threads."""
    batch = len(streams)
    streams = [np.ascontiguousarray(s, dtype=np.uint8) for s in streams]
    sp = (ctypes.c_void_p * batch)(*[s.ctypes.data for s in streams])
    sz = np.ascontiguousarray(np.asarray(sizes, dtype=np.uint64))
    eb = np.ascontiguousarray(np.asarray(bounds, dtype=np.float32))
    dp = (ctypes.c_void_p * batch)(
        *[out.ctypes.data + i * out.strides[0] for i in range(batch)])
    idx, p = _layer_args(layer_indices)
    rc = lib().kvo_decompress_batch_indexed(sp, sz.ctypes.data, batch, n,
                                            eb.ctypes.data, rate0_policy, threads,
                                            dp, p, idx.size, source_layers,
                                            elements_per_layer)
    if rc != 0:
        raise ValueError("malformed fixed-mode stream")


def int8_encode(page) -> tuple[np.ndarray, float]:
    page = _as_u16(page)
    q = np.empty(page.size, dtype=np.int8)
    scale = lib().kvo_int8_encode(page.ctypes.data, page.size, q.ctypes.data)
    return q, float(scale)


def int8_decode(q: np.ndarray, scale: float) -> np.ndarray:
    out = np.empty(q.size, dtype=np.uint16)
    lib().kvo_int8_decode(q.ctypes.data, q.size, scale, out.ctypes.data)
    return out
