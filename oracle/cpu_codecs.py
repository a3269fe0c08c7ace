"""Host codec baselines -- TEST/BENCH INFRASTRUCTURE ONLY.

Times the reference's host-side KV codecs on BF16 page bytes, on one thread
and with the pages split across threads (the codecs run in C and release the
interpreter lock), for bench.py's reported CPU baselines:
  * zstd level 1 and LZ4 default, called through the system libraries like
    integration/compression_pipeline/native_lossless.py:90-154 does;
  * INT8 (vllm_v1_compressed_offload.py:711-724, 2090-2123), via the oracle's
    C restatement.
"""

from __future__ import annotations

import ctypes
import time

import numpy as np

import oracle

_zstd = None
_lz4 = None


def _libs():
    global _zstd, _lz4
    if _zstd is None:
        z = ctypes.CDLL("libzstd.so.1")
        z.ZSTD_compressBound.restype = ctypes.c_size_t
        z.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
        z.ZSTD_compress.restype = ctypes.c_size_t
        z.ZSTD_compress.argtypes = [ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        z.ZSTD_decompress.restype = ctypes.c_size_t
        z.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p, ctypes.c_size_t]
        z.ZSTD_isError.restype = ctypes.c_uint
        z.ZSTD_isError.argtypes = [ctypes.c_size_t]
        l = ctypes.CDLL("liblz4.so.1")
        l.LZ4_compressBound.restype = ctypes.c_int
        l.LZ4_compressBound.argtypes = [ctypes.c_int]
        l.LZ4_compress_default.restype = ctypes.c_int
        l.LZ4_compress_default.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_int]
        l.LZ4_decompress_safe.restype = ctypes.c_int
        l.LZ4_decompress_safe.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_int, ctypes.c_int]
        _zstd, _lz4 = z, l
    return _zstd, _lz4


def _time_lossless(pages: np.ndarray, codec: str, verify: bool = True) -> dict:
    z, l = _libs()
    n_bytes = pages.shape[1] * 2
    if codec == "zstd":
        cap = int(z.ZSTD_compressBound(n_bytes))
    else:
        cap = int(l.LZ4_compressBound(n_bytes))
    dst = np.empty(cap, dtype=np.uint8)
    back = np.empty(n_bytes, dtype=np.uint8)
    t_c = t_d = 0.0
    total = 0
    for page in pages:
        src = np.ascontiguousarray(page)
        t0 = time.perf_counter()
        if codec == "zstd":
            size = int(z.ZSTD_compress(dst.ctypes.data, cap, src.ctypes.data,
                                       n_bytes, 1))
            if z.ZSTD_isError(size):
                raise RuntimeError("zstd failure")
        else:
            size = int(l.LZ4_compress_default(src.ctypes.data, dst.ctypes.data,
                                              n_bytes, cap))
            if size <= 0:
                raise RuntimeError("lz4 failure")
        t1 = time.perf_counter()
        if codec == "zstd":
            got = int(z.ZSTD_decompress(back.ctypes.data, n_bytes,
                                        dst.ctypes.data, size))
        else:
            got = int(l.LZ4_decompress_safe(dst.ctypes.data, back.ctypes.data,
                                            size, n_bytes))
        t2 = time.perf_counter()
        if got != n_bytes or (verify and not np.array_equal(back.view(np.uint16), src)):
            raise RuntimeError(f"{codec} round trip failed")
        t_c += t1 - t0
        t_d += t2 - t1
        total += size
    raw = pages.size * 2
    return {"ratio": round(raw / total, 4),
            "compress_gbps": round(raw / t_c / 1e9, 4),
            "decompress_gbps": round(raw / t_d / 1e9, 4),
            "store_restore_gbps": round(raw / (t_c + t_d) / 1e9, 4)}


def _time_int8(pages: np.ndarray) -> dict:
    t_c = t_d = 0.0
    for page in pages:
        t0 = time.perf_counter()
        q, scale = oracle.int8_encode(page)
        t1 = time.perf_counter()
        oracle.int8_decode(q, scale)
        t2 = time.perf_counter()
        t_c += t1 - t0
        t_d += t2 - t1
    raw = pages.size * 2
    return {"ratio": round(raw / (pages.shape[0] * (pages.shape[1] + 4)), 4),
            "compress_gbps": round(raw / t_c / 1e9, 4),
            "decompress_gbps": round(raw / t_d / 1e9, 4),
            "store_restore_gbps": round(raw / (t_c + t_d) / 1e9, 4)}


def _parallel(pages: np.ndarray, fn, threads: int) -> dict:
    """fn over `threads` page shares at once; GB/s from the wall time of the
    slowest share, ratio over all pages."""
    from concurrent.futures import ThreadPoolExecutor

    shares = [pages[i::threads] for i in range(threads) if pages[i::threads].size]
    t0 = time.perf_counter()
    with ThreadPoolExecutor(len(shares)) as ex:
        parts = list(ex.map(fn, shares))
    wall = time.perf_counter() - t0
    raw = pages.size * 2
    stored = sum(s.size * 2 / p["ratio"] for s, p in zip(shares, parts))
    return {"ratio": round(raw / stored, 4),
            "store_restore_gbps": round(raw / wall / 1e9, 4)}


def time_all(pages: np.ndarray, threads: int = 1) -> dict:
    """pages: [B, n] uint16 BF16 bit patterns.  threads > 1: also the pages
    split across that many threads (store and restore per share)."""
    out = {"cores": 1, "pages": int(pages.shape[0]),
           "zstd1": _time_lossless(pages, "zstd"),
           "lz4": _time_lossless(pages, "lz4"),
           "int8": _time_int8(pages)}
    if threads > 1:
        out["all_cores"] = {
            "cores": threads,
            "zstd1": _parallel(pages, lambda s: _time_lossless(s, "zstd", False), threads),
            "lz4": _parallel(pages, lambda s: _time_lossless(s, "lz4", False), threads),
            "int8": _parallel(pages, _time_int8, threads)}
    return out
