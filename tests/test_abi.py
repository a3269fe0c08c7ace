"""The C ABI (include/kvszp.h) as seen without a GPU: the built library
loads, exports every declared entry point, and the ctypes table in kvszp.py
covers exactly the declared set.  Pure functions are called; nothing that
touches a device is."""

from __future__ import annotations

import os
import re

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "kvszp.h")


def declared_functions() -> set[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(kvszp_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    import kvszp

    if not os.path.exists(kvszp.LIB_PATH):
        pytest.fail("libkvszp.so is not built (run __graft_entry__.build())")
    return kvszp.load()


def test_header_declares_the_reference_surface():
    names = declared_functions()
    for required in ("kvszp_create", "kvszp_destroy",
                     "kvszp_compress_batch_fixed_bf16",
                     "kvszp_compress_batch_fixed_bf16_indexed",
                     "kvszp_compress_batch_fixed_bf16_indexed_groups",
                     "kvszp_decompress_batch_fixed_bf16",
                     "kvszp_decompress_batch_fixed_bf16_scatter",
                     "kvszp_decompress_batch_fixed_bf16_indexed_scatter",
                     "kvszp_estimate_compressed_buffer_size",
                     "kvszp_get_config", "kvszp_update_config",
                     "kvszp_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    import kvszp

    assert {name for name, _, _ in kvszp.EXPORTS} == declared_functions()


def test_pure_entry_points(lib):
    import kvszp

    # cuszp_wrapper.cpp:1319-1321: 2 x bytes
    assert kvszp.estimate_compressed_buffer_size(4 * 229376) == 8 * 229376
    # R = 1024 * ceil(n / 32768)
    for n, r in ((1, 1024), (32768, 1024), (32769, 2048), (229376, 7168),
                 (172032, 6144), (57344, 2048)):
        assert kvszp.header_bytes(n) == r
    assert kvszp.last_error() == ""
