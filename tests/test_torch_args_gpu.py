"""kvszp_torch_args on device tensors: the C++ marshalling helper and the
Python checks it replaces return the same pointers and byte sizes, or both
refuse, for every condition the drop-in module checks (device, dtype,
contiguity, exact or minimum element count)."""

from __future__ import annotations

import importlib
from array import array

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def shim():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    m = importlib.import_module("cuszp_wrapper_cpp")
    assert m._targs is not None, "kvszp_torch_args is not built"
    return m


def _both(shim, monkeypatch, *args, **kwargs):
    native = shim._describe(*args, **kwargs)
    with monkeypatch.context() as m:
        m.setattr(shim, "_targs", None)
        python = shim._describe(*args, **kwargs)
    return native, python


def test_pointers_and_sizes(shim, monkeypatch):
    dev = torch.device("cuda:0")
    ts = [torch.empty(100 + i, dtype=torch.bfloat16, device=dev) for i in range(5)]
    native, python = _both(shim, monkeypatch, ts, 0, torch.bfloat16, 100)
    assert native == python
    ptrs, sizes = array("Q"), array("Q")
    ptrs.frombytes(native[0])
    sizes.frombytes(native[1])
    assert list(ptrs) == [t.data_ptr() for t in ts]
    assert list(sizes) == [2 * t.numel() for t in ts]


@pytest.mark.parametrize("case", ["dtype", "short", "exact", "strided", "cpu",
                                  "any_dtype", "strided_allowed"])
def test_refusals_match(shim, monkeypatch, case):
    dev = torch.device("cuda:0")
    good = [torch.empty(64, dtype=torch.bfloat16, device=dev) for _ in range(3)]
    kwargs = {}
    dtype = torch.bfloat16
    min_numel = 64
    ts = list(good)
    if case == "dtype":
        ts[1] = torch.empty(64, dtype=torch.float16, device=dev)
    elif case == "short":
        ts[2] = torch.empty(63, dtype=torch.bfloat16, device=dev)
    elif case == "exact":
        ts[0] = torch.empty(65, dtype=torch.bfloat16, device=dev)
        kwargs["exact"] = True
    elif case == "strided":
        ts[1] = torch.empty(128, dtype=torch.bfloat16, device=dev)[::2]
    elif case == "cpu":
        ts[2] = torch.empty(64, dtype=torch.bfloat16)
    elif case == "any_dtype":
        ts[1] = torch.empty(64, dtype=torch.uint8, device=dev)
        dtype = None
    elif case == "strided_allowed":
        ts[1] = torch.empty(128, dtype=torch.bfloat16, device=dev)[::2]
        kwargs["contiguous"] = False
    native, python = _both(shim, monkeypatch, ts, 0, dtype, min_numel, **kwargs)
    assert native == python
    refused = case in ("dtype", "short", "exact", "strided", "cpu")
    assert (native is None) == refused
