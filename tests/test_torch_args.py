"""The drop-in module's argument marshalling: kvszp_torch_args (C++) and the
Python checks it replaces give the same answer for every kind of tensor
list.  CPU half: the helper is built and loads, and it refuses what is not a
device tensor, as the Python path does.  The device half is in
test_torch_args_gpu.py."""

from __future__ import annotations

import importlib
import os

import pytest
import torch

from conftest import PKG


@pytest.fixture(scope="module")
def shim():
    return importlib.import_module("cuszp_wrapper_cpp")


def test_helper_is_built_and_loaded(shim):
    assert os.path.exists(os.path.join(PKG, "kvszp_torch_args.so")), \
        "kvszp_torch_args.so is not built (run __graft_entry__.build())"
    assert shim._targs is not None


def test_dtype_codes_are_distinct(shim):
    dtypes = [torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64,
              torch.float16, torch.float32, torch.float64, torch.bfloat16,
              torch.bool]
    codes = [shim._targs.dtype_code(d) for d in dtypes]
    assert len(set(codes)) == len(codes)
    assert all(c >= 0 for c in codes)


def _both(shim, monkeypatch, *args, **kwargs):
    native = shim._describe(*args, **kwargs)
    with monkeypatch.context() as m:
        m.setattr(shim, "_targs", None)
        python = shim._describe(*args, **kwargs)
    return native, python


@pytest.mark.parametrize("case", ["empty", "cpu", "not_a_tensor", "tuple"])
def test_native_and_python_agree_without_device(shim, monkeypatch, case):
    cpu = [torch.zeros(64, dtype=torch.bfloat16) for _ in range(3)]
    tensors = {"empty": [], "cpu": cpu, "not_a_tensor": [cpu[0], 7],
               "tuple": tuple(cpu)}[case]
    native, python = _both(shim, monkeypatch, tensors, 0, torch.bfloat16, 64)
    assert native == python
    if case == "empty":
        assert native == (b"", b"")
    else:
        assert native is None
