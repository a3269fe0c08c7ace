"""Drop-in replacement for the reference's ``cuszp_wrapper_cpp`` module.

The reference builds this module with pybind11 from
``integration/cuszp_wrapper/pybind11_bindings.cpp``; its caller,
``integration/compression_pipeline/vllm_v1_compressed_offload.py``, does
``import cuszp_wrapper_cpp`` after putting the module's directory on
``sys.path`` (:41-45).  Put this directory on ``sys.path`` instead and the
connector runs on the MI355X HIP codec unchanged.

Kept exactly: enum names and values (:13-28), ``CompressionConfig`` fields and
defaults (:31-43), ``CuSZpWrapper(config, device_id=0)`` and the method
names, argument names and order, and return shapes of the batched BF16
fixed-mode path (:84-163, :190-256), ``estimate_compressed_buffer_size``
(:260-261), ``get_config``/``update_config`` (:262-263).  Validation follows
the reference's C++ checks (cuszp_wrapper.cpp:431-868, 1034-1313): a failed
check returns ``False`` (or a ``False`` tuple) instead of raising.  Every
call runs on ``torch.cuda.current_stream()`` (the reference captures
``c10::cuda::getCurrentCUDAStream()`` per call); compress calls block until
the sizes are on the host, decompress calls only enqueue.

The single-page fp32 entry points (``compress``, ``compress_batch_fixed``,
``decompress``, ``decompress_batch``) run the same kernels with fp32 loads and
stores in fixed mode (the reference uses upstream cuSZp's fp32 kernels, whose
stream layout the batched BF16 codec shares); the plain and outlier modes run
this library's residual codes (kvszp_compress_f32 in include/kvszp.h).

Lists of tensors are checked and turned into pointer arrays in one C++ pass
by ``kvszp_torch_args`` (csrc/kvszp_torch_args.cpp, built by build.py next to
this file), as the reference's pybind11 methods do in C++; without it the
same checks run in Python.
"""

from __future__ import annotations

import ctypes
import enum
import os
import sys
from array import array

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

import kvszp  # noqa: E402  (the C ABI; raises if libkvszp.so is missing)

kvszp.load()

try:  # argument marshalling in C++ (host code, no device code)
    import kvszp_torch_args as _targs  # noqa: E402
except ImportError:
    _targs = None

_DTYPE_CODES: dict = {}


def _describe(tensors, device: int, dtype, min_numel: int = 0, exact: bool = False,
              contiguous: bool = True):
    """(pointers, byte sizes) of `tensors` as packed uint64 bytes, or None
    when any is not a tensor on CUDA device `device` of `dtype` (any dtype
    for None), contiguous when `contiguous`, with numel == min_numel
    (`exact`) or >= min_numel."""
    if not isinstance(tensors, list):
        tensors = list(tensors)
    if _targs is not None:
        code = -1
        if dtype is not None:
            code = _DTYPE_CODES.get(dtype)
            if code is None:
                code = _DTYPE_CODES[dtype] = _targs.dtype_code(dtype)
        return _targs.describe(tensors, device, code, min_numel, exact, contiguous)
    ptrs, sizes = array("Q"), array("Q")
    for t in tensors:
        if (not isinstance(t, torch.Tensor) or not t.is_cuda or t.get_device() != device
                or (dtype is not None and t.dtype != dtype)
                or (contiguous and not t.is_contiguous())):
            return None
        numel = t.numel()
        if (numel != min_numel) if exact else (numel < min_numel):
            return None
        ptrs.append(t.data_ptr())
        sizes.append(numel * t.element_size())
    return ptrs.tobytes(), sizes.tobytes()


def _u64s(packed: bytes):
    """A C uint64 array from packed bytes (pointers or sizes)."""
    return (ctypes.c_uint64 * (len(packed) // 8)).from_buffer_copy(packed)


def _u64_values(values):
    """A C uint64 array of integers (sizes, offsets)."""
    a = array("Q", values)
    return (ctypes.c_uint64 * len(a)).from_buffer(a), a


def _f32_values(values):
    """A C float array, each value rounded to the nearest float as pybind11
    converts a Python float to C float."""
    a = array("f", values)
    return (ctypes.c_float * len(a)).from_buffer(a), a


def _as_list(c_array, fmt: str) -> list:
    """Python ints ('Q') or floats ('f') of a C array, through its buffer:
    iterating the ctypes array instead costs ~50 us per 1024 values."""
    return memoryview(c_array).cast("B").cast(fmt).tolist()


class CuszpDim(enum.IntEnum):
    DIM_1D = kvszp.DIM_1D
    DIM_2D = kvszp.DIM_2D
    DIM_3D = kvszp.DIM_3D


class CuszpMode(enum.IntEnum):
    MODE_FIXED = kvszp.MODE_FIXED
    MODE_PLAIN = kvszp.MODE_PLAIN
    MODE_OUTLIER = kvszp.MODE_OUTLIER


class CuszpType(enum.IntEnum):
    TYPE_FLOAT = kvszp.TYPE_FLOAT
    TYPE_DOUBLE = kvszp.TYPE_DOUBLE


# pybind11's export_values() also puts the enumerators in the module scope.
DIM_1D, DIM_2D, DIM_3D = CuszpDim.DIM_1D, CuszpDim.DIM_2D, CuszpDim.DIM_3D
MODE_FIXED, MODE_PLAIN, MODE_OUTLIER = (
    CuszpMode.MODE_FIXED, CuszpMode.MODE_PLAIN, CuszpMode.MODE_OUTLIER)
TYPE_FLOAT, TYPE_DOUBLE = CuszpType.TYPE_FLOAT, CuszpType.TYPE_DOUBLE


def _f32(value: float) -> float:
    """Rounds a Python float through C float, as pybind11 does."""
    return float(np.float32(value))


class CompressionConfig:
    """CuSZpWrapper::CompressionConfig (cuszp_wrapper.h:11-17)."""

    def __init__(self, error_bound: float = 1e-4,
                 use_relative_error: bool = True,
                 processing_dim: CuszpDim = CuszpDim.DIM_1D,
                 encoding_mode: CuszpMode = CuszpMode.MODE_PLAIN,
                 data_type: CuszpType = CuszpType.TYPE_FLOAT):
        self.error_bound = error_bound
        self.use_relative_error = use_relative_error
        self.processing_dim = processing_dim
        self.encoding_mode = encoding_mode
        self.data_type = data_type

    @property
    def error_bound(self) -> float:
        return self._error_bound

    @error_bound.setter
    def error_bound(self, value: float) -> None:
        self._error_bound = _f32(value)

    @property
    def use_relative_error(self) -> bool:
        return self._use_relative_error

    @use_relative_error.setter
    def use_relative_error(self, value: bool) -> None:
        self._use_relative_error = bool(value)

    @property
    def processing_dim(self) -> CuszpDim:
        return self._processing_dim

    @processing_dim.setter
    def processing_dim(self, value) -> None:
        self._processing_dim = CuszpDim(int(value))

    @property
    def encoding_mode(self) -> CuszpMode:
        return self._encoding_mode

    @encoding_mode.setter
    def encoding_mode(self, value) -> None:
        self._encoding_mode = CuszpMode(int(value))

    @property
    def data_type(self) -> CuszpType:
        return self._data_type

    @data_type.setter
    def data_type(self, value) -> None:
        self._data_type = CuszpType(int(value))

    def _to_c(self) -> kvszp.Config:
        return kvszp.Config(self.error_bound, int(self.use_relative_error),
                            int(self.processing_dim), int(self.encoding_mode),
                            int(self.data_type))

    def _copy(self) -> "CompressionConfig":
        return CompressionConfig(self.error_bound, self.use_relative_error,
                                 self.processing_dim, self.encoding_mode,
                                 self.data_type)

    def __repr__(self) -> str:
        return (f"CompressionConfig(error_bound={self.error_bound}, "
                f"use_relative_error={self.use_relative_error}, "
                f"processing_dim={self.processing_dim.name}, "
                f"encoding_mode={self.encoding_mode.name}, "
                f"data_type={self.data_type.name})")


def _stream_handle(device_id: int) -> int:
    return torch.cuda.current_stream(device_id).cuda_stream


def _report(where: str) -> None:
    # The reference prints its failures to stderr and returns false
    # (cuszp_wrapper.cpp:11-19, cuszp_batched_fixed.cu:654-659).
    msg = kvszp.last_error()
    if msg:
        print(f"Error: {where}: {msg}", file=sys.stderr)


class CuSZpWrapper:
    """CuSZpWrapper (cuszp_wrapper.h:9-158) on the MI355X HIP codec."""

    def __init__(self, config: CompressionConfig, device_id: int = 0):
        self._config = config._copy()
        self._device_id = int(device_id)
        self._ctx = kvszp.Context(self._config._to_c(), self._device_id)

    # ---- configuration -------------------------------------------------

    def get_config(self) -> CompressionConfig:
        return self._config._copy()

    def update_config(self, config: CompressionConfig) -> None:
        self._config = config._copy()
        self._ctx.update_config(self._config._to_c())

    def set_codec_options(self, quantizer: int = kvszp.QUANT_TWO_ROUNDINGS,
                          rate0_policy: int = kvszp.RATE0_ZERO) -> None:
        """Codec switches with no reference counterpart: the quantizer
        reading of the reference's PTX, and whether rate-0 blocks are written
        as +0.0 or left untouched (the reference leaves them untouched)."""
        self._ctx.set_options(quantizer, rate0_policy)

    @staticmethod
    def estimate_compressed_buffer_size(original_size: int) -> int:
        return int(original_size) * 2  # cuszp_wrapper.cpp:1319-1321

    # ---- helpers ---------------------------------------------------------

    def _on_device(self, t: torch.Tensor) -> bool:
        return t.is_cuda and t.get_device() == self._device_id

    @staticmethod
    def _eps_array(eps_overrides, batch: int):
        if not eps_overrides:
            return None
        return _f32_values(eps_overrides)[0]

    def _fixed_mode(self) -> bool:
        c = self._config
        return (c.processing_dim == CuszpDim.DIM_1D
                and c.data_type == CuszpType.TYPE_FLOAT
                and c.encoding_mode == CuszpMode.MODE_FIXED)

    def _f32_1d(self) -> bool:
        # the single-page fp32 methods take any encoding mode
        # (cuszp_wrapper.cpp:268-313, 886-939)
        c = self._config
        return (c.processing_dim == CuszpDim.DIM_1D
                and c.data_type == CuszpType.TYPE_FLOAT
                and c.encoding_mode in (CuszpMode.MODE_FIXED, CuszpMode.MODE_PLAIN,
                                        CuszpMode.MODE_OUTLIER))

    def _finish_compress(self, rc: int, batch: int, sizes, bounds, where: str):
        if rc != kvszp.OK:
            _report(where)
            return (False, [], [])
        return (True, _as_list(sizes, "Q"), _as_list(bounds, "f"))

    # ---- batched BF16 compress -----------------------------------------

    def compress_batch_fixed_bf16(self, input_tensors, compressed_buffers,
                                  eps_overrides):
        """pybind11_bindings.cpp:84-101 -> cuszp_wrapper.cpp:431-544."""
        batch = len(input_tensors)
        if (batch == 0 or len(compressed_buffers) != batch
                or (eps_overrides and len(eps_overrides) != batch)
                or not self._fixed_mode()):
            return (False, [], [])
        n = input_tensors[0].numel()
        ins = _describe(input_tensors, self._device_id, torch.bfloat16, n, exact=True)
        outs = None if ins is None else _describe(
            compressed_buffers, self._device_id, torch.uint8,
            self.estimate_compressed_buffer_size(4 * n))
        if outs is None:
            return (False, [], [])
        sizes = (ctypes.c_uint64 * batch)()
        bounds = (ctypes.c_float * batch)()
        rc = self._ctx.compress(
            _u64s(ins[0]), _u64s(outs[0]), _u64s(outs[1]),
            self._eps_array(eps_overrides, batch), batch, n,
            _stream_handle(self._device_id), sizes, bounds)
        return self._finish_compress(rc, batch, sizes, bounds,
                                     "fixed BF16 batch compression failed")

    def _layer_index_ok(self, layer_indices: torch.Tensor,
                        source_layers: int) -> bool:
        sel = layer_indices.numel()
        return (sel > 0 and sel <= source_layers and self._on_device(layer_indices)
                and layer_indices.dtype == torch.int64
                and layer_indices.is_contiguous())

    def compress_batch_fixed_bf16_indexed(self, input_tensors,
                                          compressed_buffers, layer_indices,
                                          prefix_count, source_layers,
                                          elements_per_layer, eps_overrides):
        """pybind11_bindings.cpp:104-132 -> cuszp_wrapper.cpp:548-681."""
        batch = len(input_tensors)
        if (batch == 0 or len(compressed_buffers) != batch
                or (eps_overrides and len(eps_overrides) != batch)
                or prefix_count == 0 or source_layers == 0
                or elements_per_layer == 0
                or not self._layer_index_ok(layer_indices, source_layers)
                or not self._fixed_mode()):
            return (False, [], [])
        sel = layer_indices.numel()
        source_elements = prefix_count * source_layers * elements_per_layer
        n = prefix_count * sel * elements_per_layer
        ins = _describe(input_tensors, self._device_id, torch.bfloat16, source_elements)
        outs = None if ins is None else _describe(
            compressed_buffers, self._device_id, torch.uint8,
            self.estimate_compressed_buffer_size(4 * n))
        if outs is None:
            return (False, [], [])
        sizes = (ctypes.c_uint64 * batch)()
        bounds = (ctypes.c_float * batch)()
        rc = self._ctx.compress_indexed(
            _u64s(ins[0]), _u64s(outs[0]), _u64s(outs[1]),
            layer_indices.data_ptr(), sel, prefix_count, source_layers,
            elements_per_layer, self._eps_array(eps_overrides, batch), batch,
            _stream_handle(self._device_id), sizes, bounds)
        return self._finish_compress(rc, batch, sizes, bounds,
                                     "indexed fixed BF16 batch compression failed")

    def compress_batch_fixed_bf16_indexed_groups(self, input_tensors,
                                                 compressed_buffers,
                                                 layer_indices, group_sizes,
                                                 prefix_count, source_layers,
                                                 elements_per_layer,
                                                 eps_overrides):
        """pybind11_bindings.cpp:133-163 -> cuszp_wrapper.cpp:683-868."""
        batch = len(input_tensors)
        if (batch == 0 or len(compressed_buffers) != batch
                or (eps_overrides and len(eps_overrides) != batch)
                or not layer_indices or len(layer_indices) != len(group_sizes)
                or prefix_count == 0 or source_layers == 0
                or elements_per_layer == 0 or not self._fixed_mode()):
            return (False, [], [])
        for size, idx in zip(group_sizes, layer_indices):
            if size == 0 or not self._layer_index_ok(idx, source_layers):
                return (False, [], [])
        if sum(group_sizes) != batch:
            return (False, [], [])
        source_elements = prefix_count * source_layers * elements_per_layer
        ins = _describe(input_tensors, self._device_id, torch.bfloat16, source_elements)
        if ins is None:
            return (False, [], [])
        out_ptrs, out_caps = [], []
        buffers = list(compressed_buffers)
        offset = 0
        for size, idx in zip(group_sizes, layer_indices):
            n = prefix_count * idx.numel() * elements_per_layer
            outs = _describe(buffers[offset:offset + size], self._device_id, torch.uint8,
                             self.estimate_compressed_buffer_size(4 * n))
            if outs is None:
                return (False, [], [])
            out_ptrs.append(outs[0])
            out_caps.append(outs[1])
            offset += size
        groups = len(group_sizes)
        sizes = (ctypes.c_uint64 * batch)()
        bounds = (ctypes.c_float * batch)()
        rc = self._ctx.compress_indexed_groups(
            _u64s(ins[0]), _u64s(b"".join(out_ptrs)), _u64s(b"".join(out_caps)),
            kvszp.ptr_array([t.data_ptr() for t in layer_indices]),
            kvszp.size_array([t.numel() for t in layer_indices]),
            kvszp.size_array([int(s) for s in group_sizes]), groups,
            prefix_count, source_layers, elements_per_layer,
            self._eps_array(eps_overrides, batch), batch,
            _stream_handle(self._device_id), sizes, bounds)
        return self._finish_compress(
            rc, batch, sizes, bounds,
            "grouped indexed fixed BF16 batch compression failed")

    # ---- batched BF16 decompress -----------------------------------------

    def _streams(self, compressed_buffers, compressed_sizes, actual_error_bounds):
        """(stream pointers, sizes, bounds) for the C ABI, or None when a
        stream is not on the device or a size is 0 (cuszp_wrapper.cpp:1065-
        1077)."""
        streams = _describe(compressed_buffers, self._device_id, None, contiguous=False)
        if streams is None:
            return None
        sizes, keep_s = _u64_values(compressed_sizes)
        if 0 in keep_s:
            return None
        bounds, keep_b = _f32_values(actual_error_bounds)
        return _u64s(streams[0]), sizes, bounds, (keep_s, keep_b)

    def decompress_batch_fixed_bf16(self, compressed_buffers,
                                    compressed_sizes, output_tensor,
                                    num_elements_per_page,
                                    actual_error_bounds):
        """pybind11_bindings.cpp:190-207 -> cuszp_wrapper.cpp:1034-1110."""
        batch = len(compressed_buffers)
        if batch == 0:
            return True
        if (len(compressed_sizes) != batch or len(actual_error_bounds) != batch
                or num_elements_per_page == 0 or not output_tensor.is_cuda
                or output_tensor.dtype != torch.bfloat16
                or output_tensor.numel() < batch * num_elements_per_page
                or not self._fixed_mode()):
            print("Error: invalid cuSZp fixed BF16 batch metadata", file=sys.stderr)
            return False
        st = self._streams(compressed_buffers, compressed_sizes, actual_error_bounds)
        if st is None:
            print("Error: invalid cuSZp fixed BF16 batch metadata", file=sys.stderr)
            return False
        rc = self._ctx.decompress(
            st[0], st[1], st[2], batch,
            output_tensor.data_ptr(), output_tensor.numel(),
            num_elements_per_page, _stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("fixed BF16 batch decompression failed")
            return False
        return True

    def decompress_batch_fixed_bf16_scatter(self, compressed_buffers,
                                            compressed_sizes, output_tensors,
                                            num_elements_per_page,
                                            destinations_per_page,
                                            elements_per_destination,
                                            actual_error_bounds):
        """pybind11_bindings.cpp:208-230 -> cuszp_wrapper.cpp:1111-1212."""
        batch = len(compressed_buffers)
        if batch == 0:
            return True
        if (len(compressed_sizes) != batch or len(actual_error_bounds) != batch
                or destinations_per_page == 0 or elements_per_destination == 0
                or num_elements_per_page
                != destinations_per_page * elements_per_destination
                or len(output_tensors) != batch * destinations_per_page
                or not self._fixed_mode()):
            print("Error: invalid cuSZp direct-scatter metadata", file=sys.stderr)
            return False
        st = self._streams(compressed_buffers, compressed_sizes, actual_error_bounds)
        if st is None:
            print("Error: invalid cuSZp direct-scatter metadata", file=sys.stderr)
            return False
        outs = _describe(output_tensors, self._device_id, torch.bfloat16,
                         elements_per_destination)
        if outs is None:
            print("Error: invalid BF16 direct-scatter destination", file=sys.stderr)
            return False
        rc = self._ctx.decompress_scatter(
            st[0], st[1], st[2], batch, _u64s(outs[0]),
            num_elements_per_page, destinations_per_page,
            elements_per_destination, _stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("fixed BF16 direct-scatter decompression failed")
            return False
        return True

    def decompress_batch_fixed_bf16_indexed_scatter(self, compressed_buffers,
                                                    compressed_sizes,
                                                    output_tensors,
                                                    layer_indices,
                                                    prefix_count,
                                                    source_layers,
                                                    elements_per_layer,
                                                    actual_error_bounds):
        """pybind11_bindings.cpp:232-256 -> cuszp_wrapper.cpp:1214-1313."""
        batch = len(compressed_buffers)
        if batch == 0:
            return True
        if (len(compressed_sizes) != batch or len(actual_error_bounds) != batch
                or len(output_tensors) != batch or prefix_count == 0
                or source_layers == 0 or elements_per_layer == 0
                or not self._layer_index_ok(layer_indices, source_layers)
                or not self._fixed_mode()):
            return False
        source_elements = prefix_count * source_layers * elements_per_layer
        st = self._streams(compressed_buffers, compressed_sizes, actual_error_bounds)
        outs = None if st is None else _describe(
            output_tensors, self._device_id, torch.bfloat16, source_elements)
        if outs is None:
            return False
        rc = self._ctx.decompress_indexed_scatter(
            st[0], st[1], st[2], batch, _u64s(outs[0]),
            layer_indices.data_ptr(), layer_indices.numel(), prefix_count,
            source_layers, elements_per_layer, _stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("indexed fixed BF16 scatter decompression failed")
            return False
        return True

    def decompress_batch_fixed_bf16_indexed_scatter_groups(
            self, compressed_buffers, compressed_sizes, output_tensors,
            layer_indices, group_sizes, prefix_count, source_layers,
            elements_per_layer, actual_error_bounds):
        """Several decompress_batch_fixed_bf16_indexed_scatter calls (one per
        layer group, vllm_v1_compressed_offload.py:1815-2006) in one launch.
        Requests are laid out group by group: group g covers the next
        group_sizes[g] entries and scatters through layer_indices[g].  No
        reference counterpart; same argument checks and result as the
        per-group calls."""
        batch = len(compressed_buffers)
        if batch == 0:
            return True
        if (len(compressed_sizes) != batch or len(actual_error_bounds) != batch
                or len(output_tensors) != batch or not layer_indices
                or len(layer_indices) != len(group_sizes)
                or prefix_count == 0 or source_layers == 0
                or elements_per_layer == 0 or not self._fixed_mode()):
            return False
        for size, idx in zip(group_sizes, layer_indices):
            if int(size) == 0 or not self._layer_index_ok(idx, source_layers):
                return False
        if sum(int(s) for s in group_sizes) != batch:
            return False
        source_elements = prefix_count * source_layers * elements_per_layer
        st = self._streams(compressed_buffers, compressed_sizes, actual_error_bounds)
        outs = None if st is None else _describe(
            output_tensors, self._device_id, torch.bfloat16, source_elements)
        if outs is None:
            return False
        rc = self._ctx.decompress_indexed_scatter_groups(
            st[0], st[1], st[2], batch, _u64s(outs[0]),
            kvszp.ptr_array([t.data_ptr() for t in layer_indices]),
            kvszp.size_array([t.numel() for t in layer_indices]),
            kvszp.size_array([int(s) for s in group_sizes]),
            len(group_sizes), prefix_count, source_layers,
            elements_per_layer, _stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("grouped indexed fixed BF16 scatter decompression failed")
            return False
        return True

    # ---- packed publication and restore (no pybind counterpart) ----------

    def pack_payloads(self, payloads, slab):
        """The device half of CompressedPageStore.put_many_packed
        (vllm_v1_compressed_offload.py:371-447): every payload (a uint8 device
        tensor: a stream slice or a raw page's bytes) goes to `slab` at the
        8-byte-aligned exclusive scan of the sizes, gaps zeroed.  `slab` is
        normally a pinned host uint8 tensor: one gather kernel then writes the
        payloads across the link (the device-to-host copy itself).  Blocks
        until the slab is complete.  Returns (ok, offsets, packed_bytes)."""
        count = len(payloads)
        if count == 0 or slab.dtype != torch.uint8 or not slab.is_contiguous():
            return (False, [], 0)
        if not (slab.is_pinned() or self._on_device(slab)):
            return (False, [], 0)
        src = _describe(payloads, self._device_id, None)
        if src is None:
            return (False, [], 0)
        offsets = (ctypes.c_uint64 * count)()
        total = ctypes.c_uint64()
        rc = self._ctx.pack(
            _u64s(src[0]), _u64s(src[1]), count, slab.data_ptr(), slab.numel(), _stream_handle(self._device_id),
            offsets, ctypes.byref(total))
        if rc != kvszp.OK:
            _report("packing payloads failed")
            return (False, [], 0)
        return (True, _as_list(offsets, "Q"), int(total.value))

    def decompress_batch_fixed_bf16_indexed_scatter_groups_packed(
            self, packed, packed_bytes, staging, offsets, compressed_sizes,
            output_tensors, layer_indices, group_sizes, prefix_count,
            source_layers, elements_per_layer, actual_error_bounds):
        """The packed restore (vllm_v1_compressed_offload.py:1618-1711): one
        host-to-device copy of the pinned slab `packed` into the uint8 device
        tensor `staging`, then the grouped indexed scatter of the streams at
        `offsets`; staging None: the decoder reads the streams straight from
        the pinned slab.  Enqueue only."""
        batch = len(offsets)
        if batch == 0:
            return True
        if (len(compressed_sizes) != batch or len(actual_error_bounds) != batch
                or len(output_tensors) != batch or not layer_indices
                or len(layer_indices) != len(group_sizes)
                or not self._fixed_mode() or not packed.is_pinned()
                or (staging is not None and (not self._on_device(staging)
                                             or staging.dtype != torch.uint8))
                or sum(int(g) for g in group_sizes) != batch):
            return False
        for idx in layer_indices:
            if not self._layer_index_ok(idx, source_layers):
                return False
        source_elements = prefix_count * source_layers * elements_per_layer
        outs = _describe(output_tensors, self._device_id, torch.bfloat16,
                         source_elements)
        if outs is None:
            return False
        offs, keep_o = _u64_values(offsets)
        sizes, keep_s = _u64_values(compressed_sizes)
        bounds, keep_b = _f32_values(actual_error_bounds)
        rc = self._ctx.decompress_indexed_scatter_groups_packed(
            packed.data_ptr(), int(packed_bytes),
            None if staging is None else staging.data_ptr(),
            0 if staging is None else staging.numel(),
            offs, sizes, bounds, batch, _u64s(outs[0]),
            kvszp.ptr_array([t.data_ptr() for t in layer_indices]),
            kvszp.size_array([t.numel() for t in layer_indices]),
            kvszp.size_array([int(g) for g in group_sizes]), len(group_sizes),
            prefix_count, source_layers, elements_per_layer,
            _stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("packed grouped indexed scatter decompression failed")
            return False
        return True

    def synchronize(self) -> bool:
        """Waits for the current stream and reports device-side errors of
        earlier (enqueue-only) decompress calls.  No reference counterpart."""
        rc = self._ctx.synchronize(_stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("device-side codec error")
            return False
        return True

    # ---- single-page fp32 API ------------------------------------------
    # The reference runs upstream cuSZp's fp32 kernels here
    # (cuszp_fastpath.cu:5-64).  Fixed mode: the stream layout is the
    # batched BF16 one (cuszp_batched_fixed.cu:52-54), so the same HIP
    # kernels serve it with fp32 loads and stores.  Plain and outlier modes
    # (upstream's cuSZp_compress/cuSZp_decompress, :302-313, 922-933): this
    # library's residual codes (kvszp_compress_f32 in include/kvszp.h), whose
    # streams only this library decodes.

    def _fp32_ok(self, t: torch.Tensor) -> bool:
        # The reference reads data_ptr() as a dense float array without
        # checking; other dtypes or layouts are refused here instead.
        return (self._on_device(t) and t.dtype == torch.float32
                and t.is_contiguous() and t.numel() > 0)

    def compress(self, input_tensor, compressed_buffer, eps_override=-1.0):
        """pybind11_bindings.cpp:49-64 -> cuszp_wrapper.cpp:216-325.  Returns
        (ok, buffer, size, actual_error_bound); a buffer smaller than
        estimate_compressed_buffer_size(nbytes) is replaced by a new one, as
        in the reference (:229-237)."""
        if not input_tensor.is_cuda:
            print("Error: Input tensor must be on GPU", file=sys.stderr)
            return (False, compressed_buffer, 0, 0.0)
        if not self._f32_1d() or not self._fp32_ok(input_tensor):
            print("Error: cuSZp compression failed (fp32 1D only)",
                  file=sys.stderr)
            return (False, compressed_buffer, 0, 0.0)
        n = input_tensor.numel()
        # estimate(nbytes) = 8n, raised to the worst-case stream for tiny
        # inputs (a 1024-byte header per 32 768 values, 128 bytes per block,
        # 136 in the plain/outlier codes), which 8n does not cover below
        # 147 (156) values.
        per_block = 128 if self._fixed_mode() else 136
        estimated = max(self.estimate_compressed_buffer_size(4 * n),
                        kvszp.header_bytes(n) + per_block * ((n + 31) // 32))
        if (compressed_buffer.numel() * compressed_buffer.element_size()
                < estimated or not self._on_device(compressed_buffer)
                or not compressed_buffer.is_contiguous()):
            compressed_buffer = torch.empty(estimated, dtype=torch.uint8,
                                            device=input_tensor.device)
        size = ctypes.c_uint64()
        bound = ctypes.c_float()
        rc = self._ctx.compress_f32_mode(
            input_tensor.data_ptr(), n, compressed_buffer.data_ptr(),
            compressed_buffer.numel() * compressed_buffer.element_size(),
            _f32(eps_override), _stream_handle(self._device_id),
            ctypes.byref(size), ctypes.byref(bound))
        if rc != kvszp.OK:
            _report("cuSZp compression failed")
            return (False, compressed_buffer, 0, 0.0)
        return (True, compressed_buffer, int(size.value), float(bound.value))

    def compress_batch_fixed(self, input_tensors, compressed_buffers,
                             eps_overrides):
        """pybind11_bindings.cpp:65-82 -> cuszp_wrapper.cpp:327-429."""
        batch = len(input_tensors)
        if (batch == 0 or len(compressed_buffers) != batch
                or (eps_overrides and len(eps_overrides) != batch)
                or not self._fixed_mode()):
            return (False, [], [])
        n = input_tensors[0].numel()
        ins = None if n == 0 else _describe(input_tensors, self._device_id,
                                            torch.float32, n, exact=True)
        outs = None if ins is None else _describe(
            compressed_buffers, self._device_id, torch.uint8,
            self.estimate_compressed_buffer_size(4 * n))
        if outs is None:
            return (False, [], [])
        sizes = (ctypes.c_uint64 * batch)()
        bounds = (ctypes.c_float * batch)()
        rc = self._ctx.compress_batch_f32(
            _u64s(ins[0]), _u64s(outs[0]), _u64s(outs[1]),
            self._eps_array(eps_overrides, batch), batch, n,
            _stream_handle(self._device_id), sizes, bounds)
        return self._finish_compress(rc, batch, sizes, bounds,
                                     "cuSZp fixed batch compression failed")

    def decompress(self, compressed_buffer, compressed_size, output_tensor,
                   actual_error_bound):
        """pybind11_bindings.cpp:164-173 -> cuszp_wrapper.cpp:870-943: decodes
        output_tensor.numel() fp32 values; enqueue only."""
        if not compressed_buffer.is_cuda or not output_tensor.is_cuda:
            print("Error: Both compressed buffer and output tensor must be on "
                  "GPU", file=sys.stderr)
            return False
        if (not self._f32_1d() or not self._fp32_ok(output_tensor)
                or not self._on_device(compressed_buffer)
                or int(compressed_size) == 0):
            print("Error: cuSZp decompression failed (fp32 1D only)",
                  file=sys.stderr)
            return False
        rc = self._ctx.decompress_f32_mode(
            compressed_buffer.data_ptr(), int(compressed_size),
            output_tensor.data_ptr(), output_tensor.numel(),
            _f32(actual_error_bound), _stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("cuSZp fast decompression failed")
            return False
        return True

    def decompress_batch(self, compressed_buffers, compressed_sizes,
                         output_tensors, actual_error_bounds):
        """pybind11_bindings.cpp:174-189 -> cuszp_wrapper.cpp:944-1033: page i
        to output_tensors[i] (fp32, any length); enqueue only."""
        batch = len(compressed_buffers)
        if batch == 0:
            return True
        if (len(compressed_sizes) != batch or len(output_tensors) != batch
                or len(actual_error_bounds) != batch):
            print("Error: cuSZp batch metadata lengths differ", file=sys.stderr)
            return False
        if not self._f32_1d():
            print("Error: cuSZp batch fast path requires 1D f32",
                  file=sys.stderr)
            return False
        st = self._streams(compressed_buffers, compressed_sizes, actual_error_bounds)
        outs = None if st is None else _describe(
            output_tensors, self._device_id, torch.float32, 1)
        if outs is None:
            print("Error: invalid tensor in cuSZp batch", file=sys.stderr)
            return False
        out_bytes = array("Q")
        out_bytes.frombytes(outs[1])
        counts, keep_c = _u64_values(b // 4 for b in out_bytes)
        rc = self._ctx.decompress_batch_f32_mode(
            st[0], st[1], st[2], batch, _u64s(outs[0]), counts,
            _stream_handle(self._device_id))
        if rc != kvszp.OK:
            _report("cuSZp batched decompression failed")
            return False
        return True
