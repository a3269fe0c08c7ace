"""ctypes bindings for libkvszp.so, the C ABI in include/kvszp.h.

This module is the thin host layer between Python and the HIP codec.  It
takes device addresses (ints) and host-side arrays, never framework tensors,
so it can be driven from torch, from raw pointers, or from the benchmark.
The ``cuszp_wrapper_cpp`` module builds the reference's tensor API on top of
it.

If the shared library is missing this module raises at import time: there is
no CPU fallback for the codec.
"""

from __future__ import annotations

import ctypes
import os
from typing import Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkvszp.so")

OK = 0
EINVAL = -1
EHIP = -2
ENOMEM = -3
EDEVICE = -4

DIM_1D, DIM_2D, DIM_3D = 0, 1, 2
MODE_FIXED, MODE_PLAIN, MODE_OUTLIER = 0, 1, 2
TYPE_FLOAT, TYPE_DOUBLE = 0, 1
QUANT_TWO_ROUNDINGS, QUANT_FUSED = 0, 1
RATE0_SKIP, RATE0_ZERO = 0, 1
KERNEL_COMPRESS, KERNEL_DECOMPRESS = 0, 1
TIME_COMPRESS, TIME_DECOMPRESS = 1 << KERNEL_COMPRESS, 1 << KERNEL_DECOMPRESS
TIME_ALL = TIME_COMPRESS | TIME_DECOMPRESS

# (name, restype, argtypes) of every entry point declared in include/kvszp.h.
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i = ctypes.c_int
EXPORTS = [
    ("kvszp_create", _i, [_vp, _i, _vp]),
    ("kvszp_destroy", _i, [_vp]),
    ("kvszp_get_config", _i, [_vp, _vp]),
    ("kvszp_update_config", _i, [_vp, _vp]),
    ("kvszp_set_options", _i, [_vp, _i, _i]),
    ("kvszp_estimate_compressed_buffer_size", _sz, [_sz]),
    ("kvszp_header_bytes", _sz, [_sz]),
    ("kvszp_compress_batch_fixed_bf16", _i,
     [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    ("kvszp_compress_batch_fixed_bf16_noalloc", _i,
     [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    ("kvszp_compress_batch_fixed_bf16_indexed", _i,
     [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _vp]),
    ("kvszp_compress_batch_fixed_bf16_indexed_groups", _i,
     [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp,
      _vp, _vp]),
    ("kvszp_decompress_batch_fixed_bf16", _i,
     [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _sz, _vp]),
    ("kvszp_decompress_batch_fixed_bf16_scatter", _i,
     [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _sz, _sz, _vp]),
    ("kvszp_decompress_batch_fixed_bf16_indexed_scatter", _i,
     [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz, _vp]),
    ("kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups", _i,
     [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp]),
    ("kvszp_compress_fixed_f32", _i,
     [_vp, _vp, _sz, _vp, ctypes.c_uint64, ctypes.c_float, _vp, _vp, _vp]),
    ("kvszp_compress_batch_fixed_f32", _i,
     [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    ("kvszp_decompress_fixed_f32", _i,
     [_vp, _vp, ctypes.c_uint64, _vp, _sz, ctypes.c_float, _vp]),
    ("kvszp_decompress_batch_fixed_f32", _i,
     [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp]),
    ("kvszp_compress_f32", _i,
     [_vp, _vp, _sz, _vp, ctypes.c_uint64, ctypes.c_float, _vp, _vp, _vp]),
    ("kvszp_decompress_f32", _i,
     [_vp, _vp, ctypes.c_uint64, _vp, _sz, ctypes.c_float, _vp]),
    ("kvszp_decompress_batch_f32", _i,
     [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp]),
    ("kvszp_pack_streams", _i,
     [_vp, _vp, _vp, _sz, _vp, ctypes.c_uint64, _vp, _vp, _vp]),
    ("kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups_packed", _i,
     [_vp, _vp, ctypes.c_uint64, _vp, ctypes.c_uint64, _vp, _vp, _vp, _sz, _vp,
      _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp]),
    ("kvszp_synchronize", _i, [_vp, _vp]),
    ("kvszp_enable_timing", _i, [_vp, _i]),
    ("kvszp_drain_timing", _i, [_vp, _vp, _vp, _vp, _vp]),
    ("kvszp_timing_durations", _i, [_vp, _i, _vp, _i, _vp]),
    ("kvszp_reencode_count", _i, [_vp, _vp]),
    ("kvszp_set_wait_bound", _i, [_vp, ctypes.c_double]),
    ("kvszp_schedule_counts", _i, [_vp, _vp, _vp]),
    ("kvszp_last_error", ctypes.c_char_p, []),
]


class Config(ctypes.Structure):
    """kvszp_config (include/kvszp.h)."""

    _fields_ = [
        ("error_bound", ctypes.c_float),
        ("use_relative_error", ctypes.c_int),
        ("processing_dim", ctypes.c_int),
        ("encoding_mode", ctypes.c_int),
        ("data_type", ctypes.c_int),
    ]


class KvszpError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"kvszp error {code}: {message}")
        self.code = code


_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads libkvszp.so; raises if it has not been built.

    PyTorch-ROCm bundles its own HIP runtime under the same SONAME
    (libamdhip64.so.7) as the system ROCm one libkvszp.so is linked against.
    Whichever is loaded first serves the process; loading both breaks device
    discovery.  So when torch is installed it is imported first and the
    codec runs on torch's runtime, sharing its streams."""
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with build.py (hipcc, gfx950)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, restype, argtypes in EXPORTS:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().kvszp_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(code: int) -> None:
    if code != OK:
        raise KvszpError(code, last_error())


def ptr_array(values: Sequence[int]):
    return (ctypes.c_void_p * len(values))(*values)


def u64_array(values: Sequence[int]):
    return (ctypes.c_uint64 * len(values))(*values)


def f32_array(values: Sequence[float]):
    return (ctypes.c_float * len(values))(*values)


def size_array(values: Sequence[int]):
    return (ctypes.c_size_t * len(values))(*values)


class Context:
    """Owns one kvszp_ctx (device workspaces).  Not thread-safe; use one per
    stream, like the reference's CuSZpWrapper."""

    def __init__(self, config: Config | None = None, device_id: int = 0):
        self._lib = load()
        handle = ctypes.c_void_p()
        check(self._lib.kvszp_create(
            None if config is None else ctypes.byref(config), device_id,
            ctypes.byref(handle)))
        self.handle = handle
        self.device_id = device_id

    def close(self) -> None:
        if self.handle:
            self._lib.kvszp_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def get_config(self) -> Config:
        cfg = Config()
        check(self._lib.kvszp_get_config(self.handle, ctypes.byref(cfg)))
        return cfg

    def update_config(self, cfg: Config) -> None:
        check(self._lib.kvszp_update_config(self.handle, ctypes.byref(cfg)))

    def set_options(self, quantizer: int = QUANT_TWO_ROUNDINGS,
                    rate0_policy: int = RATE0_ZERO) -> None:
        check(self._lib.kvszp_set_options(self.handle, quantizer, rate0_policy))

    # Every method below returns the raw status code; callers decide whether
    # to raise (the tensor shim maps failures to the reference's False).

    def compress(self, inputs, outputs, capacities, eps, batch, n, stream,
                 sizes_out, bounds_out) -> int:
        return self._lib.kvszp_compress_batch_fixed_bf16(
            self.handle, inputs, outputs, capacities, eps, batch, n, stream,
            sizes_out, bounds_out)

    def compress_noalloc(self, inputs, outputs, capacities, eps, batch, n,
                         stream, sizes_out, bounds_out) -> int:
        """kvszp_compress_batch_fixed_bf16 without any allocation in the call
        (device state in the library's per-GPU scratch array)."""
        return self._lib.kvszp_compress_batch_fixed_bf16_noalloc(
            self.handle, inputs, outputs, capacities, eps, batch, n, stream,
            sizes_out, bounds_out)

    def compress_indexed(self, inputs, outputs, capacities, layer_indices,
                         selected_layers, prefix_count, source_layers,
                         elements_per_layer, eps, batch, stream, sizes_out,
                         bounds_out) -> int:
        return self._lib.kvszp_compress_batch_fixed_bf16_indexed(
            self.handle, inputs, outputs, capacities, layer_indices,
            selected_layers, prefix_count, source_layers, elements_per_layer,
            eps, batch, stream, sizes_out, bounds_out)

    def compress_indexed_groups(self, inputs, outputs, capacities,
                                layer_indices, selected_layers, group_sizes,
                                num_groups, prefix_count, source_layers,
                                elements_per_layer, eps, batch, stream,
                                sizes_out, bounds_out) -> int:
        return self._lib.kvszp_compress_batch_fixed_bf16_indexed_groups(
            self.handle, inputs, outputs, capacities, layer_indices,
            selected_layers, group_sizes, num_groups, prefix_count,
            source_layers, elements_per_layer, eps, batch, stream, sizes_out,
            bounds_out)

    def decompress(self, compressed, sizes, bounds, batch, output,
                   output_elements, n, stream) -> int:
        return self._lib.kvszp_decompress_batch_fixed_bf16(
            self.handle, compressed, sizes, bounds, batch, output,
            output_elements, n, stream)

    def decompress_scatter(self, compressed, sizes, bounds, batch,
                           destinations, n, destinations_per_page,
                           elements_per_destination, stream) -> int:
        return self._lib.kvszp_decompress_batch_fixed_bf16_scatter(
            self.handle, compressed, sizes, bounds, batch, destinations, n,
            destinations_per_page, elements_per_destination, stream)

    def decompress_indexed_scatter(self, compressed, sizes, bounds, batch,
                                   destinations, layer_indices,
                                   selected_layers, prefix_count,
                                   source_layers, elements_per_layer,
                                   stream) -> int:
        return self._lib.kvszp_decompress_batch_fixed_bf16_indexed_scatter(
            self.handle, compressed, sizes, bounds, batch, destinations,
            layer_indices, selected_layers, prefix_count, source_layers,
            elements_per_layer, stream)

    def decompress_indexed_scatter_groups(self, compressed, sizes, bounds,
                                          batch, destinations, layer_indices,
                                          selected_layers, group_sizes,
                                          num_groups, prefix_count,
                                          source_layers, elements_per_layer,
                                          stream) -> int:
        return self._lib.kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups(
            self.handle, compressed, sizes, bounds, batch, destinations,
            layer_indices, selected_layers, group_sizes, num_groups,
            prefix_count, source_layers, elements_per_layer, stream)

    def compress_f32(self, input_ptr, n, output_ptr, capacity, eps_override,
                     stream, size_out, bound_out) -> int:
        return self._lib.kvszp_compress_fixed_f32(
            self.handle, input_ptr, n, output_ptr, capacity, eps_override,
            stream, size_out, bound_out)

    def compress_batch_f32(self, inputs, outputs, capacities, eps, batch, n,
                           stream, sizes_out, bounds_out) -> int:
        return self._lib.kvszp_compress_batch_fixed_f32(
            self.handle, inputs, outputs, capacities, eps, batch, n, stream,
            sizes_out, bounds_out)

    def decompress_f32(self, compressed_ptr, size, output_ptr, n, eb,
                       stream) -> int:
        return self._lib.kvszp_decompress_fixed_f32(
            self.handle, compressed_ptr, size, output_ptr, n, eb, stream)

    def decompress_batch_f32(self, compressed, sizes, bounds, batch, outputs,
                             numels, stream) -> int:
        return self._lib.kvszp_decompress_batch_fixed_f32(
            self.handle, compressed, sizes, bounds, batch, outputs, numels,
            stream)

    # The context's encoding mode (fixed, plain or outlier).
    def compress_f32_mode(self, input_ptr, n, output_ptr, capacity, eps_override,
                          stream, size_out, bound_out) -> int:
        return self._lib.kvszp_compress_f32(
            self.handle, input_ptr, n, output_ptr, capacity, eps_override,
            stream, size_out, bound_out)

    def decompress_f32_mode(self, compressed_ptr, size, output_ptr, n, eb,
                            stream) -> int:
        return self._lib.kvszp_decompress_f32(
            self.handle, compressed_ptr, size, output_ptr, n, eb, stream)

    def decompress_batch_f32_mode(self, compressed, sizes, bounds, batch, outputs,
                                  numels, stream) -> int:
        return self._lib.kvszp_decompress_batch_f32(
            self.handle, compressed, sizes, bounds, batch, outputs, numels,
            stream)

    def pack(self, payloads, sizes, count, slab, slab_capacity, stream,
             offsets_out, packed_bytes_out) -> int:
        return self._lib.kvszp_pack_streams(
            self.handle, payloads, sizes, count, slab, slab_capacity, stream,
            offsets_out, packed_bytes_out)

    def decompress_indexed_scatter_groups_packed(
            self, packed, packed_bytes, staging, staging_capacity, offsets,
            sizes, bounds, batch, destinations, layer_indices, selected_layers,
            group_sizes, num_groups, prefix_count, source_layers,
            elements_per_layer, stream) -> int:
        return self._lib.kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups_packed(
            self.handle, packed, packed_bytes, staging, staging_capacity,
            offsets, sizes, bounds, batch, destinations, layer_indices,
            selected_layers, group_sizes, num_groups, prefix_count,
            source_layers, elements_per_layer, stream)

    def timing_durations(self, kind: int, capacity: int = 1 << 16) -> list:
        """Per-launch durations (ms) of the timed launches of `kind`
        (KERNEL_COMPRESS / KERNEL_DECOMPRESS) since the last drain."""
        buf = (ctypes.c_double * capacity)()
        n = ctypes.c_int()
        check(self._lib.kvszp_timing_durations(self.handle, kind, buf, capacity,
                                               ctypes.byref(n)))
        return [buf[i] for i in range(n.value)]

    def reencode_count(self) -> int:
        """Compress calls encoded again with the pre-pass schedule (a
        bounded wait gave up, or the persistent staging overflowed)."""
        n = ctypes.c_uint64()
        check(self._lib.kvszp_reencode_count(self.handle, ctypes.byref(n)))
        return n.value

    def schedule_counts(self) -> dict:
        """Compress calls encoded again (a give-up or a staging overflow)
        and calls run on the schedule that needs no residency because of a
        recent give-up."""
        r, s = ctypes.c_uint64(), ctypes.c_uint64()
        check(self._lib.kvszp_schedule_counts(self.handle, ctypes.byref(r), ctypes.byref(s)))
        return {"reencoded": r.value, "safe_calls": s.value}

    def set_wait_bound(self, microseconds: float) -> None:
        """Time bound of the encoders' cross-workgroup waits (us)."""
        check(self._lib.kvszp_set_wait_bound(self.handle, float(microseconds)))

    def synchronize(self, stream) -> int:
        return self._lib.kvszp_synchronize(self.handle, stream)

    def enable_timing(self, kinds: int | bool = TIME_ALL) -> None:
        """Times the launches of the kernel kinds in ``kinds`` (a mask of
        TIME_*; True means all, False or 0 none)."""
        if isinstance(kinds, bool):
            kinds = TIME_ALL if kinds else 0
        check(self._lib.kvszp_enable_timing(self.handle, int(kinds)))

    def drain_timing(self) -> dict:
        """Summed kernel milliseconds and launch counts since the last drain,
        from HIP events recorded on the launch stream."""
        cms, dms = ctypes.c_double(), ctypes.c_double()
        cc, dc = ctypes.c_int(), ctypes.c_int()
        check(self._lib.kvszp_drain_timing(
            self.handle, ctypes.byref(cms), ctypes.byref(cc), ctypes.byref(dms),
            ctypes.byref(dc)))
        return {"compress_ms": cms.value, "compress_launches": cc.value,
                "decompress_ms": dms.value, "decompress_launches": dc.value}


def header_bytes(n: int) -> int:
    return int(load().kvszp_header_bytes(n))


def estimate_compressed_buffer_size(original_size: int) -> int:
    return int(load().kvszp_estimate_compressed_buffer_size(original_size))
