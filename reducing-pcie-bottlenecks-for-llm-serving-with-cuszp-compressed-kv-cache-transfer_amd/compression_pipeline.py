"""Codec-facing half of the reference's KV offload connector, on the MI355X
codec.

The reference's ``CompressedOffloadingHandler``
(integration/compression_pipeline/vllm_v1_compressed_offload.py:481-2184)
turns vLLM offload jobs into calls of the batched fixed-mode BF16 codec and
back.  This module keeps exactly that part -- the page bundling, the
minimum-size padding, the raw fallback, the grouping of layers by error
bound, the choice of restore path and the packed host store -- with the same
names, metadata and decisions, and leaves out what belongs to vLLM (transfer
specs, job threads, metrics, the adaptive bound controller, the host-side
zlib/zstd/LZ4/INT8 codecs).

A page is ``kv_tensors[tensor_idx][gpu_block_id]`` (the reference's
``kv_caches.tensors[tensor_idx].tensor[gpu_block_id]``); an operation is
``(tensor_indices, gpu_block_id, cpu_block_id)`` as produced by the
reference's ``_iter_page_operations`` (:458-478).

Each method returns ``None`` where the reference's does, so a caller falls
back exactly as the connector would.
"""

from __future__ import annotations

import threading
import time
from dataclasses import dataclass
from typing import Sequence

import torch

import cuszp_wrapper_cpp

MIN_CUSZP_ELEMENTS = 36864  # vllm_v1_compressed_offload.py:49
CUSZP_MODES = {
    "plain": cuszp_wrapper_cpp.CuszpMode.MODE_PLAIN,
    "fixed": cuszp_wrapper_cpp.CuszpMode.MODE_FIXED,
    "outlier": cuszp_wrapper_cpp.CuszpMode.MODE_OUTLIER,
}


# ---- metadata (vllm_v1_compressed_offload.py:58-113) -------------------------

@dataclass
class BundleComponent:
    tensor_idx: int
    original_shape: tuple[int, ...]
    original_dtype: torch.dtype
    numel: int
    layer_axis: int | None = None
    layer_indices: tuple[int, ...] = ()
    destination_view_shape: tuple[int, ...] = ()


@dataclass
class EncodedSegment:
    payload: torch.Tensor
    compressed_size: int
    actual_error_bound: float
    encoding: str
    components: tuple[BundleComponent, ...]
    unpadded_numel: int
    compressed_numel: int
    original_bytes: int
    requested_error_bound: float
    quant_scale: float | None = None
    cuszp_mode: str | None = None


@dataclass
class CompressedBundle:
    segments: tuple[EncodedSegment, ...]
    compressed_size: int
    original_bytes: int


@dataclass
class RestoreStageTimings:
    cpu_decode_seconds: float = 0.0
    h2d_seconds: float = 0.0
    gpu_decode_seconds: float = 0.0
    scatter_seconds: float = 0.0

    def add(self, other: "RestoreStageTimings") -> None:
        self.cpu_decode_seconds += other.cpu_decode_seconds
        self.h2d_seconds += other.h2d_seconds
        self.gpu_decode_seconds += other.gpu_decode_seconds
        self.scatter_seconds += other.scatter_seconds

    def as_dict(self) -> dict[str, float]:
        return {"cpu_decode_seconds": self.cpu_decode_seconds,
                "h2d_seconds": self.h2d_seconds,
                "gpu_decode_seconds": self.gpu_decode_seconds,
                "scatter_seconds": self.scatter_seconds}


def _bundle(segments) -> CompressedBundle:
    segments = tuple(segments)
    return CompressedBundle(
        segments=segments,
        compressed_size=sum(s.compressed_size for s in segments),
        original_bytes=sum(s.original_bytes for s in segments))


def _as_bf16(storage: torch.Tensor) -> torch.Tensor:
    """KV caches may be byte tensors holding BF16 (:876-880)."""
    if storage.dtype in (torch.uint8, torch.int8):
        return storage.view(torch.uint8).view(torch.bfloat16)
    return storage


# ---- packed host store (vllm_v1_compressed_offload.py:360-455) ---------------

class CompressedPageStore:
    """Variable-length host storage shared by the offload and restore
    directions.  ``put_many_packed`` copies one job's payloads into a single
    pinned slab (8-byte aligned), with one device-to-host copy when they all
    live on one GPU."""

    ALIGNMENT = 8

    def __init__(self):
        self._pages: dict[int, CompressedBundle] = {}
        self._lock = threading.Lock()
        self._gpu_pack_slab: torch.Tensor | None = None

    def put(self, cpu_block_id: int, bundle: CompressedBundle) -> None:
        with self._lock:
            self._pages[cpu_block_id] = bundle

    def put_many_packed(self, entries: list[tuple[int, CompressedBundle]]) -> None:
        segments = [s for _, bundle in entries for s in bundle.segments]
        payloads = [s.payload.view(torch.uint8).view(-1) for s in segments]
        layout = []
        total = 0
        for seg, pay in zip(segments, payloads):
            start = -(-total // self.ALIGNMENT) * self.ALIGNMENT
            end = start + int(pay.numel())
            layout.append((seg, pay, start, end))
            total = end
        try:
            slab = torch.empty(total, dtype=torch.uint8, pin_memory=True)
        except RuntimeError:
            slab = torch.empty(total, dtype=torch.uint8)
        on_one_gpu = bool(payloads) and all(
            p.is_cuda and p.device == payloads[0].device for p in payloads)
        if on_one_gpu:
            device = payloads[0].device
            if (self._gpu_pack_slab is None
                    or self._gpu_pack_slab.device != device
                    or self._gpu_pack_slab.numel() < total):
                self._gpu_pack_slab = torch.empty(total, dtype=torch.uint8,
                                                  device=device)
            packed = self._gpu_pack_slab[:total]
            if len(layout) == 1 and layout[0][2] == 0:
                packed.copy_(layout[0][1])
            else:
                pad = torch.empty(self.ALIGNMENT, dtype=torch.uint8, device=device)
                parts, cursor = [], 0
                for _, pay, start, end in layout:
                    if start > cursor:
                        parts.append(pad[:start - cursor])
                    parts.append(pay)
                    cursor = end
                torch.cat(parts, out=packed)
            slab.copy_(packed, non_blocking=True)
            torch.cuda.current_stream(device).synchronize()
        else:
            devices = set()
            for _, pay, start, end in layout:
                slab[start:end].copy_(pay, non_blocking=pay.is_cuda)
                if pay.is_cuda:
                    devices.add(pay.device)
            for device in devices:
                torch.cuda.current_stream(device).synchronize()
        for seg, _, start, end in layout:
            seg.payload = slab[start:end]
        with self._lock:
            for cpu_block_id, bundle in entries:
                self._pages[cpu_block_id] = bundle

    def get(self, cpu_block_id: int) -> CompressedBundle:
        with self._lock:
            bundle = self._pages.get(cpu_block_id)
        if bundle is None:
            raise KeyError(f"compressed bundle not found for CPU block {cpu_block_id}")
        return bundle


# ---- the codec-facing handler -------------------------------------------------

class KVPageCodec:
    """Batched cuSZp fixed-mode store/restore of KV pages, as the reference's
    ``CompressedOffloadingHandler`` drives it (codec ``"cuszp"``).

    ``compressors`` defaults to one ``CuSZpWrapper`` per cuSZp mode, built
    like the reference's (:540-553); any object with the same methods works
    (the host tests pass a recording stand-in)."""

    def __init__(self, kv_tensors: Sequence, error_bound: float = 1e-4,
                 device_id: int = 0,
                 layer_error_bounds: dict[int, float] | None = None,
                 flat_layer_prefix: int = 2, cuszp_mode: str = "fixed",
                 compressors: dict | None = None):
        if cuszp_mode not in CUSZP_MODES:
            raise ValueError(f"unsupported cuSZp encoding mode: {cuszp_mode}")
        self.kv_tensors = list(kv_tensors)
        self.error_bound = float(error_bound)
        self.device_id = int(device_id)
        self.layer_error_bounds = layer_error_bounds
        self.flat_layer_prefix = int(flat_layer_prefix)
        self.codec = "cuszp"
        self.cuszp_mode = cuszp_mode
        self._compression_output_slab: torch.Tensor | None = None
        self._layer_index_cache: dict[tuple[str, tuple[int, ...]], torch.Tensor] = {}
        if compressors is None:
            compressors = {}
            for mode, encoding_mode in CUSZP_MODES.items():
                cfg = cuszp_wrapper_cpp.CompressionConfig(
                    error_bound=self.error_bound, use_relative_error=True,
                    processing_dim=cuszp_wrapper_cpp.CuszpDim.DIM_1D,
                    encoding_mode=encoding_mode,
                    data_type=cuszp_wrapper_cpp.CuszpType.TYPE_FLOAT)
                compressors[mode] = cuszp_wrapper_cpp.CuSZpWrapper(cfg, self.device_id)
        self.compressors = compressors

    # -- helpers ---------------------------------------------------------------

    def page(self, tensor_idx: int, gpu_block_id: int) -> torch.Tensor:
        t = self.kv_tensors[tensor_idx]
        t = getattr(t, "tensor", t)
        return t[gpu_block_id]

    def layer_index(self, device: torch.device,
                    layer_indices: tuple[int, ...]) -> torch.Tensor:
        """Cached device index tensors (:555-564)."""
        key = (str(device), tuple(layer_indices))
        index = self._layer_index_cache.get(key)
        if index is None:
            index = torch.tensor(layer_indices, dtype=torch.long, device=device)
            self._layer_index_cache[key] = index
        return index

    def _output_slab(self, nbytes: int, device) -> torch.Tensor:
        slab = self._compression_output_slab
        if slab is None or slab.device != device or slab.numel() < nbytes:
            slab = torch.empty(nbytes, dtype=torch.uint8, device=device)
            self._compression_output_slab = slab
        return slab

    # -- store: uniform bound (vllm_v1_compressed_offload.py:825-1028) ---------

    def compress_fixed_bundles_batched(
            self, operations, active_bounds: dict[int, float] | None = None,
            active_mode: str = "fixed"):
        """Whole pages with one bound in one native call; MIN-pad small
        pages; keep a page raw when its stream is not smaller."""
        bounds = self.layer_error_bounds if active_bounds is None else active_bounds
        batch_bound = self.error_bound
        if bounds:
            layer_ids = sorted(bounds)
            if layer_ids != list(range(len(layer_ids))):
                return None
            distinct = {float(bounds[i]) for i in layer_ids}
            if len(distinct) != 1:
                return None
            batch_bound = next(iter(distinct))
        if (self.codec != "cuszp" or active_mode != "fixed" or batch_bound <= 0
                or len(operations) <= 1):
            return None
        compress = getattr(self.compressors["fixed"], "compress_batch_fixed_bf16", None)
        if compress is None:
            return None

        prepared = []
        common_numel = common_device = None
        for page_index, (tensor_indices, gpu_block_id, cpu_block_id) in enumerate(operations):
            components, pieces, raw_pieces, original_bytes = [], [], [], 0
            for tensor_idx in tensor_indices:
                storage = self.page(tensor_idx, gpu_block_id)
                source = _as_bf16(storage)
                selected = source.contiguous()
                if selected.dtype != torch.bfloat16:
                    return None
                pieces.append(selected.view(-1))
                raw_pieces.append(selected.view(torch.uint8).view(-1))
                components.append(BundleComponent(
                    tensor_idx=tensor_idx, original_shape=tuple(selected.shape),
                    original_dtype=source.dtype, numel=selected.numel(),
                    layer_axis=None, layer_indices=(),
                    destination_view_shape=tuple(source.shape)))
                original_bytes += selected.numel() * selected.element_size()
            unpadded = sum(c.numel for c in components)
            numeric = pieces[0] if len(pieces) == 1 else torch.cat(pieces).contiguous()
            if unpadded < MIN_CUSZP_ELEMENTS:
                numeric = torch.nn.functional.pad(
                    numeric, (0, MIN_CUSZP_ELEMENTS - unpadded)).contiguous()
            if common_numel is None:
                common_numel, common_device = numeric.numel(), numeric.device
            elif numeric.numel() != common_numel or numeric.device != common_device:
                return None
            capacity = cuszp_wrapper_cpp.CuSZpWrapper.estimate_compressed_buffer_size(
                numeric.numel() * 4)
            slab = self._output_slab(len(operations) * capacity, numeric.device)
            compressed = slab[page_index * capacity:(page_index + 1) * capacity]
            raw = raw_pieces[0] if len(raw_pieces) == 1 else torch.cat(raw_pieces).contiguous()
            prepared.append((cpu_block_id, tuple(components), numeric, compressed,
                             raw, unpadded, int(original_bytes)))

        ok, sizes, actual = compress([p[2] for p in prepared], [p[3] for p in prepared],
                                     [batch_bound] * len(prepared))
        if not ok or len(sizes) != len(prepared) or len(actual) != len(prepared):
            return None
        entries = []
        for (cpu_block_id, components, numeric, compressed, raw, unpadded,
             original_bytes), size, bound in zip(prepared, sizes, actual):
            size = int(size)
            if size <= 0 or size > compressed.numel():
                return None
            if size < original_bytes:
                seg = EncodedSegment(
                    payload=compressed[:size], compressed_size=size,
                    actual_error_bound=float(bound), encoding="cuszp",
                    components=components, unpadded_numel=unpadded,
                    compressed_numel=numeric.numel(), original_bytes=original_bytes,
                    requested_error_bound=batch_bound, cuszp_mode="fixed")
            else:  # raw fallback (:994-1005)
                seg = EncodedSegment(
                    payload=raw, compressed_size=original_bytes,
                    actual_error_bound=0.0, encoding="raw", components=components,
                    unpadded_numel=unpadded, compressed_numel=numeric.numel(),
                    original_bytes=original_bytes, requested_error_bound=batch_bound,
                    cuszp_mode=None)
            entries.append((cpu_block_id, _bundle([seg])))
        return entries

    # -- store: per-layer bounds (vllm_v1_compressed_offload.py:1286-1569) -----

    def compress_adaptive_fixed_bundles_indexed(
            self, operations, active_bounds: dict[int, float],
            active_mode: str = "fixed"):
        """Layers grouped by bound; each group of each page is one
        layer-indexed segment, all groups in one native call.  Bound <= 0
        keeps a group raw; any stream that is not smaller than its raw bytes
        sends the whole job back to the caller (returns None)."""
        if (self.codec != "cuszp" or active_mode != "fixed" or not active_bounds
                or len(operations) <= 1
                or any(len(ti) != 1 for ti, _, _ in operations)):
            return None
        compressor = self.compressors["fixed"]
        per_group = getattr(compressor, "compress_batch_fixed_bf16_indexed", None)
        if per_group is None:
            return None
        num_layers = len(active_bounds)
        prefix = self.flat_layer_prefix
        if num_layers <= 0 or prefix <= 0:
            return None
        grouped: dict[float, list[int]] = {}
        for layer in range(num_layers):
            grouped.setdefault(float(active_bounds.get(layer, self.error_bound)),
                               []).append(layer)
        if len(grouped) <= 1:
            return None
        groups = sorted(grouped.items())

        page_segments = [[None] * len(groups) for _ in operations]
        requests, cpu_ids = [], []
        epl = device = None
        for page_index, (tensor_indices, gpu_block_id, cpu_block_id) in enumerate(operations):
            cpu_ids.append(cpu_block_id)
            tensor_idx = tensor_indices[0]
            source = _as_bf16(self.page(tensor_idx, gpu_block_id))
            divisor = prefix * num_layers
            if (source.dtype != torch.bfloat16 or source.ndim != 1
                    or source.numel() % divisor):
                return None
            e = source.numel() // divisor
            if epl is None:
                epl, device = e, source.device
            elif e != epl or source.device != device:
                return None
            view = source.view(prefix, num_layers, e)
            for seg_index, (bound, layers) in enumerate(groups):
                layers = tuple(layers)
                numel = prefix * len(layers) * e
                component = BundleComponent(
                    tensor_idx=tensor_idx, original_shape=(prefix, len(layers), e),
                    original_dtype=source.dtype, numel=numel, layer_axis=1,
                    layer_indices=layers, destination_view_shape=tuple(view.shape))
                if bound <= 0:
                    index = self.layer_index(source.device, layers)
                    raw = view.index_select(1, index).contiguous().view(torch.uint8).view(-1)
                    nbytes = numel * source.element_size()
                    page_segments[page_index][seg_index] = EncodedSegment(
                        payload=raw, compressed_size=nbytes, actual_error_bound=0.0,
                        encoding="raw", components=(component,), unpadded_numel=numel,
                        compressed_numel=numel, original_bytes=nbytes,
                        requested_error_bound=bound)
                    continue
                if numel < MIN_CUSZP_ELEMENTS:
                    return None
                requests.append(dict(
                    page_index=page_index, segment_index=seg_index, bound=bound,
                    source=source.contiguous(), selected_layers=layers,
                    selected_index=self.layer_index(source.device, layers),
                    component=component, selected_numel=numel,
                    original_bytes=numel * source.element_size(),
                    capacity=cuszp_wrapper_cpp.CuSZpWrapper.estimate_compressed_buffer_size(
                        numel * 4)))
        if not requests:
            return None
        slab = self._output_slab(sum(r["capacity"] for r in requests), device)
        offset = 0
        request_groups: dict[tuple, list[dict]] = {}
        for r in requests:
            r["compressed"] = slab[offset:offset + r["capacity"]]
            offset += r["capacity"]
            request_groups.setdefault((r["bound"], r["selected_layers"]), []).append(r)
        grouped_requests = list(request_groups.values())

        results = []
        grouped_call = getattr(compressor, "compress_batch_fixed_bf16_indexed_groups", None)
        if grouped_call is not None and len(grouped_requests) > 1:
            flat = [r for rs in grouped_requests for r in rs]
            ok, sizes, actual = grouped_call(
                [r["source"] for r in flat], [r["compressed"] for r in flat],
                [rs[0]["selected_index"] for rs in grouped_requests],
                [len(rs) for rs in grouped_requests], prefix, num_layers, epl,
                [r["bound"] for r in flat])
            if ok and len(sizes) == len(flat) and len(actual) == len(flat):
                results.append((flat, sizes, actual))
        if not results:
            for rs in grouped_requests:
                ok, sizes, actual = per_group(
                    [r["source"] for r in rs], [r["compressed"] for r in rs],
                    rs[0]["selected_index"], prefix, num_layers, epl,
                    [r["bound"] for r in rs])
                if not ok or len(sizes) != len(rs) or len(actual) != len(rs):
                    return None
                results.append((rs, sizes, actual))
        for rs, sizes, actual in results:
            for r, size, bound in zip(rs, sizes, actual):
                size = int(size)
                if size <= 0 or size > r["compressed"].numel() or size >= r["original_bytes"]:
                    return None
                page_segments[r["page_index"]][r["segment_index"]] = EncodedSegment(
                    payload=r["compressed"][:size], compressed_size=size,
                    actual_error_bound=float(bound), encoding="cuszp",
                    components=(r["component"],), unpadded_numel=r["selected_numel"],
                    compressed_numel=r["selected_numel"],
                    original_bytes=r["original_bytes"], requested_error_bound=r["bound"],
                    cuszp_mode="fixed")
        entries = []
        for cpu_block_id, segs in zip(cpu_ids, page_segments):
            if any(s is None for s in segs):
                return None
            entries.append((cpu_block_id, _bundle(segs)))
        return entries

    # -- restore (vllm_v1_compressed_offload.py:1578-2184) ---------------------

    def restore_raw_direct_batched(self, items) -> RestoreStageTimings:
        """Raw whole-component segments copied straight into their pages."""
        for gpu_block_id, segment in items:
            offset = 0
            for c in segment.components:
                dst = self.page(c.tensor_idx, gpu_block_id).view(
                    c.original_dtype).view(c.destination_view_shape)
                if c.layer_axis is not None or tuple(dst.shape) != c.original_shape:
                    raise ValueError("raw direct destination is not a complete KV component")
                end = offset + c.numel * dst.element_size()
                src = segment.payload[offset:end].view(c.original_dtype).view(c.original_shape)
                dst.copy_(src, non_blocking=True)
                offset = end
            if offset != segment.compressed_size:
                raise RuntimeError("raw direct metadata does not cover the payload")
        return RestoreStageTimings()

    def decompress_bundles_batched(self, bundles) -> RestoreStageTimings:
        """Restores a job: raw whole components by direct copy; every other
        segment's payload is copied to the GPU in one packed transfer, then
        cuSZp segments are decoded in batches (:1618-1711)."""
        timings = RestoreStageTimings()
        direct, raw_direct = [], []
        for gpu_block_id, bundle in bundles:
            for seg in bundle.segments:
                if seg.encoding == "raw" and all(c.layer_axis is None for c in seg.components):
                    raw_direct.append((gpu_block_id, seg))
                elif seg.encoding in ("cuszp", "raw"):
                    direct.append((gpu_block_id, seg))
                else:
                    raise ValueError(f"encoding {seg.encoding!r} is not part of this codec")
        if raw_direct:
            timings.add(self.restore_raw_direct_batched(raw_direct))
        prefetched = []
        if direct:
            device = self.page(direct[0][1].components[0].tensor_idx, direct[0][0]).device
            payloads = [seg.payload for _, seg in direct]
            total = sum(int(p.numel()) for p in payloads)
            packed = torch.empty(total, dtype=torch.uint8, device=device)
            first = payloads[0]
            contiguous = True
            ptr, expect = first.untyped_storage().data_ptr(), first.storage_offset()
            for p in payloads:
                if p.untyped_storage().data_ptr() != ptr or p.storage_offset() != expect:
                    contiguous = False
                    break
                expect += p.numel()
            if contiguous:
                packed.copy_(first.as_strided((total,), (1,), first.storage_offset()),
                             non_blocking=True)
            offset = 0
            for (gpu_block_id, seg), p in zip(direct, payloads):
                view = packed[offset:offset + p.numel()]
                if not contiguous:
                    view.copy_(p, non_blocking=True)
                prefetched.append((gpu_block_id, seg, view))
                offset += p.numel()
        cuszp = [it for it in prefetched if it[1].encoding == "cuszp"]
        if cuszp:
            timings.add(self.decode_cuszp_prefetched_batched(cuszp))
        for gpu_block_id, seg, payload_gpu in prefetched:
            if seg.encoding != "cuszp":
                timings.add(self.decode_segment(gpu_block_id, seg, payload_gpu))
        return timings

    def fixed_bf16_indexed_destinations(self, items):
        """Full destination pages plus the shared layer index, when every
        segment is the same layer-indexed BF16 component (:1713-1773)."""
        first = items[0][1]
        if len(first.components) != 1:
            return None
        c0 = first.components[0]
        layers = c0.layer_indices
        if (c0.layer_axis != 1 or c0.original_dtype != torch.bfloat16 or not layers
                or len(c0.destination_view_shape) != 3):
            return None
        prefix, src_layers, epl = c0.destination_view_shape
        expected = (prefix, len(layers), epl)
        outputs = []
        for gpu_block_id, seg, _ in items:
            if len(seg.components) != 1 or seg.unpadded_numel != seg.compressed_numel:
                return None
            c = seg.components[0]
            if (c.layer_axis != 1 or c.original_dtype != torch.bfloat16
                    or c.layer_indices != layers
                    or c.destination_view_shape != c0.destination_view_shape
                    or c.original_shape != expected):
                return None
            dst = self.page(c.tensor_idx, gpu_block_id).view(torch.uint8).view(
                torch.bfloat16).view(-1)
            if not dst.is_contiguous() or dst.numel() < prefix * src_layers * epl:
                return None
            outputs.append(dst)
        return outputs, self.layer_index(outputs[0].device, layers), prefix, src_layers, epl

    def fixed_bf16_direct_destinations(self, items):
        """Whole-component destinations of equal size (:1775-1812)."""
        count = len(items[0][1].components)
        if count == 0:
            return None
        per = items[0][1].components[0].numel
        dests = []
        for gpu_block_id, seg, _ in items:
            if (len(seg.components) != count or seg.unpadded_numel != seg.compressed_numel
                    or seg.compressed_numel != count * per):
                return None
            for c in seg.components:
                if (c.layer_axis is not None or c.original_dtype != torch.bfloat16
                        or c.numel != per):
                    return None
                dst = self.page(c.tensor_idx, gpu_block_id).view(
                    c.original_dtype).view(c.destination_view_shape)
                if tuple(dst.shape) != c.original_shape or not dst.is_contiguous():
                    return None
                dests.append(dst.view(-1))
        return dests, count, per

    def decode_cuszp_prefetched_batched(self, prefetched) -> RestoreStageTimings:
        """Batches of compatible segments: indexed scatter into full pages,
        else direct scatter, else contiguous staging plus per-segment scatter
        (:1815-2006)."""
        timings = RestoreStageTimings()
        grouped: dict[tuple, list] = {}
        for item in prefetched:
            seg = item[1]
            mode = seg.cuszp_mode or self.cuszp_mode
            if mode == "fixed":
                layout = tuple((c.tensor_idx, c.original_shape, c.original_dtype, c.numel,
                                c.layer_axis, c.layer_indices, c.destination_view_shape)
                               for c in seg.components)
                key = (mode, seg.compressed_numel, seg.unpadded_numel, layout)
            else:
                key = (mode,)
            grouped.setdefault(key, []).append(item)
        # Layer groups that scatter into full pages with the same page shape
        # are restored by one grouped launch (the reference issues one
        # indexed-scatter call per group; the values written are the same).
        indexed = []
        for key, items in grouped.items():
            mode = str(key[0])
            compressor = self.compressors.get(mode)
            if compressor is None:
                raise ValueError(f"unknown cuSZp mode in segment: {mode}")
            dtypes = {c.original_dtype for _, s, _ in items for c in s.components}
            numels = {s.compressed_numel for _, s, _ in items}
            if not (mode == "fixed" and dtypes == {torch.bfloat16} and len(numels) == 1):
                raise ValueError("only BF16 fixed-mode cuSZp segments are decodable here")
            started = time.perf_counter()
            idx = self.fixed_bf16_indexed_destinations(items)
            if idx is not None:
                indexed.append((compressor, items, idx))
                timings.gpu_decode_seconds += time.perf_counter() - started
                continue
            direct = self.fixed_bf16_direct_destinations(items)
            if direct is not None:
                outputs, per_page, per_output = direct
                ok = compressor.decompress_batch_fixed_bf16_scatter(
                    [it[2] for it in items], [it[1].compressed_size for it in items],
                    outputs, next(iter(numels)), per_page, per_output,
                    [it[1].actual_error_bound for it in items])
                timings.gpu_decode_seconds += time.perf_counter() - started
                if not ok:
                    raise RuntimeError("cuSZp failed to direct-scatter a KV batch")
                continue
            total = sum(s.compressed_numel for _, s, _ in items)
            storage = torch.empty(total, dtype=torch.bfloat16, device=items[0][2].device)
            ok = compressor.decompress_batch_fixed_bf16(
                [it[2] for it in items], [it[1].compressed_size for it in items],
                storage, next(iter(numels)), [it[1].actual_error_bound for it in items])
            timings.gpu_decode_seconds += time.perf_counter() - started
            if not ok:
                raise RuntimeError("cuSZp failed to decompress a KV batch")
            offset = 0
            for gpu_block_id, seg, payload_gpu in items:
                restored = storage[offset:offset + seg.compressed_numel]
                offset += seg.compressed_numel
                timings.add(self.decode_segment(gpu_block_id, seg, payload_gpu, restored))
        if indexed:
            started = time.perf_counter()
            self.restore_indexed_groups(indexed)
            timings.gpu_decode_seconds += time.perf_counter() - started
        return timings

    @staticmethod
    def restore_indexed_groups(indexed) -> None:
        """Indexed-scatter restores: one launch for all groups sharing the
        compressor and page geometry (prefix, source layers, elements per
        layer), else one call per group as in :1899-1908."""
        by_shape: dict[tuple, list] = {}
        for compressor, items, idx in indexed:
            _, _, prefix, src_layers, epl = idx
            by_shape.setdefault((id(compressor), prefix, src_layers, epl), []).append(
                (compressor, items, idx))
        for (_, prefix, src_layers, epl), groups in by_shape.items():
            compressor = groups[0][0]
            streams, sizes, outputs, bounds, indices, counts = [], [], [], [], [], []
            for _, items, idx in groups:
                streams += [it[2] for it in items]
                sizes += [it[1].compressed_size for it in items]
                bounds += [it[1].actual_error_bound for it in items]
                outputs += idx[0]
                indices.append(idx[1])
                counts.append(len(items))
            if len(groups) == 1:
                ok = compressor.decompress_batch_fixed_bf16_indexed_scatter(
                    streams, sizes, outputs, indices[0], prefix, src_layers, epl, bounds)
            else:
                ok = compressor.decompress_batch_fixed_bf16_indexed_scatter_groups(
                    streams, sizes, outputs, indices, counts, prefix, src_layers, epl, bounds)
            if not ok:
                raise RuntimeError("cuSZp failed to indexed-scatter a KV batch")

    def decode_segment(self, gpu_block_id: int, segment: EncodedSegment,
                       payload_gpu: torch.Tensor,
                       restored: torch.Tensor | None = None) -> RestoreStageTimings:
        """Scatters one segment into its pages: raw payload bytes, or the
        values a batched decode left in ``restored`` (:2021-2184)."""
        if segment.encoding == "raw":
            offset = 0
            for c in segment.components:
                dst = self.page(c.tensor_idx, gpu_block_id).view(
                    c.original_dtype).view(c.destination_view_shape)
                end = offset + c.numel * dst.element_size()
                src = payload_gpu[offset:end].view(c.original_dtype).view(c.original_shape)
                if c.layer_axis is None:
                    dst.copy_(src)
                else:
                    dst.index_copy_(c.layer_axis, self.layer_index(dst.device, c.layer_indices), src)
                offset = end
            if offset != segment.compressed_size:
                raise RuntimeError("raw bundle metadata does not cover the payload")
            return RestoreStageTimings()
        if segment.encoding != "cuszp":
            raise ValueError(f"unknown KV bundle encoding: {segment.encoding}")
        if restored is None or restored.numel() != segment.compressed_numel:
            raise ValueError("cuSZp segments are restored through the batched decoder")
        offset = 0
        for c in segment.components:
            dst = self.page(c.tensor_idx, gpu_block_id).view(
                c.original_dtype).view(c.destination_view_shape)
            if c.layer_axis is None:
                ok = tuple(dst.shape) == c.original_shape
            else:
                shape = list(dst.shape)
                shape[c.layer_axis] = len(c.layer_indices)
                ok = tuple(shape) == c.original_shape
            if not ok:
                raise ValueError("destination KV page shape changed since offload")
            end = offset + c.numel
            vals = restored[offset:end].view(c.original_shape).to(c.original_dtype)
            if c.layer_axis is None:
                dst.copy_(vals)
            else:
                dst.index_copy_(c.layer_axis, self.layer_index(dst.device, c.layer_indices), vals)
            offset = end
        if offset != segment.unpadded_numel:
            raise RuntimeError("compressed bundle metadata does not cover the payload")
        return RestoreStageTimings()
