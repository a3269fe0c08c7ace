#!/usr/bin/env python3
"""Benchmark: batched fixed-mode BF16 KV-page store + restore on one MI355X.

Metric: KV compress/decompress GB/s of BF16 input, % of HBM
peak, compression ratio.  One step is what the reference's connector does
for one transfer job (vllm_v1_compressed_offload.py:825-1028 / 1286-1569 for
the store, :1815-2006 for the restore), through the C ABI (libkvszp.so) with
every pointer table built once and the pages resident in HBM:

  --config 1 (default; the metric's configuration): the full Qwen2.5-1.5B
      4K-context KV cache, 256 vLLM pages of [2, 28, 16, 2, 128] BF16, layers
      {0,1,2,5,19,20,21} at REL 1e-5 and the other 21 at 1e-4:
      store   = one compress_batch_fixed_bf16_indexed_groups call over all
                512 (page, layer group) requests (blocking: sizes come back)
      restore = one decompress_batch_fixed_bf16_indexed_scatter_groups launch
                into fresh pages (--restore-per-group: the reference's one
                indexed_scatter call per group)
  --config 0: one layer's K and V (2 pages of 1 048 576), REL 1e-4, uniform
      store + contiguous restore
  --config 2: 8192 pages of a 16 x 8192-token pool in page-table order,
      REL 1e-4, uniform store + restore into permuted fresh slots
  --config 3: Qwen2.5-7B 32K (2048 pages of 458 752, RoPE-like K), REL 1e-5,
      uniform store + restore into permuted fresh slots
  --config 4: Llama-3-8B 64K stress pages (4096 pages of 1 048 576: zero,
      constant, heavy-tailed, Gaussian), per-layer REL 1e-4/1e-5 alternating:
      grouped indexed store + grouped restore

Reported (one JSON line):
  value            BF16 bytes of the job / wall time per step (store+restore)
                   over K timed steps (per-step wall times in step_ms).  Each step uses the next of --rotate
                   buffer sets (pages, streams, destinations), so that a step
                   re-reads nothing the 256 MB Infinity Cache still holds from
                   the step before (default 3 sets for configs 0 and 1, whose
                   working set is below 256 MB; the other configs exceed it).
                   value_mall_warm: the same steps on one buffer set.
  kernel times     per-launch durations from HIP events recorded by the
                   library on the launch stream: mean, min, median.
  roofline         the encoder (dominant kernel): algorithmic bytes per launch
                   (2N read + S written per segment) / mean launch duration,
                   against 8 TB/s; traffic = FETCH_SIZE + WRITE_SIZE bytes per
                   launch from rocprofv3 (profiles/traffic_*.json, used only
                   while the kernel source it was measured on is unchanged).
  pcie             config 1 with the link: store = encode + kvszp_pack_streams
                   into a pinned host slab, restore = one host-to-device copy
                   + grouped decode (the reference's packed store and restore)
  ratio            BF16 bytes / stream bytes of the step; ratio_uniform_1e-4:
                   config 1's pages at a uniform REL 1e-4 (the metric's eb)
  cpu_baseline     the scalar CPU oracle (C, -O2) on a sample of the same
                   pages, store + restore, all host cores; one_core beside it;
                   cpu_host_codecs: the reference's host codecs (zstd-1, LZ4,
                   INT8), one core and all cores
"""

from __future__ import annotations

import argparse
import ctypes
import gc
import hashlib
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(
    REPO,
    "reducing-pcie-bottlenecks-for-llm-serving-with-cuszp-compressed-kv-cache-transfer_amd")
sys.path.insert(0, PKG)

METRIC = "KV compress/decompress GB/s (BF16 in), % of HBM peak, ratio at eb=1e-4"
HBM_PEAK_GBPS = 8000.0
# The device code: the kernels and the headers they include.
KERNELS_SRC = [os.path.join(PKG, "csrc", f) for f in
               ("kvszp_kernels.hip", "kvszp_internal.h", "kvszp_plan.h", "kvszp_bits.h")]


def traffic_file(config: int) -> str:
    name = {1: "qwen15b_4k_store_restore"}.get(config, f"config{config}")
    return os.path.join(REPO, "profiles", f"traffic_{name}.json")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def kernels_sha() -> str:
    h = hashlib.sha256()
    for path in KERNELS_SRC:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


# ---- workloads -------------------------------------------------------------------

class Workload:
    """Pages, stream slabs and destinations of one configuration, `sets`
    copies at distinct addresses; pointer tables built once per set."""

    grouped = False

    def __init__(self, config: int, seed: int, sets: int):
        import kvszp
        import torch

        self.k = kvszp
        self.torch = torch
        self.config = config
        self.build(seed)
        self.num_pages, self.page_numel = self.pages.shape
        cfg = kvszp.Config(1e-4, 1, kvszp.DIM_1D, kvszp.MODE_FIXED, kvszp.TYPE_FLOAT)
        self.ctx = kvszp.Context(cfg, 0)
        self.stream = torch.cuda.current_stream().cuda_stream
        self.sets = [self.make_set(s) for s in range(sets)]

    # requests: self.req_pages[i] (index of the input page), self.req_eps[i],
    # self.req_n[i] (logical values); set up by build()

    def make_set(self, s: int) -> dict:
        torch, k = self.torch, self.k
        pages = self.pages if s == 0 else self.pages.clone()
        caps = [8 * n for n in self.req_n]
        slab = torch.empty(sum(caps), dtype=torch.uint8, device="cuda")
        offs, o = [], 0
        for c in caps:
            offs.append(o)
            o += c
        base = slab.data_ptr()
        st = {
            "pages": pages, "slab": slab,
            "dest": torch.zeros_like(self.dest_template()),
            "inputs": k.ptr_array([pages[p].data_ptr() for p in self.req_pages]),
            "outputs": k.ptr_array([base + x for x in offs]),
            "stream_ptrs": [base + x for x in offs],
            "caps": k.u64_array(caps),
            "eps": k.f32_array(self.req_eps),
            "sizes": (ctypes.c_uint64 * len(caps))(),
            "bounds": (ctypes.c_float * len(caps))(),
        }
        st["stream_table"] = k.ptr_array(st["stream_ptrs"])
        self.make_restore_tables(st)
        return st

    def dest_template(self):
        return self.pages

    @property
    def batch(self) -> int:
        return len(self.req_n)

    @property
    def bf16_bytes(self) -> int:
        return 2 * sum(self.req_n)

    def stream_bytes(self, s: int = 0) -> int:
        st = self.sets[s]
        return int(sum(st["sizes"][i] for i in range(self.batch)))

    def step(self, s: int) -> None:
        self.store(s)
        self.restore(s)


class Grouped(Workload):
    """Configs 1 and 4: layer groups by bound, one grouped indexed store and
    one grouped indexed restore."""

    grouped = True

    def __init__(self, config, seed, sets, per_group_restore=False):
        self.per_group_restore = per_group_restore
        super().__init__(config, seed, sets)

    def build(self, seed):
        import kv_synth

        torch = self.torch
        if self.config == 1:
            self.shape = kv_synth.QWEN25_1P5B_4K
            self.pages = kv_synth.paged_kv(self.shape, seed=seed, device="cuda")
            self.groups = kv_synth.mixed_bound_groups()
            self.name = ("qwen2.5-1.5b 4k store+restore (configs[1]): 256 pages x "
                         "[2,28,16,2,128] bf16, layers {0,1,2,5,19,20,21} REL 1e-5 + "
                         "21 layers REL 1e-4, indexed_groups compress + "
                         "indexed_scatter_groups restore")
        else:
            self.shape = kv_synth.LLAMA3_8B_64K
            self.pages, self.classes = kv_synth.stress_pages(self.shape, seed=seed,
                                                             device="cuda")
            self.groups = kv_synth.alternating_bound_groups(self.shape.layers)
            self.name = ("llama-3-8b 64k stress pages (configs[4]): 4096 pages x "
                         "[2,32,16,8,128] bf16, per-layer REL 1e-4/1e-5 alternating, "
                         "indexed_groups compress + indexed_scatter_groups restore")
        self.epl = self.shape.elements_per_layer
        npages = self.pages.shape[0]
        self.req_pages, self.req_eps, self.req_n = [], [], []
        for bound, layers in self.groups:
            for p in range(npages):
                self.req_pages.append(p)
                self.req_eps.append(bound)
                self.req_n.append(2 * len(layers) * self.epl)
        self.layer_idx = [torch.tensor(ls, dtype=torch.long, device="cuda")
                          for _, ls in self.groups]
        k = __import__("kvszp")
        self.idx_ptrs = k.ptr_array([t.data_ptr() for t in self.layer_idx])
        self.sel = k.size_array([len(ls) for _, ls in self.groups])
        self.group_sizes = k.size_array([npages] * len(self.groups))

    def make_restore_tables(self, st):
        k = self.k
        dest_ptrs = [st["dest"][p].data_ptr() for p in range(self.num_pages)]
        st["dest_table"] = k.ptr_array(dest_ptrs * len(self.groups))
        st["per_group"] = []
        for g in range(len(self.groups)):
            lo, hi = g * self.num_pages, (g + 1) * self.num_pages
            st["per_group"].append((
                k.ptr_array(st["stream_ptrs"][lo:hi]),
                (ctypes.c_uint64 * (hi - lo)).from_buffer(st["sizes"], lo * 8),
                (ctypes.c_float * (hi - lo)).from_buffer(st["bounds"], lo * 4),
                hi - lo, k.ptr_array(dest_ptrs), self.layer_idx[g].data_ptr(),
                len(self.groups[g][1])))

    def store(self, s):
        st = self.sets[s]
        self.k.check(self.ctx.compress_indexed_groups(
            st["inputs"], st["outputs"], st["caps"], self.idx_ptrs, self.sel,
            self.group_sizes, len(self.groups), 2, self.shape.layers, self.epl,
            st["eps"], self.batch, self.stream, st["sizes"], st["bounds"]))

    def restore(self, s):
        st = self.sets[s]
        if self.per_group_restore:
            for comp, sizes, bounds, cnt, dests, idx, sel in st["per_group"]:
                self.k.check(self.ctx.decompress_indexed_scatter(
                    comp, sizes, bounds, cnt, dests, idx, sel, 2,
                    self.shape.layers, self.epl, self.stream))
            return
        self.k.check(self.ctx.decompress_indexed_scatter_groups(
            st["stream_table"], st["sizes"], st["bounds"], self.batch,
            st["dest_table"], self.idx_ptrs, self.sel, self.group_sizes,
            len(self.groups), 2, self.shape.layers, self.epl, self.stream))

    def verify(self) -> dict:
        """Restored values within 2*eb of the input on every element of the
        restored layers (the reference's BF16 tolerance, tests :457, :639).
        Constant pages (config 4) saturate the quantizer under a relative
        bound (eb = eps * 1e-6) and are left out: the connector stores them
        raw (vllm_v1_compressed_offload.py:994-1005)."""
        torch = self.torch
        st = self.sets[0]
        err = (st["dest"].float() - self.pages.float()).abs().view(
            self.num_pages, 2, self.shape.layers, self.epl)
        keep = torch.tensor([c != "constant" for c in getattr(
            self, "classes", ["gaussian"] * self.num_pages)], device="cuda")
        worst = 0.0
        for g, (_, layers) in enumerate(self.groups):
            lo = g * self.num_pages
            eb = torch.tensor([st["bounds"][lo + p] for p in range(self.num_pages)],
                              device="cuda")
            e = err[:, :, list(layers)].amax(dim=(1, 2, 3))
            finite = torch.isfinite(e) & keep
            worst = max(worst, float((e[finite] / (2 * eb[finite] + 1e-30)).max()))
        return {"max_err_over_2eb": worst, "ok": worst <= 1.0}


class Uniform(Workload):
    """Configs 0, 2, 3: one bound for all pages, compress_batch_fixed_bf16,
    restore contiguous (config 0) or into permuted fresh page slots."""

    def build(self, seed):
        import kv_synth

        torch = self.torch
        g = torch.Generator().manual_seed(seed + 17)
        if self.config == 0:
            shape = kv_synth.QWEN25_1P5B_4K
            kk, vv = kv_synth.layer_kv(shape, layer=0, seed=seed, device="cuda")
            self.pages = torch.stack([kk.reshape(-1), vv.reshape(-1)])
            self.eps, self.slots = 1e-4, None
            self.name = ("qwen2.5-1.5b single layer (configs[0]): K and V [4096,2,128] "
                         "bf16 as 2 pages, REL 1e-4, compress_batch_fixed_bf16 + "
                         "decompress_batch_fixed_bf16")
        elif self.config == 2:
            shape = kv_synth.QWEN25_1P5B_4K
            pool = kv_synth.paged_kv(shape, seed=seed, device="cuda", tokens=16 * 8192)
            order = torch.randperm(pool.shape[0], generator=g)
            self.pool, self.order = pool, order
            self.pages = pool
            self.eps = 1e-4
            self.slots = torch.randperm(pool.shape[0], generator=g).tolist()
            self.name = ("qwen2.5-1.5b 16x8k pool (configs[2]): 8192 pages x "
                         "[2,28,16,2,128] bf16 in page-table order, REL 1e-4, "
                         "compress_batch_fixed_bf16 + scatter restore to permuted slots")
        else:
            shape = kv_synth.QWEN25_7B_32K
            self.pages = kv_synth.rope_kv(shape, seed=seed, device="cuda")
            self.eps = 1e-5
            self.slots = torch.randperm(self.pages.shape[0], generator=g).tolist()
            self.name = ("qwen2.5-7b 32k (configs[3]): 2048 pages x [2,28,16,4,128] "
                         "bf16, RoPE-like K, REL 1e-5, compress_batch_fixed_bf16 + "
                         "scatter restore to permuted slots")
        npages, n = self.pages.shape
        if self.config == 2:
            self.req_pages = self.order.tolist()
        else:
            self.req_pages = list(range(npages))
        self.req_eps = [self.eps] * npages
        self.req_n = [n] * npages

    def make_restore_tables(self, st):
        k = self.k
        if self.slots is None:
            return
        st["slot_table"] = k.ptr_array([st["dest"][s].data_ptr() for s in self.slots])

    def store(self, s):
        st = self.sets[s]
        self.k.check(self.ctx.compress(
            st["inputs"], st["outputs"], st["caps"], st["eps"], self.batch,
            self.page_numel, self.stream, st["sizes"], st["bounds"]))

    def restore(self, s):
        st = self.sets[s]
        if self.slots is None:
            self.k.check(self.ctx.decompress(
                st["stream_table"], st["sizes"], st["bounds"], self.batch,
                st["dest"].data_ptr(), st["dest"].numel(), self.page_numel,
                self.stream))
            return
        self.k.check(self.ctx.decompress_scatter(
            st["stream_table"], st["sizes"], st["bounds"], self.batch,
            st["slot_table"], self.page_numel, 1, self.page_numel, self.stream))

    def verify(self) -> dict:
        torch = self.torch
        st = self.sets[0]
        src = self.pages[self.req_pages] if self.config == 2 else self.pages
        out = st["dest"] if self.slots is None else st["dest"][self.slots]
        e = (out.float() - src.float()).abs().amax(dim=1)
        eb = torch.tensor([st["bounds"][i] for i in range(self.batch)], device="cuda")
        finite = torch.isfinite(e)
        worst = float((e[finite] / (2 * eb[finite] + 1e-30)).max())
        return {"max_err_over_2eb": worst, "ok": worst <= 1.0}


def make_workload(config: int, seed: int, sets: int, per_group_restore: bool):
    if config in (1, 4):
        return Grouped(config, seed, sets, per_group_restore)
    return Uniform(config, seed, sets)


# ---- measurement --------------------------------------------------------------------

def kernel_stats(ms: list) -> dict:
    if not ms:
        return {}
    return {"mean_ms": round(statistics.fmean(ms), 5), "min_ms": round(min(ms), 5),
            "median_ms": round(statistics.median(ms), 5), "launches": len(ms)}


def timed_steps(w: Workload, steps: int, sets: int) -> dict:
    """K steps over `sets` buffer sets: wall time, then the encoder's and the
    decoder's per-launch durations (each from its own pass of K steps; an
    event pair costs a little GPU time, so only one kind is timed at once).

    Each step's own wall time is kept too (from the end of the step before,
    so the per-step times add up to the whole pass): the store blocks until
    its sizes are on the host, and the restore is enqueued behind it, so a
    step ends with its restore still queued and the next step's store waits
    for it."""
    torch, k = w.torch, w.k
    torch.cuda.synchronize()
    w.ctx.enable_timing(0)
    marks = [time.perf_counter()]
    for i in range(steps):
        w.step(i % sets)
        marks.append(time.perf_counter())
    torch.cuda.synchronize()
    end = time.perf_counter()
    wall = end - marks[0]
    per = [(b - a) * 1e3 for a, b in zip(marks, marks[1:])]
    if per:
        per[-1] += (end - marks[-1]) * 1e3  # the last restore's drain
    out = {"ms_per_step": wall / steps * 1e3,
           "step_ms": {"mean": round(statistics.fmean(per), 4) if per else 0.0,
                       "median": round(statistics.median(per), 4) if per else 0.0,
                       "min": round(min(per), 4) if per else 0.0,
                       "max": round(max(per), 4) if per else 0.0,
                       "first": round(per[0], 4) if per else 0.0}}
    if os.environ.get("KVSZP_BENCH_STEP_LOG"):
        log("step ms: " + " ".join(f"{x:.4f}" for x in per))
    for kind, key in ((k.KERNEL_COMPRESS, "compress"), (k.KERNEL_DECOMPRESS, "decompress")):
        w.ctx.timing_durations(kind)
        w.ctx.enable_timing(1 << kind)
        for i in range(steps):
            w.step(i % sets)
        torch.cuda.synchronize()
        w.ctx.enable_timing(0)
        ms = w.ctx.timing_durations(kind)
        if os.environ.get("KVSZP_BENCH_STEP_LOG"):
            log(f"{key} us: " + " ".join(f"{x * 1e3:.1f}" for x in ms))
        per_step = len(ms) // steps if steps else 0
        out[key] = kernel_stats(ms)
        out[key]["launches_per_step"] = per_step
        # a step's kernel time (several launches per step: one per 16 groups)
        out[key]["ms_per_step"] = sum(ms) / steps if steps else 0.0
    return out


def pcie_steps(w: Grouped, steps: int) -> dict:
    """Config 1 across the link: store = encode + publication of the packed
    slab in pinned host memory (blocking, like put_many_packed), restore =
    the grouped decode of that slab; `steps` steps on buffer set 0 for each
    combination of the two store and the two restore modes.

    Store modes: "link" = the pack kernel writes the slab across the link;
    "staged" = it packs into device memory and one DMA copy moves the slab.
    Restore modes: "link" = the decoder reads the pinned slab itself;
    "staged" = one DMA copy into device memory, then the decode."""
    torch, k = w.torch, w.k
    st = w.sets[0]
    w.store(0)
    sizes = [st["sizes"][i] for i in range(w.batch)]
    cap = sum(sizes) + 8 * w.batch + (64 << 20)
    slab = torch.empty(cap, dtype=torch.uint8).pin_memory()
    staging = torch.empty(cap, dtype=torch.uint8, device="cuda")
    offsets = (ctypes.c_uint64 * w.batch)()
    packed = ctypes.c_uint64()
    lens = (ctypes.c_uint64 * w.batch)()
    b = w.bf16_bytes
    out = {"packed_bytes": 0, "steps": steps}
    best = None
    for smode in ("link", "staged"):
        for rmode in ("link", "staged"):
            t_store = t_restore = 0.0
            torch.cuda.synchronize()
            for it in range(steps + 3):  # 3 untimed steps per combination first
                if it == 3:
                    t_store = t_restore = 0.0
                t0 = time.perf_counter()
                w.store(0)
                for i in range(w.batch):
                    lens[i] = st["sizes"][i]
                if smode == "link":
                    k.check(w.ctx.pack(st["stream_table"], lens, w.batch, slab.data_ptr(),
                                       cap, w.stream, offsets, ctypes.byref(packed)))
                else:
                    k.check(w.ctx.pack(st["stream_table"], lens, w.batch,
                                       staging.data_ptr(), cap, w.stream, offsets,
                                       ctypes.byref(packed)))
                    slab[:packed.value].copy_(staging[:packed.value])
                    torch.cuda.synchronize()
                t1 = time.perf_counter()
                k.check(w.ctx.decompress_indexed_scatter_groups_packed(
                    slab.data_ptr(), packed.value,
                    staging.data_ptr() if rmode == "staged" else None, cap, offsets, lens,
                    st["bounds"], w.batch, st["dest_table"], w.idx_ptrs, w.sel,
                    w.group_sizes, len(w.groups), 2, w.shape.layers, w.epl, w.stream))
                torch.cuda.synchronize()
                t2 = time.perf_counter()
                t_store += t1 - t0
                t_restore += t2 - t1
            out["packed_bytes"] = int(packed.value)
            key = f"{smode}_store_{rmode}_restore"
            out[key] = {
                "store_restore_gbps": round(b * steps / (t_store + t_restore) / 1e9, 2),
                "store_gbps": round(b * steps / t_store / 1e9, 2),
                "restore_gbps": round(b * steps / t_restore / 1e9, 2),
                "ms_per_step": round((t_store + t_restore) / steps * 1e3, 4),
                "link_gbps": round(2 * packed.value * steps / (t_store + t_restore) / 1e9, 2)}
            if best is None or out[key]["store_restore_gbps"] > out[best]["store_restore_gbps"]:
                best = key
    out["store_restore_gbps"] = out[best]["store_restore_gbps"]
    out["best_modes"] = best
    return out


def contended_store(w: Workload, calls: int = 16) -> dict:
    """The store beside a busy stream: three BF16 products of 8192 x 8192
    matrices queued on a second stream hold the CUs while the store runs on
    the current stream, as the connector's store thread runs beside the
    model's kernels (vllm_v1_compressed_offload.py:2365-2385).

    Each call is classed by what the library did: "persistent" (the
    persistent encoder ran through), "gave_up" (a bounded wait gave up and
    the call was encoded again with the schedule that needs no residency),
    "safe" (a recent give-up sent the call to that schedule at once).
    Reported: the median wall time per class, solo (idle device) and
    contended, and how many calls fell in each."""
    torch = w.torch
    a = torch.randn(8192, 8192, dtype=torch.bfloat16, device="cuda")
    b = torch.randn(8192, 8192, dtype=torch.bfloat16, device="cuda")
    busy = torch.cuda.Stream()

    def one(contended: bool):
        before = w.ctx.schedule_counts()
        if contended:
            with torch.cuda.stream(busy):
                for _ in range(3):
                    torch.mm(a, b)
        t0 = time.perf_counter()
        w.store(0)
        ms = (time.perf_counter() - t0) * 1e3
        torch.cuda.synchronize()
        after = w.ctx.schedule_counts()
        kind = ("gave_up" if after["reencoded"] > before["reencoded"]
                else "safe" if after["safe_calls"] > before["safe_calls"] else "persistent")
        return kind, ms

    def summary(rows):
        out = {}
        for kind in ("persistent", "gave_up", "safe"):
            ms = [m for k, m in rows if k == kind]
            if ms:
                out[kind] = {"calls": len(ms), "median_ms": round(statistics.median(ms), 4)}
        return out

    torch.cuda.synchronize()
    solo = [one(False) for _ in range(calls)]
    # one forced give-up (a zero wait bound), then the idle device's calls
    # on the schedule that needs no residency
    w.ctx.set_wait_bound(0.0)
    forced = one(False)
    w.ctx.set_wait_bound(200.0)
    solo += [forced] + [one(False) for _ in range(calls)]
    contended = [one(True) for _ in range(3 * calls)]
    del a, b
    torch.cuda.empty_cache()
    return {"solo": summary(solo), "contended": summary(contended),
            "busy_stream": "3 x torch.mm of 8192x8192 bf16 per call",
            "wait_bound_us": 200.0}


def uniform_ratio(w: Grouped) -> float:
    """Config 1's pages at a uniform REL 1e-4 (the metric's eb): one
    compress_batch_fixed_bf16 call over the 256 whole pages."""
    torch, k = w.torch, w.k
    n = w.page_numel
    slab = torch.empty(w.num_pages * 8 * n, dtype=torch.uint8, device="cuda")
    sizes = (ctypes.c_uint64 * w.num_pages)()
    bounds = (ctypes.c_float * w.num_pages)()
    k.check(w.ctx.compress(
        k.ptr_array([w.pages[p].data_ptr() for p in range(w.num_pages)]),
        k.ptr_array([slab.data_ptr() + p * 8 * n for p in range(w.num_pages)]),
        k.u64_array([8 * n] * w.num_pages), k.f32_array([1e-4] * w.num_pages),
        w.num_pages, n, w.stream, sizes, bounds))
    return round(2 * n * w.num_pages / sum(sizes), 4)


def host_info() -> dict:
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"nproc": cores, "cpu_model": model}


def cpu_baseline(w: Grouped, max_pages: int, threads: int) -> dict:
    """The scalar CPU oracle on config 1's first `max_pages` pages, store +
    restore of both layer groups, on `threads` threads and on one."""
    import numpy as np

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle

    host = w.pages[:max_pages].contiguous().cpu().view(w.torch.int16).numpy().view(np.uint16)
    nbytes = 2 * host.size

    def run(nthreads):
        t_c = t_d = 0.0
        for bound, layers in w.groups:
            streams, sizes, bounds, enc_s = oracle.compress_batch(
                host, [bound] * host.shape[0], relative=True, threads=nthreads,
                layer_indices=list(layers), source_layers=w.shape.layers,
                elements_per_layer=w.epl, return_elapsed=True)
            out = np.zeros_like(host)
            n = 2 * len(layers) * w.epl
            t1 = time.perf_counter()
            oracle.decompress_batch_indexed(streams, sizes, n, bounds, out, list(layers),
                                            w.shape.layers, w.epl, threads=nthreads)
            t_d += time.perf_counter() - t1
            t_c += enc_s
        return {"value": round(nbytes / (t_c + t_d) / 1e9, 4), "unit": "GB/s",
                "cores": nthreads,
                "compress_gbps": round(nbytes / t_c / 1e9, 4),
                "decompress_gbps": round(nbytes / t_d / 1e9, 4)}

    one = run(1)
    allc = run(threads) if threads > 1 else dict(one)
    allc.update({"kind": "port",
                 "sample": f"{host.shape[0]} of 256 config-1 pages, both layer groups, "
                           "store+restore (oracle/kvszp_oracle.c, gcc -O2)",
                 "one_core": one})
    return allc


def host_codec_baselines(w: Grouped, max_pages: int, threads: int) -> dict:
    import numpy as np

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import cpu_codecs

    host = w.pages[:max_pages].contiguous().cpu().view(w.torch.int16).numpy().view(np.uint16)
    return cpu_codecs.time_all(host, threads=threads)


# ---- rocprof traffic post-processing (no GPU) ----------------------------------------

def _pmc_per_dispatch(run_dir: str, counter: str) -> dict:
    """{kernel kind: [value per dispatch, KiB]} from a rocprofv3 --pmc CSV."""
    import csv
    from collections import defaultdict

    path = os.path.join(run_dir, "run_counter_collection.csv")
    per = defaultdict(float)
    names = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            did = int(row["Dispatch_Id"])
            per[did] += float(row["Counter_Value"])
            names[did] = row["Kernel_Name"]
    out = defaultdict(list)
    for did in sorted(per):
        name = names[did]
        if "kvszp::" in name and "decompress" in name:
            kind = "decompress_kernel"
        elif "kvszp::" in name and "compress" in name and "minmax" not in name:
            kind = "compress_kernel"
        elif "copyBuffer" in name:
            kind = "copy"
        else:
            continue
        out[kind].append(per[did])
    return out


def traffic_from(base: str, config: int) -> int:
    """HBM bytes per launch from FETCH_SIZE / WRITE_SIZE (KiB per dispatch),
    each scaled so that a plain device copy of known size reads and writes
    exactly its own bytes; written with the kernel source's hash."""
    with open(os.path.join(base, "copy_calibration.json")) as f:
        copy_bytes = json.load(f)["copy_bytes_each_way"]
    cf = _pmc_per_dispatch(os.path.join(base, "copy_fetch"), "FETCH_SIZE")["copy"]
    cw = _pmc_per_dispatch(os.path.join(base, "copy_write"), "WRITE_SIZE")["copy"]
    fetch_factor = copy_bytes / (sum(cf) / len(cf) * 1024)
    write_factor = copy_bytes / (sum(cw) / len(cw) * 1024)
    bf = _pmc_per_dispatch(os.path.join(base, "bench_fetch"), "FETCH_SIZE")
    bw = _pmc_per_dispatch(os.path.join(base, "bench_write"), "WRITE_SIZE")
    result = {"fetch_factor": round(fetch_factor, 4),
              "write_factor": round(write_factor, 4),
              "kernels_sha": kernels_sha()}
    for kind in ("compress_kernel", "decompress_kernel"):
        fetch = sum(bf[kind]) / len(bf[kind]) * 1024 * fetch_factor
        write = sum(bw[kind]) / len(bw[kind]) * 1024 * write_factor
        result[kind] = int(round(fetch + write))
        result[kind + "_fetch"] = int(round(fetch))
        result[kind + "_write"] = int(round(write))
    path = traffic_file(config)
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w") as f:
        json.dump(result, f, indent=1)
    print(json.dumps(result))
    return 0


def bw_probe(sets: int = 4) -> dict:
    """Achievable HBM rate of plain device copies (torch copy_), read + write
    bytes per second, on buffers rotated so that a copy reads nothing the
    Infinity Cache holds, and on one buffer pair (cache-warm)."""
    import torch

    out = {}
    for mib in (64, 117, 256, 1024):
        n = (mib << 20) // 2
        srcs = [torch.ones(n, dtype=torch.bfloat16, device="cuda") for _ in range(sets)]
        dsts = [torch.empty_like(s) for s in srcs]
        res = {}
        for label, rot in (("cold", sets), ("warm", 1)):
            ts = []
            for r in range(24):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                dsts[r % rot].copy_(srcs[r % rot])
                b.record()
                b.synchronize()
                ts.append(a.elapsed_time(b))
            ms = statistics.median(ts[4:])
            res[label] = round(2 * n * 2 / (ms * 1e-3) / 1e9, 1)
        out[f"{mib}MiB"] = res
        del srcs, dsts
        torch.cuda.empty_cache()
    return out


def link_probe(mib: int = 70) -> dict:
    """Host-device link rates: DMA copies (torch copy_ between a pinned host
    tensor and device memory) against kvszp_pack_streams writing one payload
    of the same size straight into pinned memory with its gather kernel."""
    import kvszp
    import torch

    n = mib << 20
    host = torch.empty(n, dtype=torch.uint8).pin_memory()
    dev = torch.ones(n, dtype=torch.uint8, device="cuda")
    cfg = kvszp.Config(1e-4, 1, kvszp.DIM_1D, kvszp.MODE_FIXED, kvszp.TYPE_FLOAT)
    ctx = kvszp.Context(cfg, 0)
    stream = torch.cuda.current_stream().cuda_stream
    offsets = (ctypes.c_uint64 * 1)()
    packed = ctypes.c_uint64()

    def pack():
        kvszp.check(ctx.pack(kvszp.ptr_array([dev.data_ptr()]), kvszp.u64_array([n]), 1,
                             host.data_ptr(), n, stream, offsets, ctypes.byref(packed)))

    out = {}
    for name, fn in (("dma_d2h", lambda: host.copy_(dev, non_blocking=True)),
                     ("dma_h2d", lambda: dev.copy_(host, non_blocking=True)),
                     ("pack_kernel_d2h", pack)):
        ts = []
        for _ in range(12):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        out[name] = round(n / statistics.median(ts[2:]) / 1e9, 2)
    return {"bytes": n, "gbps": out}


# ---- main ---------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=1, choices=(0, 1, 2, 3, 4))
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 200 for configs 0/1, 20 otherwise)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--rotate", type=int, default=None,
                    help="buffer sets the steps rotate through (default 3 for "
                         "configs 0/1, 1 otherwise)")
    ap.add_argument("--cpu-pages", type=int, default=256,
                    help="config-1 pages of the CPU oracle sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-pcie", action="store_true")
    ap.add_argument("--no-contended", action="store_true")
    ap.add_argument("--restore-per-group", action="store_true",
                    help="grouped configs: one indexed_scatter call per layer group "
                         "(the reference's call pattern) instead of one grouped launch")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy (the reference kernel "
                         "for scaling rocprof FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--bw-probe", action="store_true",
                    help="only measure plain device-copy rates (cache-cold and warm)")
    ap.add_argument("--link-probe", action="store_true",
                    help="only measure host-device link rates (DMA and the pack kernel)")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="no GPU work: turn the rocprofv3 --pmc runs under DIR "
                         "(copy_fetch, copy_write, bench_fetch, bench_write) into HBM "
                         "bytes per launch for --config")
    args = ap.parse_args()
    if args.traffic_from:
        return traffic_from(args.traffic_from, args.config)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (KV pages "
              "are private to the GPU that owns them, and each GPU's connector stores "
              "and restores its own pages).", file=sys.stderr)
        return 2

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        src = torch.ones(128 << 20, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 2, "copies": 3}), flush=True)
        return 0
    if args.bw_probe:
        print(json.dumps({"bw_probe_gbps_read_plus_write": bw_probe()}), flush=True)
        return 0
    if args.link_probe:
        print(json.dumps({"link_probe": link_probe()}), flush=True)
        return 0

    small = args.config in (0, 1)
    steps = args.steps if args.steps is not None else (200 if small else 20)
    warmup = args.warmup if args.warmup is not None else (20 if small else 3)
    sets = args.rotate if args.rotate is not None else (3 if small else 1)
    log(f"building config {args.config} ({sets} buffer sets)")
    w = make_workload(args.config, args.seed, sets, args.restore_per_group)
    log(f"{w.num_pages} pages x {w.page_numel} BF16, {w.batch} requests")
    # The timed passes follow the warm-up directly (no idle gap before the
    # first timed step).  Python's cyclic garbage collector stays off while
    # they run (a full collection in a process holding torch takes
    # milliseconds, and would land inside one step).
    gc.collect()
    gc.disable()
    try:
        for i in range(max(1, warmup)):
            w.step(i % sets)
        cold = timed_steps(w, steps, sets)
        warm = timed_steps(w, steps, 1) if sets > 1 else cold
    finally:
        gc.enable()
    # Every step writes the same restored pages, so the round trip of the
    # timed steps is checked afterwards.
    check = w.verify()
    log(f"round trip check: {check}")
    if not check["ok"]:
        print("error bound violated", file=sys.stderr)
        return 1
    s_bytes = w.stream_bytes(0)
    ratio = w.bf16_bytes / s_bytes
    step_ms = cold["ms_per_step"]
    enc, dec = cold["compress"], cold["decompress"]
    enc_launch_bytes = (w.bf16_bytes + s_bytes) / max(1, enc["launches_per_step"])
    enc_hbm = enc_launch_bytes / (enc["mean_ms"] * 1e-3) / 1e9
    dec_hbm = (w.bf16_bytes + s_bytes) / (dec["ms_per_step"] * 1e-3) / 1e9
    traffic = None
    tf = traffic_file(args.config)
    if os.path.exists(tf):
        with open(tf) as f:
            t = json.load(f)
        if t.get("kernels_sha") == kernels_sha():
            traffic = t.get("compress_kernel")

    result = {
        "metric": METRIC,
        "value": round(w.bf16_bytes / (step_ms * 1e-3) / 1e9, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(step_ms, 4),
        "step_ms": cold["step_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": w.name + (" (per-group restore)" if args.restore_per_group else ""),
            "config_index": args.config,
            "pages": w.num_pages,
            "page_elements": w.page_numel,
            "segment_requests": w.batch,
            "kv_bytes": w.bf16_bytes,
            "buffer_sets": sets,
            "parallelism": "single GPU",
        },
        "value_mall_warm": round(w.bf16_bytes / (warm["ms_per_step"] * 1e-3) / 1e9, 3),
        "ratio": round(ratio, 4),
        "compress_gbps": round(w.bf16_bytes / (enc["ms_per_step"] * 1e-3) / 1e9, 2),
        "decompress_gbps": round(w.bf16_bytes / (dec["ms_per_step"] * 1e-3) / 1e9, 2),
        "compress_kernel": enc,
        "decompress_kernel": dec,
        "compress_hbm_frac": round(enc_hbm / HBM_PEAK_GBPS, 4),
        "decompress_hbm_frac": round(dec_hbm / HBM_PEAK_GBPS, 4),
        # the same launches on the uncompressed basis (2N bytes only); the
        # algorithmic-traffic fractions above are larger by 1 + S / 2N
        "compress_bf16_frac": round(
            w.bf16_bytes / (enc["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "decompress_bf16_frac": round(
            w.bf16_bytes / (dec["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "mall_warm": {"compress_kernel": warm["compress"],
                      "decompress_kernel": warm["decompress"],
                      "ms_per_step": round(warm["ms_per_step"], 4)},
        "roofline": {
            # the encoder launches timed as "compress_kernel" above: the
            # persistent schedule, which rocprofv3 lists as
            # compress_persistent[_argtable]_kernel<quantizer, early>
            "kernel": "encoder (compress_persistent*_kernel)",
            "bound": "hbm",
            "achieved": round(enc_hbm, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(enc_hbm / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": int(enc_launch_bytes),
        },
        "reencoded_calls": w.ctx.reencode_count(),
        "round_trip_check": check,
    }
    if args.config == 1:
        result["ratio_uniform_1e-4"] = uniform_ratio(w)
        if not args.no_contended:
            log("store beside a busy stream")
            result["contended_store"] = contended_store(w)
        if not args.no_pcie:
            log("pcie store+restore")
            result["pcie"] = pcie_steps(w, 20)
        if not args.no_cpu:
            info = host_info()
            # the GPU box's share of host cores is 16, whatever nproc says
            threads = max(1, min(info["nproc"] or 1, 16))
            log(f"cpu baseline ({threads} threads)")
            result["cpu_baseline"] = cpu_baseline(w, args.cpu_pages, threads)
            result["cpu_baseline"].update(info)
            try:
                result["cpu_host_codecs"] = host_codec_baselines(
                    w, min(args.cpu_pages, 64), threads)
            except Exception as exc:  # system codec libraries may be absent
                result["cpu_host_codecs"] = {"error": str(exc)}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
