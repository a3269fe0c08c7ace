#!/usr/bin/env python3
"""Benchmark: batched fixed-mode BF16 KV-page store + restore on one MI355X.

Workload: the full Qwen2.5-1.5B 4K-context KV
cache, 28 layers x K/V x [4096 tokens, 2 heads, 128] BF16, laid out as 256
vLLM pages of [2, 28, 16, 2, 128] (229 376 values, 448 KiB each).  Layer
bounds follow the reference's measured mixed profile: layers
{0,1,2,5,19,20,21} at REL 1e-5, the other 21 at REL 1e-4, so every page is
two layer-selected segments.  One step is what the reference's connector
does for this job (vllm_v1_compressed_offload.py:1286-1569 and 1815-2006):

  store   : one compress_batch_fixed_bf16_indexed_groups call over all 512
            (page, segment) requests (blocking: sizes come back to the host)
  restore : the reference's one decompress_batch_fixed_bf16_indexed_scatter
            call per group, writing straight into fresh KV pages -- by
            default as ONE decompress_batch_fixed_bf16_indexed_scatter_groups
            launch over both groups (same output; --restore-per-group runs
            the per-group calls instead)

Calls go through the C ABI (libkvszp.so) with the page-pointer arrays built
once, inputs resident in HBM.  `value` = uncompressed BF16 bytes of the KV
cache / (store + restore time per step).  Kernel-only throughput and the
roofline fraction come from HIP events recorded on the launch stream.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(
    REPO,
    "reducing-pcie-bottlenecks-for-llm-serving-with-cuszp-compressed-kv-cache-transfer_amd")
sys.path.insert(0, PKG)

METRIC = "KV compress/decompress GB/s (BF16 in), % of HBM peak, ratio at eb=1e-4"
HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic_qwen15b_4k_store_restore.json")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Workload:
    """Config 1 pages, compressed slabs and pointer tables, built once."""

    def __init__(self, seed: int, tokens: int | None = None,
                 grouped_restore: bool = True):
        import torch

        import kv_synth
        import kvszp

        self.kvszp = kvszp
        self.shape = kv_synth.QWEN25_1P5B_4K
        self.pages = kv_synth.paged_kv(self.shape, seed=seed, device="cuda",
                                       tokens=tokens)
        self.dest = torch.zeros_like(self.pages)
        self.num_pages, self.page_numel = self.pages.shape
        self.epl = self.shape.elements_per_layer
        self.groups = kv_synth.mixed_bound_groups()
        self.layer_idx = [torch.tensor(ls, dtype=torch.long, device="cuda")
                          for _, ls in self.groups]
        # requests group by group, page by page (the connector's order)
        caps, eps, self.seg_numel = [], [], []
        for bound, layers in self.groups:
            n = 2 * len(layers) * self.epl
            for _ in range(self.num_pages):
                caps.append(8 * n)
                eps.append(bound)
                self.seg_numel.append(n)
        self.batch = len(caps)
        self.slab = torch.empty(sum(caps), dtype=torch.uint8, device="cuda")
        offs = [0]
        for c in caps[:-1]:
            offs.append(offs[-1] + c)
        base = self.slab.data_ptr()
        page_ptrs = [p.data_ptr() for p in self.pages]
        dest_ptrs = [p.data_ptr() for p in self.dest]
        self.inputs = kvszp.ptr_array(page_ptrs * len(self.groups))
        self.outputs = kvszp.ptr_array([base + o for o in offs])
        self.stream_ptrs = [base + o for o in offs]
        self.caps = kvszp.u64_array(caps)
        self.eps = kvszp.f32_array(eps)
        self.idx_ptrs = kvszp.ptr_array([t.data_ptr() for t in self.layer_idx])
        self.sel = kvszp.size_array([len(ls) for _, ls in self.groups])
        self.group_sizes = kvszp.size_array([self.num_pages] * len(self.groups))
        self.dest_ptrs = kvszp.ptr_array(dest_ptrs)
        self.sizes = (ctypes.c_uint64 * self.batch)()
        self.bounds = (ctypes.c_float * self.batch)()
        cfg = kvszp.Config(1e-4, 1, kvszp.DIM_1D, kvszp.MODE_FIXED,
                           kvszp.TYPE_FLOAT)
        self.ctx = kvszp.Context(cfg, 0)
        self.stream = torch.cuda.current_stream().cuda_stream
        self.group_slices = []
        start = 0
        for _ in self.groups:
            self.group_slices.append((start, start + self.num_pages))
            start += self.num_pages
        # Per-group restore arguments, built once like the other tables.
        self.grouped_restore = grouped_restore
        self.stream_table = kvszp.ptr_array(self.stream_ptrs)
        # one destination page per request: every group restores into the
        # same fresh pages
        self.dest_table = kvszp.ptr_array(dest_ptrs * len(self.groups))
        self.restore_args = []
        for g, (lo, hi) in enumerate(self.group_slices):
            cnt = hi - lo
            self.restore_args.append((
                kvszp.ptr_array(self.stream_ptrs[lo:hi]),
                (ctypes.c_uint64 * cnt).from_buffer(self.sizes, lo * 8),
                (ctypes.c_float * cnt).from_buffer(self.bounds, lo * 4),
                cnt, self.layer_idx[g].data_ptr(), len(self.groups[g][1])))

    def store(self) -> None:
        k = self.kvszp
        k.check(self.ctx.compress_indexed_groups(
            self.inputs, self.outputs, self.caps, self.idx_ptrs, self.sel,
            self.group_sizes, len(self.groups), 2, self.shape.layers, self.epl,
            self.eps, self.batch, self.stream, self.sizes, self.bounds))

    def restore(self) -> None:
        k = self.kvszp
        if self.grouped_restore:
            k.check(self.ctx.decompress_indexed_scatter_groups(
                self.stream_table, self.sizes, self.bounds, self.batch,
                self.dest_table, self.idx_ptrs, self.sel, self.group_sizes,
                len(self.groups), 2, self.shape.layers, self.epl,
                self.stream))
            return
        for comp, sizes, bounds, cnt, idx, sel in self.restore_args:
            k.check(self.ctx.decompress_indexed_scatter(
                comp, sizes, bounds, cnt, self.dest_ptrs, idx, sel, 2,
                self.shape.layers, self.epl, self.stream))

    def step(self) -> None:
        self.store()
        self.restore()

    @property
    def bf16_bytes(self) -> int:
        return 2 * self.num_pages * self.page_numel

    def stream_bytes(self) -> int:
        return int(sum(self.sizes[i] for i in range(self.batch)))


def verify(w: Workload) -> dict:
    """Round-trip checks on the measured data: restored pages within 2*eb of
    the input on every element (the reference's BF16 tolerance, tests
    :457, :639), and stream sizes/bounds consistent."""
    import torch

    err = (w.dest.float() - w.pages.float()).abs().view(
        w.num_pages, 2, w.shape.layers, w.epl)
    worst = 0.0
    for g, (bound, layers) in enumerate(w.groups):
        lo, hi = w.group_slices[g]
        eb = torch.tensor([w.bounds[i] for i in range(lo, hi)], device="cuda")
        e = err[:, :, list(layers)].amax(dim=(1, 2, 3))
        worst = max(worst, float((e / (2 * eb + 1e-12)).max()))
    return {"max_err_over_2eb": worst, "ok": worst <= 1.0}


def cpu_baseline(w: Workload, max_pages: int) -> dict:
    """The scalar CPU oracle (one thread) on the same pages: store + restore
    of `max_pages` pages, reported as BF16 GB/s like the GPU value."""
    import numpy as np

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle

    import torch

    host = w.pages[:max_pages].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    n_pages = host.shape[0]
    t_c = t_d = 0.0
    for bound, layers in w.groups:
        streams, sizes, bounds, enc_s = oracle.compress_batch(
            host, [bound] * n_pages, relative=True, threads=1,
            layer_indices=list(layers), source_layers=w.shape.layers,
            elements_per_layer=w.epl, return_elapsed=True)
        n = 2 * len(layers) * w.epl
        out = np.zeros_like(host)
        t1 = time.perf_counter()
        for i in range(n_pages):
            oracle.decompress_indexed(streams[i], n, float(bounds[i]), out[i],
                                      list(layers), w.shape.layers, w.epl)
        t2 = time.perf_counter()
        t_c += enc_s
        t_d += t2 - t1
    nbytes = 2 * host.size
    return {"value": round(nbytes / (t_c + t_d) / 1e9, 4), "unit": "GB/s",
            "cores": 1, "kind": "port",
            "sample": f"{n_pages} of 256 pages (both layer groups), store+restore",
            "compress_gbps": round(nbytes / t_c / 1e9, 4),
            "decompress_gbps": round(nbytes / t_d / 1e9, 4)}


def host_codec_baselines(w: Workload, max_pages: int) -> dict:
    """The reference's host codecs (zstd level 1, LZ4 default, INT8) on the
    same BF16 page bytes, one thread, as reported extras."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import cpu_codecs

    host = w.pages[:max_pages].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    return cpu_codecs.time_all(host)


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
            kind = "decompress_kernel"   # decompress_kernel / decompress_persistent_kernel
        elif "kvszp::" in name and "compress" in name and "minmax" not in name:
            kind = "compress_kernel"     # compress_kernel / compress_persistent_kernel
        elif "copyBuffer" in name:
            kind = "copy"
        else:
            continue
        out[kind].append(per[did])
    return out


def traffic_from(base: str) -> int:
    """HBM bytes per launch from FETCH_SIZE / WRITE_SIZE (KiB per dispatch),
    each scaled so that a plain device copy of known size reads and writes
    exactly its own bytes."""
    with open(os.path.join(base, "copy_calibration.json")) as f:
        copy_bytes = json.load(f)["copy_bytes_each_way"]
    cf = _pmc_per_dispatch(os.path.join(base, "copy_fetch"), "FETCH_SIZE")["copy"]
    cw = _pmc_per_dispatch(os.path.join(base, "copy_write"), "WRITE_SIZE")["copy"]
    fetch_factor = copy_bytes / (sum(cf) / len(cf) * 1024)
    write_factor = copy_bytes / (sum(cw) / len(cw) * 1024)
    bf = _pmc_per_dispatch(os.path.join(base, "bench_fetch"), "FETCH_SIZE")
    bw = _pmc_per_dispatch(os.path.join(base, "bench_write"), "WRITE_SIZE")
    result = {"fetch_factor": round(fetch_factor, 4),
              "write_factor": round(write_factor, 4)}
    for kind in ("compress_kernel", "decompress_kernel"):
        fetch = sum(bf[kind]) / len(bf[kind]) * 1024 * fetch_factor
        write = sum(bw[kind]) / len(bw[kind]) * 1024 * write_factor
        result[kind] = int(round(fetch + write))
        result[kind + "_fetch"] = int(round(fetch))
        result[kind + "_write"] = int(round(write))
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(result, f, indent=1)
    print(json.dumps(result))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # A step is ~0.12 ms: 200 timed steps (~25 ms of GPU time) give a steady
    # state; 20 steps read ~5 % low from first-step effects.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-pages", type=int, default=256,
                    help="pages of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--restore-per-group", action="store_true",
                    help="restore with one indexed_scatter call per layer "
                         "group (the reference's call pattern) instead of "
                         "one grouped launch")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy (the reference "
                         "kernel for scaling rocprof FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="no GPU work: turn the rocprofv3 --pmc runs under DIR "
                         "(copy_fetch, copy_write, bench_fetch, bench_write) into "
                         "HBM bytes per launch, written to " + TRAFFIC_FILE)
    args = ap.parse_args()
    if args.traffic_from:
        return traffic_from(args.traffic_from)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(KV pages are private to the GPU that owns them; see DESIGN.md "
              "for how the path shards).", file=sys.stderr)
        return 2

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        src = torch.ones(128 << 20, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 2,
                          "copies": 3}), flush=True)
        return 0
    log("building workload")
    w = Workload(args.seed, grouped_restore=not args.restore_per_group)
    log(f"workload: {w.num_pages} pages x {w.page_numel} BF16, "
        f"{w.batch} segment requests")
    for _ in range(max(1, args.warmup)):
        w.step()
    torch.cuda.synchronize()
    check = verify(w)
    log(f"round trip check: {check}")
    if not check["ok"]:
        print("error bound violated", file=sys.stderr)
        return 1
    ratio = w.bf16_bytes / w.stream_bytes()

    # Timed region: whole steps, with HIP events around the dominant kernel
    # (the encoder) only -- each event record costs GPU time.
    w.ctx.drain_timing()
    w.ctx.enable_timing(w.kvszp.TIME_COMPRESS)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        w.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    w.ctx.enable_timing(0)
    kt = w.ctx.drain_timing()
    step_s = (t1 - t0) / args.steps
    # Decoder launch durations from a second pass of the same steps (not
    # part of `value`).
    w.ctx.enable_timing(w.kvszp.TIME_DECOMPRESS)
    for _ in range(args.steps):
        w.step()
    torch.cuda.synchronize()
    w.ctx.enable_timing(0)
    dt = w.ctx.drain_timing()
    kt["decompress_ms"] = dt["decompress_ms"]
    dec_launches = max(1, dt["decompress_launches"] // max(1, args.steps))

    # Algorithmic bytes per launch: compress reads 2N and writes S per
    # segment; restore reads S and writes 2N.
    s_bytes = w.stream_bytes()
    comp_launch_bytes = w.bf16_bytes + s_bytes
    comp_ms = kt["compress_ms"] / max(1, kt["compress_launches"])
    dec_ms_step = kt["decompress_ms"] / args.steps
    comp_gbps = w.bf16_bytes / (comp_ms * 1e-3) / 1e9
    dec_gbps = w.bf16_bytes / (dec_ms_step * 1e-3) / 1e9
    comp_hbm = comp_launch_bytes / (comp_ms * 1e-3) / 1e9
    dec_hbm = (w.bf16_bytes + s_bytes) / (dec_ms_step * 1e-3) / 1e9
    if comp_ms >= dec_ms_step:
        dom = ("compress_kernel", comp_hbm, comp_launch_bytes)
    else:
        dom = ("decompress_kernel", dec_hbm,
               (w.bf16_bytes + s_bytes) / dec_launches)
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get(dom[0])

    result = {
        "metric": METRIC,
        "value": round(w.bf16_bytes / step_s / 1e9, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "qwen2.5-1.5b 4k store+restore (configs[1]): 256 pages "
                        "x [2,28,16,2,128] bf16, layers {0,1,2,5,19,20,21} REL "
                        "1e-5 + 21 layers REL 1e-4, indexed_groups compress + "
                        + ("2x indexed_scatter restore" if args.restore_per_group
                           else "indexed_scatter_groups restore"),
            "pages": w.num_pages,
            "page_elements": w.page_numel,
            "segment_requests": w.batch,
            "kv_bytes": w.bf16_bytes,
            "parallelism": "single GPU",
        },
        "ratio": round(ratio, 4),
        "compress_gbps": round(comp_gbps, 2),
        "decompress_gbps": round(dec_gbps, 2),
        "compress_kernel_ms": round(comp_ms, 4),
        "decompress_kernel_ms_per_step": round(dec_ms_step, 4),
        "compress_hbm_frac": round(comp_hbm / HBM_PEAK_GBPS, 4),
        "decompress_hbm_frac": round(dec_hbm / HBM_PEAK_GBPS, 4),
        "roofline": {
            "kernel": dom[0],
            "bound": "hbm",
            "achieved": round(dom[1], 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dom[1] / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": int(dom[2]),
        },
        "round_trip_check": check,
    }
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_pages)
        try:
            result["cpu_host_codecs"] = host_codec_baselines(w, min(args.cpu_pages, 64))
        except Exception as exc:  # system codec libraries may be absent
            result["cpu_host_codecs"] = {"error": str(exc)}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
