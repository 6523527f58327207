#!/usr/bin/env python3
"""Benchmark of the submanifold sparse conv3d path on one MI355X.

Headline (the JSON line's `value`): the neighbor-map build on ~1.5M voxels of a 1-voxel shell in
a 512^3 grid, shuffled rows ("map512").  One step = one tsc_map_build over the whole coordinate
set, inputs already resident in HBM.  value = algorithmic bytes (128 B/voxel: 16 B coords in,
4 B sorted key + 108 B neighbor row out) / time, in GB/s.

`secondary` carries the conv workloads measured in the same run (ms per conv, effective
TFLOP/s counting only valid taps, algorithmic GB/s, roofline fraction):
  conv64_f32       conv 64->64 fp32, ~25k voxels (64^3, 2-voxel shell)
  narrow512_f16    conv 32->32 and 32->64 fp16 on the map512 voxels
  narrow512s2_f16  the same convs on ~3.0M voxels of a 2-voxel shell in 512^3 (the thickness a
                   subdivided 1-voxel shell has); both narrow workloads also time the unplanned
                   (direct) kernel in the map's row order
  wide128_bf16     conv 512->512 bf16, 4 x ~61k voxels (128^3 shells)
  resblock64_bf16  4 x ResBlock (conv-LN-SiLU-conv-+x) at C=1024 bf16, 2 x ~32k voxels
and the decoder upsample (tsc_subdivide) on the wide128 voxels with 512 bf16 channels, all 8
children and a random keep mask (ms, algorithmic GB/s = coords + rows in and out, HBM fraction),
and a sparse ConvNeXt block (conv + two linears, C=512, hidden 2048, bf16) on the same voxels,
varlen self-attention over the resblock64 voxels (12 heads x 128, bf16 and fp32: TFLOP/s, MFMA
fraction), and a 340 MB safetensors weight file streamed to the device (as stored, and widened to
fp32).

`roofline` is for the map build's dominant kernel, timed with hipEvents around each launch on
the stream the library launches on; `cpu_baseline` times the PyTorch-CPU restatement of the
reference's hashmap_fallback (torch.sort + torch.searchsorted) on the same coordinates.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-secondary]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ms/conv + effective TFLOP/s (or GB/s) for 3^3 sparse conv at N active voxels"
PEAK_HBM = 8.0e12          # B/s, MI355X HBM3E
PEAK_MFMA = {"bfloat16": 2.5e15, "float16": 2.5e15, "float32": 157.3e12}  # dense FLOP/s
MAP_BYTES_PER_VOXEL = 128  # 16 coords + 4 key + 108 table
# Algorithmic bytes per voxel of each map-build kernel (inputs it must read + outputs it writes).
MAP_KERNEL_BYTES = {
    "map_mark": 16, "map_place": 16 + 4 + 4, "map_fill": 4 + 4 + 108,   # bitmap path
    "radix_pack": 16 + 4 + 4,          # coords in; (key, row) out
    "radix_partition": 8 + 8,          # (key, row) in and out
    "radix_buckets": 8 + 8,            # (key, row) in; sorted key + row out (column table extra)
    "radix_fill": 4 + 4 + 108,         # sorted key + row in; 27 neighbor rows out
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_steps(fn, steps: int, warmup: int) -> float:
    """Mean ms per step over `steps` after `warmup`, bracketed by syncs and events."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def kernel_times(ctx, fn, steps: int) -> dict:
    """{kernel: (avg ms per launch, launches per step)} from library hipEvents."""
    import torch

    torch.cuda.synchronize()
    ctx.profile_reset()
    ctx.profile(True)
    for _ in range(steps):
        fn()
    ctx.profile(False)
    res = ctx.profile_results()
    ctx.profile_reset()
    return {k: (ms / n, n / steps) for k, (ms, n) in res.items()}


# Library profiler names -> the kernel names of profiles/workload_counters.json (rocprofv3
# symbols shortened by trellis.2-stableprojectorz_amd/profiling.py).
ROCPROF_NAME = {"map_fill": "fill_columns_kernel<bitmap>", "map_mark": "mark_kernel<int32>",
                "map_place": "place_kernel<int32>", "radix_fill": "fill_window_kernel<int32>",
                "radix_buckets": "bucket_sort_kernel<int32>",
                "radix_partition": "partition_kernel<int32>", "radix_pack": "pack_sort_kernel<int32>",
                "radix_scan": "scan_kernel", "attention": "attn_mma_kernel",
                "layernorm": "layernorm_kernel", "layernorm_silu": "layernorm_kernel",
                "conv_tile_cost": "tile_cost_kernel", "conv_tile_schedule": "tile_schedule_kernel"}


COUNTERS_FILE = ROOT / "profiles" / "workload_counters.json"


def load_counters() -> dict:
    """{workload: {kernel: record}} from profiles/workload_counters.json (profiling.py merge of
    the per-workload rocprofv3 runs), or {}."""
    if not COUNTERS_FILE.exists():
        return {}
    try:
        return json.loads(COUNTERS_FILE.read_text()).get("workloads", {})
    except ValueError:
        return {}


def load_traffic(counters: dict, workload: str, kernel: str):
    """HBM bytes per launch of `kernel` in `workload` (FETCH_SIZE + WRITE_SIZE runs)."""
    rec = counters.get(workload, {}).get(ROCPROF_NAME.get(kernel, kernel))
    if not rec or rec.get("fetch_bytes") is None or rec.get("write_bytes") is None:
        return None
    return rec["fetch_bytes"] + rec["write_bytes"]


def write_floor_record(ctx, nmap, n: int, fill_ms: float, steps: int) -> dict:
    """The fill's store pattern alone (tsc_map_write_floor): the (N,27) rows written at the map's
    original rows (perm, what the fill does) and at sequential rows, each launch timed with
    hipEvents.  fill_over_floor = the fill's time / the scattered floor."""
    import torch

    out = torch.empty((n, 27), dtype=torch.int32, device=nmap.nbr.device)
    res = {"kernel": "map_write_floor", "bytes_per_launch": 112 * n,
           "note": "tsc_map_write_floor: 112 B per voxel (4 B row index in, 108 B row out), the "
                   "fill's blocks, lanes and 12-byte stores without its loads and searches"}
    for label, rows in (("scattered_ms", nmap.perm), ("sequential_ms", None)):
        def run():
            _check(ctx, ctx.lib.tsc_map_write_floor(ctx.bind(), None if rows is None else
                                                    rows.data_ptr(), n, out.data_ptr()))
        for _ in range(3):
            run()
        kt = kernel_times(ctx, run, steps)
        res[label] = round(kt["map_write_floor"][0], 4)
    res["scattered_gbps"] = round(112 * n / (res["scattered_ms"] / 1e3) / 1e9, 1)
    res["fill_over_floor"] = round(fill_ms / res["scattered_ms"], 3)
    log(f"write floor: scattered {res['scattered_ms']} ms ({res['scattered_gbps']} GB/s), "
        f"sequential {res['sequential_ms']} ms; fill / floor = {res['fill_over_floor']}")
    return res


def _check(ctx, status: int) -> None:
    if status:
        raise RuntimeError(f"tsc status {status}: {ctx.lib.tsc_last_error().decode()}")


# Workloads of the rocprofv3 counter runs (bench.py --profile-pass --workload NAME).  Each run
# sets the workload up, runs it PROFILE_WARM times, makes a 256 MiB device copy (the counters'
# byte scale), then runs it PROFILE_REPS more times; profiling.py keeps the dispatches after the
# copy, so each counter record belongs to one workload and to warm launches.
PROFILE_WARM, PROFILE_REPS = 3, 3
PROFILE_WORKLOADS = ("map512", "conv64_f32", "narrow512_f16_32x32", "narrow512_f16_32x64",
                     "narrow512s2_f16_32x32", "narrow512s2_f16_32x64", "wide128_bf16", "resblock64_bf16", "map_prep", "subdivide", "convnext",
                     "attention_bf16")


def profile_key(rec: dict) -> str:
    """The PROFILE_WORKLOADS name a BENCH record's counters come from."""
    if "profile_workload" in rec:
        return rec["profile_workload"]
    w = rec.get("workload", "")
    if w in ("narrow512_f16", "narrow512s2_f16"):
        return f"{w}_{rec['ci']}x{rec['co']}"
    return w


def profile_setup(pkg, dev, name: str):
    """(callable running the workload once, description) for one PROFILE_WORKLOADS entry."""
    import numpy as np
    import torch

    wl = pkg.workloads
    dts = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
    if name in ("map512", "map_prep"):
        coords = wl.make_coords("map512")
        cd = torch.from_numpy(coords).to(dev)
        shape = wl.grid_shape("map512")
        if name == "map512":
            return (lambda: pkg.build_neighbor_map(cd, shape, 1, validate=False)), \
                "tsc_map_build on map512"
        nmap = pkg.build_neighbor_map(cd, shape, 1)

        def prep():
            pkg.map_conv_order(nmap.nbr, nmap.perm)
            pkg.map_gather_plan(cd, nmap.nbr, 1, shape)
        return prep, "tsc_map_conv_order + tsc_map_gather_plan on map512"
    if name in ("subdivide", "convnext"):
        coords = wl.make_coords("wide128_bf16")
        n = coords.shape[0]
        if name == "subdivide":
            sc = torch.from_numpy(coords).to(dev)
            sf = torch.from_numpy(wl.features(n, SUBDIV_C, 4)).to(dev).to(torch.bfloat16)
            return (lambda: pkg.sparse_subdivide(sc, sf)), \
                f"tsc_subdivide, wide128 voxels x {SUBDIV_C} bf16, all children"
        c, hid, dt = CONVNEXT_C, CONVNEXT_HIDDEN, torch.bfloat16
        g = torch.Generator(device="cpu").manual_seed(7)

        def rnd(*shape, scale=1.0):
            return (torch.randn(*shape, generator=g) * scale).to(dev).to(dt)
        x = pkg.SparseTensor(rnd(n, c), torch.from_numpy(coords).to(dev))
        blk = pkg.SparseConvNeXtBlock3d(torch.from_numpy(wl.conv_weight(c, c, 3)).to(dev).to(dt),
                                       rnd(c, scale=0.1), rnd(hid, c, scale=c ** -0.5),
                                       rnd(hid, scale=0.1), rnd(c, hid, scale=hid ** -0.5),
                                       rnd(c, scale=0.1))
        return (lambda: blk(x)), f"ConvNeXt block, wide128 voxels, C={c}, hidden={hid}, bf16"
    if name == "attention_bf16":
        ac = wl.make_coords("resblock64_bf16")
        counts = np.bincount(ac[:, 0])
        cu = torch.tensor([0, *np.cumsum(counts).tolist()], dtype=torch.int32, device=dev)
        n = int(counts.sum())
        q, k, v = (torch.randn((n, ATTN_HEADS, ATTN_DIM), device=dev).to(torch.bfloat16)
                   for _ in range(3))
        o = torch.empty_like(q)
        return (lambda: pkg.sparse_attention(q, k, v, cu, out=o, max_seqlen_q=int(counts.max()))), \
            f"varlen attention bf16, resblock64 voxels, {ATTN_HEADS} x {ATTN_DIM}"
    base = name[:-6] if name.startswith("narrow512") else name
    w = wl.WORKLOADS[base]
    coords = wl.make_coords(base)
    nmap = pkg.build_neighbor_map(torch.from_numpy(coords).to(dev), wl.grid_shape(base),
                                  int(coords[:, 0].max()) + 1)
    n = coords.shape[0]
    ci, co = ((32, int(name[-2:])) if name.startswith("narrow512") else w.channels[0])
    dt = dts[w.dtype]
    f = torch.from_numpy(wl.features(n, ci, 1)).to(dev).to(dt)
    if base == "resblock64_bf16":
        ws = [(torch.from_numpy(wl.conv_weight(co, ci, 10 + i)).to(dev).to(dt),
               torch.from_numpy(wl.conv_weight(co, ci, 20 + i)).to(dev).to(dt)) for i in range(4)]
        zero = torch.zeros(co, device=dev, dtype=dt)
        bufs = [torch.empty_like(f) for _ in range(2)]

        def chain():
            h = f
            for i, (w1, w2) in enumerate(ws):
                h = pkg.sparse_resblock(h, nmap, w1, zero, w2, zero, eps=1e-6, out=bufs[i % 2])
        return chain, f"4 x ResBlock, resblock64 voxels, C={co}, bf16"
    wt = torch.from_numpy(wl.conv_weight(co, ci, 2)).to(dev).to(dt)
    b = torch.zeros(co, device=dev, dtype=dt)
    o = torch.empty((n, co), device=dev, dtype=dt)
    return (lambda: pkg.sparse_conv3d(f, wt, b, nmap, out=o)), \
        f"conv {base} {ci}->{co} {w.dtype}"


def profile_pass(pkg, dev, name: str) -> None:
    """Short fixed run of one workload for rocprofv3: set-up, PROFILE_WARM launches, the
    calibration copy (256 MiB device copy: the counters' byte scale, and the mark after which
    profiling.py counts dispatches), then PROFILE_REPS launches (the ones profiling.py keeps)."""
    import torch

    if name not in PROFILE_WORKLOADS:
        raise SystemExit(f"unknown profile workload {name!r}; one of {', '.join(PROFILE_WORKLOADS)}")
    run, desc = profile_setup(pkg, dev, name)
    torch.cuda.synchronize()
    log(f"{name}: {desc}: set up")
    for _ in range(PROFILE_WARM):
        run()
    torch.cuda.synchronize()
    c = torch.ones(1 << 26, dtype=torch.int32, device=dev)
    d = torch.empty_like(c)
    d.copy_(c)
    torch.cuda.synchronize()
    del c, d
    log("calibration copy 256 MiB done")
    for _ in range(PROFILE_REPS):
        run()
    torch.cuda.synchronize()
    log(f"{name}: {PROFILE_WARM} warm-up + {PROFILE_REPS} profiled launches done")


# Decoder upsample measured on the 2-voxel shell in 128^3 (4 x ~60k voxels) with 512 bf16
# channels: every voxel -> its 8 children, then a random keep mask (~half the children).
SUBDIV_C = 512


def subdivide_records(pkg, dev, steps, warmup) -> list:
    import numpy as np
    import torch

    wl = pkg.workloads
    coords = wl.make_coords("wide128_bf16")
    n = coords.shape[0]
    c = torch.from_numpy(coords).to(dev)
    f = torch.from_numpy(wl.features(n, SUBDIV_C, 4)).to(dev).to(torch.bfloat16)
    keep = torch.from_numpy(np.random.default_rng(5).integers(0, 256, n).astype(np.uint8)).to(dev)
    row = SUBDIV_C * 2
    out = []
    ctx = pkg._lib.context(dev.index)
    for label, k in (("all 8 children", None), ("random keep mask", keep)):
        m = 8 * n if k is None else pkg.subdivide_count(k)
        co = torch.empty((m, 4), dtype=torch.int32, device=dev)
        fo = torch.empty((m, SUBDIV_C), dtype=torch.bfloat16, device=dev)

        def run():
            pkg._lib.check(ctx.lib.tsc_subdivide(ctx.bind(), c.data_ptr(), n, 2, f.data_ptr(),
                                                 SUBDIV_C, None if k is None else k.data_ptr(),
                                                 co.data_ptr(), fo.data_ptr()))
        ms = time_steps(run, steps, warmup)
        nbytes = n * (16 + row) + m * (16 + row) + (0 if k is None else n)
        rec = {"workload": f"subdivide wide128 shell, {SUBDIV_C} bf16 channels, {label}",
               "profile_workload": "subdivide" if k is None else None,
               "voxels": n, "children": m, "ms": round(ms, 4),
               "gbps_algorithmic": round(nbytes / (ms / 1e3) / 1e9, 1), "bound": "hbm",
               "roofline_frac": round(nbytes / (ms / 1e3) / PEAK_HBM, 4),
               "kernels": {kn: {"avg_ms": round(a, 4), "launches_per_step": cnt}
                           for kn, (a, cnt) in kernel_times(ctx, run, 3).items()}}
        log(f"subdivide ({label}): {ms:.4f} ms, {rec['gbps_algorithmic']} GB/s, "
            f"roofline {rec['roofline_frac']}")
        if rec["profile_workload"]:
            attach_counters(rec, load_counters(), None, nbytes)
        else:
            del rec["profile_workload"]
        out.append(rec)
        del co, fo
        torch.cuda.empty_cache()
    return out


CONVNEXT_C, CONVNEXT_HIDDEN = 512, 2048


def convnext_record(pkg, dev, steps, warmup) -> dict:
    """Sparse ConvNeXt block (conv -> LN -> Linear C->4C -> LN+SiLU -> Linear 4C->C + skip) on the
    wide128 voxels, bf16: ms per block, effective TFLOP/s (valid-tap conv + both linears)."""
    import torch

    wl = pkg.workloads
    coords = wl.make_coords("wide128_bf16")
    n = coords.shape[0]
    c, hid, dt = CONVNEXT_C, CONVNEXT_HIDDEN, torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(7)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dev).to(dt)
    x = pkg.SparseTensor(rnd(n, c), torch.from_numpy(coords).to(dev))
    blk = pkg.SparseConvNeXtBlock3d(torch.from_numpy(wl.conv_weight(c, c, 3)).to(dev).to(dt),
                                   rnd(c, scale=0.1), rnd(hid, c, scale=c ** -0.5),
                                   rnd(hid, scale=0.1), rnd(c, hid, scale=hid ** -0.5),
                                   rnd(c, scale=0.1))
    nmap = pkg.get_neighbor_map(x)
    nmap.conv_order()
    p = int((nmap.nbr >= 0).sum().item())
    ms = time_steps(lambda: blk(x), steps, warmup)
    ctx = pkg._lib.context(dev.index)
    kt = kernel_times(ctx, lambda: blk(x), 3)
    flops_conv = 2.0 * p * c * c
    flops_lin = 2.0 * 2 * n * c * hid
    lin_ms = kt.get("linear", (0.0, 0))[0] * kt.get("linear", (0.0, 0))[1]
    rec = {"workload": f"ConvNeXt block on wide128 ({n} voxels), C={c}, hidden={hid}, bf16",
           "profile_workload": "convnext",
           "voxels": n, "ms_per_block": round(ms, 4),
           "tflops_effective": round((flops_conv + flops_lin) / (ms / 1e3) / 1e12, 1),
           "linear_tflops": round(flops_lin / (lin_ms / 1e3) / 1e12, 1) if lin_ms else None,
           "bound": "mfma", "mfma_frac": round((flops_conv + flops_lin) / (ms / 1e3) / PEAK_MFMA["bfloat16"], 4),
           "kernels": {k: {"avg_ms": round(a, 4), "launches_per_step": cnt} for k, (a, cnt) in kt.items()}}
    log(f"convnext block: {ms:.4f} ms, {rec['tflops_effective']} TFLOP/s eff, "
        f"linears {rec['linear_tflops']} TFLOP/s")
    attach_counters(rec, load_counters())
    return rec


ATTN_HEADS, ATTN_DIM = 12, 128  # SLat flow transformer: 1536 channels, 12 heads


def attention_record(pkg, dev, steps) -> dict:
    """Varlen self-attention over the voxels of the resblock64 shells (2 sequences, one per
    sample), 12 heads x 128, as the SLat flow's blocks run it: ms per call, TFLOP/s (4*D flops per
    query-key pair and head), MFMA fraction; bf16 and fp32.  The CPU leg is the same attention in
    numpy fp32 (BLAS) on one head of 2048 queries against all keys of sample 0."""
    import numpy as np
    import torch

    wl = pkg.workloads
    coords = wl.make_coords("resblock64_bf16")
    counts = np.bincount(coords[:, 0])
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    n, h, d = int(cu[-1]), ATTN_HEADS, ATTN_DIM
    pairs = float((counts.astype(np.float64) ** 2).sum())
    flops = 4.0 * h * d * pairs
    g = torch.Generator(device="cpu").manual_seed(11)
    out = {"workload": f"varlen self-attention over the resblock64 voxels ({len(counts)} sequences, "
                       f"{n} tokens), {h} heads x {d}",
           "tokens": n, "sequences": [int(c) for c in counts], "flops_per_call": flops}
    ctx = pkg._lib.context(dev.index)
    for dt, name in ((torch.bfloat16, "bfloat16"), (torch.float32, "float32")):
        q, k, v = (torch.randn((n, h, d), generator=g).to(dev).to(dt) for _ in range(3))
        cu_d = torch.from_numpy(cu.astype(np.int32)).to(dev)
        o = torch.empty_like(q)

        def run():
            return pkg.sparse_attention(q, k, v, cu_d, out=o, max_seqlen_q=int(counts.max()))
        reps = steps if dt == torch.bfloat16 else max(2, steps // 8)
        ms = time_steps(run, reps, 2)
        kt = kernel_times(ctx, run, 2)
        tf = flops / (ms / 1e3)
        out[name] = {"ms": round(ms, 3), "tflops": round(tf / 1e12, 1),
                     "mfma_frac": round(tf / PEAK_MFMA[name], 4),
                     "kernels": {kk: {"avg_ms": round(a, 4), "launches_per_step": c}
                                 for kk, (a, c) in kt.items()}}
        if dt == torch.bfloat16:
            out[name]["profile_workload"] = "attention_bf16"
            attach_counters(out[name], load_counters(), flops)
        log(f"attention {name}: {ms:.3f} ms, {tf / 1e12:.1f} TFLOP/s, "
            f"{tf / PEAK_MFMA[name]:.3f} of MFMA peak")
        del q, k, v, o
        torch.cuda.empty_cache()
    rng = np.random.default_rng(0)
    nq, nk = 2048, int(counts[0])
    qh, kh, vh = (rng.standard_normal((m, d)).astype(np.float32) for m in (nq, nk, nk))
    t0 = time.perf_counter()
    s = qh @ kh.T * np.float32(d ** -0.5)
    s -= s.max(axis=1, keepdims=True)
    np.exp(s, out=s)
    s /= s.sum(axis=1, keepdims=True)
    _ = s @ vh
    tc = time.perf_counter() - t0
    out["cpu_numpy_fp32"] = {"tflops": round(4.0 * d * nq * nk / tc / 1e12, 4),
                             "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
                             "kind": "port",
                             "sample": f"1 head, {nq} queries x {nk} keys, numpy BLAS fp32"}
    return out


ST_TENSORS, ST_C = 24, 512
PEAK_HOST_LINK = 64e9  # B/s, PCIe 5.0 x16 host -> device, one direction


def safetensors_record(pkg, steps) -> dict:
    """Decoder-sized weight file (24 conv weights (512,3,3,3,512) bf16, 340 MB) streamed from a
    file in the page cache to the device: as stored (bf16) and converted to fp32 on the GPU.
    GB/s = file bytes / wall time of loading every tensor; the CPU leg is the reference's
    readTensorF32 (host read + bf16 -> f32 widening) restated in numpy, on 4 of the tensors."""
    import tempfile

    import numpy as np
    import torch
    from safetensors.torch import save_file

    from oracle import st_reader

    wl = pkg.workloads
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "decoder.safetensors")
        base = torch.from_numpy(wl.conv_weight(ST_C, ST_C, 9)).to(torch.bfloat16)
        save_file({f"blocks.{i}.conv.weight": base.roll(i, 0).contiguous() for i in range(ST_TENSORS)},
                  path)
        nbytes = os.path.getsize(path)
        res = {}
        with pkg.SafetensorsFile(path, "cuda:0") as sf:
            names = sf.list_tensors()
            for label, dt in (("bf16 as stored", None), ("bf16 -> fp32 on the GPU", torch.float32)):
                outs = []
                for _ in range(2):  # warm-up (pinned staging, workspace, page cache)
                    outs = [sf.read_tensor(n, dt) for n in names]
                torch.cuda.synchronize()
                del outs
                times = []
                for _ in range(max(3, steps // 4)):
                    t0 = time.perf_counter()
                    outs = [sf.read_tensor(n, dt) for n in names]
                    torch.cuda.synchronize()
                    times.append(time.perf_counter() - t0)
                    del outs
                t = statistics.median(times)
                res[label] = {"ms": round(t * 1e3, 2), "gbps": round(nbytes / t / 1e9, 2),
                              "host_link_frac": round(nbytes / t / PEAK_HOST_LINK, 4)}
                log(f"safetensors load ({label}): {t * 1e3:.1f} ms, {nbytes / t / 1e9:.2f} GB/s")
        sample = names[:4]
        st_reader.read_f32(path, sample[0])
        t0 = time.perf_counter()
        for n in sample:
            st_reader.read_f32(path, n)
        tc = time.perf_counter() - t0
        cpu_bytes = nbytes * len(sample) / len(names)
    return {"workload": f"safetensors weight file: {ST_TENSORS} conv weights ({ST_C},3,3,3,{ST_C}) "
                        f"bf16, {nbytes / 1e6:.0f} MB, page cache -> device",
            "file_bytes": nbytes, "loads": res, "bound": "host link (PCIe 5.0 x16, 64 GB/s)",
            "cpu_reference_reader": {"gbps": round(cpu_bytes / tc / 1e9, 2), "cores": 1,
                                     "kind": "port",
                                     "sample": f"{len(sample)} tensors, numpy read + bf16->f32 "
                                               f"widening (readTensorF32)"}}


def cpu_info(threads: int) -> dict:
    """Host facts recorded beside every CPU leg: threads used, os.cpu_count(), CPU model."""
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"torch_threads": threads, "os_cpu_count": os.cpu_count(), "cpu_model": model}


def conv_cpu_baseline(f_np, w_np, nbr, dtype: str, threads: int, budget_s: float = 20.0) -> dict:
    """The reference's conv_none restated in PyTorch-CPU (oracle/torch_path.py: per tap
    index_select of the valid neighbor rows -> mm with W[:,v,:]^T -> index_add), timed on this
    host: median of up to 3 runs after one warm-up, fewer when a run takes long (wall-clock).
    fp16 / bf16 inputs are rounded to that type and computed in fp32 (torch's CPU half matmuls
    are not a fair baseline)."""
    import torch

    from oracle import torch_path

    dts = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
    torch.set_num_threads(threads)
    f = torch.from_numpy(f_np).to(dts[dtype]).float()
    w = torch.from_numpy(w_np).to(dts[dtype]).float()
    nb = nbr.cpu() if hasattr(nbr, "cpu") else torch.from_numpy(nbr)
    times = []
    t_all = time.perf_counter()
    warm = True
    while len(times) < 3:
        t0 = time.perf_counter()
        torch_path.conv_none(f, w, None, nb, acc_dtype=torch.float32)
        dt = time.perf_counter() - t0
        if warm and dt < 2.0:  # short runs: the first one is a warm-up
            warm = False
            continue
        warm = False
        times.append(dt)
        if time.perf_counter() - t_all > budget_s:
            break
    t = statistics.median(times)
    rec = {"value": round(t * 1e3, 2), "unit": "ms/conv", "cores": threads, "kind": "port",
           "runs": len(times),
           "sample": f"full conv, conv_none restated in torch {torch.__version__} on the CPU "
                     f"(fp32 compute{'' if dtype == 'float32' else ' on ' + dtype + '-rounded inputs'})"}
    rec.update(cpu_info(threads))
    return rec


def cpu_baseline(coords_np, shape, threads: int) -> dict:
    import torch

    from oracle import torch_path

    torch.set_num_threads(threads)
    c = torch.from_numpy(coords_np)
    n = c.shape[0]
    torch_path.hashmap_fallback(c[:1000], shape)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch_path.hashmap_fallback(c, shape)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    rec = {"value": round(MAP_BYTES_PER_VOXEL * n / t / 1e9, 4), "unit": "GB/s", "cores": threads,
           "kind": "port", "ms": round(t * 1e3, 2),
           "sample": f"full map512 coordinate set (N={n}), torch.sort + 27 torch.searchsorted, "
                     f"median of 3 after a warm-up, torch {torch.__version__}"}
    rec.update(cpu_info(threads))
    return rec


def conv_record(name, ms, n, p, ci, co, dtype, extra=None) -> dict:
    s = 4 if dtype == "float32" else 2
    flops = 2.0 * p * ci * co
    nbytes = n * ci * s + n * co * s + 27 * ci * co * s + co * s + 108 * n
    t = ms / 1e3
    ideal = max(flops / PEAK_MFMA[dtype], nbytes / PEAK_HBM)
    bound = "mfma" if flops / PEAK_MFMA[dtype] >= nbytes / PEAK_HBM else "hbm"
    rec = {"workload": name, "dtype": dtype, "voxels": n, "valid_pairs": p, "ci": ci, "co": co,
           "ms_per_conv": round(ms, 4), "voxels_per_s": round(n / t, 1),
           "tflops_effective": round(flops / t / 1e12, 2), "gbps_algorithmic": round(nbytes / t / 1e9, 1),
           "bound": bound, "roofline_frac": round(ideal / t, 4),
           "mfma_frac": round(flops / t / PEAK_MFMA[dtype], 4)}
    if extra:
        rec.update(extra)
    return rec


def attach_counters(rec: dict, counters: dict, flops: float | None = None,
                    alg_bytes: float | None = None) -> None:
    """Add the rocprofv3 figures of the record's kernels, from the counter runs of the record's
    own workload (profiles/workload_counters.json): MFMA busy, executed MFMA TFLOP/s, clock, HBM
    bytes, the counter run's duration over this run's, and for the dominant kernel the executed
    MFMA work over the valid-tap work and the HBM bytes over the algorithmic bytes."""
    key = profile_key(rec)
    wl = counters.get(key)
    if not wl:
        return
    ks = rec.get("kernels", {})
    dom = max(ks, key=lambda k: ks[k]["avg_ms"] * ks[k]["launches_per_step"]) if ks else None
    got = {}
    symbols = [ROCPROF_NAME.get(k, k) for k in ks]
    for k, kr in ks.items():
        sym = ROCPROF_NAME.get(k, k)
        if symbols.count(sym) > 1:
            continue  # one kernel symbol for several launches of the record: not separable
        c = wl.get(sym)
        if not c:
            continue
        e = {key2: round(c[key2], 4) for key2 in ("mfma_busy", "mfma_tflops_hw", "clock_ghz", "avg_us")
             if key2 in c}
        for b in ("fetch_bytes", "write_bytes"):
            if b in c:
                e[b] = c[b]
        if kr.get("avg_ms"):
            e["counter_run_over_bench_duration"] = round(c["avg_us"] / 1e3 / kr["avg_ms"], 3)
        if k == dom and flops and c.get("mfma_tflops_hw"):
            # > 1: zero-padded taps were multiplied too
            e["mfma_work_over_algorithmic"] = round(c["mfma_tflops_hw"] * 1e12 * c["avg_us"] * 1e-6
                                                    / flops, 3)
        if k == dom and alg_bytes and "fetch_bytes" in c and "write_bytes" in c:
            e["hbm_bytes_over_algorithmic"] = round((c["fetch_bytes"] + c["write_bytes"]) / alg_bytes, 3)
        got[k] = e
    if got:
        rec["counters"] = {"source": "profiles/workload_counters.txt", "workload": key,
                           "kernels": got}


def copy_ceiling(dev, steps: int) -> dict:
    """A 1 GiB device-to-device copy (torch): the HBM rate this box sustains for a plain
    streaming kernel, counting the bytes read and the bytes written."""
    import torch

    a = torch.ones(1 << 28, dtype=torch.int32, device=dev)
    b = torch.empty_like(a)
    ms = time_steps(lambda: b.copy_(a), max(5, steps // 2), 3)
    nbytes = 2 * a.numel() * 4
    del a, b
    torch.cuda.empty_cache()
    rec = {"what": "torch copy of 1 GiB on the device (bytes read + written)", "ms": round(ms, 4),
           "gbps": round(nbytes / (ms / 1e3) / 1e9, 1),
           "hbm_frac": round(nbytes / (ms / 1e3) / PEAK_HBM, 4)}
    log(f"copy ceiling: {rec['gbps']} GB/s ({rec['hbm_frac']} of HBM peak)")
    return rec


def dense_gemm_ceiling(dev, m: int, k: int, n: int, steps: int) -> dict:
    """torch.matmul (hipBLASLt) in bf16 of a conv's implicit-GEMM shape with every tap present
    (M = voxels, K = 27 * Ci, N = Co): the rate the chip's own GEMM library sustains on the
    dense work of that shape, beside which the sparse conv's MFMA fraction is read."""
    import torch

    g = torch.Generator(device="cpu").manual_seed(3)
    a = torch.randn((m, k), generator=g, dtype=torch.float32).to(torch.bfloat16).to(dev)
    b = torch.randn((k, n), generator=g, dtype=torch.float32).to(torch.bfloat16).to(dev)
    ms = time_steps(lambda: torch.matmul(a, b), max(3, steps // 4), 2)
    flops = 2.0 * m * k * n
    del a, b
    torch.cuda.empty_cache()
    return {"what": "torch.matmul bf16 (hipBLASLt), dense implicit-GEMM shape of the conv",
            "shape_mkn": [m, k, n], "ms": round(ms, 4),
            "tflops": round(flops / (ms / 1e3) / 1e12, 1),
            "mfma_frac": round(flops / (ms / 1e3) / PEAK_MFMA["bfloat16"], 4)}


def secondary(pkg, dev, steps, warmup, map512_coords, cpu_threads=None, copy=None) -> list:
    import numpy as np
    import torch

    wl = pkg.workloads
    counters = load_counters()
    out = []
    dts = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
    for name in ("conv64_f32", "narrow512_f16", "narrow512s2_f16", "wide128_bf16",
                 "resblock64_bf16"):
        w = wl.WORKLOADS[name]
        coords = map512_coords if w.shell == "map512" else wl.make_coords(name)
        shape = wl.grid_shape(name)
        batch = int(coords[:, 0].max()) + 1
        c_dev = torch.from_numpy(coords).to(dev)
        nmap = pkg.build_neighbor_map(c_dev, shape, batch)
        n = coords.shape[0]
        p = int((nmap.nbr >= 0).sum().item())
        dt = dts[w.dtype]
        for ci, co in w.channels:
            f = torch.from_numpy(wl.features(n, ci, 1)).to(dev).to(dt)
            if name == "resblock64_bf16":
                ws = [(torch.from_numpy(wl.conv_weight(co, ci, 10 + i)).to(dev).to(dt),
                       torch.from_numpy(wl.conv_weight(co, ci, 20 + i)).to(dev).to(dt)) for i in range(4)]
                zero = torch.zeros(co, device=dev, dtype=dt)
                bufs = [torch.empty_like(f) for _ in range(2)]

                def chain():
                    h = f
                    for i, (w1, w2) in enumerate(ws):
                        h = pkg.sparse_resblock(h, nmap, w1, zero, w2, zero, eps=1e-6, out=bufs[i % 2])
                    return h
                ms = time_steps(chain, max(3, steps // 4), 2)
                rec = conv_record(name, ms / 8, n, p, ci, co, w.dtype,
                                  {"ms_per_chain": round(ms, 3), "chain": "4 x (conv-LN-SiLU-conv-+x)",
                                   "note": "ms_per_conv = chain time / 8 (LN+SiLU time included)"})
                kt = kernel_times(pkg._lib.context(dev.index), chain, 2)
            else:
                wt = torch.from_numpy(wl.conv_weight(co, ci, 2)).to(dev).to(dt)
                b = torch.zeros(co, device=dev, dtype=dt)
                o = torch.empty((n, co), device=dev, dtype=dt)

                def conv():
                    return pkg.sparse_conv3d(f, wt, b, nmap, out=o)
                ms = time_steps(conv, steps, warmup)
                rec = conv_record(name, ms, n, p, ci, co, w.dtype)
                kt = kernel_times(pkg._lib.context(dev.index), conv, 3)
                if name.startswith("narrow512"):
                    # the same conv without the gather plan: the direct kernel in the map's
                    # cached row order (what an order argument selects)
                    order = nmap.conv_order()
                    rec["unplanned_ms"] = round(time_steps(
                        lambda: pkg.sparse_conv3d(f, wt, b, nmap, order=order, out=o), steps,
                        warmup), 4)
                    log(f"  unplanned kernel (row order): {rec['unplanned_ms']} ms")
            rec["kernels"] = {k: {"avg_ms": round(a, 4), "launches_per_step": c} for k, (a, c) in kt.items()}
            s_el = 4 if w.dtype == "float32" else 2
            attach_counters(rec, counters, 2.0 * p * ci * co,
                            n * ci * s_el + n * co * s_el + 27 * ci * co * s_el + co * s_el + 108 * n)
            if rec["bound"] == "hbm" and copy:
                rec["frac_of_copy_ceiling"] = round(rec["gbps_algorithmic"] / copy["gbps"], 4)
            if rec["bound"] == "mfma" and w.dtype == "bfloat16":
                rec["dense_gemm_ceiling"] = dense_gemm_ceiling(dev, n, 27 * ci, co, steps)
                rec["frac_of_dense_gemm_ceiling"] = round(
                    rec["tflops_effective"] / rec["dense_gemm_ceiling"]["tflops"], 4)
                log(f"  dense GEMM ceiling {rec['dense_gemm_ceiling']['tflops']} TFLOP/s "
                    f"({rec['dense_gemm_ceiling']['mfma_frac']} of peak)")
            if cpu_threads:
                log(f"{name} {ci}->{co}: CPU conv_none baseline on {cpu_threads} threads ...")
                rec["cpu_baseline"] = conv_cpu_baseline(wl.features(n, ci, 1),
                                                        wl.conv_weight(co, ci, 2), nmap.nbr,
                                                        w.dtype, cpu_threads)
                log(f"  cpu: {rec['cpu_baseline']['value']} ms/conv")
            out.append(rec)
            log(f"{name} {ci}->{co} {w.dtype}: {rec['ms_per_conv']} ms/conv, "
                f"{rec['tflops_effective']} TFLOP/s eff, {rec['gbps_algorithmic']} GB/s, "
                f"roofline {rec['roofline_frac']}")
        del nmap, c_dev
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--profile-pass", action="store_true",
                    help="run one short fixed workload (--workload) for rocprofv3 runs and exit")
    ap.add_argument("--workload", default="map512", choices=PROFILE_WORKLOADS,
                    help="the --profile-pass workload")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build's sparse-conv path runs on a single "
              "MI355X (multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    if args.profile_pass:
        profile_pass(pkg, dev, args.workload)
        return 0
    wl = pkg.workloads
    t0 = time.time()
    coords = wl.make_coords("map512")
    shape = wl.grid_shape("map512")
    n = coords.shape[0]
    log(f"map512: N={n} voxels generated in {time.time() - t0:.1f}s")
    c_dev = torch.from_numpy(coords).to(dev)
    nmap = pkg.build_neighbor_map(c_dev, shape, 1)  # validated once (duplicates / range)
    torch.cuda.synchronize()

    def step():
        return pkg.build_neighbor_map(c_dev, shape, 1, validate=False)

    ms = time_steps(step, args.steps, args.warmup)
    log(f"map build: {ms:.4f} ms/step, {MAP_BYTES_PER_VOXEL * n / ms / 1e6:.1f} GB/s algorithmic")
    ctx = pkg._lib.context(dev.index)
    kt = kernel_times(ctx, step, args.steps)
    dom = max(kt, key=lambda k: kt[k][0] * kt[k][1])
    dom_ms = kt[dom][0]
    per_voxel = MAP_KERNEL_BYTES.get(dom)
    achieved = (per_voxel * n / (dom_ms / 1e3)) if per_voxel else None
    counters = load_counters()
    traffic = load_traffic(counters, "map512", dom)
    roofline = {"kernel": dom, "bound": "hbm",
                "achieved": round(achieved / 1e9, 1) if achieved else None, "peak": PEAK_HBM / 1e9,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4) if achieved else None,
                "traffic": traffic, "avg_ms": round(dom_ms, 4),
                "alg_bytes_per_launch": per_voxel * n if per_voxel else None,
                "kernels": {k: {"avg_ms": round(a, 4), "launches_per_step": c} for k, (a, c) in kt.items()}}
    log(f"dominant kernel {dom}: {dom_ms:.4f} ms; all: " +
        ", ".join(f"{k}={a:.4f}" for k, (a, c) in kt.items()))
    roofline["write_floor"] = write_floor_record(ctx, nmap, n, dom_ms, args.steps)
    copy = copy_ceiling(dev, args.steps)
    roofline["copy_ceiling"] = copy
    if achieved:
        roofline["frac_of_copy_ceiling"] = round(achieved / 1e9 / copy["gbps"], 4)
    roofline["build_frac_of_copy_ceiling"] = round(MAP_BYTES_PER_VOXEL * n / (ms / 1e3) / 1e9
                                                   / copy["gbps"], 4)
    roofline["profile_workload"] = "map512"
    attach_counters(roofline, load_counters(), None, per_voxel * n if per_voxel else None)
    # One-time per coordinate set, cached with the map: the row order the convs use.
    order_ms = time_steps(lambda: pkg.map_conv_order(nmap.nbr, nmap.perm), args.steps, args.warmup)
    log(f"conv row order (tsc_map_conv_order): {order_ms:.4f} ms")
    plan_ms = time_steps(lambda: pkg.map_gather_plan(c_dev, nmap.nbr, 1, shape), args.steps,
                         args.warmup)
    log(f"narrow-conv gather plan (tsc_map_gather_plan): {plan_ms:.4f} ms")
    del nmap
    sec = []
    if not args.no_secondary:
        sec = secondary(pkg, dev, args.steps, args.warmup, coords,
                        None if args.no_cpu_baseline else args.cpu_threads, copy)
        for r in subdivide_records(pkg, dev, args.steps, args.warmup):
            r["frac_of_copy_ceiling"] = round(r["gbps_algorithmic"] / copy["gbps"], 4)
            sec.append(r)
        sec.append(convnext_record(pkg, dev, args.steps, args.warmup))
        sec.append(attention_record(pkg, dev, args.steps))
        sec.append(safetensors_record(pkg, args.steps))
    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline on {args.cpu_threads} threads ...")
        cpu = cpu_baseline(coords, shape, args.cpu_threads)
        log(f"cpu baseline: {cpu['ms']} ms ({cpu['value']} GB/s)")
    line = {
        "metric": METRIC, "value": round(MAP_BYTES_PER_VOXEL * n / (ms / 1e3) / 1e9, 2), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int32",
        "data": "synthetic",
        "config": {"workload": f"map512: neighbor-map build, {n} voxels, 1-voxel shell of a perturbed "
                               f"ellipsoid in 512^3, shuffled rows, 3x3x3 dilation 1",
                   "voxels": n, "grid": list(shape), "batch": 1,
                   "bytes_per_voxel_algorithmic": MAP_BYTES_PER_VOXEL},
        "roofline": roofline, "cpu_baseline": cpu,
        "map_prep": {"conv_order_ms": round(order_ms, 4), "gather_plan_ms": round(plan_ms, 4),
                     "map_ready_ms": round(ms + order_ms, 4),
                     "map_ready_narrow_ms": round(ms + plan_ms, 4),
                     "note": "tsc_map_conv_order and tsc_map_gather_plan, once per coordinate set "
                             "(cached with the map); not part of ms_per_step.  map_ready = build + "
                             "row order (what a wide conv needs first), map_ready_narrow = build + "
                             "gather plan (what a narrow 16-bit conv needs first)"},
        "secondary": sec,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
