"""Benchmark of the fused 28-field embedding-bag step on one MI355X.

A step pools one batch of the bf16-2m workload: 28 fields, bf16 tables of 2,000,000 x 128,
B = 4096 samples, geometric(mean 8) bag lengths, Zipf(1.1) ids, mean pooling, bf16 output
[4096, 28*128]. Tables and several independently seeded index sets (each with its own hot rows)
are resident in HBM before timing; step k uses index set k mod n_sets, so consecutive steps do
not find each other's rows in L2 / MALL.

`--int8` row-quantises every table on the device first (online_best/infer.py:895-901) and pools
the int8 rows with their fp32 scales (online_best/infer.py:904-942); the algorithmic bytes count
1 byte per element plus the 4-byte scale of each looked-up row.

`--stage h2d` measures the step end to end from host memory (online_best/infer.py:742-779): each
step moves one flat-layout batch (int64 ids and offsets in pageable host memory, as the collate
leaves them) to the GPU and pools it with the reference launch (one shared table, sum), through
(a) the reference's `.to(device, non_blocking=True)`, (b) the pinned, double-buffered InputStager
with int64 inputs, (c) the same with ids and offsets narrowed to int32 on the host. The line
reports bags/s per variant, the copy-only and pool-only times, and the bytes moved per batch.

`--stage encoder` times the encoder's front end on the workload's batches (reference layout, one
shared table as in the reference, sum pooling, online_best/infer.py:1050-1085): RepEncoder.forward's
order (pooling, the LayerNorm kernel in place, torch's Linear(28*D -> 512)) is the line's value;
beside it the LayerNorm statistics with the matrix-core kernel that normalises the pooled block's
tiles as it loads them and multiplies them with the Linear's weight, and the pooling with the
LayerNorm fused into it followed by torch's Linear; each kernel alone too.

`--stage layout` times the device layout kernels against the reference's way of doing the same
work: merging the 8 sub-batches of lazy-32k into one flat layout (online_best/infer.py:581-631,
torch ops on host tensors there; one kernel over device tensors here) and packing 28 per-slot
(values, offsets) pairs of a bf16-2m batch into the flat layout (online_best/infer.py:960-974,
two torch.cat and a host list copied to the device there; one kernel here).

`--stage small` times the reference's small-batch call pattern (online_best/infer.py:2849-2863,
:2689): wall-clock µs per call of the drop-in launch at B in {2, 128, 512, 1024} with length-1
bags (Python checks included; the raw C call; a HIP-graph replay; RepEncoder.pooled / forward
on the per-slot batch), and lazy-32k's sub-batches pooled call by call against one merged call.

`--stage layernorm` times the encoder's input LayerNorm instead (online_best/infer.py:1061-1076):
the workload's batches are pooled once, and each step normalises one pooled block
[B, sum(D)] (rows/s; roofline bytes = the block read and written plus gamma and beta).

Printed (one JSON line): pooled bags/s over the timed steps, plus
  roofline     HBM bytes per launch / mean launch duration (one pair of HIP events around the
               K timed launches, on the stream the kernels run on), against 8 TB/s: `traffic` is
               the HBM traffic per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE summary
               committed under profiles/ (`achieved` and `frac` are null when it is absent);
               `effective_gbs` / `effective_frac` count every lookup's row (the algorithmic
               bytes, which L2 / MALL hits let pass the peak), `compulsory_*` each distinct row
               once
  plain_launch the same steps without a dispatch order (when the batches carry one)
  cpu_baseline the reference's CPU pooling loop (F.embedding_bag per field, the oracle's
               restatement) on this host, on a bounded sample of the same batch
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "pooled bags/sec + achieved HBM GB/s (% of peak), B=4096×28 fields, D=128 bf16"
WORKLOAD_TEXT = {
    "bf16-2m": "28 fields, bf16 tables 2,000,000 x 128, B=4096, geometric(mean 8) bag lengths clipped to "
               "[0, 256], Zipf(1.1) ids, mean pooling, bf16 output [4096, 28, 128]",
    "fp32-1m": "28 fields, fp32 tables 1,000,000 x 128, B=4096, geometric(mean 8) lengths, Zipf(1.1) ids, sum",
    "hetero-bf16": "28 fields, bf16 tables of width 32/64/128, log-uniform vocab [1e3, 5e6], B=8192, "
                   "20 Poisson(2) + 8 lognormal(median 64, max 2048) fields, sum",
    "lazy-32k": "28 fields, bf16 tables 4,000,000 x 128, B=32768 from 8 merged sub-batches, Zipf(0.8), mean",
    "small-fp32": "28 fields, fp32 tables 10,000 x 64, B=256, Poisson(3) lengths, sum",
    "reference-5m": "28 slots over one shared bf16 table 5,000,000 x 512 (the reference's nn.Embedding), B=4096, "
                    "geometric(mean 8) lengths, Zipf(1.1) ids, sum, bf16 output [4096, 28*512]",
}
# Workloads whose launches end faster when tiles start longest-first (the order is made one step
# ahead inside the previous launch). lazy-32k is slower with it (its launch is DRAM-bound and the
# reordered tiles read values out of address order), small-fp32 too (launch-bound), int8 unchanged.
ORDERED_BY_DEFAULT = {"bf16-2m", "fp32-1m"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_from_profiles(workload, kernel="pool_kernel", keys=("hbm_bytes_per_launch",)):
    """HBM bytes per launch recorded by the rocprofv3 counter runs, read from the first of the
    lines `<key>: N` (in the order of `keys`) of profiles/<kernel>_<workload>.md, as
    (bytes, "profiles/<file>") or (None, None)."""
    name = f"{kernel}_{workload}.md"
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None, None
    with open(path) as fh:
        lines = [line.strip() for line in fh]
    for key in keys:
        for line in lines:
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1].strip()), f"profiles/{name}"
    return None, None


def roofline(nbytes, launch_s, kernel, traffic_key=None, compulsory_bytes=None, streaming=False, **extra):
    """The bench line's roofline object for one kernel launch of `launch_s` seconds (mean).

    `achieved` / `frac` are HBM bytes moved per second against the 8 TB/s peak: the HBM traffic
    the rocprofv3 FETCH_SIZE / WRITE_SIZE passes measured for one launch of the same kernel and
    workload (`traffic`, read from `traffic_source`), or, for a streaming kernel that reads and
    writes each of its bytes once (`streaming`), its algorithmic bytes. Without either, `achieved`
    is null. `effective_gbs` / `effective_frac` count every lookup's row (the algorithmic bytes
    `nbytes`, most of them served by L2 / MALL under Zipf ids, so they can pass the peak), and
    `compulsory_gbs` / `compulsory_frac` each distinct row once."""
    traffic, source = traffic_from_profiles(*traffic_key) if traffic_key else (None, None)
    if traffic is None and streaming:
        traffic, source = nbytes, "algorithmic bytes (each byte read or written once)"
    achieved = traffic / launch_s / 1e9 if traffic else None
    rec = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": achieved / HBM_PEAK_GBS if achieved else None, "traffic": traffic,
           "traffic_source": source, "kernel": kernel, "launch_us_mean": launch_s * 1e6,
           "bytes_per_launch": nbytes, "effective_gbs": nbytes / launch_s / 1e9,
           "effective_frac": nbytes / launch_s / 1e9 / HBM_PEAK_GBS}
    if compulsory_bytes is not None:
        rec.update(compulsory_bytes_per_launch=compulsory_bytes, compulsory_gbs=compulsory_bytes / launch_s / 1e9,
                   compulsory_frac=compulsory_bytes / launch_s / 1e9 / HBM_PEAK_GBS)
    rec.update(extra)
    return rec


def host_cpus():
    """The host's CPU counts: logical CPUs, the ones this process may run on, physical cores, and
    the CPU share its cgroup grants (cpu.max quota / period), when these are visible."""
    info = {"logical": os.cpu_count()}
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        info["affinity"] = info["logical"]
    try:
        import psutil

        info["physical"] = psutil.cpu_count(logical=False)
    except Exception:  # psutil missing or unable to read the topology
        info["physical"] = None
    info["cgroup_share"] = None
    for path in ("/sys/fs/cgroup/cpu.max", "/sys/fs/cgroup/cpu/cpu.cfs_quota_us"):
        try:
            with open(path) as fh:
                parts = fh.read().split()
            if path.endswith("cpu.max") and parts[0] != "max":
                info["cgroup_share"] = float(parts[0]) / float(parts[1])
            elif path.endswith("quota_us") and int(parts[0]) > 0:
                with open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as fh:
                    info["cgroup_share"] = int(parts[0]) / int(fh.read())
            break
        except (OSError, ValueError, IndexError):
            continue
    return info


def cpu_baseline(wl, tables_dev, seconds):
    """Time the reference's CPU pooling on this host, on host tables holding the rows this batch
    reads (full-size tables, untouched rows left as zero pages): the oracle's F.embedding_bag loop
    (the reported baseline) and the literal baseline loop (clamp + F.embedding + segment_reduce +
    cat, baseline/infer.py:256-263), each pass timed separately for about `seconds` / 2 of CPU work
    (at least 5 passes); medians are reported."""
    import numpy as np
    import torch

    from oracle import cpu_loops

    cpus = host_cpus()
    # every CPU this process may run on, capped by the CPU share its cgroup grants (threads beyond
    # the share only queue for it)
    threads = cpus["affinity"] or 1
    if cpus["cgroup_share"]:
        threads = max(1, min(threads, int(cpus["cgroup_share"])))
    torch.set_num_threads(threads)
    host = []
    for f, t in enumerate(tables_dev):
        s, e = int(wl.offsets[f * wl.batch]), int(wl.offsets[(f + 1) * wl.batch])
        rows = np.unique(np.clip(wl.values[s:e], 0, wl.vocab[f] - 1))
        data = t.index_select(0, torch.from_numpy(rows).to(t.device)).cpu()
        if t.dtype == torch.float32:
            h = torch.from_numpy(np.zeros(tuple(t.shape), np.float32))
        else:
            h = torch.from_numpy(np.zeros(tuple(t.shape), np.int16)).view(t.dtype)
        h[torch.from_numpy(rows)] = data
        host.append(h)
    values = torch.from_numpy(wl.values)
    offsets = torch.from_numpy(wl.offsets)

    def timed(loop):
        loop(values, offsets, host, wl.pooling, wl.batch)  # warm-up
        times, t_start = [], time.perf_counter()
        while len(times) < 5 or (time.perf_counter() - t_start < seconds / 2 and len(times) < 100_000):
            t0 = time.perf_counter()
            loop(values, offsets, host, wl.pooling, wl.batch)
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times), time.perf_counter() - t_start

    med_bag, n_bag, el_bag = timed(cpu_loops.embedding_bag_loop)
    med_lit, n_lit, el_lit = timed(cpu_loops.baseline_loop)
    return {"value": wl.num_bags / med_bag, "unit": "bags/s", "cores": threads, "kind": "port",
            "host_logical_cpus": cpus["logical"], "host_physical_cores": cpus["physical"],
            "process_affinity_cpus": cpus["affinity"], "cgroup_cpu_share": cpus["cgroup_share"],
            "sample": f"median of {n_bag} full passes ({el_bag:.1f} s) of the timed batch ({wl.num_bags} bags) "
                      f"through F.embedding_bag per field (oracle/cpu_loops.py), {wl.table_dtype} tables in host "
                      f"memory, torch intra-op threads = {threads}",
            "baseline_loop": {"value": wl.num_bags / med_lit, "unit": "bags/s",
                              "sample": f"median of {n_lit} passes ({el_lit:.1f} s) of the literal loop: clamp + "
                                        "F.embedding + segment_reduce + cat (baseline/infer.py:256-263)"}}


def bench_h2d(args, pkg, wls, dev):
    """End-to-end steps from host flat-layout batches: transfer + the reference pooling launch."""
    import numpy as np
    import torch

    wl0 = wls[0]
    F, B, D = wl0.num_fields, wl0.batch, wl0.dims[0]
    V = max(wl0.vocab)
    host = []
    for wl in wls:
        off = wl.offsets
        ro = np.stack([off[f * B:(f + 1) * B + 1] - off[f * B] for f in range(F)]).reshape(-1)
        vo = off[0:F * B:B].copy()
        host.append({"_flat_values": torch.from_numpy(wl.values.copy()), "_flat_row_offsets": torch.from_numpy(ro),
                     "_val_offsets": torch.from_numpy(vo)})
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    weight = torch.empty((V, D), dtype=wl0.table_dtype, device=dev)
    weight.normal_(0.0, 0.01, generator=g)
    out = torch.empty((B, F * D), dtype=wl0.table_dtype, device=dev)
    max_nnz = max(h["_flat_values"].numel() for h in host)
    n = len(host)

    def pool(db):
        pkg.fused_all_slots_embedding(db["_flat_values"], db["_val_offsets"], db["_flat_row_offsets"], weight, out,
                                      B, D, V - 1, tile_order=db.get("_tile_order"))

    def run(step, K, W):
        for i in range(W):
            step(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(K):
            step(W + i)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / K

    results = {}

    def reference(i):
        pool(pkg.move_model_inputs_to_device(host[i % n], dev, F))

    log("reference transfer (.to(device, non_blocking=True) of pageable int64)")
    results["reference_pageable_int64"] = run(reference, args.steps, args.warmup)
    # host batches whose producer already emits int32 (saturated) ids and offsets
    host32 = []
    for h in host:
        h32 = {}
        for k, t in h.items():
            d = torch.empty(t.numel(), dtype=torch.int32)
            pkg._capi.check(pkg._capi.lib().cti_ebag_narrow_ids(t.data_ptr(), t.numel(), d.data_ptr(), 16))
            h32[k] = d
        host32.append(h32)
    # the same int32 batches with the order their producer made (a collate in DataLoader workers
    # would make it beside the flat layout, off the serving thread)
    host32o = [dict(h, _tile_order=pkg.make_tile_order(h["_flat_row_offsets"], B, F, wl0.table_dtype, D))
               for h in host32]
    for name, compact, src, order in (("pinned_int64_overlapped", False, host, False),
                                      ("pinned_int32_overlapped", True, host, False),
                                      ("pinned_int32_from_int32_overlapped", True, host32, False),
                                      ("pinned_int32_ordered_overlapped", True, host, True),
                                      ("pinned_int32_from_int32_with_order_overlapped", True, host32o, True)):
        stager = pkg.InputStager(max_nnz, F, B, dev, depth=2, compact=compact,
                                 order_for=(wl0.table_dtype, D) if order else None)

        def staged(i, stager=stager, src=src):
            db = pkg.move_model_inputs_to_device(src[i % n], dev, F, stager=stager)
            pool(db)
            stager.release(db)

        def copy_only(i, stager=stager, src=src):
            stager.release(stager.stage(src[i % n]))

        log(name)
        results[name] = run(staged, args.steps, args.warmup)
        results[name.replace("overlapped", "copy_only")] = run(copy_only, args.steps, args.warmup)
        torch.cuda.synchronize()
        del stager
    # the DMA alone: host data already in pinned buffers
    for width, dt in ((8, torch.int64), (4, torch.int32)):
        hbuf = torch.empty(max_nnz + F * (B + 2), dtype=dt, pin_memory=True)
        dbuf = torch.empty_like(hbuf, device=dev)
        results[f"dma_only_int{width * 8}"] = run(lambda i: dbuf.copy_(hbuf, non_blocking=True), args.steps,
                                                  args.warmup)
        del hbuf, dbuf
    resident = [pkg.move_model_inputs_to_device(h, dev, F) for h in host]
    results["pool_only_resident_int64"] = run(lambda i: pool(resident[i % n]), args.steps, args.warmup)
    # the same resident batches, each with the order its collate would make on the host
    for h, r in zip(host, resident):
        r["_tile_order"] = pkg.make_tile_order(h["_flat_row_offsets"], B, F, wl0.table_dtype, D).to(dev)
    results["pool_only_resident_int64_ordered"] = run(lambda i: pool(resident[i % n]), args.steps, args.warmup)
    bags = wl0.num_bags
    nnz_mean = float(np.mean([h["_flat_values"].numel() for h in host]))
    bytes64 = 8 * (nnz_mean + F * (B + 1) + F)
    best = min(("reference_pageable_int64", "pinned_int64_overlapped", "pinned_int32_overlapped",
                "pinned_int32_from_int32_overlapped", "pinned_int32_ordered_overlapped",
                "pinned_int32_from_int32_with_order_overlapped"), key=lambda k: results[k])
    rec = {
        "metric": "end-to-end pooled bags/sec from host flat-layout batches (H2D + pooling), B=4096x28 fields, D=128 bf16",
        "value": bags / results[best],
        "unit": "bags/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": results[best] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic: {n} seeded index sets rotated, host batches in pageable int64 tensors",
        "config": {"workload": f"{args.workload}: {WORKLOAD_TEXT[args.workload]}; one shared table "
                               f"[{V}, {D}], sum (the reference launch)", "best_variant": best},
        "us_per_step": {k: v * 1e6 for k, v in results.items()},
        "bags_per_s": {k: bags / v for k, v in results.items()},
        "h2d_bytes_per_batch": {"int64": bytes64, "int32": bytes64 / 2},
    }
    print(json.dumps(rec), flush=True)


def bench_encoder(args, pkg, wls, dev):
    """Pooling + input LayerNorm: two kernels against the fused kernel (reference layout)."""
    import numpy as np
    import torch

    wl0 = wls[0]
    F, B, D = wl0.num_fields, wl0.batch, wl0.dims[0]
    V = max(wl0.vocab)
    batches = []
    for wl in wls:
        off = wl.offsets
        ro = np.stack([off[f * B:(f + 1) * B + 1] - off[f * B] for f in range(F)]).reshape(-1)
        batches.append((torch.from_numpy(wl.values).to(dev), torch.from_numpy(off[0:F * B:B].copy()).to(dev),
                        torch.from_numpy(ro).to(dev)))
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    weight = torch.empty((V, D), dtype=wl0.table_dtype, device=dev)
    weight.normal_(0.0, 0.01, generator=g)
    gamma = torch.empty(F * D, dtype=wl0.table_dtype, device=dev).normal_(1.0, 0.1, generator=g)
    beta = torch.empty(F * D, dtype=wl0.table_dtype, device=dev).normal_(0.0, 0.1, generator=g)
    out = torch.empty((B, F * D), dtype=wl0.table_dtype, device=dev)
    n = len(batches)

    # each batch's dispatch order, as its collate would make it on the host from the offsets
    orders = [pkg.make_tile_order(ro.cpu(), B, F, wl0.table_dtype, D).to(dev) for _, _, ro in batches]

    def pool_plain(i):
        v, vo, ro = batches[i % n]
        pkg.fused_all_slots_embedding(v, vo, ro, weight, out, B, D, V - 1)

    def pool_ordered(i):
        v, vo, ro = batches[i % n]
        pkg.fused_all_slots_embedding(v, vo, ro, weight, out, B, D, V - 1, tile_order=orders[i % n])

    def separate(i):
        v, vo, ro = batches[i % n]
        pkg.fused_all_slots_embedding(v, vo, ro, weight, out, B, D, V - 1, tile_order=orders[i % n])
        pkg.layer_norm(out, gamma, beta, 1e-5, out=out)

    def fused(i):
        v, vo, ro = batches[i % n]
        pkg.fused_all_slots_embedding_layernorm(v, vo, ro, weight, out, B, D, V - 1, gamma, beta, 1e-5)

    def timed(step):
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.steps):
            step(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps / 1e3

    # the encoder's Linear(F*D -> d_model) after the LayerNorm (online_best/infer.py:1085, nn.Linear
    # of the reference's model, d_model = 512)
    d_model = 512
    lin_w = torch.empty((d_model, F * D), dtype=torch.bfloat16, device=dev).normal_(0.0, (F * D) ** -0.5, generator=g)
    lin_b = torch.empty(d_model, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.1, generator=g)
    y = torch.empty((B, d_model), dtype=torch.bfloat16, device=dev)
    mean = torch.empty(B, dtype=torch.float32, device=dev)
    rstd = torch.empty(B, dtype=torch.float32, device=dev)
    gamma_b, beta_b = gamma.to(torch.bfloat16), beta.to(torch.bfloat16)

    def front_mfma(i):  # RepEncoder.forward(fused_linear=True): pooling, statistics, LayerNorm inside the Linear
        pool_ordered(i)
        pkg.layer_norm_stats(out, 1e-5, mean, rstd)
        pkg.layer_norm_linear(out, lin_w, lin_b, mean=mean, rstd=rstd, norm_weight=gamma_b, norm_bias=beta_b, out=y)

    def front_fused_norm_torch_linear(i):  # pooling + LayerNorm in one kernel, then torch's Linear
        fused(i)
        torch.nn.functional.linear(out, lin_w, lin_b)

    def front_separate_torch_linear(i):  # RepEncoder.forward: pooling, the LayerNorm kernel, torch's Linear
        separate(i)
        torch.nn.functional.linear(out, lin_w, lin_b)

    def ln_linear_only(i):
        pkg.layer_norm_linear(out, lin_w, lin_b, mean=mean, rstd=rstd, norm_weight=gamma_b, norm_bias=beta_b, out=y)

    def torch_linear_only(i):
        torch.nn.functional.linear(out, lin_w, lin_b)

    def stats_only(i):
        pkg.layer_norm_stats(out, 1e-5, mean, rstd)

    log("drop-in pooling, plain and with host-made orders")
    t_plain = timed(pool_plain)
    t_ordered = timed(pool_ordered)
    log("pooling then LayerNorm")
    t_sep = timed(separate)
    log("fused")
    t_fused = timed(fused)
    log("front end with the Linear: torch's Linear after the LayerNorm, and statistics + LayerNorm-Linear kernel")
    t_front = timed(front_mfma)
    t_front_torch = timed(front_fused_norm_torch_linear)
    t_front_sep = timed(front_separate_torch_linear)
    pool_ordered(0)
    pkg.layer_norm_stats(out, 1e-5, mean, rstd)
    t_lin = timed(ln_linear_only)
    t_tlin = timed(torch_linear_only)
    t_stats = timed(stats_only)
    # the pooling's algorithmic bytes with the reference layout's offsets (row offsets + slot bases)
    pool_bytes = float(np.mean([wl.bytes_algorithmic() - wl.offsets.size * 8 + (F * (B + 1) + F) * 8 for wl in wls]))
    fused_bytes = pool_bytes + 2 * F * D * 2  # + gamma and beta
    lin_flops = 2.0 * B * d_model * F * D
    lin_bytes = B * F * D * 2 + d_model * F * D * 2 + B * d_model * 2 + B * 8
    log(f"front end {t_front_sep * 1e6:.1f} us (pooling, LayerNorm kernel, torch Linear; with the LayerNorm-Linear "
        f"kernel {t_front * 1e6:.1f}; pool+LN fused then torch Linear {t_front_torch * 1e6:.1f}); LayerNorm-Linear "
        f"{t_lin * 1e6:.1f} us = {lin_flops / t_lin / 1e12:.0f} TFLOP/s, torch Linear {t_tlin * 1e6:.1f} us")
    rec = {
        "metric": f"encoder front end rows/sec (pooling, input LayerNorm, Linear({F * D}->{d_model})), "
                  f"B={B}x{F} fields, D={D} bf16",
        "value": B / t_front_sep,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_front_sep * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic: {n} seeded index sets rotated, one shared N(0, 0.01) table [{V}, {D}], "
                "gamma ~ N(1, 0.1), beta ~ N(0, 0.1), Linear weight ~ N(0, 1/K), bias ~ N(0, 0.1)",
        "config": {"workload": f"{args.workload}: {WORKLOAD_TEXT[args.workload]}; reference layout, one shared "
                               f"table, sum pooling, LayerNorm over [B, {F * D}], Linear to {d_model}"},
        "us_per_step": {"front_end_pool_then_layernorm_then_torch_linear": t_front_sep * 1e6,
                        "front_end_pool_stats_layernorm_linear": t_front * 1e6,
                        "front_end_pool_layernorm_fused_then_torch_linear": t_front_torch * 1e6,
                        "layernorm_linear_kernel": t_lin * 1e6, "torch_linear": t_tlin * 1e6,
                        "layernorm_statistics": t_stats * 1e6,
                        "pool_then_layernorm": t_sep * 1e6, "fused_pool_layernorm": t_fused * 1e6,
                        "pool_drop_in": t_plain * 1e6, "pool_drop_in_host_order": t_ordered * 1e6},
        "roofline": {"bound": "mfma", "kernel": "ln_linear_kernel", "achieved": lin_flops / t_lin / 1e12,
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": lin_flops / t_lin / 1e12 / 2500.0,
                     "flops_per_launch": lin_flops, "launch_us_mean": t_lin * 1e6,
                     "hbm_bytes_per_launch_algorithmic": lin_bytes,
                     "hbm_gbs_algorithmic": lin_bytes / t_lin / 1e9,
                     "traffic": traffic_from_profiles(args.workload + "-shared", "ln_linear_kernel")[0],
                     "torch_linear_tflops": lin_flops / t_tlin / 1e12},
        "roofline_fused_pool_layernorm": roofline(fused_bytes, t_fused, "pool_norm_kernel",
                                                  (args.workload + "-shared", "pool_norm_kernel")),
        "cpu_baseline": None,
    }
    print(json.dumps(rec), flush=True)


def reference_layout(wl, dev):
    """(values, val_offsets, row_offsets) of a workload in the reference's flat layout, on dev."""
    import numpy as np
    import torch

    F, B = wl.num_fields, wl.batch
    off = wl.offsets
    ro = np.stack([off[f * B:(f + 1) * B + 1] - off[f * B] for f in range(F)]).reshape(-1)
    return (torch.from_numpy(wl.values).to(dev), torch.from_numpy(off[0:F * B:B].copy()).to(dev),
            torch.from_numpy(ro).to(dev))


def bench_reference(args, pkg, dev):
    """The reference's own shape: 28 slots over one shared bf16 [5,000,000, 512] table (5.12 GB,
    so rows past 4 GiB are addressed with 64-bit offsets), reference layout, sum: the drop-in
    pooling launch, pooling with the input LayerNorm over 14,336 columns fused, and the int8
    table. A second leg compares the two addressing paths on identical batches: ids below
    4,194,303 pooled from the 5M-row table (64-bit addresses) and from a 4,194,303-row table
    (which fits the 32-bit buffer path)."""
    import numpy as np
    import torch

    W = pkg.workloads
    V, D, F = 5_000_000, 512, 28
    log(f"reference-5m: generating {args.sets} index sets")
    wls = [W.make("reference-5m", seed=s) for s in range(1, args.sets + 1)]
    B = wls[0].batch
    batches = [reference_layout(wl, dev) for wl in wls]
    log("filling the shared [5,000,000, 512] bf16 table")
    weight = W.make_tables(wls[0], dev, seed=0)[0]
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    gamma = torch.empty(F * D, dtype=torch.bfloat16, device=dev).normal_(1.0, 0.1, generator=g)
    beta = torch.empty(F * D, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.1, generator=g)
    out = torch.empty((B, F * D), dtype=torch.bfloat16, device=dev)
    n = len(batches)

    def timed(step):
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.steps):
            step(args.warmup + i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps / 1e3

    def pool(i, w=weight, bs=batches):
        v, vo, ro = bs[i % len(bs)]
        pkg.fused_all_slots_embedding(v, vo, ro, w, out, B, D, w.shape[0] - 1)

    def fused(i):
        v, vo, ro = batches[i % n]
        pkg.fused_all_slots_embedding_layernorm(v, vo, ro, weight, out, B, D, V - 1, gamma, beta, 1e-5)

    legs = set(args.legs.split(","))
    us = {}
    if "pool" in legs:
        log("drop-in pooling")
        us["pool"] = timed(pool) * 1e6
    if "fused" in legs:
        log("pooling + LayerNorm fused")
        us["pool_layernorm_fused"] = timed(fused) * 1e6

    def pool_int8(i):
        v, vo, ro = batches[i % n]
        pkg.fused_all_slots_embedding_int8(v, vo, ro, q, sc, out, B, D, V - 1)

    if "int8" in legs:
        log("quantising the table to int8")
        q, sc = pkg.quantize_embedding_int8(weight)
        log("int8 pooling")
        us["pool_int8"] = timed(pool_int8) * 1e6
        del q, sc
        torch.cuda.empty_cache()

    wl4 = []
    if "addressing" in legs:
        # the addressing paths on identical batches: ids < 4,194,303 (so no clamp differs)
        V4 = (1 << 32) // (D * 2) - 1
        log("addressing paths: index sets over 4,194,303 rows")
        wl4 = [W.make("reference-5m", seed=s, vocab=V4) for s in range(1, args.sets + 1)]
        b4 = [reference_layout(wl, dev) for wl in wl4]
        us["pool_64bit_addresses_ids_below_4gib"] = timed(lambda i: pool(i, weight, b4)) * 1e6
        del weight
        torch.cuda.empty_cache()
        w4 = torch.empty((V4, D), dtype=torch.bfloat16, device=dev).normal_(0.0, 0.01, generator=g)
        us["pool_buffer_path_table_below_4gib"] = timed(lambda i: pool(i, w4, b4)) * 1e6

    def alg_bytes(wl, tb=2, extra=0):
        # each lookup's row, ids, the reference layout's offsets, the output
        return wl.nnz * (D * tb + extra) + wl.nnz * 8 + (F * (B + 1) + F) * 8 + B * F * D * 2

    pool_bytes = float(np.mean([alg_bytes(wl) for wl in wls]))
    int8_bytes = float(np.mean([alg_bytes(wl, 1, 4) for wl in wls]))
    fused_bytes = pool_bytes + 2 * F * D * 2
    if "pool" not in legs:
        print(json.dumps({"us_per_step": us}), flush=True)
        return
    t = us["pool"] / 1e6
    rec = {
        "metric": "pooled bags/sec at the reference's own table shape (one shared bf16 [5e6, 512] table, 28 slots)",
        "value": B * F / t, "unit": "bags/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": t * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": f"synthetic: {n} seeded index sets rotated, shared N(0, 0.01) table, gamma ~ N(1, 0.1), "
                "beta ~ N(0, 0.1)",
        "config": {"workload": f"reference-5m: {WORKLOAD_TEXT['reference-5m']}",
                   "nnz_mean": float(np.mean([wl.nnz for wl in wls]))},
        "us_per_step": us,
        "roofline": roofline(pool_bytes, t, "pool_kernel", ("reference-5m", "pool_kernel")),
        "cpu_baseline": None,
    }
    if "fused" in legs:
        tf = us["pool_layernorm_fused"] / 1e6
        rec["roofline_fused_layernorm"] = roofline(fused_bytes, tf, "pool_norm_kernel",
                                                   ("reference-5m", "pool_norm_kernel"))
    if "int8" in legs:
        ti = us["pool_int8"] / 1e6
        rec["roofline_int8"] = roofline(int8_bytes, ti, "pool_kernel", ("reference-5m-int8", "pool_kernel"))
    if wl4:
        b4_bytes = float(np.mean([alg_bytes(wl) for wl in wl4]))
        rec["addressing"] = {
            "bytes_per_launch": b4_bytes,
            "frac_64bit": b4_bytes / (us["pool_64bit_addresses_ids_below_4gib"] / 1e6) / 1e9 / HBM_PEAK_GBS,
            "frac_buffer": b4_bytes / (us["pool_buffer_path_table_below_4gib"] / 1e6) / 1e9 / HBM_PEAK_GBS}
    print(json.dumps(rec), flush=True)


def reference_merge_cpu(batches, slot_num=28):
    """The flat-layout part of _timed_lazy_merge_group_cpu (online_best/infer.py:592-620) on host
    tensors: per slot, slice each sub-batch, rebase its local offsets, concatenate."""
    import torch

    parts_v, parts_o, vo = [], [], [0]
    for slot in range(slot_num):
        sv, so = [], []
        base = 0
        for b in batches:
            vals, ro, vos = b["_flat_values"], b["_flat_row_offsets"], b["_val_offsets"]
            seq_len = ro.numel() // slot_num - 1
            start = int(vos[slot])
            end = int(vos[slot + 1]) if slot + 1 < slot_num else int(vals.numel())
            sv.append(vals[start:end])
            so.append(ro[slot * (seq_len + 1):(slot + 1) * (seq_len + 1)][:-1] + base)
            base += end - start
        parts_v.append(torch.cat(sv).long())
        parts_o.append(torch.cat(so + [torch.tensor([base], dtype=torch.long)]).long())
        vo.append(vo[-1] + base)
    return {"_flat_values": torch.cat(parts_v).long(), "_flat_row_offsets": torch.cat(parts_o).long(),
            "_val_offsets": torch.tensor(vo[:-1], dtype=torch.long)}


def reference_pack(slots, dev):
    """online_best/infer.py:960-974 on device slot tensors: two torch.cat and val_offsets built
    from the slot sizes on the host, then copied to the device."""
    import torch

    val_lens = [0]
    for v, _ in slots:
        val_lens.append(val_lens[-1] + v.shape[0])
    return {"_flat_values": torch.cat([v for v, _ in slots]), "_flat_row_offsets": torch.cat([o for _, o in slots]),
            "_val_offsets": torch.tensor(val_lens[:-1], device=dev, dtype=torch.long)}


def bench_layout(args, pkg, dev):
    """Device merge and pack kernels against the reference's merge (host) and pack (torch.cat)."""
    import numpy as np
    import torch

    W = pkg.workloads

    def flat(wl, device):
        F, B = wl.num_fields, wl.batch
        off = wl.offsets
        ro = np.stack([off[f * B:(f + 1) * B + 1] - off[f * B] for f in range(F)]).reshape(-1)
        return {"_flat_values": torch.from_numpy(wl.values).to(device),
                "_flat_row_offsets": torch.from_numpy(ro).to(device),
                "_val_offsets": torch.from_numpy(off[0:F * B:B].copy()).to(device)}

    def same(a, b):
        return all(torch.equal(a[k].cpu(), b[k].cpu()) for k in ("_flat_values", "_flat_row_offsets", "_val_offsets"))

    def gpu_timed(fn, K):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(K):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / K, e0.elapsed_time(e1) / 1e3 / K

    def host_timed(fn, seconds):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            if time.perf_counter() - t0 > seconds:
                return (time.perf_counter() - t0) / n

    log("lazy-32k: generating the 8 sub-batches")
    lazy = W.make("lazy-32k", seed=1)
    host_subs = [flat(s, "cpu") for s in lazy.sub_batches]
    dev_subs = [flat(s, dev) for s in lazy.sub_batches]
    F = lazy.num_fields
    merged_ref = reference_merge_cpu(host_subs, F)
    if not same(merged_ref, pkg.merge_batches(dev_subs, F)):
        raise RuntimeError("device merge differs from the reference merge")
    log("timing the reference merge on the host")
    t_ref_merge = host_timed(lambda: reference_merge_cpu(host_subs, F), 3.0)
    log("timing the device merge")
    wall_merge, k_merge_py = gpu_timed(lambda: pkg.merge_batches(dev_subs, F), args.steps)
    # the raw C call with its argument arrays built once (what a serving loop would do)
    lay, lib, C = pkg.layout, pkg._capi.lib(), pkg._capi
    merged = pkg.merge_batches(dev_subs, F)
    stream = torch.cuda.current_stream(dev).cuda_stream
    margs = (lay._ptr_array([d["_flat_values"] for d in dev_subs]), lay._ptr_array([d["_val_offsets"] for d in dev_subs]),
             lay._ptr_array([d["_flat_row_offsets"] for d in dev_subs]),
             lay._i64_array([d["_flat_row_offsets"].numel() // F - 1 for d in dev_subs]),
             lay._i64_array([d["_flat_values"].numel() for d in dev_subs]), len(dev_subs), F,
             merged["_flat_values"].data_ptr(), merged["_flat_row_offsets"].data_ptr(),
             merged["_val_offsets"].data_ptr(), None, stream)
    wall_merge_raw, k_merge = gpu_timed(lambda: C.check(lib.cti_ebag_merge_batches(*margs)), args.steps)
    n_vals, n_offs = lazy.nnz, F * (lazy.batch + 1)
    merge_bytes = 16 * n_vals + 8 * sum(s["_flat_row_offsets"].numel() for s in host_subs) + 8 * n_offs + 16 * F

    log("bf16-2m: per-slot pairs on the device")
    wl = W.make("bf16-2m", seed=1)
    B = wl.batch
    slots = []
    for f in range(F):
        o = wl.offsets[f * B:(f + 1) * B + 1]
        slots.append((torch.from_numpy(wl.values[o[0]:o[-1]].copy()).to(dev), torch.from_numpy(o - o[0]).to(dev)))
    if not same(reference_pack(slots, dev), pkg.pack_slots(slots)):
        raise RuntimeError("device pack differs from the reference pack")
    log("timing the reference pack and the device pack")
    wall_ref_pack, k_ref_pack = gpu_timed(lambda: reference_pack(slots, dev), args.steps)
    wall_pack, k_pack_py = gpu_timed(lambda: pkg.pack_slots(slots), args.steps)
    packed = pkg.pack_slots(slots)
    pargs = (lay._ptr_array([v for v, _ in slots]), lay._ptr_array([o for _, o in slots]),
             lay._i64_array([v.numel() for v, _ in slots]), F, B, packed["_flat_values"].data_ptr(),
             packed["_flat_row_offsets"].data_ptr(), packed["_val_offsets"].data_ptr(), None, stream)
    wall_pack_raw, k_pack = gpu_timed(lambda: C.check(lib.cti_ebag_pack_slots(*pargs)), args.steps)
    pack_bytes = 16 * wl.nnz + 16 * F * (B + 1) + 8 * F

    achieved = merge_bytes / k_merge / 1e9
    rec = {
        "metric": "flat-layout merge of 8 sub-batches (lazy-32k, 28 fields, B=8x4096) and per-slot pack "
                  "(bf16-2m batch): bags/s",
        "value": lazy.batch * F / wall_merge_raw,
        "unit": "bags/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall_merge_raw * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int64",
        "data": "synthetic: lazy-32k sub-batches and one bf16-2m batch (seed 1)",
        "config": {"workload": "lazy-32k merge (8 x 4096 samples, 28 fields, nnz "
                               f"{n_vals}) and bf16-2m per-slot pack (4096 samples, nnz {wl.nnz})"},
        "us_per_call": {"reference_merge_host": t_ref_merge * 1e6, "device_merge_python": wall_merge * 1e6,
                        "device_merge_raw": wall_merge_raw * 1e6, "device_merge_gpu": k_merge * 1e6,
                        "reference_pack": wall_ref_pack * 1e6, "reference_pack_gpu": k_ref_pack * 1e6,
                        "device_pack_python": wall_pack * 1e6, "device_pack_raw": wall_pack_raw * 1e6,
                        "device_pack_gpu": k_pack * 1e6},
        "roofline": roofline(merge_bytes, k_merge, "merge_kernel", streaming=True,
                             pack_bytes_per_launch=pack_bytes, pack_achieved=pack_bytes / k_pack / 1e9),
        "cpu_baseline": {"value": lazy.batch * F / t_ref_merge, "unit": "bags/s", "cores": torch.get_num_threads(),
                         "kind": "port", "sample": "the reference merge (torch ops on host tensors) of the same "
                                                   "8 sub-batches, repeated for 3 s"},
    }
    print(json.dumps(rec), flush=True)


def bench_layernorm(args, pkg, plan, inputs, wl0, dev):
    """Time the input LayerNorm over pooled blocks of the workload (one block per step, rotated)."""
    import torch

    blocks = [plan(v, o) for v, o in inputs[:4]]
    width = blocks[0].shape[1]
    gen = torch.Generator(device=dev).manual_seed(0)
    gamma = (1 + 0.1 * torch.randn(width, device=dev, generator=gen)).to(wl0.out_dtype)
    beta = (0.1 * torch.randn(width, device=dev, generator=gen)).to(wl0.out_dtype)
    out = torch.empty_like(blocks[0])
    for i in range(args.warmup):
        pkg.layer_norm(blocks[i % 4], gamma, beta, 1e-5, out=out)
    K = args.steps
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    log(f"timing {K} LayerNorm steps over [{blocks[0].shape[0]}, {width}] {wl0.out_dtype}")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for i in range(K):
        pkg.layer_norm(blocks[i % 4], gamma, beta, 1e-5, out=out)
    ev1.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    launch_s = ev0.elapsed_time(ev1) / 1e3 / K
    nbytes = 2 * blocks[0].numel() * blocks[0].element_size() + 2 * width * gamma.element_size()
    achieved = nbytes / launch_s / 1e9
    log(f"{launch_s * 1e6:.2f} us/step on the GPU, {achieved:.0f} GB/s")
    rec = {
        "metric": "input LayerNorm rows/sec over the pooled block", "value": blocks[0].shape[0] / (elapsed / K),
        "unit": "rows/s", "n_gpus": 1, "steps": K, "warmup": args.warmup, "ms_per_step": elapsed / K * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float32: "f32", torch.float16: "f16"}[wl0.out_dtype],
        "data": "synthetic: pooled blocks of 4 seeded index sets rotated",
        "config": {"workload": f"layernorm over the pooled {args.workload} block", "rows": blocks[0].shape[0],
                   "cols": width},
        "roofline": roofline(nbytes, launch_s, "norm_rows_kernel", streaming=True),
        "cpu_baseline": None,
    }
    print(json.dumps(rec), flush=True)


def bench_small(args, pkg, dev):
    """The reference's small-batch call pattern: _warmup_model drives RepEncoder with per-slot
    batches of B in {2, 128, 512, 1024} length-1 bags (all ids 1, online_best/infer.py:2849-2863),
    and grouped serving calls the encoder once per sub-batch (:2689) and concatenates. Per B:
    wall-clock µs per call (Python argument checks included) of the drop-in launch
    (fused_all_slots_embedding on the flat layout), of the raw C call with its arguments built
    once, of a HIP-graph replay of the drop-in launch, of RepEncoder.pooled on the per-slot batch
    (device packing + launch) and of RepEncoder.forward (pooling, LayerNorm kernel, torch's Linear;
    and with fused_linear=True: statistics and the LayerNorm-Linear kernel);
    and the GPU time of the launch. Then lazy-32k's 8 sub-batches of 4096: 8 drop-in calls into
    slices of one output against one call on the merged batch."""
    import ctypes

    import numpy as np
    import torch

    C = pkg._capi
    lib = C.lib()
    V, D, S, d_model = 5_000_000, 512, 28, 512
    log("building RepEncoder(5,000,000, 512, 28 slots, d_model 512) in bf16")
    torch.manual_seed(0)
    enc = pkg.RepEncoder(V, D, slot_num=S, d_model=d_model).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        enc.emb.weight.normal_(0.0, 0.01)
    weight = enc.emb.weight.detach()
    n_calls = max(args.steps, 50)

    def wall(fn, n=n_calls):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    def gpu(fn, n=n_calls):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n * 1e3

    per_b = {}
    for B in (2, 128, 512, 1024):
        offs = torch.arange(B + 1, dtype=torch.long, device=dev)
        vals = torch.ones(B, dtype=torch.long, device=dev)
        slot_batch = {s: (vals, offs) for s in range(1, S + 1)}
        flat = pkg.pack_slots([slot_batch[s] for s in range(1, S + 1)])
        fv, vo, ro = flat["_flat_values"], flat["_val_offsets"], flat["_flat_row_offsets"]
        out = torch.empty((B, S * D), dtype=weight.dtype, device=dev)

        def drop_in():
            pkg.fused_all_slots_embedding(fv, vo, ro, weight, out, B, D, V - 1)

        stream = torch.cuda.current_stream(dev).cuda_stream
        raw_args = (fv.data_ptr(), vo.data_ptr(), ro.data_ptr(), weight.data_ptr(), C.BF16, out.data_ptr(), B, S, D,
                    V - 1, fv.numel(), stream)

        def raw():
            C.check(lib.cti_ebag_fused_all_slots(*raw_args))

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            drop_in()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            drop_in()
        torch.cuda.synchronize()
        want = out.clone()
        rec = {"drop_in_call_us": wall(drop_in), "raw_c_call_us": wall(raw), "graph_replay_us": wall(graph.replay),
               "rep_encoder_pooled_us": wall(lambda: enc.pooled(slot_batch)),
               "rep_encoder_forward_us": wall(lambda: enc(slot_batch)),
               "rep_encoder_forward_fused_linear_us": wall(lambda: enc(slot_batch, fused_linear=True)),
               "launch_gpu_us": gpu(drop_in)}
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(out.view(torch.int16), want.view(torch.int16)):
            raise RuntimeError(f"B={B}: the graph replay differs from the eager launch")
        per_b[B] = rec
        log(f"B={B}: " + ", ".join(f"{k} {v:.1f}" for k, v in rec.items()))
        del graph

    log("lazy-32k sub-batches: 8 calls into one output against one call on the merged batch")
    lazy = pkg.workloads.make("lazy-32k", seed=1, vocab=V)
    subs = []
    for sb in lazy.sub_batches:
        ro_s = np.concatenate([sb.offsets[f * sb.batch:(f + 1) * sb.batch + 1] - sb.offsets[f * sb.batch]
                               for f in range(S)]).astype(np.int64)
        subs.append((torch.from_numpy(sb.values).to(dev), torch.from_numpy(sb.offsets[0:S * sb.batch:sb.batch].copy()).to(dev),
                     torch.from_numpy(ro_s).to(dev), sb.batch))
    merged = pkg.merge_batches([{"_flat_values": v, "_val_offsets": o, "_flat_row_offsets": r} for v, o, r, _ in subs], S)
    Bm = lazy.batch
    out_m = torch.empty((Bm, S * D), dtype=weight.dtype, device=dev)
    out_s = torch.empty_like(out_m)

    def per_sub():
        row = 0
        for v, o, r, b in subs:
            pkg.fused_all_slots_embedding(v, o, r, weight, out_s[row:row + b], b, D, V - 1)
            row += b

    def one_merged():
        pkg.fused_all_slots_embedding(merged["_flat_values"], merged["_val_offsets"], merged["_flat_row_offsets"],
                                      weight, out_m, Bm, D, V - 1)

    sub_rec = {"per_sub_batch_calls_us": wall(per_sub, 20), "merged_call_us": wall(one_merged, 20),
               "per_sub_batch_gpu_us": gpu(per_sub, 20), "merged_gpu_us": gpu(one_merged, 20)}
    per_sub()
    one_merged()
    torch.cuda.synchronize()
    if not torch.equal(out_s.view(torch.int16), out_m.view(torch.int16)):
        raise RuntimeError("per-sub-batch pooling differs from the merged batch's")
    log("sub-batches: " + ", ".join(f"{k} {v:.1f}" for k, v in sub_rec.items()))
    ref = per_b[128]
    rec = {
        "metric": "drop-in pooling calls/sec at the reference's warmup batch sizes (B=128 shown; "
                  "one shared bf16 [5e6, 512] table, 28 slots, length-1 bags)",
        "value": 1e6 / ref["drop_in_call_us"], "unit": "calls/s", "n_gpus": 1, "steps": n_calls, "warmup": 10,
        "ms_per_step": ref["drop_in_call_us"] / 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: per-slot batches of length-1 bags with id 1 (as online_best/infer.py:2849-2863); "
                "lazy-32k sub-batches (seed 1)",
        "config": {"workload": "reference warmup batches B in {2, 128, 512, 1024}; lazy-32k's 8 sub-batches of 4096"},
        "us_per_call": {str(k): v for k, v in per_b.items()}, "sub_batches": sub_rec,
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(rec), flush=True)


def main_kernel_name(wl, args):
    """The pooling launch sequence's kernels: fields of several row widths share one mixed-width
    launch sequence; binning adds its pass and the list kernel."""
    main_kernel = "pool_mixed_kernel" if len(set(wl.dims)) > 1 else "pool_kernel"
    return f"bin_kernel + {main_kernel} + pool_long_kernel" if args.bins else main_kernel


def main_prof_kernel(wl, args):
    """The name under which the launch sequence's profiles are kept in profiles/."""
    mixed = len(set(wl.dims)) > 1
    if args.bins:
        return "bin_mixed_long_kernels" if mixed else "bin_pool_long_kernels"
    return "pool_mixed_kernel" if mixed else "pool_kernel"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # 1000 untimed steps (~37 ms): the first ~10-30 ms of sustained load run 0.5-3 us per step slower
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--workload", default="bf16-2m", choices=sorted(WORKLOAD_TEXT))
    ap.add_argument("--sets", type=int, default=8, help="independently seeded index sets rotated over")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--long-threshold", type=int, default=0)
    ap.add_argument("--bins", action="store_true", help="run the device length-binning pass")
    ap.add_argument("--block-threshold", type=int, default=0)
    ap.add_argument("--split-threshold", type=int, default=0)
    ap.add_argument("--stage", default="pool",
                    choices=["pool", "layernorm", "h2d", "encoder", "layout", "reference", "small"],
                    help="time the pooling step (default), the input LayerNorm over pooled blocks, or the "
                         "step end to end from host batches")
    ap.add_argument("--int8", action="store_true", help="int8 row-quantised tables (quantised on the device)")
    ap.add_argument("--index-dtype", choices=["int64", "int32"], default="int64",
                    help="ids as the kernel reads them: int64 as the reference's collate produces them (default), "
                         "or int32 as InputStager delivers them to the device")
    ap.add_argument("--legs", default="pool,fused,int8,addressing",
                    help="--stage reference: which of pool, fused, int8, addressing to time")
    ap.add_argument("--dispatch-order", choices=["auto", "host", "launch", "off"], default="auto",
                    help="host: each batch carries its tile order (most rows per bag first in each XCD's share), "
                         "made on the host from its offsets where the batch is produced; launch: each step also "
                         "sorts the next batch's tiles on the device and follows the order the previous step made; "
                         "auto: host for the workloads where ordering was measured to pay (%s) without --bins"
                         % ", ".join(sorted(ORDERED_BY_DEFAULT)))
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only copy 1 GiB device-to-device 3 times (scales rocprofv3 FETCH/WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.dispatch_order == "auto":
        args.dispatch_order = "host" if args.workload in ORDERED_BY_DEFAULT and not args.bins else "off"

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE={world}).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.calibrate_copy:
        n = 1 << 28  # 2^28 fp32 = 1 GiB read + 1 GiB written per copy
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copied 1 GiB three times")
        return

    from __graft_entry__ import load_package

    pkg = load_package()
    W = pkg.workloads
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.stage == "layout":
        return bench_layout(args, pkg, dev)
    if args.stage == "reference":
        return bench_reference(args, pkg, dev)
    if args.stage == "small":
        return bench_small(args, pkg, dev)
    log(f"workload {args.workload}: generating {args.sets} index sets")
    wls = [W.make(args.workload, seed=s) for s in range(1, args.sets + 1)]
    wl0 = wls[0]
    if args.stage == "h2d":
        return bench_h2d(args, pkg, wls, dev)
    if args.stage == "encoder":
        return bench_encoder(args, pkg, wls, dev)
    # host-side preparation first (byte counts, the batches' dispatch orders, the inputs' copies),
    # so that the table fill, the GPU's own work, runs right before the warm-up steps
    ib = 4 if args.index_dtype == "int32" else 8
    bytes_alg = [wl.bytes_algorithmic(int8=args.int8, index_bytes=ib) for wl in wls]
    bytes_comp = [wl.bytes_compulsory(int8=args.int8, index_bytes=ib) for wl in wls]
    orders = None
    if args.dispatch_order == "host":
        # each batch's order, made on the host from its offsets as its producer would make it
        tdt = torch.int8 if args.int8 else wl0.table_dtype
        orders = [pkg.make_tile_order(torch.from_numpy(wl.offsets), wl.batch, wl.num_fields, tdt, wl.dims[0]).to(dev)
                  for wl in wls]
    idx_dtype = torch.int32 if args.index_dtype == "int32" else torch.int64
    inputs = [W.to_device(wl, dev, index_dtype=idx_dtype) for wl in wls]
    log("filling tables on the device")
    tables = W.make_tables(wl0, dev, seed=0)
    pooled_tables = tables
    if args.int8:
        log("quantising the tables to int8")
        pooled_tables = [pkg.quantize_embedding_int8(t) for t in tables]
    plan = pkg.PooledEmbedding(pooled_tables, pooling=wl0.pooling, out_dtype=wl0.out_dtype,
                               long_threshold=args.long_threshold, use_bins=args.bins,
                               block_threshold=args.block_threshold, max_batch=wl0.batch,
                               split_threshold=args.split_threshold, dispatch_order=args.dispatch_order == "launch")
    out = torch.empty((wl0.batch, sum(wl0.dims)), dtype=wl0.out_dtype, device=dev)
    if args.stage == "layernorm":
        return bench_layernorm(args, pkg, plan, inputs, wl0, dev)
    torch.cuda.synchronize()

    def step(i):
        v, o = inputs[i % args.sets]
        if args.dispatch_order == "launch":
            plan(v, o, out, next_offsets=inputs[(i + 1) % args.sets][1])
        elif orders is not None:
            plan(v, o, out, tile_order=orders[i % args.sets])
        else:
            plan(v, o, out)

    log(f"warmup {args.warmup} steps")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Timed region: K back-to-back steps, bracketed by one pair of HIP events recorded on the
    # stream the kernels run on (per-step events would add a gap between kernels).
    K = args.steps

    def timed_region(step_fn):
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        for i in range(args.warmup, args.warmup + K):  # continues the warm-up's sequence of index sets
            step_fn(i)
        ev1.record()
        torch.cuda.synchronize()
        return time.perf_counter() - t0, ev0.elapsed_time(ev1) / 1e3 / K

    log(f"timing {K} steps")
    elapsed, mean_launch_s = timed_region(step)
    timed = range(args.warmup, args.warmup + K)
    used_bytes = float(np.mean([bytes_alg[i % args.sets] for i in timed]))
    used_comp = float(np.mean([bytes_comp[i % args.sets] for i in timed]))
    ms_per_step = elapsed / K * 1e3
    value = wl0.num_bags / (elapsed / K)
    achieved = used_bytes / mean_launch_s / 1e9
    log(f"{ms_per_step * 1e3:.1f} us/step wall, {mean_launch_s * 1e6:.1f} us/step on the GPU, "
        f"{achieved:.0f} GB/s algorithmic, {used_comp / mean_launch_s / 1e9:.0f} GB/s compulsory")

    plain = None
    if orders is not None or args.dispatch_order == "launch":
        # the same steps without a dispatch order: what the reference's call site gets with no
        # change to the batch's producer
        for i in range(200):
            plan(*inputs[i % args.sets], out)
        plain_elapsed, plain_launch_s = timed_region(lambda i: plan(*inputs[i % args.sets], out))
        log(f"without a dispatch order: {plain_launch_s * 1e6:.1f} us/step on the GPU")
        plain = {"dispatch_order": "off", "value": wl0.num_bags / (plain_elapsed / K), "unit": "bags/s",
                 "ms_per_step": plain_elapsed / K * 1e3,
                 "roofline": roofline(used_bytes, plain_launch_s, main_kernel_name(wl0, args),
                                      None if args.index_dtype == "int32" else
                                      (args.workload + ("-int8" if args.int8 else ""), main_prof_kernel(wl0, args),
                                       ("hbm_bytes_per_launch_order_off", "hbm_bytes_per_launch")),
                                      compulsory_bytes=used_comp)}

    accuracy = None
    if args.int8:
        # int8 pooled rows against the same batch pooled from the float tables (fp32 output)
        v, o = inputs[0]
        ref = pkg.PooledEmbedding(tables, pooling=wl0.pooling, out_dtype=torch.float32)(v, o)
        got = pkg.PooledEmbedding(pooled_tables, pooling=wl0.pooling, out_dtype=torch.float32)(v, o)
        err = (got - ref).float()
        accuracy = {"vs": "float tables, fp32 output, index set 1",
                    "max_abs_err": err.abs().max().item(),
                    "rel_rms_err": (err.pow(2).mean().sqrt() / ref.float().pow(2).mean().sqrt()).item()}
        del ref, got, err

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(wl0, tables, args.cpu_seconds)
        if args.int8:
            cpu["sample"] += " (the reference's CPU path has no int8 tables: this is its float loop)"

    kernel_name = main_kernel_name(wl0, args)
    prof_kernel = main_prof_kernel(wl0, args)
    rec = {
        "metric": METRIC,
        "value": value,
        "unit": "bags/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8" if args.int8 else {torch.bfloat16: "bf16", torch.float32: "f32",
                                          torch.float16: "f16"}[wl0.table_dtype],
        "data": f"synthetic: {args.sets} seeded index sets rotated, random N(0, 0.01) tables"
                + (", row-quantised to int8 on the device" if args.int8 else "")
                + ("; each batch carries its tile order, made on the host from its offsets" if orders is not None
                   else ""),
        "config": {"workload": f"{args.workload}: {WORKLOAD_TEXT[args.workload]}", "batch": wl0.batch,
                   "fields": wl0.num_fields, "dims": sorted(set(wl0.dims)), "pooling": wl0.pooling,
                   "nnz_mean": float(np.mean([wl.nnz for wl in wls])), "index_sets": args.sets,
                   "length_binning": bool(args.bins), "int8_tables": bool(args.int8),
                   "dispatch_order": args.dispatch_order, "index_dtype": args.index_dtype},
        # the profiles' counters were taken with int64 ids: int32 launches report no traffic
        "roofline": roofline(used_bytes, mean_launch_s, kernel_name,
                             None if args.index_dtype == "int32" else
                             (args.workload + ("-int8" if args.int8 else ""), prof_kernel,
                              {"host": ("hbm_bytes_per_launch",),
                               "launch": ("hbm_bytes_per_launch_order_launch", "hbm_bytes_per_launch"),
                               "off": ("hbm_bytes_per_launch_order_off", "hbm_bytes_per_launch")}[args.dispatch_order]),
                             compulsory_bytes=used_comp),
        "plain_launch": plain,
        "cpu_baseline": cpu,
    }
    if accuracy is not None:
        rec["int8_accuracy"] = accuracy
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
