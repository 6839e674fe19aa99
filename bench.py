"""Benchmark of the lookup / interaction forward path on one MI355X.

Default workload: the single-hot pooled lookup (26 tables, rows log-uniform
in [1e3, 4e7], dim 128 bf16, one Zipf(1.05) id per bag, batch 65,536, sum,
fp32 out).  ``--workload`` selects another of the five workloads.  A step is
one forward of the path over one batch already resident in HBM.

Prints ONE JSON line with the throughput, the roofline of the dominant kernel
(algorithmic bytes or FLOPs per launch over its HIP-event-timed average
duration) and a CPU baseline (the C oracle on the host cores, bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "embedding lookups/sec + achieved HBM GB/s (% peak); OneTrans block samples/sec"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_from_profiles(workload: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    calibrated against a copy kernel, as recorded in profiles/traffic.txt:
    lines ``<workload> <bytes per launch>``."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) >= 2 and parts[0] == workload and not line.startswith("#"):
            try:
                return float(parts[1])
            except ValueError:
                return None
    return None


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def time_cpu(fn, reps: int = 5) -> float:
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


# ----------------------------------------------------------------------------------------------
# pooled workloads
# ----------------------------------------------------------------------------------------------

def setup_pooled(pdm, torch, dev, w, weight_std: float):
    """Builds the tables of workload ``w`` on the device and returns the step closure."""
    L = pdm._lib
    dt_code = {"fp32": L.PDM_F32, "bf16": L.PDM_BF16, "int8": L.PDM_I8_SB_F16}[w.dtype]
    pool = {"sum": L.PDM_POOL_SUM, "mean": L.PDM_POOL_MEAN}[w.pooling]
    row_bytes = {"fp32": 4 * w.dim, "bf16": 2 * w.dim, "int8": (4 + w.dim + 3) & ~3}[w.dtype]
    offs, off = [], 0
    for r in w.rows:
        off = (off + 255) // 256 * 256
        offs.append(off)
        off += r * row_bytes
    log(f"allocating {off / 1e9:.2f} GB of tables")
    flat = torch.empty(off, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1000)
    chunk = 1 << 20
    for t, r in enumerate(w.rows):
        for r0 in range(0, r, chunk):
            n = min(chunk, r - r0)
            src = torch.empty((n, w.dim), dtype=torch.float32, device=dev)
            if w.weight_init == "uniform0.01":
                src.uniform_(-0.01, 0.01, generator=gen)
            else:
                src.normal_(0.0, weight_std, generator=gen)
            dst = flat.narrow(0, offs[t] + r0 * row_bytes, n * row_bytes)
            if w.dtype == "int8":
                dst.copy_(pdm.ops.int8_rowwise_quantize(src, row_bytes).view(-1))
            elif w.dtype == "bf16":
                dst.view(torch.bfloat16).copy_(src.view(-1))
            else:
                dst.view(torch.float32).copy_(src.view(-1))
    slots, col = [], 0
    for t, r in enumerate(w.rows):
        slots.append(dict(rows=r, weights_offset=offs[t], dim=w.dim, dtype=dt_code, pooling=pool,
                          row_bytes=row_bytes, out_offset=col))
        col += w.dim
    plan = pdm.ops.TbePlan(slots, dev)
    indices = torch.from_numpy(w.indices).to(dev)
    offsets = torch.from_numpy(w.offsets).to(dev)
    out_dtype = {"fp32": torch.float32, "fp16": torch.float16}[w.out_dtype]
    out = torch.empty((w.batch, col), dtype=out_dtype, device=dev)

    def step():
        pdm.ops.tbe_pooled_raw(plan, flat, indices, offsets, w.batch, out_dtype, -1, out=out)

    osize = 4 if w.out_dtype == "fp32" else 2
    n = w.num_lookups
    alg_bytes = n * row_bytes + n * 8 + w.offsets.size * 8 + w.batch * col * osize
    return step, alg_bytes, (flat, plan, indices, offsets, out)


def cpu_pooled(orc, w, threads: int, row_cap: int, weight_std: float):
    """The oracle over the same ids on tables capped at ``row_cap`` rows (ids of a
    capped table are drawn with the same distribution over the capped rows)."""
    import primus_dlrm_amd.synthetic as syn

    g = np.random.default_rng(5)
    rows = [min(r, row_cap) for r in w.rows]
    row_bytes = {"fp32": 4 * w.dim, "bf16": 2 * w.dim, "int8": (4 + w.dim + 3) & ~3}[w.dtype]
    chunks, slots, off, col = [], [], 0, 0
    for t, r in enumerate(rows):
        # random finite values: the timing does not depend on them
        if w.dtype == "int8":
            b = g.integers(0, 256, (r, row_bytes), dtype=np.uint8)
            b[:, 0:4] = np.frombuffer(np.array([weight_std / 64, -weight_std], np.float16).tobytes(), np.uint8)
        elif w.dtype == "bf16":
            b = (g.integers(0, 1 << 16, (r, w.dim), dtype=np.uint16) & 0x807F) | 0x3C00
        else:
            b = g.random((r, w.dim), dtype=np.float32) * np.float32(0.02) - np.float32(0.01)
        b = b.view(np.uint8).reshape(-1)
        slots.append(dict(rows=r, weights_offset=off, dim=w.dim, dtype=w.dtype, pooling=w.pooling,
                          row_bytes=row_bytes if w.dtype == "int8" else 0, out_offset=col))
        chunks.append(b)
        off += b.size
        col += w.dim
    flat = np.concatenate(chunks)
    idx = w.indices.copy()
    for t, r in enumerate(w.rows):
        if r > row_cap:
            seg = slice(w.offsets[t * w.batch], w.offsets[(t + 1) * w.batch])
            idx[seg] = syn.zipf_rows(syn.rng(99, t), idx[seg].size, row_cap, 1.05) if w.dtype != "int8" \
                else idx[seg] % row_cap
    od = "fp32" if w.out_dtype == "fp32" else "fp16"
    sec = time_cpu(lambda: orc.tbe_pooled(flat, slots, idx, w.offsets, w.batch, -1, od, threads=threads))
    return w.num_lookups / sec, sec


# ----------------------------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="single_hot",
                    choices=["single_hot", "ebc_fp32", "int8_mean", "seq_gather", "onetrans"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (no collectives or sharding); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import __graft_entry__ as ge

    pdm = ge.pdm_import()
    import primus_dlrm_amd.synthetic as syn
    from oracle import oracle as orc

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    threads = cpu_threads()

    cfg = {}
    if args.workload in ("single_hot", "ebc_fp32", "int8_mean"):
        if args.workload == "single_hot":
            w, std, cap = syn.single_hot_bf16(), 0.02, 500_000
        elif args.workload == "ebc_fp32":
            w, std, cap = syn.ebc_fp32(), 0.01, 100_000
        else:
            w, std, cap = syn.int8_mean(), 0.05, 200_000
        step, alg_bytes, keep = setup_pooled(pdm, torch, dev, w, std)
        units_per_step, unit = w.num_lookups, "lookups/s"
        dtype = {"bf16": "bf16->f32", "fp32": "f32", "int8": "u8->f32"}[w.dtype]
        cfg = {"workload": w.name, "tables": w.num_tables, "rows_total": int(sum(w.rows)), "dim": w.dim,
               "batch": w.batch, "lookups_per_batch": w.num_lookups, "pooling": w.pooling,
               "weights": w.dtype, "out": w.out_dtype}
        bound = "hbm"
    else:
        raise SystemExit(f"workload {args.workload} is not wired into bench.py yet")

    stream = torch.cuda.current_stream(dev)
    log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # per-launch HIP events on the launch stream give the kernel's average duration
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
    ms_per_step = elapsed * 1e3 / args.steps
    value = units_per_step * args.steps / elapsed
    achieved = alg_bytes / (kernel_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles(args.workload)
    roofline = {"bound": bound, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "algorithmic_bytes": int(alg_bytes), "kernel_ms": round(kernel_ms, 5)}
    log(f"{value:.4g} {unit}, kernel {kernel_ms:.4f} ms, {achieved:.1f} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline on {threads} threads")
        cpu_val, sec = cpu_pooled(orc, w, threads, cap, std)
        cpu = {"value": round(cpu_val, 1), "unit": unit, "cores": threads, "kind": "port",
               "sample": f"C oracle, full batch of {w.num_lookups} lookups on tables capped at {cap} rows "
                         f"(ids redrawn over the capped rows), median of 5 reps = {sec:.3f} s"}

    line = {"metric": METRIC, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic",
            "config": cfg, "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
