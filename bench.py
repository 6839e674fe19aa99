"""Benchmark of the lookup / interaction forward path on one MI355X.

Default workload: the quantized-inference TBE, the largest single-GPU lookup
(64 tables x 5,000,000 rows x dim 128 int8 rowwise with fp16 scale and bias,
mean pooling over Poisson(20) bags in [1, 100] of Zipf(1.2) ids, batch
16,384, fp16 out: 42.2 GB of tables, about 21 M lookups per batch).
``--workload`` selects another:

  int8_mean   (default, above)
  ebc_fp32    8 tables x 100,000 x 64 fp32, sum, Poisson(10) bags, B=2048; also timed as 64 back-to-back
              batches in one HIP graph (steady state, launch overhead amortised)
  single_hot  26 tables, rows log-uniform in [1e3, 4e7], dim 128 bf16, one Zipf(1.05) id per bag, B=65,536,
              sum, fp32 out
  seq_gather  3 behaviour pools, item 10M x 256 + artist 1M x 64 + album 2M x 64 bf16, B=1024
  seq_tokenize  the seq_gather workload fused with one SequentialTokenizer per pool (Linear 384 -> 256,
              GELU, Linear 256 -> 256, + pos_emb of 2048 x 256 fp32), fp32 S-tokens [1024, 768, 256]
  ns_tokenize NS tokens: uid/item/artist/album rows (1M/9.4M/1.3M/3.4M x 64 bf16) + dense parts 64/6/6/64 -> 396
              wide NS input -> AutoSplitTokenizer Linear(396, 4096) + GELU + Linear(4096, 4096), B=1024
  onetrans    4-layer OneTrans block stack, B=1024, 384 S + 16 NS tokens, d 256, schedule 384/256/128/64
  onetrans_l  OneTransL: 8-layer stack, B=1024, 1500 S + 16 NS tokens, d 384, 6 heads, the pyramid schedule
              1500 -> 16 (1500, 1288, 1076, 864, 652, 440, 228, 16)
  cross_hash  cross-feature ids: xxHash64 of (uid, artist_id) int64 pairs % 100,000,000, 16,777,216 rows
  train_adam  pooled backward + fused Adam (lr 1e-2, eps 1e-8, wd 1e-5): 8 tables x 10,000,000 x 64 fp32,
              sum, Poisson(10) bags in [0, 50], uniform ids, B=65,536 (about 5.2 M lookups)
  train_rowwise_adagrad  the same with fused row-wise Adagrad (L2 weight decay 1e-5)
  train_seq_adam  S-token gather backward + fused Adam over the seq_gather workload's tables in fp32
              (item 10M x 256, artist 1M x 64, album 2M x 64; B=1024, 768 slots, row-0 padding)
  kjt_build   device KJT build: 26 features x 65,536 rows x 20 int64 ids, 30 % padding id 0 filtered
              (lengths, offsets, compacted values; no host sync)
  copy_1gib   calibration only: a 1 GiB device-to-device copy (the HBM counters' reference kernel)

A step is one forward of the path over one batch already resident in HBM.
Prints ONE JSON line with the throughput, the roofline of the dominant kernel
(algorithmic bytes or FLOPs per launch over its HIP-event-timed average
duration on the launch stream) and a CPU baseline: the reference's own CPU
path (the PyTorch CPU operators that the unsharded TorchRec modules and the
OneTrans model reduce to) on the host cores, on the same seeded inputs or a
bounded sample of them.
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


def traffic_fields(workload: str) -> dict:
    """Memory traffic per launch of ``workload`` as measured with rocprofv3 --pmc and recorded in
    profiles/traffic.txt, lines ``<workload> <read bytes> <write bytes> <DRAM-bound read bytes> <DRAM-bound write
    bytes>``: the L2's read and write requests to the memory fabric weighted by their size (read requests carry
    128 B, TCC_EA0_RDREQ_32B ones 32 B; TCC_EA0_WRREQ_64B write requests 64 B, the others 32 B), and the requests
    the L2 sent towards DRAM (TCC_EA0_RDREQ_DRAM, TCC_EA0_WRREQ_DRAM) at the same mean request size.  The
    Infinity Cache sits behind that interface, so its hits are counted too."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return {"traffic": None}
    for line in open(path):
        parts = line.split()
        if len(parts) >= 5 and parts[0] == workload and not line.startswith("#"):
            try:
                rd, wr, drd, dwr = (float(v) for v in parts[1:5])
            except ValueError:
                return {"traffic": None}
            return {"traffic": rd + wr, "traffic_read": rd, "traffic_write": wr, "traffic_dram": drd + dwr,
                    "traffic_note": TRAFFIC_NOTE}
    return {"traffic": None}


def cpu_env():
    """(threads used, cores in this process's affinity, CPU model).  Every affinity core is used, except
    that a set OMP_NUM_THREADS (the host's CPU share for this process) caps the count."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    used = min(aff, int(cap)) if cap.isdigit() and int(cap) > 0 else aff
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return max(1, used), aff, model


def host_mem_available() -> int:
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except OSError:
        pass
    return 0


def time_cpu(fn, reps: int = 5, slow_s: float = 4.0) -> tuple:
    """Median wall time of ``reps`` calls after one warmup call (3 reps when one call takes over ``slow_s``).
    Returns (seconds, reps)."""
    t0 = time.perf_counter()
    fn()
    if time.perf_counter() - t0 > slow_s:
        reps = min(reps, 3)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), reps


def fill_tiled(torch, dst, block):
    """Fills the rows of ``dst`` [rows, C] with repeated copies of ``block`` [b, C] (host tables for the CPU
    baseline: the values do not change the timing, and tiling fills tens of GB in seconds)."""
    b, rows = block.shape[0], dst.shape[0]
    full = rows // b
    if full:
        dst[:full * b].view(full, b, -1).copy_(block.unsqueeze(0).expand(full, -1, -1))
    if rows % b:
        dst[full * b:].copy_(block[:rows % b])


def cpu_result(value, unit, threads, path, sample, sec, reps, **extra):
    used, aff, model = cpu_env()
    out = {"value": round(value, 1), "unit": unit, "cores": threads, "kind": "port", "path": path,
           "sample": f"{sample}, median of {reps} reps = {sec:.4g} s", "cpu_model": model, "affinity_cores": aff}
    out.update(extra)
    return out


GRAPH_BATCHES = 64


def graph_steady_state(torch, dev, step, n: int, reps: int = 20) -> float:
    """Milliseconds per batch of ``n`` back-to-back launches of ``step`` captured in one HIP graph and replayed
    ``reps`` times (launch overhead amortised: the steady-state rate of a stream of batches)."""
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(n):
            step()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (reps * n)


def cpu_cross_hash(a, b, table_size: int):
    """The reference's cross ids on the CPU: ``cross_hash_batch`` is a Python loop of ``xxhash.xxh64`` over
    ``struct.pack("<qq", a, b)`` modulo the table size (primus_dlrm/data/hashing.py:86-112)."""
    import struct
    import xxhash

    pack = struct.Struct("<2q").pack
    al, bl = a.tolist(), b.tolist()

    def run():
        return [xxhash.xxh64(pack(x, y), seed=0).intdigest() % table_size for x, y in zip(al, bl)]

    sec, reps = time_cpu(run, reps=3)
    return sec, reps, "python loop of xxhash.xxh64 over struct-packed int64 pairs (hashing.py cross_hash_batch)"


def cpu_kjt(torch, mats, padding_idx: int, threads: int):
    """``_build_pooled_kjt`` (primus_dlrm/models/embedding.py:179-204) on the CPU: per feature ``mask = ids != pad``,
    ``lengths = mask.sum(1)``, ``values = ids[mask]``, concatenated, offsets by a cumulative sum."""
    torch.set_num_threads(threads)
    feats = [torch.from_numpy(m) for m in mats]

    def run():
        vals, lens = [], []
        for ids in feats:
            mask = ids != padding_idx
            lens.append(mask.sum(1).to(torch.int32))
            vals.append(ids[mask])
        lengths = torch.cat(lens)
        return torch.cat(vals), lengths, torch.cumsum(lengths.to(torch.int64), 0)

    return time_cpu(run)


# ----------------------------------------------------------------------------------------------
# pooled workloads (ebc_fp32, single_hot, int8_mean)
# ----------------------------------------------------------------------------------------------

def setup_pooled(pdm, torch, dev, w, weight_std: float):
    """Builds the tables of workload ``w`` on the device; returns (step, algorithmic bytes, keepalive)."""
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


def cpu_pooled(torch, w, threads: int, weight_std: float):
    """The unsharded TorchRec EmbeddingBagCollection's CPU path: one ``F.embedding_bag(include_last_offset=True)``
    per table (int8 tables: torch's ``quantized::embedding_bag_byte_rowwise_offsets`` on rows repacked with an
    fp32 scale and bias after the codes), outputs concatenated in table order (the KeyedTensor values), on the
    full batch.  Tables are full size when host memory holds them, else every table is row-subsampled to fit
    and the ids of a subsampled table redrawn over its rows from the same distribution."""
    import torch.nn.functional as Fn
    import primus_dlrm_amd.synthetic as syn

    torch.set_num_threads(threads)
    T, B = len(w.rows), w.batch
    bpr = {"fp32": 4 * w.dim, "bf16": 2 * w.dim, "int8": w.dim + 8}[w.dtype]
    budget = int(0.6 * host_mem_available())
    cap = max(w.rows)
    if sum(w.rows) * bpr > budget:
        cap = max(1, budget // (T * bpr))
    rows = [min(r, cap) for r in w.rows]
    g = torch.Generator().manual_seed(5)
    tables = []
    for r in rows:
        nb = min(r, 1 << 16)
        if w.dtype == "int8":
            t = torch.empty((r, w.dim + 8), dtype=torch.uint8)
            block = torch.randint(0, 256, (nb, w.dim + 8), dtype=torch.uint8, generator=g)
            block[:, w.dim:] = torch.tensor([weight_std / 64, -2 * weight_std], dtype=torch.float32).view(torch.uint8)
        else:
            dt = torch.float32 if w.dtype == "fp32" else torch.bfloat16
            t = torch.empty((r, w.dim), dtype=dt)
            block = (torch.randn(nb, w.dim, generator=g) * weight_std).to(dt)
        fill_tiled(torch, t, block)
        tables.append(t)
    idx, offs = [], []
    alpha = {"bf16": 1.05, "int8": 1.2}.get(w.dtype)
    for t in range(T):
        lo, hi = int(w.offsets[t * B]), int(w.offsets[(t + 1) * B])
        ids = w.indices[lo:hi]
        if rows[t] < w.rows[t]:
            ids = syn.zipf_rows(syn.rng(99, t), hi - lo, rows[t], alpha) if alpha else \
                syn.rng(99, t).integers(0, rows[t], hi - lo)
        idx.append(torch.from_numpy(np.ascontiguousarray(ids)))
        offs.append(torch.from_numpy(w.offsets[t * B:(t + 1) * B + 1] - lo))
    out_dt = torch.float32 if w.out_dtype == "fp32" else torch.float16
    mode = 0 if w.pooling == "sum" else 1

    def run():
        outs = []
        for t in range(T):
            if w.dtype == "int8":
                outs.append(torch.ops.quantized.embedding_bag_byte_rowwise_offsets(
                    tables[t], idx[t], offs[t], False, mode, False, None, None, True))
            else:
                outs.append(Fn.embedding_bag(idx[t], tables[t], offs[t], mode=w.pooling, include_last_offset=True))
        return torch.cat(outs, 1).to(out_dt)

    sec, reps = time_cpu(run)
    size = "full-size tables" if cap >= max(w.rows) else \
        f"tables row-subsampled to {cap} rows to fit host memory (ids redrawn, same distribution)"
    op = "quantized::embedding_bag_byte_rowwise_offsets (fp32 scale/bias repack)" if w.dtype == "int8" else \
        "F.embedding_bag"
    return w.num_lookups / sec, sec, reps, op, f"full batch of {w.num_lookups} lookups on {size}, " \
        f"{sum(r * bpr for r in rows) / 1e9:.1f} GB of host tables"


# ----------------------------------------------------------------------------------------------
# pooled backward + fused optimizer
# ----------------------------------------------------------------------------------------------

def setup_train(pdm, torch, dev, w, optimizer: str):
    """fp32 tables of ``w`` with zeroed optimizer state; a step is one fused backward + update over the
    batch with a fixed output gradient.  Returns (step, algorithmic bytes, distinct rows, keepalive)."""
    L = pdm._lib
    D = w.dim
    offs, off = [], 0
    for r in w.rows:
        off = (off + 255) // 256 * 256
        offs.append(off)
        off += r * D * 4
    log(f"allocating {off / 1e9:.2f} GB of fp32 tables (+ optimizer state)")
    flat = torch.empty(off // 4, dtype=torch.float32, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1007)
    for r0 in range(0, flat.numel(), 1 << 26):
        flat[r0:r0 + (1 << 26)].uniform_(-0.01, 0.01, generator=gen)
    slots, col = [], 0
    for t, r in enumerate(w.rows):
        slots.append(dict(rows=r, weights_offset=offs[t], dim=D, dtype=L.PDM_F32, pooling=L.PDM_POOL_SUM,
                          row_bytes=4 * D, out_offset=col))
        col += D
    plan = pdm.ops.TbePlan(slots, dev)
    adam = optimizer == "adam"
    m1 = torch.zeros_like(flat) if adam else torch.zeros(plan.total_rows, dtype=torch.float32, device=dev)
    m2 = torch.zeros_like(flat) if adam else None
    indices = torch.from_numpy(w.indices).to(dev)
    offsets = torch.from_numpy(w.offsets).to(dev)
    grad = torch.randn(w.batch, col, device=dev, generator=gen)
    ws = pdm.ops.tbe_backward_workspace(plan, indices.numel(), w.batch, dev)
    counter = [0]
    opt = L.PDM_OPT_ADAM if adam else L.PDM_OPT_ROWWISE_ADAGRAD

    def step():
        counter[0] += 1
        pdm.ops.tbe_backward_fused_raw(plan, flat, m1, m2, indices, offsets, w.batch, grad, optimizer=opt,
                                       learning_rate=0.01, eps=1e-8, weight_decay=1e-5,
                                       weight_decay_mode=L.PDM_WD_L2, step=counter[0], workspace=ws)

    distinct = 0
    for t in range(len(w.rows)):
        seg = w.indices[w.offsets[t * w.batch]:w.offsets[(t + 1) * w.batch]]
        distinct += int(np.unique(seg).size)
    n = w.num_lookups
    per_row = 6 * D * 4 if adam else 2 * D * 4 + 8  # weights (+ state) read and written once per distinct row
    alg_bytes = n * 8 + w.offsets.size * 8 + w.batch * col * 4 + distinct * per_row
    return step, alg_bytes, distinct, (flat, m1, m2, plan, indices, offsets, grad, ws)


def cpu_train(torch, w, optimizer: str, batch: int, row_cap: int, threads: int):
    """The PyTorch CPU form of an embedding backward + row-sparse update: per table ``F.embedding_bag`` with a
    sparse gradient, ``backward`` of the fixed output gradient, then ``torch.optim.SparseAdam`` (Adam; no weight
    decay there) or ``torch.optim.Adagrad`` (element-wise: torch has no row-wise Adagrad) over the first
    ``batch`` bags of every table, tables capped at ``row_cap`` rows (ids taken modulo)."""
    import torch.nn.functional as Fn

    torch.set_num_threads(threads)
    D, T = w.dim, len(w.rows)
    rows = [min(r, row_cap) for r in w.rows]
    g = torch.Generator().manual_seed(8)
    params, idx, offs = [], [], []
    for t, r in enumerate(rows):
        p = torch.empty(r, D)
        fill_tiled(torch, p, torch.rand(min(r, 1 << 16), D, generator=g) * 0.02 - 0.01)
        params.append(p.requires_grad_())
        lo = int(w.offsets[t * w.batch])
        o = w.offsets[t * w.batch:t * w.batch + batch + 1] - lo
        idx.append(torch.from_numpy(w.indices[lo:lo + int(o[-1])] % r))
        offs.append(torch.from_numpy(o))
    grad = torch.randn(batch, D, generator=g)
    opt = torch.optim.SparseAdam(params, lr=0.01, eps=1e-8) if optimizer == "adam" else \
        torch.optim.Adagrad(params, lr=0.01, eps=1e-8)

    def run():
        for t in range(T):
            out = Fn.embedding_bag(idx[t], params[t], offs[t], mode="sum", sparse=True, include_last_offset=True)
            out.backward(grad)
        opt.step()
        opt.zero_grad(set_to_none=True)

    sec, reps = time_cpu(run)
    return int(sum(i.numel() for i in idx)), sec, reps


def setup_train_seq(pdm, torch, dev, w):
    """fp32 feature tables of the S-token workload with zeroed Adam state; a step is one gather backward +
    fused update with a fixed token gradient.  Returns (step, algorithmic bytes, distinct rows, keepalive)."""
    L = pdm._lib
    offs, off = [], 0
    for r, d in zip(w.table_rows, w.table_dims):
        off = (off + 255) // 256 * 256
        offs.append(off)
        off += r * d * 4
    log(f"allocating {off / 1e9:.2f} GB of fp32 tables (+ Adam state)")
    flat = torch.empty(off // 4, dtype=torch.float32, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1008)
    for r0 in range(0, flat.numel(), 1 << 26):
        flat[r0:r0 + (1 << 26)].uniform_(-0.01, 0.01, generator=gen)
    slots, col = [], 0
    for f, (r, d) in enumerate(zip(w.table_rows, w.table_dims)):
        slots.append(dict(rows=r, weights_offset=offs[f], dim=d, dtype=L.PDM_F32, pooling=L.PDM_POOL_SUM,
                          row_bytes=4 * d, out_offset=col))
        col += d
    plan = pdm.ops.TbePlan(slots, dev)
    m1, m2 = torch.zeros_like(flat), torch.zeros_like(flat)
    ids = [[torch.from_numpy(a).to(dev) for a in row] for row in w.ids]
    offsets = [torch.from_numpy(o).to(dev) for o in w.offsets]
    S = sum(w.max_len)
    grad = torch.randn(w.batch, S, col, device=dev, generator=gen)
    ws = pdm.ops.tbe_backward_workspace(plan, len(slots) * w.batch * S, w.batch * S, dev)
    counter = [0]

    def step():
        counter[0] += 1
        pdm.ops.seq_gather_backward_fused_raw(plan, flat, m1, m2, w.table_rows, w.table_dims, ids, offsets,
                                              w.max_len, grad, learning_rate=0.01, eps=1e-8, weight_decay=1e-5,
                                              step=counter[0], workspace=ws)

    # distinct rows: the kept events' ids per table, plus row 0 when some slot is padding; each distinct row's
    # weights and both Adam moments are read and written once
    distinct, kept, upd = 0, 0, 0
    for f, d in enumerate(w.table_dims):
        seen, pad = [], False
        for p, (o, m) in enumerate(zip(w.offsets, w.max_len)):
            k = np.minimum(np.diff(o), m)
            pad = pad or bool((k < m).any())
            sel = np.concatenate([np.arange(a, a + n) for a, n in zip(o[1:] - k, k)])
            seen.append(w.ids[p][f][sel])
            if f == 0:
                kept += int(k.sum())
        u = np.unique(np.concatenate(seen + ([np.zeros(1, np.int64)] if pad else [])))
        distinct += int(u.size)
        upd += int(u.size) * 6 * 4 * d
    alg_bytes = kept * 3 * 8 + sum(o.size * 8 for o in w.offsets) + w.batch * S * col * 4 + upd
    return step, alg_bytes, distinct, kept, (flat, m1, m2, plan, ids, offsets, grad, ws)


def cpu_train_seq(torch, w, batch: int, row_cap: int, threads: int):
    """The PyTorch CPU form of the S-token gather backward + Adam: the padded lookups of ``cpu_seq`` with sparse
    gradients on fp32 tables, ``backward`` of the fixed token gradient, ``torch.optim.SparseAdam``, over the
    first ``batch`` samples, tables capped at ``row_cap`` rows (ids taken modulo)."""
    import torch.nn.functional as Fn

    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(9)
    rows = [min(r, row_cap) for r in w.table_rows]
    params = []
    for r, d in zip(rows, w.table_dims):
        p = torch.empty(r, d)
        fill_tiled(torch, p, torch.rand(min(r, 1 << 16), d, generator=g) * 0.02 - 0.01)
        params.append(p.requires_grad_())
    padded = _padded_ids(torch, [[a % r for a, r in zip(row, rows)] for row in w.ids], w.offsets, w.max_len, batch)
    S = sum(w.max_len)
    grad = torch.randn(batch, S, sum(w.table_dims), generator=g)
    opt = torch.optim.SparseAdam(params, lr=0.01, eps=1e-8)

    def run():
        parts = [torch.cat([Fn.embedding(pid, params[f], sparse=True) for f, pid in enumerate(pool)], -1)
                 for pool, _ in padded]
        torch.cat(parts, 1).backward(grad)
        opt.step()
        opt.zero_grad(set_to_none=True)

    sec, reps = time_cpu(run)
    return batch * S, sec, reps


# ----------------------------------------------------------------------------------------------
# S-token gather
# ----------------------------------------------------------------------------------------------

def setup_seq(pdm, torch, dev, w):
    gen = torch.Generator(device=dev)
    gen.manual_seed(1004)
    tables = []
    for rows, dim in zip(w.table_rows, w.table_dims):
        t = torch.empty((rows, dim), dtype=torch.bfloat16, device=dev)
        for r0 in range(0, rows, 1 << 20):
            n = min(1 << 20, rows - r0)
            t[r0:r0 + n].copy_(torch.empty((n, dim), device=dev).normal_(0.0, 0.02, generator=gen))
        tables.append(t)
    ids = [[torch.from_numpy(a).to(dev) for a in row] for row in w.ids]
    offs = [torch.from_numpy(o).to(dev) for o in w.offsets]

    def step():
        pdm.ops.seq_gather_raw(tables, ids, offs, w.max_len)

    S = sum(w.max_len)
    row_bytes = sum(w.table_dims) * 2
    events = w.num_events
    kept = sum(int(np.minimum(np.diff(o), m).sum()) for o, m in zip(w.offsets, w.max_len))
    # rows read for kept events + row 0 per padded slot (cached) counted once per slot is ignored;
    # ids read (3 x int64 per kept event), offsets, padded output and mask written
    alg_bytes = kept * row_bytes + kept * 3 * 8 + sum(o.size * 8 for o in w.offsets) + \
        w.batch * S * row_bytes + w.batch * S
    return step, alg_bytes, kept, (tables, ids, offs)


def _padded_ids(torch, ids, offsets, max_len, batch=None):
    """The dataset's jagged -> padded step (primus_dlrm/data/dataset.py:604-626) on the CPU: per pool the last
    ``L`` events of each sample, right aligned, left padded with id 0; returns [(per-feature [B, L] ids, mask)]."""
    out = []
    for p, L in enumerate(max_len):
        off = torch.from_numpy(offsets[p] if batch is None else offsets[p][:batch + 1])
        n = (off[1:] - off[:-1]).clamp(max=L)
        k = torch.arange(L).unsqueeze(0) - (L - n).unsqueeze(1)
        valid = k >= 0
        src = (off[1:] - n).unsqueeze(1) + k.clamp(min=0)
        feats = []
        for a in ids[p]:
            t = torch.from_numpy(a)
            feats.append(torch.where(valid, t[src.clamp(max=max(t.numel() - 1, 0))], 0) if t.numel() else
                         torch.zeros_like(src))
        out.append((feats, valid))
    return out


def cpu_seq(torch, w, threads: int):
    """The reference's S-token input on the CPU: the jagged -> padded ids (dataset.py:604-626), ``W[ids]`` per
    feature (EmbeddingCollection rows, ``values().view(B, L, D)``), ``cat`` of item | artist | album per pool
    (onetrans.py:515-520) and of the pools along the sequence (:553-558), with the padding mask, on the full
    batch over full-size bf16 tables."""
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(6)
    tables = []
    for r, d in zip(w.table_rows, w.table_dims):
        t = torch.empty((r, d), dtype=torch.bfloat16)
        fill_tiled(torch, t, (torch.randn(min(r, 1 << 16), d, generator=g) * 0.02).to(torch.bfloat16))
        tables.append(t)

    def run():
        parts, masks = [], []
        for feats, valid in _padded_ids(torch, w.ids, w.offsets, w.max_len):
            parts.append(torch.cat([tables[f][pid] for f, pid in enumerate(feats)], -1))
            masks.append(valid)
        return torch.cat(parts, 1), torch.cat(masks, 1)

    sec, reps = time_cpu(run)
    return sec, reps, sum(r * d * 2 for r, d in zip(w.table_rows, w.table_dims))


# ----------------------------------------------------------------------------------------------
# S-token gather fused with the sequential tokenizers
# ----------------------------------------------------------------------------------------------

TOK_D, TOK_POS_ROWS = 256, 2048


def setup_tokenize(pdm, torch, dev, w):
    _, _, kept, (tables, ids, offs) = setup_seq(pdm, torch, dev, w)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1010)
    K, d = sum(w.table_dims), TOK_D
    bf = lambda *shape: (torch.randn(*shape, device=dev, generator=gen) * 0.05).to(torch.bfloat16)  # noqa: E731
    weights = [dict(w1=bf(d, K), b1=bf(d), w2=bf(d, d), b2=bf(d),
                    pos=torch.randn(TOK_POS_ROWS, d, device=dev, generator=gen)) for _ in w.max_len]
    S = sum(w.max_len)
    out = torch.empty(w.batch, S, d, device=dev)
    work = pdm.ops.seq_tokenize_workspace(tables, ids, offs, w.max_len, d)

    def step():
        pdm.ops.seq_tokenize_raw(tables, ids, offs, w.max_len, weights, out=out, workspace=work)

    # HBM bytes a perfect kernel moves: kept events' rows and ids, offsets, the fp32 S-tokens and mask written,
    # the tokenizer weights and the used position rows read once
    row_bytes = K * 2
    alg_bytes = kept * row_bytes + kept * 3 * 8 + sum(o.size * 8 for o in w.offsets) + \
        w.batch * S * (d * 4 + 1) + len(w.max_len) * ((K * d + d * d + 2 * d) * 2 + max(w.max_len) * d * 4)
    # MFMA work: the MLP of every kept event plus one padding row per pool
    flops = 2.0 * (K * d + d * d) * (kept + len(w.max_len))
    return step, alg_bytes, flops, kept, (tables, ids, offs, weights, out, work)


def unfused_tokenize_ms(pdm, torch, keep, w, reps: int = 20) -> float:
    """The same S-tokens the reference's way on this GPU: the S-token gather to [B, S, 384] bf16, then per pool
    torch bf16 Linear (+bias), exact GELU, Linear (+bias) and + pos_emb in fp32, concatenated (reported beside
    the fused call, not the bench value)."""
    import torch.nn.functional as Fn

    tables, ids, offs, weights, _, _ = keep
    S = sum(w.max_len)

    def run():
        raw, _ = pdm.ops.seq_gather_raw(tables, ids, offs, w.max_len)
        parts, s0 = [], 0
        for p, L in enumerate(w.max_len):
            wt = weights[p]
            hdn = Fn.gelu(Fn.linear(raw[:, s0:s0 + L], wt["w1"], wt["b1"]))
            parts.append(Fn.linear(hdn, wt["w2"], wt["b2"]).float() + wt["pos"][:L])
            s0 += L
        return torch.cat(parts, dim=1)

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        run()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def cpu_tokenize(torch, w, threads: int, batch: int):
    """The reference's S-tokens on the CPU in fp32: the padded lookups and concat of ``cpu_seq`` (full-size
    tables) for the first ``batch`` samples, then per pool ``SequentialTokenizer`` (Linear(384, 256), exact GELU,
    Linear(256, 256), + pos_emb(arange(L)); onetrans.py:238-257) and the concat along the sequence."""
    import torch.nn.functional as Fn

    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(6)
    tables = []
    for r, d in zip(w.table_rows, w.table_dims):
        t = torch.empty((r, d))
        fill_tiled(torch, t, torch.randn(min(r, 1 << 16), d, generator=g) * 0.02)
        tables.append(t)
    K = sum(w.table_dims)
    ws = [dict(w1=torch.randn(TOK_D, K, generator=g) * 0.05, b1=torch.randn(TOK_D, generator=g) * 0.05,
               w2=torch.randn(TOK_D, TOK_D, generator=g) * 0.05, b2=torch.randn(TOK_D, generator=g) * 0.05,
               pos=torch.randn(TOK_POS_ROWS, TOK_D, generator=g)) for _ in w.max_len]

    def run():
        parts = []
        for p, (feats, _) in enumerate(_padded_ids(torch, w.ids, w.offsets, w.max_len, batch)):
            raw = torch.cat([tables[f][pid] for f, pid in enumerate(feats)], -1)
            wt = ws[p]
            h = Fn.gelu(Fn.linear(raw, wt["w1"], wt["b1"]))
            parts.append(Fn.linear(h, wt["w2"], wt["b2"]) + wt["pos"][:raw.shape[1]])
        return torch.cat(parts, 1)

    return time_cpu(run, reps=3)


# ----------------------------------------------------------------------------------------------
# NS tokens (scalar-feature rows + dense parts through the AutoSplitTokenizer)
# ----------------------------------------------------------------------------------------------

NS_TABLES = [("uid", 1_000_001), ("item", 9_390_624), ("artist", 1_293_395), ("album", 3_367_692)]
NS_DIM, NS_DENSE, NS_D, NS_N = 64, [64, 6, 6, 64], 256, 16


def setup_ns(pdm, torch, dev, batch: int):
    gen = torch.Generator(device=dev)
    gen.manual_seed(1011)
    tables = []
    for _, rows in NS_TABLES:
        t = torch.empty((rows, NS_DIM), dtype=torch.bfloat16, device=dev)
        for r0 in range(0, rows, 1 << 21):
            n = min(1 << 21, rows - r0)
            t[r0:r0 + n].copy_(torch.empty((n, NS_DIM), device=dev).uniform_(-0.05, 0.05, generator=gen))
        tables.append(t)
    rng = np.random.default_rng(1012)
    ids = [torch.from_numpy(rng.integers(0, rows, batch)).to(dev) for _, rows in NS_TABLES]
    dense = [torch.randn(batch, d, device=dev, generator=gen) for d in NS_DENSE]
    K, N = NS_DIM * len(NS_TABLES) + sum(NS_DENSE), NS_D * NS_N
    bf = lambda *shape: (torch.randn(*shape, device=dev, generator=gen) * 0.02).to(torch.bfloat16)  # noqa: E731
    w1, b1, w2, b2 = bf(N, K), bf(N), bf(N, N), bf(N)
    out = torch.empty(batch, NS_N, NS_D, device=dev)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)

    def step():
        pdm.ops.ns_tokenize_raw(tables, ids, dense, w1, b1, w2, b2, NS_N, out=out, workspace=ws)

    flops = 2.0 * batch * (K * N + N * N)
    return step, flops, K, N, (tables, ids, dense, w1, b1, w2, b2, out, ws)


def unfused_ns_ms(pdm, torch, keep, reps: int = 20) -> float:
    """The same NS tokens the reference's way on this GPU: row lookups + cat to [B, 396] bf16, then torch bf16
    F.linear + bias, F.gelu, F.linear + bias, viewed [B, n_ns, d] and converted to fp32 (reported beside the
    fused call)."""
    import torch.nn.functional as Fn

    tables, ids, dense, w1, b1, w2, b2, _, _ = keep

    def run():
        raw = torch.cat([t[i] for t, i in zip(tables, ids)] + [x.to(torch.bfloat16) for x in dense], dim=1)
        hdn = Fn.gelu(Fn.linear(raw, w1, b1))
        return Fn.linear(hdn, w2, b2).view(raw.shape[0], NS_N, NS_D).float()

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        run()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def cpu_ns(torch, threads: int, batch: int):
    """The reference's NS tokens on the CPU in fp32: one row per scalar feature from full-size tables, the dense
    parts, ``cat`` (_build_ns_raw, onetrans.py:522-532), then AutoSplitTokenizer's Linear(396, 4096), exact GELU,
    Linear(4096, 4096), viewed [B, 16, 256] (onetrans.py:260-276)."""
    import torch.nn.functional as Fn

    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(7)
    tabs = []
    for _, rows in NS_TABLES:
        t = torch.empty(rows, NS_DIM)
        fill_tiled(torch, t, torch.rand(min(rows, 1 << 16), NS_DIM, generator=g) * 0.1 - 0.05)
        tabs.append(t)
    ids = [torch.randint(0, rows, (batch,), generator=g) for _, rows in NS_TABLES]
    dense = [torch.randn(batch, d, generator=g) for d in NS_DENSE]
    K, N = NS_DIM * len(NS_TABLES) + sum(NS_DENSE), NS_D * NS_N
    w1, b1 = torch.randn(N, K, generator=g) * 0.02, torch.randn(N, generator=g) * 0.02
    w2, b2 = torch.randn(N, N, generator=g) * 0.02, torch.randn(N, generator=g) * 0.02

    def run():
        raw = torch.cat([t[i] for t, i in zip(tabs, ids)] + dense, dim=1)
        return Fn.linear(Fn.gelu(Fn.linear(raw, w1, b1)), w2, b2).view(batch, NS_N, NS_D)

    return time_cpu(run, reps=3)


# ----------------------------------------------------------------------------------------------
# OneTrans block stack
# ----------------------------------------------------------------------------------------------

def setup_onetrans(pdm, torch, dev, w):
    import primus_dlrm_amd.synthetic as syn

    D, F, n_ns = w.d_model, w.d_model * w.ffn_mult, w.n_ns
    gen = torch.Generator(device=dev)
    gen.manual_seed(1005)
    layers = []
    for _ in w.schedule:
        r = lambda *s: (torch.randn(*s, device=dev, generator=gen) * 0.02).to(torch.bfloat16)  # noqa: E731
        layers.append(dict(norm1_w=torch.ones(D, device=dev), s_qkv_w=r(3 * D, D), ns_qkv_w=r(n_ns, 3 * D, D),
                           out_w=r(D, D), norm2_w=torch.ones(D, device=dev), s_w1=r(F, D), s_w2=r(D, F),
                           ns_w1=r(n_ns, F, D), ns_w2=r(n_ns, D, F)))
    kv0 = w.l_s + n_ns
    x = torch.randn(w.batch, kv0, D, device=dev, generator=gen) * 0.02
    H = D // 64
    ws = torch.empty(pdm.ops.onetrans_stack_workspace_bytes(w.batch, kv0, D, F, n_ns, H, w.schedule),
                     dtype=torch.uint8, device=dev)
    out = torch.empty(w.batch, w.schedule[-1] + n_ns, D, device=dev)

    def step():
        # the whole 4-layer loop in one call (pdm_onetrans_stack_fwd)
        pdm.ops.onetrans_stack_raw(x, layers, H, w.schedule, out=out, workspace=ws)

    return step, syn.block_flops(w), syn.block_flops_causal(w), (x, layers, ws, out)


def _torch_block(torch, x, w, q_len: int, n_heads: int):
    """OneTransBlock.forward as the reference writes it (onetrans.py:74-231) with torch functional ops in fp32:
    RMSNorm, shared Linear QKV + per-token einsum, SDPA with the bool pyramid mask, out-projection, RMSNorm,
    shared FFN + per-token einsum FFN, residuals."""
    import torch.nn.functional as Fn

    B, kv, D = x.shape
    n_ns = w["ns_qkv"].shape[0]
    n_s, dh = kv - n_ns, D // n_heads

    def rms(t, wt):
        return (t * t.pow(2).mean(-1, keepdim=True).add(1e-6).rsqrt()) * wt

    h = rms(x, w["norm1"])
    sq = Fn.linear(h[:, :n_s], w["s_qkv"]).reshape(B, n_s, 3, n_heads, dh)
    nq = torch.einsum("btn,tmn->btm", h[:, n_s:], w["ns_qkv"]).reshape(B, n_ns, 3, n_heads, dh)
    q = torch.cat([sq[:, :, 0], nq[:, :, 0]], 1)[:, kv - q_len:]
    k = torch.cat([sq[:, :, 1], nq[:, :, 1]], 1)
    v = torch.cat([sq[:, :, 2], nq[:, :, 2]], 1)
    mask = torch.arange(kv).unsqueeze(0) <= torch.arange(q_len).unsqueeze(1) + (kv - q_len)
    o = Fn.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                        attn_mask=mask[None, None]).transpose(1, 2).reshape(B, q_len, D)
    z = Fn.linear(o, w["out"]) + x[:, kv - q_len:]
    h2 = rms(z, w["norm2"])
    n_s_out = q_len - n_ns
    s_out = Fn.linear(Fn.gelu(Fn.linear(h2[:, :n_s_out], w["s_w1"])), w["s_w2"])
    ns_h = Fn.gelu(torch.einsum("btn,tmn->btm", h2[:, n_s_out:], w["ns_w1"]))
    ns_out = torch.einsum("btm,tnm->btn", ns_h, w["ns_w2"])
    return z + torch.cat([s_out, ns_out], 1)


def cpu_onetrans(torch, w, threads: int, batch: int):
    """The reference's block stack (the block loop of onetrans.py:568-582) in fp32 torch on the CPU at
    ``batch`` samples, N(0, 0.02) weights and inputs."""
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1005)
    D, F, n_ns = w.d_model, w.d_model * w.ffn_mult, w.n_ns
    r = lambda *shape: torch.randn(*shape, generator=g) * 0.02  # noqa: E731
    layers = [dict(norm1=torch.ones(D), s_qkv=r(3 * D, D), ns_qkv=r(n_ns, 3 * D, D), out=r(D, D),
                   norm2=torch.ones(D), s_w1=r(F, D), s_w2=r(D, F), ns_w1=r(n_ns, F, D), ns_w2=r(n_ns, D, F))
              for _ in w.schedule]
    x0 = r(batch, w.l_s + n_ns, D)

    def run():
        with torch.no_grad():
            x = x0
            for lw, q_s in zip(layers, w.schedule):
                x = _torch_block(torch, x, lw, q_s + n_ns, D // 64)
        return x

    return time_cpu(run, reps=3)


# ----------------------------------------------------------------------------------------------
# timing and rooflines
# ----------------------------------------------------------------------------------------------

def time_steps(torch, stream, step, steps: int, warmup: int):
    """``warmup`` untimed steps, then ``steps`` timed steps bracketed by device synchronisations.  Returns (mean
    HIP-event duration of one step on the launch stream in ms, wall seconds of the timed region)."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    return statistics.mean(a.elapsed_time(b) for a, b in ev), elapsed


TRAFFIC_NOTE = ("traffic: bytes per launch that the L2 requested from and wrote to the memory fabric (rocprofv3 "
                "TCC_EA0 read/write requests by size, read requests 128 B); requests served by the Infinity Cache "
                "are included, so it is an upper bound on HBM bytes, not an HBM measurement; traffic_dram counts "
                "the requests bound for DRAM and equals it here")


def hbm_roofline(alg: float, kernel_ms: float, workload):
    achieved = alg / (kernel_ms * 1e-3) / 1e9
    out = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": int(alg),
           "kernel_ms": round(kernel_ms, 5)}
    if workload is not None:
        out.update(traffic_fields(workload))
    return out


def mfma_roofline(alg: float, kernel_ms: float, workload):
    achieved = alg / (kernel_ms * 1e-3) / 1e12
    out = {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
           "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None, "algorithmic_flops": alg,
           "kernel_ms": round(kernel_ms, 5)}
    if workload is not None:
        out.update(traffic_fields(workload))
    return out


def causal_roofline(causal: float, kernel_ms: float):
    """The same step against the FLOPs the causal pyramid executes (no masked keys, no dropped Q rows)."""
    ach_c = causal / (kernel_ms * 1e-3) / 1e12
    return dict(causal_flops=causal, achieved_causal=round(ach_c, 1), frac_causal=round(ach_c / BF16_PEAK_TFLOPS, 4))


def int8_uniform_leg(pdm, torch, dev, stream, keep, args):
    """The default lookup on the same 64 x 5 M int8 tables and bag lengths with uniform ids: each lookup reads
    a row that is unlikely to be in any cache, so this rate is what the kernel reaches from HBM."""
    import primus_dlrm_amd.synthetic as syn

    flat, plan, _, _, out = keep
    w = syn.int8_mean(ids="uniform")
    indices = torch.from_numpy(w.indices).to(dev)
    offsets = torch.from_numpy(w.offsets).to(dev)

    def step():
        pdm.ops.tbe_pooled_raw(plan, flat, indices, offsets, w.batch, torch.float16, -1, out=out)

    row_bytes = (4 + w.dim + 3) & ~3
    n = w.num_lookups
    alg = n * row_bytes + n * 8 + w.offsets.size * 8 + w.batch * out.shape[1] * 2
    log("uniform-id control: warmup")
    kernel_ms, elapsed = time_steps(torch, stream, step, args.steps, args.warmup)
    r = hbm_roofline(alg, kernel_ms, "int8_mean_uniform")
    log(f"uniform-id control: {kernel_ms:.4f} ms, {r['achieved']:.1f} GB/s")
    return {"workload": w.name, "ids": "uniform over each table's 5,000,000 rows", "lookups_per_batch": n,
            "value": round(n * args.steps / elapsed, 1), "unit": "lookups/s",
            "ms_per_step": round(elapsed * 1e3 / args.steps, 5), "roofline": r}


def onetrans_config(w, alg, causal):
    return {"workload": w.name, "batch": w.batch, "l_s": w.l_s, "n_ns": w.n_ns, "d_model": w.d_model,
            "n_heads": w.n_heads, "ffn": w.d_model * w.ffn_mult, "schedule": w.schedule,
            "gflop_per_step": round(alg / 1e9, 1), "causal_gflop_per_step": round(causal / 1e9, 1)}


ONETRANS_CPU_BATCH = 1024
ONETRANS_L_CPU_BATCH = 16  # OneTransL: 0.67 TFLOP per 16 samples


def onetrans_cpu_baseline(torch, w, threads: int, batch: int = ONETRANS_CPU_BATCH):
    sec, reps = cpu_onetrans(torch, w, threads, batch)
    n = len(w.schedule)
    return cpu_result(batch / sec, "samples/s", threads, f"torch fp32 OneTransBlock x{n} (Linear, einsum, "
                      "SDPA with the bool pyramid mask, RMSNorm, GELU)",
                      f"the {n}-layer stack on " + (f"the full batch of {batch} samples" if batch == w.batch else
                                                    f"{batch} of the batch's {w.batch} samples"), sec, reps)


def block_leg(pdm, torch, dev, stream, args, threads: int):
    """The OneTrans interaction block half of the metric, measured in the same run: the 4-layer stack
    (pdm_onetrans_stack_fwd) at B = 1024, 384 S + 16 NS tokens, d_model 256, schedule 384/256/128/64."""
    import primus_dlrm_amd.synthetic as syn

    w = syn.onetrans_block()
    step, alg, causal, keep = setup_onetrans(pdm, torch, dev, w)
    log("block leg: warmup")
    kernel_ms, elapsed = time_steps(torch, stream, step, args.steps, args.warmup)
    r = mfma_roofline(alg, kernel_ms, "onetrans")
    r.update(causal_roofline(causal, kernel_ms))
    log(f"block leg: {kernel_ms:.4f} ms per step, {r['achieved']:.1f} TFLOP/s")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = onetrans_cpu_baseline(torch, w, threads)
    del keep
    return {"metric": "OneTrans block samples/sec", "value": round(w.batch * args.steps / elapsed, 1),
            "unit": "samples/s", "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(elapsed * 1e3 / args.steps, 5), "dtype": "bf16",
            "config": onetrans_config(w, alg, causal), "roofline": r, "cpu_baseline": cpu}


# ----------------------------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="int8_mean",
                    choices=["single_hot", "ebc_fp32", "int8_mean", "seq_gather", "seq_tokenize", "ns_tokenize",
                             "onetrans", "onetrans_l",
                             "cross_hash",
                             "train_adam", "train_rowwise_adagrad", "train_seq_adam", "kjt_build", "copy_1gib"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ids", default="zipf", choices=["zipf", "uniform"],
                    help="id distribution of single_hot, int8_mean and seq_gather (uniform: the cold-row control)")
    ap.add_argument("--no-extra-legs", action="store_true",
                    help="default workload only: skip the uniform-id control and the OneTrans block leg")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (no collectives or sharding); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import __graft_entry__ as ge

    pdm = ge.pdm_import()
    import primus_dlrm_amd.synthetic as syn
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    threads, _, cpu_model = cpu_env()
    cpu_fn = None
    graph_fn = None

    if args.workload in ("single_hot", "ebc_fp32", "int8_mean"):
        if args.workload == "single_hot":
            w, std = syn.single_hot_bf16(ids=args.ids), 0.02
        elif args.workload == "ebc_fp32":
            w, std = syn.ebc_fp32(), 0.01
        else:
            w, std = syn.int8_mean(ids=args.ids), 0.05
        step, alg, keep = setup_pooled(pdm, torch, dev, w, std)
        units, unit, bound = w.num_lookups, "lookups/s", "hbm"
        dtype = {"bf16": "bf16->f32", "fp32": "f32", "int8": "u8->f32"}[w.dtype]
        cfg = {"workload": w.name, "tables": w.num_tables, "rows_total": int(sum(w.rows)), "dim": w.dim,
               "batch": w.batch, "lookups_per_batch": w.num_lookups, "pooling": w.pooling,
               "weights": w.dtype, "out": w.out_dtype,
               "ids": "uniform" if args.workload == "ebc_fp32" else args.ids}  # the EBC workload's ids are uniform
        if args.workload == "ebc_fp32":
            def graph_fn():
                return graph_steady_state(torch, dev, step, GRAPH_BATCHES)

        def cpu_fn():
            val, sec, reps, op, sample = cpu_pooled(torch, w, threads, std)
            return cpu_result(val, unit, threads, f"torch {op} per table + cat (unsharded TorchRec EBC)",
                              sample, sec, reps)
    elif args.workload == "seq_gather":
        w = syn.seq_gather(ids=args.ids)
        step, alg, kept, keep = setup_seq(pdm, torch, dev, w)
        units, unit, bound, dtype = kept, "events/s", "hbm", "bf16"
        cfg = {"workload": w.name, "batch": w.batch, "pools": len(w.max_len), "max_len": w.max_len,
               "tables": {"rows": w.table_rows, "dims": w.table_dims}, "events_kept": kept,
               "out": [w.batch, sum(w.max_len), sum(w.table_dims)], "ids": args.ids}

        def cpu_fn():
            sec, reps, tb = cpu_seq(torch, w, threads)
            return cpu_result(kept / sec, unit, threads, "torch jagged->padded ids + W[ids] + cat (EC rows, "
                              "_build_pool_raw, pool concat)", f"full batch of {kept} kept events on full-size "
                              f"bf16 tables ({tb / 1e9:.1f} GB)", sec, reps)
    elif args.workload == "seq_tokenize":
        w = syn.seq_gather()
        step, alg, flops, kept, keep = setup_tokenize(pdm, torch, dev, w)
        S = sum(w.max_len)
        units, unit, bound, dtype = w.batch * S, "slots/s", "hbm", "bf16->f32"
        cfg = {"workload": w.name + "_tokenize", "batch": w.batch, "pools": len(w.max_len), "max_len": w.max_len,
               "tables": {"rows": w.table_rows, "dims": w.table_dims}, "events_kept": kept,
               "tokenizer": {"raw_dim": sum(w.table_dims), "d_model": TOK_D, "pos_rows": TOK_POS_ROWS},
               "out": [w.batch, S, TOK_D], "mlp_gflop_per_step": round(flops / 1e9, 2),
               "timed": "whole fused call (list build, MLP over kept events, padding fill)"}
        cfg["unfused_same_gpu_ms"] = round(unfused_tokenize_ms(pdm, torch, keep, w), 4)
        cpu_b = w.batch

        def cpu_fn():
            sec, reps = cpu_tokenize(torch, w, threads, cpu_b)
            return cpu_result(cpu_b * S / sec, unit, threads, "torch fp32: padded lookups + cat, per pool "
                              "Linear / GELU / Linear + pos_emb (SequentialTokenizer), cat",
                              f"the full batch of {cpu_b} samples ({cpu_b * S} slots) on full-size fp32 tables", sec, reps)
    elif args.workload == "ns_tokenize":
        B_ = 1024
        step, alg, K_, N_, keep = setup_ns(pdm, torch, dev, B_)
        units, unit, bound, dtype = B_, "samples/s", "mfma", "bf16"
        cfg = {"workload": "ns_tokens_b1024_k396_n4096", "batch": B_,
               "scalar_tables": {n: r for n, r in NS_TABLES}, "scalar_dim": NS_DIM, "dense_dims": NS_DENSE,
               "ns_input": K_, "d_model": NS_D, "n_ns": NS_N, "gflop_per_step": round(alg / 1e9, 2),
               "timed": "whole call (NS rows gather, W1 padding copy, Linear 1 + bias + GELU, Linear 2 + bias)"}
        cfg["unfused_same_gpu_ms"] = round(unfused_ns_ms(pdm, torch, keep), 4)

        def cpu_fn():
            sec, reps = cpu_ns(torch, threads, B_)
            return cpu_result(B_ / sec, unit, threads, "torch fp32: scalar rows + dense cat (_build_ns_raw), "
                              "Linear / GELU / Linear (AutoSplitTokenizer)", f"full batch of {B_} samples on "
                              "full-size fp32 tables", sec, reps)
    elif args.workload == "cross_hash":
        # user_x_artist cross ids (config.py:151): one (uid, artist_id) pair per row, 100M buckets, salt 0
        n_rows, table_size = 1 << 24, 100_000_000
        rng = np.random.default_rng(1006)
        uid = rng.integers(0, 1_000_000, n_rows, dtype=np.int64)
        artist = rng.integers(0, 1_290_000, n_rows, dtype=np.int64)
        keys = [torch.from_numpy(uid).to(dev), torch.from_numpy(artist).to(dev)]
        out = torch.empty(n_rows, dtype=torch.int64, device=dev)
        keep = (keys, out)

        def step():
            pdm.ops.cross_hash_raw(keys, table_size, 0, out=out)

        alg, units, unit, bound, dtype = n_rows * 24, n_rows, "hashes/s", "hbm", "int64"
        cfg = {"workload": "cross_hash_uid_x_artist_16m", "rows": n_rows, "keys": 2, "table_size": table_size,
               "salt": 0}
        cpu_rows = 1 << 22

        def cpu_fn():
            sec, reps, path = cpu_cross_hash(uid[:cpu_rows], artist[:cpu_rows], table_size)
            return cpu_result(cpu_rows / sec, unit, 1, path, f"the first {cpu_rows} rows", sec, reps)
    elif args.workload in ("train_adam", "train_rowwise_adagrad"):
        optimizer = "adam" if args.workload == "train_adam" else "rowwise_adagrad"
        w = syn.ebc_fp32(scale_rows=100.0, batch=65_536)
        step, alg, distinct, keep = setup_train(pdm, torch, dev, w, optimizer)
        units, unit, bound, dtype = w.num_lookups, "lookups/s", "hbm", "f32"
        cfg = {"workload": f"{w.name}_{optimizer}", "tables": w.num_tables, "rows_total": int(sum(w.rows)),
               "dim": w.dim, "batch": w.batch, "lookups_per_batch": w.num_lookups, "distinct_rows": distinct,
               "pooling": "sum", "weights": "fp32", "optimizer": optimizer, "lr": 0.01, "eps": 1e-8,
               "weight_decay": 1e-5, "timed": "whole fused backward (linearise, 3 radix passes, accumulate)"}
        cpu_b, cpu_cap = 16_384, 1_000_000

        def cpu_fn():
            n, sec, reps = cpu_train(torch, w, optimizer, cpu_b, cpu_cap, threads)
            opt = "SparseAdam" if optimizer == "adam" else "Adagrad (element-wise)"
            return cpu_result(n / sec, unit, threads, f"torch F.embedding_bag(sparse=True) backward + {opt}",
                              f"the first {cpu_b} bags of each table ({n} lookups), tables capped at {cpu_cap} "
                              "rows (ids modulo)", sec, reps)
    elif args.workload == "train_seq_adam":
        w = syn.seq_gather()
        step, alg, distinct, kept, keep = setup_train_seq(pdm, torch, dev, w)
        S = sum(w.max_len)
        units, unit, bound, dtype = w.batch * S, "slots/s", "hbm", "f32"
        cfg = {"workload": "seq_gather_3pools_b1024_fp32_adam", "batch": w.batch, "slots": S,
               "tables": {"rows": w.table_rows, "dims": w.table_dims}, "events_kept": kept,
               "distinct_rows": distinct, "pad": "row0 (pad slots update row 0, as the reference's pad id 0)",
               "optimizer": "adam", "lr": 0.01, "eps": 1e-8, "weight_decay": 1e-5,
               "timed": "whole fused gather backward"}
        cpu_b, cpu_cap = w.batch, 1_000_000

        def cpu_fn():
            n, sec, reps = cpu_train_seq(torch, w, cpu_b, cpu_cap, threads)
            return cpu_result(n / sec, unit, threads, "torch padded F.embedding(sparse=True) + cat, backward, "
                              "SparseAdam", f"the first {cpu_b} samples ({n} slots x 3 features), tables capped "
                              f"at {cpu_cap} rows (ids modulo)", sec, reps)
    elif args.workload == "kjt_build":
        # the pooled-history KJT of _build_pooled_kjt (embedding.py:177-204) at the single-hot batch
        F_, B_, L_ = 26, 65_536, 20
        rng = np.random.default_rng(1009)
        mats = []
        for _ in range(F_):
            m = rng.integers(1, 1 << 40, (B_, L_), dtype=np.int64)
            m[rng.random((B_, L_)) < 0.3] = 0
            mats.append(m)
        feats = [torch.from_numpy(m).to(dev) for m in mats]
        kept = int(sum(int((m != 0).sum()) for m in mats))
        # two batches of the same size (the second: the same matrices in a rolled feature order, in their own
        # memory) alternate, so no build starts on ids the previous build left in the caches
        batches = (feats, [t.clone() for t in feats[1:] + feats[:1]])
        keep = batches
        nstep = [0]

        def step():
            pdm.ops.kjt_from_dense_raw(batches[nstep[0] & 1], 0)
            nstep[0] += 1

        rows = F_ * B_
        alg = F_ * B_ * L_ * 8 + kept * 8 + rows * 4 + (rows + 1) * 8
        units, unit, bound, dtype = F_ * B_ * L_, "ids/s", "hbm", "int64"
        cfg = {"workload": "kjt_build_26x65536x20_pad30", "features": F_, "batch": B_, "ids_per_row": L_,
               "kept": kept, "padding_idx": 0}

        def cpu_fn():
            sec, reps = cpu_kjt(torch, mats, 0, threads)
            return cpu_result(units / sec, unit, threads, "torch _build_pooled_kjt expression (mask, sum, ids[mask], "
                              "cat, offsets cumsum)", f"all {units} ids", sec, reps)
    elif args.workload == "copy_1gib":
        # calibration: a plain device copy of 1 GiB (reads 1 GiB, writes 1 GiB) for the HBM counters
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        keep = (src, dst)

        def step():
            dst.copy_(src)

        alg, units, unit, bound, dtype = 2 << 30, 2 << 30, "bytes/s", "hbm", "f32"
        cfg = {"workload": "device_copy_1gib"}
    else:
        large = args.workload == "onetrans_l"
        w = syn.onetrans_large() if large else syn.onetrans_block()
        step, alg, causal, keep = setup_onetrans(pdm, torch, dev, w)
        units, unit, bound, dtype = w.batch, "samples/s", "mfma", "bf16"
        cfg = onetrans_config(w, alg, causal)

        def cpu_fn():
            return onetrans_cpu_baseline(torch, w, threads, ONETRANS_L_CPU_BATCH if large else ONETRANS_CPU_BATCH)

    stream = torch.cuda.current_stream(dev)
    log(f"warmup {args.warmup} steps")
    kernel_ms, elapsed = time_steps(torch, stream, step, args.steps, args.warmup)
    ms_per_step = elapsed * 1e3 / args.steps
    value = units * args.steps / elapsed
    if bound == "hbm":
        roofline = hbm_roofline(alg, kernel_ms, args.workload if args.ids == "zipf" else args.workload + "_uniform")
    else:
        roofline = mfma_roofline(alg, kernel_ms, args.workload)
        if args.workload in ("onetrans", "onetrans_l"):
            roofline.update(causal_roofline(causal, kernel_ms))
    log(f"{value:.4g} {unit}, step {kernel_ms:.4f} ms, {roofline['achieved']:.1f} {roofline['unit']}")
    if graph_fn is not None:
        g_ms = graph_fn()
        g_ach = alg / (g_ms * 1e-3) / 1e9
        roofline["graph_steady_state"] = {
            "batches_per_graph": GRAPH_BATCHES, "ms_per_batch": round(g_ms, 5), "achieved": round(g_ach, 1),
            "frac": round(g_ach / HBM_PEAK_GBS, 4),
            "note": "the same launch replayed back to back from one HIP graph; the eager figure above is one "
                    "batch's launch latency"}
        log(f"graph steady state: {g_ms:.4f} ms per batch, {g_ach:.1f} GB/s")

    extra = {}
    if args.workload == "int8_mean" and args.ids == "zipf" and not args.no_extra_legs:
        # the same tables and bag lengths with uniform ids: rows that mostly come from HBM
        extra["uniform_ids_control"] = int8_uniform_leg(pdm, torch, dev, stream, keep, args)
    cpu = None
    if not args.no_cpu_baseline and cpu_fn is not None:
        log(f"cpu baseline on {threads} threads ({cpu_model})")
        cpu = cpu_fn()
    if args.workload == "int8_mean" and args.ids == "zipf" and not args.no_extra_legs:
        del keep, step
        torch.cuda.empty_cache()
        extra["block"] = block_leg(pdm, torch, dev, stream, args, threads)

    line = {"metric": METRIC, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic",
            "config": cfg, "roofline": roofline, "cpu_baseline": cpu}
    line.update(extra)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
