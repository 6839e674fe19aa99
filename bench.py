"""Benchmark of the lookup / interaction forward path on one MI355X.

Default workload: the single-hot pooled lookup (26 tables, rows log-uniform
in [1e3, 4e7], dim 128 bf16, one Zipf(1.05) id per bag, batch 65,536, sum,
fp32 out).  ``--workload`` selects another:

  ebc_fp32    8 tables x 100,000 x 64 fp32, sum, Poisson(10) bags, B=2048
  single_hot  (default, above)
  int8_mean   64 tables x 5,000,000 x 128 int8 rowwise, mean, Poisson(20) bags, B=16,384, fp16 out
  seq_gather  3 behaviour pools, item 10M x 256 + artist 1M x 64 + album 2M x 64 bf16, B=1024
  seq_tokenize  the seq_gather workload fused with one SequentialTokenizer per pool (Linear 384 -> 256,
              GELU, Linear 256 -> 256, + pos_emb of 2048 x 256 fp32), fp32 S-tokens [1024, 768, 256]
  ns_tokenize NS tokens: uid/item/artist/album rows (1M/9.4M/1.3M/3.4M x 64 bf16) + dense parts 64/6/6/64 -> 396
              wide NS input -> AutoSplitTokenizer Linear(396, 4096) + GELU + Linear(4096, 4096), B=1024
  onetrans    4-layer OneTrans block stack, B=1024, 384 S + 16 NS tokens, d 256, schedule 384/256/128/64
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
duration on the launch stream) and a CPU baseline (the oracle on the host
cores, bounded sample).
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


def cpu_pooled(orc, w, threads: int, row_cap: int, weight_std: float):
    """The oracle over the same bags on tables capped at ``row_cap`` rows (ids of a
    capped table are redrawn over the capped rows with the same distribution)."""
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
    alpha = {"bf16": 1.05, "int8": 1.2}.get(w.dtype, None)
    for t, r in enumerate(w.rows):
        if r > row_cap:
            seg = slice(w.offsets[t * w.batch], w.offsets[(t + 1) * w.batch])
            n = int(w.offsets[(t + 1) * w.batch] - w.offsets[t * w.batch])
            idx[seg] = syn.zipf_rows(syn.rng(99, t), n, row_cap, alpha) if alpha else \
                syn.rng(99, t).integers(0, row_cap, n)
    od = "fp32" if w.out_dtype == "fp32" else "fp16"
    sec = time_cpu(lambda: orc.tbe_pooled(flat, slots, idx, w.offsets, w.batch, -1, od, threads=threads))
    return w.num_lookups / sec, sec


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


def cpu_train(orc, w, optimizer: str, batch: int, row_cap: int):
    """The oracle's backward + update over the first ``batch`` bags of every table, on tables capped at
    ``row_cap`` rows (ids taken modulo)."""
    D, T = w.dim, len(w.rows)
    rows = [min(r, row_cap) for r in w.rows]
    g = np.random.default_rng(8)
    slots, off = [], 0
    for t, r in enumerate(rows):
        slots.append(dict(rows=r, weights_offset=off * 4, dim=D, dtype="fp32", pooling="sum", row_bytes=0,
                          out_offset=t * D))
        off += r * D
    lens = np.diff(w.offsets).reshape(T, w.batch)[:, :batch]
    idx = np.concatenate([w.indices[w.offsets[t * w.batch]:w.offsets[t * w.batch] + int(lens[t].sum())] % rows[t]
                          for t in range(T)])
    offsets = orc.offsets_np(lens.reshape(-1))
    grad = g.standard_normal((batch, T * D), dtype=np.float32)
    flat = (g.random(off, dtype=np.float32) - np.float32(0.5)) * np.float32(0.02)
    adam = optimizer == "adam"
    m1 = np.zeros(off if adam else sum(rows), dtype=np.float32)
    m2 = np.zeros(off if adam else 1, dtype=np.float32)
    step = [0]

    def run():
        step[0] += 1
        orc.tbe_backward(slots, idx, offsets, batch, grad, optimizer=orc.ADAM if adam else orc.ROWWISE_ADAGRAD,
                         weights=flat, m1=m1, m2=m2, lr=0.01, eps=1e-8, weight_decay=1e-5, wd_mode=orc.WD_L2,
                         step=step[0])

    sec = time_cpu(run)
    return idx.size, sec


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


def cpu_train_seq(orc, w, batch: int, row_cap: int):
    """The oracle's gather backward + Adam over the first ``batch`` samples, tables capped at ``row_cap`` rows."""
    g = np.random.default_rng(9)
    rows = [min(r, row_cap) for r in w.table_rows]
    slots, off, col = [], 0, 0
    for r, d in zip(rows, w.table_dims):
        slots.append(dict(rows=r, weights_offset=off * 4, dim=d, dtype="fp32", pooling="sum", row_bytes=0,
                          out_offset=col))
        off += r * d
        col += d
    ids = [[a[:o[batch]] % r for a, r in zip(row, rows)] for row, o in zip(w.ids, w.offsets)]
    offsets = [o[:batch + 1] for o in w.offsets]
    S = sum(w.max_len)
    grad = g.standard_normal((batch, S, col), dtype=np.float32)
    flat = (g.random(off, dtype=np.float32) - np.float32(0.5)) * np.float32(0.02)
    m1, m2 = np.zeros(off, np.float32), np.zeros(off, np.float32)
    step = [0]

    def run():
        step[0] += 1
        orc.seq_gather_backward(slots, ids, offsets, w.max_len, grad, optimizer=orc.ADAM, weights=flat, m1=m1,
                                m2=m2, lr=0.01, eps=1e-8, weight_decay=1e-5, step=step[0])

    sec = time_cpu(run)
    return batch * S, sec


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


def cpu_seq(orc, w, row_cap: int):
    g = np.random.default_rng(6)
    tabs = [g.integers(0, 1 << 16, (min(r, row_cap), d), dtype=np.uint16) for r, d in zip(w.table_rows,
                                                                                          w.table_dims)]
    ids = [[a % min(r, row_cap) for a, r in zip(row, w.table_rows)] for row in w.ids]
    sec = time_cpu(lambda: orc.seq_gather(tabs, ids, w.offsets, w.max_len))
    return sec


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


def cpu_tokenize(w, threads: int, batch: int, row_cap: int):
    """The oracle (C gather + PyTorch-CPU tokenizer in autocast emulation) on the first ``batch`` samples."""
    import torch
    from oracle import onetrans as ot

    torch.set_num_threads(threads)
    g = np.random.default_rng(6)
    # random bf16 bits with bit 14 clear: finite values of magnitude below 2
    tabs = [g.integers(0, 1 << 16, (min(r, row_cap), dm), dtype=np.uint16) & 0xBFFF
            for r, dm in zip(w.table_rows, w.table_dims)]
    offs = [o[:batch + 1] for o in w.offsets]
    ids = [[a[:int(o[batch])] % min(r, row_cap) for a, r in zip(row, w.table_rows)] for row, o in zip(w.ids, offs)]
    K = sum(w.table_dims)
    ws = [ot.random_tokenizer_weights(K, TOK_D, max(w.max_len), seed=p) for p in range(len(w.max_len))]
    sec = time_cpu(lambda: ot.seq_tokenize(tabs, ids, offs, w.max_len, ws), reps=3)
    return sec


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


def cpu_ns(threads: int, batch: int):
    import torch
    from oracle import onetrans as ot

    torch.set_num_threads(threads)
    g = np.random.default_rng(7)
    K, N = NS_DIM * len(NS_TABLES) + sum(NS_DENSE), NS_D * NS_N
    tabs = [g.normal(0, 0.05, (100_000, NS_DIM)).astype(np.float32) for _ in NS_TABLES]
    ids = [g.integers(0, 100_000, batch) for _ in NS_TABLES]
    dense = [g.normal(0, 1, (batch, d)).astype(np.float32) for d in NS_DENSE]
    w = ot.random_autosplit_weights(K, N, std=0.02, seed=3)
    return time_cpu(lambda: ot.ns_tokenize(tabs, ids, dense, w, NS_N), reps=3)


# ----------------------------------------------------------------------------------------------
# OneTrans block stack
# ----------------------------------------------------------------------------------------------

def setup_onetrans(pdm, torch, dev, w):
    from oracle import onetrans as ot  # noqa: F401  (flop convention lives with the oracle)

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
    ws_size = pdm.ops.onetrans_workspace_layout(w.batch, kv0, kv0, D, F)["total"][0]
    ws = torch.empty(ws_size, dtype=torch.uint8, device=dev)
    outs = []
    kv = kv0
    for q_s in w.schedule:
        outs.append(torch.empty(w.batch, q_s + n_ns, D, device=dev))
    H = D // 64

    def step():
        cur = x
        for layer, q_s in enumerate(w.schedule):
            pdm.ops.onetrans_block_raw(cur, layers[layer], H, q_s + n_ns, out=outs[layer], workspace=ws)
            cur = outs[layer]

    flops = 0.0
    for q_s in w.schedule:
        flops += ot.block_flops(w.batch, kv, q_s + n_ns, D, F, n_ns)
        kv = q_s + n_ns
    return step, flops, (x, layers, ws, outs)


def cpu_onetrans(w, threads: int, batch: int):
    import torch
    from oracle import onetrans as ot

    torch.set_num_threads(threads)
    D, F = w.d_model, w.d_model * w.ffn_mult
    layers = [ot.random_weights(D, F, w.n_ns, seed=i) for i in range(len(w.schedule))]
    x = torch.randn(batch, w.l_s + w.n_ns, D) * 0.02
    sec = time_cpu(lambda: ot.stack_forward(x, layers, w.schedule, D // 64), reps=3)
    return sec


# ----------------------------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="single_hot",
                    choices=["single_hot", "ebc_fp32", "int8_mean", "seq_gather", "seq_tokenize", "ns_tokenize",
                             "onetrans",
                             "cross_hash",
                             "train_adam", "train_rowwise_adagrad", "train_seq_adam", "kjt_build", "copy_1gib"])
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
    cpu_fn = None

    if args.workload in ("single_hot", "ebc_fp32", "int8_mean"):
        if args.workload == "single_hot":
            w, std, cap = syn.single_hot_bf16(), 0.02, 500_000
        elif args.workload == "ebc_fp32":
            w, std, cap = syn.ebc_fp32(), 0.01, 100_000
        else:
            w, std, cap = syn.int8_mean(), 0.05, 200_000
        step, alg, keep = setup_pooled(pdm, torch, dev, w, std)
        units, unit, bound = w.num_lookups, "lookups/s", "hbm"
        dtype = {"bf16": "bf16->f32", "fp32": "f32", "int8": "u8->f32"}[w.dtype]
        cfg = {"workload": w.name, "tables": w.num_tables, "rows_total": int(sum(w.rows)), "dim": w.dim,
               "batch": w.batch, "lookups_per_batch": w.num_lookups, "pooling": w.pooling,
               "weights": w.dtype, "out": w.out_dtype}

        def cpu_fn():
            val, sec = cpu_pooled(orc, w, threads, cap, std)
            return {"value": round(val, 1), "unit": unit, "cores": threads, "kind": "port",
                    "sample": f"C oracle, full batch of {w.num_lookups} lookups on tables capped at {cap} rows "
                              f"(ids redrawn over the capped rows), median of 5 reps = {sec:.3f} s"}
    elif args.workload == "seq_gather":
        w = syn.seq_gather()
        step, alg, kept, keep = setup_seq(pdm, torch, dev, w)
        units, unit, bound, dtype = kept, "events/s", "hbm", "bf16"
        cfg = {"workload": w.name, "batch": w.batch, "pools": len(w.max_len), "max_len": w.max_len,
               "tables": {"rows": w.table_rows, "dims": w.table_dims}, "events_kept": kept,
               "out": [w.batch, sum(w.max_len), sum(w.table_dims)]}

        def cpu_fn():
            sec = cpu_seq(orc, w, 1_000_000)
            return {"value": round(kept / sec, 1), "unit": unit, "cores": 1, "kind": "port",
                    "sample": f"C oracle (one thread), full batch of {kept} kept events, item table capped at "
                              f"1,000,000 rows (ids taken modulo), median of 5 reps = {sec:.3f} s"}
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
        cpu_b, cpu_cap = 256, 250_000

        def cpu_fn():
            sec = cpu_tokenize(w, threads, cpu_b, cpu_cap)
            return {"value": round(cpu_b * S / sec, 1), "unit": unit, "cores": threads, "kind": "port",
                    "sample": f"oracle (C gather + PyTorch-CPU tokenizers, autocast emulation) on the first {cpu_b} "
                              f"samples ({cpu_b * S} slots), tables capped at {cpu_cap} rows (ids modulo), "
                              f"median of 3 reps = {sec:.3f} s"}
    elif args.workload == "ns_tokenize":
        B_ = 1024
        step, alg, K_, N_, keep = setup_ns(pdm, torch, dev, B_)
        units, unit, bound, dtype = B_, "samples/s", "mfma", "bf16"
        cfg = {"workload": "ns_tokens_b1024_k396_n4096", "batch": B_,
               "scalar_tables": {n: r for n, r in NS_TABLES}, "scalar_dim": NS_DIM, "dense_dims": NS_DENSE,
               "ns_input": K_, "d_model": NS_D, "n_ns": NS_N, "gflop_per_step": round(alg / 1e9, 2),
               "timed": "whole call (NS rows gather, W1 padding copy, Linear 1 + bias + GELU, Linear 2 + bias)"}
        cfg["unfused_same_gpu_ms"] = round(unfused_ns_ms(pdm, torch, keep), 4)
        cpu_b = 1024

        def cpu_fn():
            sec = cpu_ns(threads, cpu_b)
            return {"value": round(cpu_b / sec, 1), "unit": unit, "cores": threads, "kind": "port",
                    "sample": f"oracle (numpy row gather + PyTorch-CPU AutoSplitTokenizer, autocast emulation) at "
                              f"batch {cpu_b}, tables of 100,000 rows, median of 3 reps = {sec:.3f} s"}
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

        def cpu_fn():
            sec = time_cpu(lambda: orc.cross_hash([uid, artist], table_size, 0))
            return {"value": round(n_rows / sec, 1), "unit": unit, "cores": threads, "kind": "port",
                    "sample": f"C oracle (XXH64 per row, OpenMP), all {n_rows} rows, median of 5 reps = {sec:.3f} s"}
    elif args.workload in ("train_adam", "train_rowwise_adagrad"):
        optimizer = "adam" if args.workload == "train_adam" else "rowwise_adagrad"
        w = syn.ebc_fp32(scale_rows=100.0, batch=65_536)
        step, alg, distinct, keep = setup_train(pdm, torch, dev, w, optimizer)
        units, unit, bound, dtype = w.num_lookups, "lookups/s", "hbm", "f32"
        cfg = {"workload": f"{w.name}_{optimizer}", "tables": w.num_tables, "rows_total": int(sum(w.rows)),
               "dim": w.dim, "batch": w.batch, "lookups_per_batch": w.num_lookups, "distinct_rows": distinct,
               "pooling": "sum", "weights": "fp32", "optimizer": optimizer, "lr": 0.01, "eps": 1e-8,
               "weight_decay": 1e-5, "timed": "whole fused backward (linearise, 3 radix passes, accumulate)"}
        cpu_b, cpu_cap = 16_384, 250_000

        def cpu_fn():
            n, sec = cpu_train(orc, w, optimizer, cpu_b, cpu_cap)
            return {"value": round(n / sec, 1), "unit": unit, "cores": 1, "kind": "port",
                    "sample": f"C oracle (one thread): backward + {optimizer} over the first {cpu_b} bags of each "
                              f"table ({n} lookups) on tables capped at {cpu_cap} rows (ids modulo), "
                              f"median of 5 reps = {sec:.3f} s"}
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
        cpu_b, cpu_cap = 256, 250_000

        def cpu_fn():
            n, sec = cpu_train_seq(orc, w, cpu_b, cpu_cap)
            return {"value": round(n / sec, 1), "unit": unit, "cores": 1, "kind": "port",
                    "sample": f"C oracle (one thread, slot placement in numpy): gather backward + Adam over the "
                              f"first {cpu_b} samples ({n} slots x 3 features) on tables capped at {cpu_cap} rows "
                              f"(ids modulo), median of 5 reps = {sec:.3f} s"}
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
        keep = feats

        def step():
            pdm.ops.kjt_from_dense_raw(feats, 0)

        rows = F_ * B_
        alg = F_ * B_ * L_ * 8 + kept * 8 + rows * 4 + (rows + 1) * 8
        units, unit, bound, dtype = F_ * B_ * L_, "ids/s", "hbm", "int64"
        cfg = {"workload": "kjt_build_26x65536x20_pad30", "features": F_, "batch": B_, "ids_per_row": L_,
               "kept": kept, "padding_idx": 0}

        def cpu_fn():
            sec = time_cpu(lambda: orc.kjt_from_dense(mats, 0))
            return {"value": round(units / sec, 1), "unit": unit, "cores": 1, "kind": "port",
                    "sample": f"numpy oracle (boolean mask per feature, one thread), all {units} ids, median of 5 "
                              f"reps = {sec:.3f} s"}
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
        w = syn.onetrans_block()
        step, alg, keep = setup_onetrans(pdm, torch, dev, w)
        units, unit, bound, dtype = w.batch, "samples/s", "mfma", "bf16"
        cfg = {"workload": w.name, "batch": w.batch, "l_s": w.l_s, "n_ns": w.n_ns, "d_model": w.d_model,
               "n_heads": w.n_heads, "ffn": w.d_model * w.ffn_mult, "schedule": w.schedule,
               "gflop_per_step": round(alg / 1e9, 1)}
        cpu_batch = 8

        def cpu_fn():
            sec = cpu_onetrans(w, threads, cpu_batch)
            return {"value": round(cpu_batch / sec, 2), "unit": unit, "cores": threads, "kind": "port",
                    "sample": f"PyTorch-CPU oracle (autocast emulation, fp32) of the 4-layer stack at batch "
                              f"{cpu_batch}, median of 3 reps = {sec:.3f} s"}

    stream = torch.cuda.current_stream(dev)
    log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
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
    value = units * args.steps / elapsed
    if bound == "hbm":
        achieved = alg / (kernel_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(args.workload),
                    "algorithmic_bytes": int(alg), "kernel_ms": round(kernel_ms, 5)}
    else:
        achieved = alg / (kernel_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": traffic_from_profiles(args.workload),
                    "algorithmic_flops": alg, "kernel_ms": round(kernel_ms, 5)}
    log(f"{value:.4g} {unit}, step {kernel_ms:.4f} ms, {achieved:.1f} {roofline['unit']}")

    cpu = None
    if not args.no_cpu_baseline and cpu_fn is not None:
        log(f"cpu baseline on {threads} threads")
        cpu = cpu_fn()

    line = {"metric": METRIC, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic",
            "config": cfg, "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
