"""Seeded synthetic inputs for the five lookup / interaction workloads.

The reference's generator draws uniform ids (primus_dlrm/data/synthetic.py:195-243);
these workloads need Poisson bag lengths and Zipf-skewed ids, so ids come
from NumPy ``Generator(PCG64)`` streams seeded ``[1000 + workload, stream]``:

* Zipf(alpha) over ``[1, N]`` by inverting the continuous power law,
  ``r = floor(((N**(1-a) - 1) * u + 1) ** (1 / (1 - a)))``; rank ``r`` maps to
  row ``(r * 2654435761) mod N`` so hot rows are scattered over the table.
* Poisson lengths clipped to ``[lo, hi]``.
* Log-uniform row counts ``round(exp(U(ln lo, ln hi)))``.

Weights are drawn on the device with torch's seeded generator.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

ZIPF_SCATTER = 2654435761  # prime > any table size used here, so the rank -> row map is a bijection


def rng(workload: int, stream: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([1000 + workload, stream]))


def zipf_rows(g: np.random.Generator, n: int, rows: int, alpha: float) -> np.ndarray:
    if rows <= 0:
        raise ValueError("rows must be > 0")
    u = g.random(n)
    if abs(alpha - 1.0) < 1e-12:
        r = np.floor(np.exp(u * math.log(rows + 1.0)))
    else:
        e = 1.0 - alpha
        r = np.floor(((rows ** e - 1.0) * u + 1.0) ** (1.0 / e))
    r = np.clip(r, 1, rows).astype(np.int64)
    return (r * ZIPF_SCATTER) % rows


def poisson_lengths(g: np.random.Generator, n: int, mean: float, lo: int, hi: int) -> np.ndarray:
    return np.clip(g.poisson(mean, n), lo, hi).astype(np.int64)


def offsets_from_lengths(lengths: np.ndarray) -> np.ndarray:
    out = np.zeros(lengths.size + 1, dtype=np.int64)
    np.cumsum(lengths, out=out[1:])
    return out


@dataclass
class PooledWorkload:
    """A table-batched pooled lookup: T tables, B bags per table, table-major offsets."""
    name: str
    rows: List[int]
    dim: int
    dtype: str            # "fp32" | "bf16" | "int8"
    pooling: str          # "sum" | "mean"
    out_dtype: str        # "fp32" | "fp16"
    batch: int
    indices: np.ndarray   # int64 [N]
    offsets: np.ndarray   # int64 [T*B+1]
    weight_init: str      # "uniform0.01" | "normal0.02" | "normal0.05"
    notes: Dict[str, str] = field(default_factory=dict)

    @property
    def num_tables(self) -> int:
        return len(self.rows)

    @property
    def num_lookups(self) -> int:
        return int(self.offsets[-1])


def ebc_fp32(scale_rows: float = 1.0, batch: int = 2048) -> PooledWorkload:
    """8 tables x 100,000 x 64 fp32, U(-0.01, 0.01), sum, lengths Poisson(10) in [0, 50], uniform ids."""
    T, rows = 8, max(1, int(100_000 * scale_rows))
    idx, lens = [], []
    for t in range(T):
        g = rng(1, t)
        ln = poisson_lengths(g, batch, 10.0, 0, 50)
        lens.append(ln)
        idx.append(g.integers(0, rows, int(ln.sum()), dtype=np.int64))
    name = f"ebc_fp32_8x{rows // 1000}k_d64_b{batch}" if rows < 1_000_000 else \
        f"ebc_fp32_8x{rows // 1_000_000}m_d64_b{batch}"
    return PooledWorkload(name, [rows] * T, 64, "fp32", "sum", "fp32", batch,
                          np.concatenate(idx), offsets_from_lengths(np.concatenate(lens)), "uniform0.01")


def draw_rows(g: np.random.Generator, n: int, rows: int, alpha: float, ids: str) -> np.ndarray:
    """``n`` row ids of a table of ``rows`` rows: Zipf(alpha) (``ids="zipf"``) or uniform (``ids="uniform"``,
    the control distribution whose rows mostly miss every cache)."""
    if ids == "zipf":
        return zipf_rows(g, n, rows, alpha)
    if ids == "uniform":
        return g.integers(0, rows, n, dtype=np.int64)
    raise ValueError(f"ids must be 'zipf' or 'uniform', got {ids!r}")


def _ids_suffix(ids: str) -> str:
    return "" if ids == "zipf" else "_" + ids


def single_hot_bf16(batch: int = 65_536, max_rows: Optional[int] = None, ids: str = "zipf") -> PooledWorkload:
    """26 tables, rows log-uniform in [1e3, 4e7], dim 128 bf16, one id per bag, Zipf(1.05) (or uniform) ids,
    sum, fp32 out."""
    T = 26
    g0 = rng(2, 1000)
    rows = [int(round(math.exp(g0.uniform(math.log(1e3), math.log(4e7))))) for _ in range(T)]
    if max_rows is not None:
        rows = [min(r, max_rows) for r in rows]
    idx = [draw_rows(rng(2, t), batch, rows[t], 1.05, ids) for t in range(T)]
    offsets = np.arange(T * batch + 1, dtype=np.int64)
    return PooledWorkload("tbe_bf16_single_hot_26t_d128_b65536" + _ids_suffix(ids), rows, 128, "bf16", "sum",
                          "fp32", batch, np.concatenate(idx), offsets, "normal0.02")


def int8_mean(batch: int = 16_384, rows: int = 5_000_000, tables: int = 64, ids: str = "zipf") -> PooledWorkload:
    """64 tables x 5,000,000 x 128 int8 rowwise (from N(0, 0.05)), lengths Poisson(20) in [1, 100],
    Zipf(1.2) (or uniform) ids, mean, fp16 out."""
    idx, lens = [], []
    for t in range(tables):
        g = rng(3, t)
        ln = poisson_lengths(g, batch, 20.0, 1, 100)
        lens.append(ln)
        idx.append(draw_rows(g, int(ln.sum()), rows, 1.2, ids))
    return PooledWorkload("tbe_int8_mean_64t_5m_d128_b16384" + _ids_suffix(ids), [rows] * tables, 128, "int8",
                          "mean", "fp16", batch, np.concatenate(idx), offsets_from_lengths(np.concatenate(lens)),
                          "normal0.05")


@dataclass
class SeqWorkload:
    """Behaviour pools (listen+, like, skip) of jagged events; item / artist / album per event."""
    name: str
    batch: int
    max_len: List[int]
    table_rows: List[int]      # item, artist, album
    table_dims: List[int]
    ids: List[List[np.ndarray]]  # [pool][feature] int64
    offsets: List[np.ndarray]    # [pool] int64 [B+1]

    @property
    def num_events(self) -> int:
        return int(sum(o[-1] for o in self.offsets))


def item_to_artist(items: np.ndarray, n_artist: int) -> np.ndarray:
    return (items * 40503 + 7) % n_artist


def item_to_album(items: np.ndarray, n_album: int) -> np.ndarray:
    return (items * 69069 + 13) % n_album


def seq_gather(batch: int = 1024, item_rows: int = 10_000_000, artist_rows: int = 1_000_000,
               album_rows: int = 2_000_000, means=(150.0, 40.0, 80.0), max_len: int = 256,
               ids: str = "zipf") -> SeqWorkload:
    """3 pools with lengths Poisson(150/40/80) clipped to [0, 256]; items Zipf(1.1) (or uniform) over 10M x 256
    bf16, artist (1M x 64) and album (2M x 64) ids from fixed maps of the item id."""
    out_ids, offs = [], []
    for p, mean in enumerate(means):
        g = rng(4, p)
        ln = poisson_lengths(g, batch, mean, 0, max_len)
        items = draw_rows(g, int(ln.sum()), item_rows, 1.1, ids)
        out_ids.append([items, item_to_artist(items, artist_rows), item_to_album(items, album_rows)])
        offs.append(offsets_from_lengths(ln))
    return SeqWorkload("seq_gather_3pools_b1024" + _ids_suffix(ids), batch, [max_len] * len(means),
                       [item_rows, artist_rows, album_rows], [256, 64, 64], out_ids, offs)


@dataclass
class BlockWorkload:
    name: str
    batch: int
    l_s: int
    n_ns: int
    d_model: int
    n_heads: int
    ffn_mult: int
    schedule: List[int]


def onetrans_block(batch: int = 1024) -> BlockWorkload:
    """B=1024, 384 S-tokens + 16 NS-tokens, d 256, 4 heads x 64, FFN 4x, 4 layers,
    pyramid 384 -> 256 -> 128 -> 64, inputs and weights N(0, 0.02)."""
    return BlockWorkload("onetrans_4layer_b1024", batch, 384, 16, 256, 4, 4, [384, 256, 128, 64])


def onetrans_large(batch: int = 1024) -> BlockWorkload:
    """OneTransL (configs/bench_onetrans_large_synthetic.yaml:1-5,28-33): B=1024, 1500 S-tokens + 16 NS-tokens,
    d 384, 6 heads x 64, FFN 4x, 8 layers, the reference's pyramid schedule 1500 -> 16
    (pyramid_schedule(1500, 16, 8): 1500, 1288, 1076, 864, 652, 440, 228, 16), inputs and weights N(0, 0.02)."""
    return BlockWorkload("onetransl_8layer_b1024", batch, 1500, 16, 384, 6, 4,
                         [1500, 1288, 1076, 864, 652, 440, 228, 16])


def block_flops(w: BlockWorkload) -> float:
    """Forward FLOPs by the reference's convention (onetrans.py:392-474 without the x3 for backward):
    S-token QKV on every kv S-token, attention counted full (no causal discount)."""
    D, H = w.d_model, w.n_heads
    dh, F = D // H, D * w.ffn_mult
    kv = w.l_s + w.n_ns
    total = 0.0
    for q_s in w.schedule:
        q = q_s + w.n_ns
        n_s = kv - w.n_ns
        total += 2 * n_s * D * 3 * D + 2 * w.n_ns * 3 * D * D
        total += 4 * H * dh * q * kv
        total += 2 * q * D * D
        total += 2 * (q - w.n_ns) * D * F * 2 + 2 * w.n_ns * D * F * 2
        kv = q
    return total * w.batch


def block_flops_causal(w: BlockWorkload) -> float:
    """Forward FLOPs of the work the causal pyramid needs: K and V of every kv token, Q only of the kept
    queries, attention over the keys each query sees (query i of a layer keeping q of kv tokens sees
    kv - q + i + 1 keys), the out-projection and FFN of the kept queries."""
    D, F = w.d_model, w.d_model * w.ffn_mult
    kv = w.l_s + w.n_ns
    total = 0.0
    for q_s in w.schedule:
        q = q_s + w.n_ns
        total += 2 * kv * D * 2 * D + 2 * q * D * D           # K, V of all tokens; Q of the kept ones
        visible = q * (kv - q) + q * (q + 1) // 2              # keys summed over the kept queries
        total += 4 * D * visible                              # S = Q K^T and O = P V
        total += 2 * q * D * D + 4 * q * D * F                # out-projection, FFN up and down
        kv = q
    return total * w.batch
