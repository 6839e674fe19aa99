"""NumPy front end of the C oracle (pdm_oracle.c).  TEST INFRASTRUCTURE ONLY.

Only the parity tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py`` use this module, as the checker.  It restates the
reference's lookup semantics on the CPU:

* ``tbe_pooled``      pooled sum / mean per (table, bag) — primus_dlrm/models/
                      sharded_embedding.py:220-227, padding filter embedding.py:188-194,
                      table-major offsets tests/test_fbgemm_tbe.py:33-35.
* ``int8_quantize``   int8 rowwise rows ([fp16 scale][fp16 bias][q]); the reference has
                      no quantized path, so this restates FBGEMM's fused rowwise SB-half
                      quantizer (fbgemm_gpu 1.5.0, absent here).
* ``seq_gather``      jagged -> padded pools: data/dataset.py:604-626 (last L events,
                      left pad with id 0), onetrans.py:515-520 (feature concat),
                      onetrans.py:553-558 (pool concat).
* ``cross_hash``      cross-feature ids: data/hashing.py:23-52 (XXH64 of the "<{n}q"
                      packed keys, seed = salt, % table_size); ``xxh64`` is the digest.
* ``tbe_backward``    pooled-lookup backward + the fused embedding optimizer TorchRec maps the
                      reference's choice to (distributed/wrapper.py:151-174): row gradients
                      summed in lookup order, then FBGEMM's ADAM or EXACT_ROWWISE_ADAGRAD
                      update per distinct row (fbgemm_gpu 2026.4.29, absent here; rules
                      restated at oracle_tbe_backward in pdm_oracle.c).  ``row_space``
                      numbers the distinct tables the way the library documents it.
* ``kjt_from_dense`` / ``kjt_permute``  KJT construction: _build_pooled_kjt (embedding.py:177-204, padding
                      filter per row, lengths, key-major concat) and key permutation (pipeline_batch.py:70-100).
* ``seq_gather_backward`` the S-token gather's backward: ``seq_token_ids`` restates the forward's slot
                      placement (dataset.py:604-626, onetrans.py:515-520,553-558) and every slot becomes
                      a one-id bag of ``tbe_backward``.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# PDM_ORACLE_LIB selects another build of the same source (the sanitizer build of ``make -C oracle sanitize``)
_LIB_PATH = os.environ.get("PDM_ORACLE_LIB") or os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

F32, F16, BF16, I8 = 0, 1, 2, 3
_DT = {"fp32": F32, "fp16": F16, "bf16": BF16, "int8": I8}
_POOL = {"sum": 0, "mean": 1}


class _Table(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_int64), ("weights_offset", ctypes.c_int64), ("dim", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("pooling", ctypes.c_int32), ("row_bytes", ctypes.c_int32),
                ("out_offset", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class _Optim(ctypes.Structure):
    _fields_ = [("optimizer", ctypes.c_int32), ("wd_mode", ctypes.c_int32), ("lr", ctypes.c_float),
                ("eps", ctypes.c_float), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
                ("weight_decay", ctypes.c_float), ("reserved", ctypes.c_int32), ("step", ctypes.c_int64)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} missing: run `make -C oracle`")
        h = ctypes.CDLL(_LIB_PATH)
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        h.oracle_f16_to_f32.restype = ctypes.c_float
        h.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        h.oracle_f32_to_f16.restype = ctypes.c_uint16
        h.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        h.oracle_f32_to_bf16.restype = ctypes.c_uint16
        h.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        h.oracle_tbe_pooled.restype = i64
        h.oracle_tbe_pooled.argtypes = [ctypes.POINTER(_Table), i32, i64, vp, vp, i32, i64, vp, i64, vp, i32,
                                        i64, i32]
        h.oracle_int8_quantize.restype = None
        h.oracle_int8_quantize.argtypes = [vp, i64, i32, vp, i32, i32]
        h.oracle_seq_gather.restype = i64
        h.oracle_seq_gather.argtypes = [i32, i32, i32, i64, vp, vp, vp, vp, vp, vp, vp, i32, i32, vp, vp]
        h.oracle_xxh64.restype = ctypes.c_uint64
        h.oracle_xxh64.argtypes = [vp, ctypes.c_size_t, ctypes.c_uint64]
        h.oracle_tbe_backward.restype = i64
        h.oracle_tbe_backward.argtypes = [ctypes.POINTER(_Table), vp, i32, i64, vp, i32, i64, vp, i64, vp, i64,
                                          vp, vp, i32, ctypes.POINTER(_Optim), vp, vp, vp, vp, vp]
        h.oracle_cross_hash.restype = None
        h.oracle_cross_hash.argtypes = [vp, vp, i32, i64, ctypes.c_uint64, ctypes.c_uint64, vp]
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- conversions -------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([lib().oracle_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([lib().oracle_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    return np.array([lib().oracle_f16_to_f32(int(v)) for v in h], dtype=np.float32)


def offsets_np(lengths) -> np.ndarray:
    lengths = np.asarray(lengths, dtype=np.int64).ravel()
    out = np.zeros(lengths.size + 1, dtype=np.int64)
    np.cumsum(lengths, out=out[1:])
    return out


# ---- pooled lookup -----------------------------------------------------------

def default_row_bytes(dtype: str, dim: int) -> int:
    return {"fp32": 4 * dim, "fp16": 2 * dim, "bf16": 2 * dim}.get(dtype, (4 + dim + 3) & ~3)


def tbe_pooled(flat: np.ndarray, slots: Sequence[dict], indices: np.ndarray, offsets: np.ndarray, batch: int,
               padding_idx: int = -1, out_dtype: str = "fp32", out_stride: Optional[int] = None,
               threads: int = 1, return_bad: bool = False):
    """flat: uint8 bytes of every table; slots: dicts rows, weights_offset, dim, dtype ("fp32" | "fp16" |
    "bf16" | "int8"), pooling ("sum" | "mean"), row_bytes (0 = default), out_offset.
    Returns [B, out_stride] float32 (out_dtype fp32) or uint16 bit patterns (fp16 / bf16)."""
    T = len(slots)
    arr = (_Table * T)()
    total = 0
    for i, s in enumerate(slots):
        arr[i] = _Table(int(s["rows"]), int(s["weights_offset"]), int(s["dim"]), _DT[s["dtype"]],
                        _POOL[s["pooling"]], int(s.get("row_bytes", 0)), int(s["out_offset"]), 0)
        total = max(total, int(s["out_offset"]) + int(s["dim"]))
    out_stride = total if out_stride is None else out_stride
    flat = np.ascontiguousarray(flat, dtype=np.uint8)
    indices = np.ascontiguousarray(indices)
    if indices.dtype not in (np.int32, np.int64):
        indices = indices.astype(np.int64)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    assert offsets.size == T * batch + 1
    out = np.zeros((batch, out_stride), dtype=np.float32 if out_dtype == "fp32" else np.uint16)
    bad = lib().oracle_tbe_pooled(arr, T, batch, _p(flat), _p(indices) if indices.size else None,
                                  32 if indices.dtype == np.int32 else 64, indices.size, _p(offsets),
                                  padding_idx, _p(out), _DT[out_dtype], out_stride, threads)
    return (out, int(bad)) if return_bad else out


def table_bytes(w) -> np.ndarray:
    """Raw bytes of a table given as a torch tensor (any dtype) or numpy array."""
    try:
        import torch
        if isinstance(w, torch.Tensor):
            w = w.detach().cpu().contiguous()
            if w.dtype in (torch.bfloat16, torch.float16):
                return w.view(torch.int16).numpy().view(np.uint8).reshape(-1)
            return w.numpy().view(np.uint8).reshape(-1)
    except ImportError:
        pass
    return np.ascontiguousarray(w).view(np.uint8).reshape(-1)


def _dtype_name(w) -> str:
    try:
        import torch
        if isinstance(w, torch.Tensor):
            return {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16",
                    torch.uint8: "int8"}[w.dtype]
    except ImportError:
        pass
    return {np.dtype(np.float32): "fp32", np.dtype(np.float16): "fp16", np.dtype(np.uint8): "int8"}[w.dtype]


def tbe_pooled_from_tables(tables: Sequence, poolings: Sequence[str], indices, offsets, batch: int,
                           out_dtype: str = "fp32", padding_idx: int = -1, dims: Optional[Sequence[int]] = None,
                           threads: int = 1):
    """Convenience form: one 2-D table per slot (int8 tables as uint8 [rows, row_bytes] with ``dims``)."""
    chunks, slots, off, col = [], [], 0, 0
    for i, w in enumerate(tables):
        b = table_bytes(w)
        dt = _dtype_name(w)
        rows = int(w.shape[0])
        dim = int(dims[i]) if dims is not None else int(w.shape[1])
        rb = int(w.shape[1]) if dt == "int8" else 0
        pad = (-off) % 16
        if pad:
            chunks.append(np.zeros(pad, dtype=np.uint8))
            off += pad
        slots.append(dict(rows=rows, weights_offset=off, dim=dim, dtype=dt, pooling=poolings[i], row_bytes=rb,
                          out_offset=col))
        chunks.append(b)
        off += b.size
        col += dim
    flat = np.concatenate(chunks) if chunks else np.zeros(1, np.uint8)
    return tbe_pooled(flat, slots, np.asarray(indices), np.asarray(offsets), batch, padding_idx, out_dtype,
                      threads=threads)


# ---- int8 rowwise ------------------------------------------------------------

def int8_quantize(src: np.ndarray, row_bytes: int = 0, threads: int = 1) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32)
    rows, dim = src.shape
    rb = row_bytes or (4 + dim + 3) & ~3
    out = np.zeros((rows, rb), dtype=np.uint8)
    lib().oracle_int8_quantize(_p(src), rows, dim, _p(out), rb, threads)
    return out


def int8_decode(q: np.ndarray, dim: int) -> np.ndarray:
    """Row decode x = float(q) * scale (fp32 rounding) + bias (fp32 rounding)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    sb = q[:, :4].copy().view(np.float16).astype(np.float32)  # [rows, 2]
    scale, bias = sb[:, 0:1], sb[:, 1:2]
    prod = (q[:, 4:4 + dim].astype(np.float32) * scale).astype(np.float32)
    return (prod + bias).astype(np.float32)


# ---- sequence gather ---------------------------------------------------------

def seq_gather(tables: Sequence[np.ndarray], ids: Sequence[Sequence[np.ndarray]], offsets: Sequence[np.ndarray],
               max_len: Sequence[int], pad_mode: int = 0, align: int = 0, return_bad: bool = False):
    """tables[f]: [rows, dim] uint16 (bf16 / fp16 bits) or float32; ids[p][f] int64; offsets[p] int64 [B+1].
    Returns (out [B, S, sum dim] in the table dtype, mask uint8 [B, S])."""
    P, F = len(offsets), len(tables)
    tables = [np.ascontiguousarray(t) for t in tables]
    esize = tables[0].dtype.itemsize
    B = offsets[0].size - 1
    S = int(sum(max_len))
    Dt = int(sum(t.shape[1] for t in tables))
    out = np.zeros((B, S, Dt), dtype=tables[0].dtype)
    mask = np.zeros((B, S), dtype=np.uint8)
    ml = np.asarray(max_len, dtype=np.int32)
    dims = np.asarray([t.shape[1] for t in tables], dtype=np.int32)
    rows = np.asarray([t.shape[0] for t in tables], dtype=np.int64)
    ids_c = [np.ascontiguousarray(ids[p][f], dtype=np.int64) for p in range(P) for f in range(F)]
    offs_c = [np.ascontiguousarray(o, dtype=np.int64) for o in offsets]
    num_ids = np.asarray([ids_c[p * F].size for p in range(P)], dtype=np.int64)
    tab_ptrs = (ctypes.c_void_p * F)(*[_p(t) for t in tables])
    id_ptrs = (ctypes.c_void_p * (P * F))(*[_p(a) for a in ids_c])
    off_ptrs = (ctypes.c_void_p * P)(*[_p(o) for o in offs_c])
    bad = lib().oracle_seq_gather(P, F, esize, B, _p(ml), _p(dims), _p(rows), tab_ptrs, id_ptrs, off_ptrs,
                                  _p(num_ids), pad_mode, align, _p(out), _p(mask))
    return (out, mask, int(bad)) if return_bad else (out, mask)


def xxh64(data: bytes, seed: int = 0) -> int:
    """XXH64 digest of ``data`` (the C restatement, any length)."""
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    return int(lib().oracle_xxh64(_p(buf), len(data), seed & (2**64 - 1)))


def cross_hash(keys: Sequence[np.ndarray], table_size: int, salt: int = 0) -> np.ndarray:
    """Cross-feature ids: per row, XXH64(seed=salt) of the little-endian int64 keys, % table_size.

    ``keys`` are int64 arrays of one length or of length 1 (broadcast), as in
    primus_dlrm/data/hashing.py:23-52 (n-way) and :72-112 (batch)."""
    ks = [np.ascontiguousarray(np.asarray(k, dtype=np.int64).ravel()) for k in keys]
    n = max(k.shape[0] for k in ks)
    strides = np.array([0 if (k.shape[0] == 1 and n != 1) else 1 for k in ks], dtype=np.int64)
    for k, st in zip(ks, strides):
        assert st == 0 or k.shape[0] == n, "key arrays must have one length (or length 1)"
    out = np.empty(n, dtype=np.int64)
    ptrs = (ctypes.c_void_p * len(ks))(*[_p(k) for k in ks])
    lib().oracle_cross_hash(ctypes.addressof(ptrs), _p(strides), len(ks), n, table_size, salt & (2**64 - 1),
                            _p(out))
    return out


# ---- pooled backward + fused optimizer ----------------------------------------

ADAM, ROWWISE_ADAGRAD, GRAD_ONLY = 0, 1, 2
WD_NONE, WD_L2 = 0, 1


def row_space(slots: Sequence[dict]):
    """Row id of row 0 of each slot's table and the total row count: distinct tables (equal
    weights_offset, rows, dim, dtype, row_bytes) numbered group by group ((dtype, dim) groups in
    first-appearance order), in slot order inside a group."""
    def ident(s):
        return (int(s["weights_offset"]), int(s["rows"]), int(s["dim"]), s["dtype"],
                int(s.get("row_bytes", 0)) or default_row_bytes(s["dtype"], int(s["dim"])))
    groups: List[tuple] = []
    for s in slots:
        g = (s["dtype"], int(s["dim"]))
        if g not in groups:
            groups.append(g)
    row_off = [0] * len(slots)
    seen = {}
    total = 0
    for g in groups:
        for i, s in enumerate(slots):
            if (s["dtype"], int(s["dim"])) != g:
                continue
            k = ident(s)
            if k in seen:
                row_off[i] = seen[k]
            else:
                seen[k] = row_off[i] = total
                total += int(s["rows"])
    return row_off, total


def tbe_backward(slots: Sequence[dict], indices: np.ndarray, offsets: np.ndarray, batch: int, grad: np.ndarray,
                 padding_idx: int = -1, optimizer: int = GRAD_ONLY, weights: Optional[np.ndarray] = None,
                 m1: Optional[np.ndarray] = None, m2: Optional[np.ndarray] = None, lr: float = 0.01,
                 eps: float = 1e-8, beta1: float = 0.9, beta2: float = 0.999, weight_decay: float = 0.0,
                 wd_mode: int = WD_NONE, step: int = 1, row_off: Optional[Sequence[int]] = None):
    """slots as for ``tbe_pooled`` (fp32 tables); grad: float32 [B, grad_stride].
    weights / m1 / m2: float32 arrays updated in place (weights and Adam state indexed by
    weights_offset / 4 + row * dim; row-wise state by row id).
    Returns (row_ids, row_grads [U, max dim] (a row of a narrower table is zero past its dim), bad)."""
    T = len(slots)
    arr = (_Table * T)()
    for i, s in enumerate(slots):
        arr[i] = _Table(int(s["rows"]), int(s["weights_offset"]), int(s["dim"]), _DT[s["dtype"]],
                        _POOL[s["pooling"]], int(s.get("row_bytes", 0)), int(s["out_offset"]), 0)
    if row_off is None:
        row_off, _ = row_space(slots)
    ro = np.ascontiguousarray(row_off, dtype=np.int64)
    indices = np.ascontiguousarray(indices)
    if indices.dtype not in (np.int32, np.int64):
        indices = indices.astype(np.int64)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    assert offsets.size == T * batch + 1
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    n = max(indices.size, 1)
    D = max(int(s["dim"]) for s in slots)
    ids = np.zeros(n, dtype=np.int64)
    rows = np.zeros((n, D), dtype=np.float32)
    entries = np.zeros(n * 40, dtype=np.uint8)
    bad = ctypes.c_int64(0)
    opt = _Optim(optimizer, wd_mode, lr, eps, beta1, beta2, weight_decay, 0, step)
    for a in (weights, m1, m2):
        assert a is None or (a.dtype == np.float32 and a.flags.c_contiguous)
    u = lib().oracle_tbe_backward(arr, _p(ro), T, batch, _p(indices) if indices.size else None,
                                  32 if indices.dtype == np.int32 else 64, indices.size, _p(offsets), padding_idx,
                                  _p(grad) if grad.size else None, grad.shape[1] if grad.ndim == 2 else 0,
                                  _p(ids), _p(rows), D, ctypes.byref(opt),
                                  _p(weights) if weights is not None else None, _p(m1) if m1 is not None else None,
                                  _p(m2) if m2 is not None else None, _p(entries), ctypes.byref(bad))
    return ids[:u], rows[:u], int(bad.value)


SEQ_PAD = 1 << 62  # slot marker the sequence backward skips (padding in ZERO mode)


def seq_token_ids(ids: Sequence[Sequence[np.ndarray]], offsets: Sequence[np.ndarray], max_len: Sequence[int],
                  pad_mode: str = "row0", align: str = "right") -> np.ndarray:
    """Id of every S-token slot, [F, B, S]: pool p keeps the last min(len, L_p) events of each sample, right
    aligned with left padding (data/dataset.py:604-626) or left aligned; a padding slot holds id 0 (row0, the
    reference's pad id) or SEQ_PAD (zero: the slot looks nothing up)."""
    P, F = len(offsets), len(ids[0])
    B = offsets[0].size - 1
    S = int(sum(max_len))
    out = np.full((F, B, S), 0 if pad_mode == "row0" else SEQ_PAD, dtype=np.int64)
    s0 = 0
    for p in range(P):
        L = int(max_len[p])
        for b in range(B):
            beg, end = int(offsets[p][b]), int(offsets[p][b + 1])
            if beg < 0 or end < beg or end > len(ids[p][0]):
                beg = end = 0  # malformed offsets: the forward treats the sample as empty
            n = min(end - beg, L)
            first = L - n if align == "right" else 0
            for f in range(F):
                out[f, b, s0 + first:s0 + first + n] = ids[p][f][end - n:end]
        s0 += L
    return out


def seq_gather_backward(slots: Sequence[dict], ids, offsets, max_len, grad: np.ndarray, pad_mode: str = "row0",
                        align: str = "right", **kw):
    """Backward of the S-token gather + fused optimizer: every (feature, slot) is a one-id bag of slot f whose
    gradient is token row (b, s), columns of feature f; ``slots`` are the features' fp32 tables (sum pooling,
    out_offset = column).  Returns what ``tbe_backward`` returns."""
    tok = seq_token_ids(ids, offsets, max_len, pad_mode, align)
    F, B, S = tok.shape
    g2 = np.ascontiguousarray(grad, dtype=np.float32).reshape(B * S, -1)
    return tbe_backward(slots, tok.reshape(-1), np.arange(F * B * S + 1, dtype=np.int64), B * S, g2,
                        padding_idx=SEQ_PAD, **kw)


# ---- KeyedJaggedTensor construction ----------------------------------------------------------

def kjt_from_dense(mats: Sequence[np.ndarray], padding_idx: int = -1):
    """Per feature, per row of the dense [B, L] ids, the ids != padding_idx in row order, features concatenated;
    returns (values, lengths int32 [F*B], offsets int64 [F*B+1])."""
    vals, lens = [], []
    for m in mats:
        m = np.asarray(m)
        keep = np.ones(m.shape, bool) if padding_idx < 0 else m != padding_idx
        vals.append(m[keep])
        lens.append(keep.sum(axis=1).astype(np.int32))
    lengths = np.concatenate(lens) if lens else np.zeros(0, np.int32)
    values = np.concatenate(vals) if vals else np.zeros(0, np.int64)
    return values, lengths, offsets_np(lengths)


def kjt_permute(values: np.ndarray, offsets: np.ndarray, num_keys: int, batch: int, perm: Sequence[int]):
    """Output key k = input key perm[k]: its B bags copied in order."""
    segs, lens = [], []
    for k in perm:
        for b in range(batch):
            lo, hi = int(offsets[k * batch + b]), int(offsets[k * batch + b + 1])
            segs.append(values[lo:hi])
            lens.append(hi - lo)
    lengths = np.asarray(lens, np.int32)
    return (np.concatenate(segs) if segs else values[:0]), lengths, offsets_np(lengths)
