"""Tables whose rows lie beyond 4 GiB of their base pointer: the 64-bit row addressing that the
full-size workloads rely on (26 bf16 tables of 34 GB, 64 int8 tables of 42 GB, a 5.1 GB item table).

Each device table is several GiB, and only the rows that the lookups touch are written; the oracle
runs on a compact copy of exactly those rows (ids remapped to their rank), so the comparison stays
bit-exact (the fused tokenizer leg: the tokenizer tests' per-element bf16 bound) without a host copy of the
whole table.  Ids concentrate on the last rows, whose byte
offsets exceed 2^32 both within a table and as a table's start in the flat buffer."""
import numpy as np
import pytest
import torch

from oracle import oracle as o

pytestmark = pytest.mark.gpu

GIB = 1 << 30


def _ids(g, rows, n):
    """n ids: 60 % among the last 4096 rows, the rest uniform (row 0 included once)."""
    tail = g.integers(max(rows - 4096, 0), rows, int(n * 0.6))
    rest = g.integers(0, rows, n - tail.size)
    ids = np.concatenate([tail, rest])
    g.shuffle(ids)
    ids[0] = 0
    return ids.astype(np.int64)


def _row_payload(g, dtype, n, dim):
    if dtype == "int8":
        return o.int8_quantize(g.normal(0, 0.05, (n, dim)).astype(np.float32))
    tdt = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype]
    t = torch.from_numpy(g.normal(0, 0.5, (n, dim)).astype(np.float32)).to(tdt)
    return o.table_bytes(t).reshape(n, -1)


def _scatter_rows(flat, base, row_bytes, rows, ids_u, payload, dev):
    view = flat[base:base + rows * row_bytes].view(rows, row_bytes)
    view.index_copy_(0, torch.from_numpy(ids_u).to(dev), torch.from_numpy(payload).to(dev))


def _codes(pdm):
    L = pdm._lib
    return ({"fp32": L.PDM_F32, "bf16": L.PDM_BF16, "int8": L.PDM_I8_SB_F16},
            {"sum": L.PDM_POOL_SUM, "mean": L.PDM_POOL_MEAN})


@pytest.fixture(scope="module")
def big_tables(pdm, dev):
    """A 5.2 GiB flat buffer: a 20 M x 128 bf16 table at offset 0 (5.12 GB), then an int8 and an fp32 table
    that start past 2^32 bytes."""
    g = np.random.default_rng(4242)
    specs = [("bf16", 20_000_000, 128, "sum"), ("int8", 300_000, 128, "mean"), ("fp32", 200_000, 64, "sum")]
    slots, off = [], 0
    for dt, rows, dim, pool in specs:
        rb = o.default_row_bytes(dt, dim)
        off = (off + 255) // 256 * 256
        slots.append(dict(rows=rows, weights_offset=off, dim=dim, dtype=dt, pooling=pool, row_bytes=rb))
        off += rows * rb
    assert slots[0]["rows"] * slots[0]["row_bytes"] > 4 * GIB and slots[1]["weights_offset"] > 4 * GIB
    print(f"flat table buffer {off / GIB:.2f} GiB", flush=True)
    flat = torch.empty(off, dtype=torch.uint8, device=dev)
    col = 0
    for s in slots:
        s["out_offset"] = col
        col += s["dim"]
    uniq, compact_slots, chunks, coff = [], [], [], 0
    for s in slots:
        pad = (-coff) % 256
        if pad:
            chunks.append(np.zeros(pad, np.uint8))
            coff += pad
        ids_u = np.unique(np.concatenate([_ids(g, s["rows"], 3000), [0, s["rows"] - 1]]))
        payload = _row_payload(g, s["dtype"], ids_u.size, s["dim"])
        _scatter_rows(flat, s["weights_offset"], s["row_bytes"], s["rows"], ids_u, payload, dev)
        uniq.append(ids_u)
        compact_slots.append(dict(s, rows=ids_u.size, weights_offset=coff))
        chunks.append(payload.reshape(-1))
        coff += payload.size
    torch.cuda.synchronize()
    yield dict(flat=flat, slots=slots, compact_slots=compact_slots, host=np.concatenate(chunks), uniq=uniq, g=g)
    del flat
    torch.cuda.empty_cache()


def _lookup(pdm, dev, bt, lens, pick, out_dtype="fp32"):
    B = lens.size // len(bt["slots"])
    dts, pools = _codes(pdm)
    idx_real, idx_compact = [], []
    for t, u in enumerate(bt["uniq"]):
        n = int(lens[t * B:(t + 1) * B].sum())
        r = pick(u.size, n)
        idx_real.append(u[r])
        idx_compact.append(r.astype(np.int64))
    idx_real, idx_compact = np.concatenate(idx_real), np.concatenate(idx_compact)
    offs = o.offsets_np(lens)
    plan = pdm.ops.TbePlan([dict(s, dtype=dts[s["dtype"]], pooling=pools[s["pooling"]]) for s in bt["slots"]], dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    tdt = {"fp32": torch.float32, "fp16": torch.float16}[out_dtype]
    got = pdm.ops.tbe_pooled_raw(plan, bt["flat"], torch.from_numpy(idx_real).to(dev), torch.from_numpy(offs).to(dev),
                                 B, tdt, err_flag=err)
    torch.cuda.synchronize()
    plan.release()
    want = o.tbe_pooled(bt["host"], bt["compact_slots"], idx_compact, offs, B, -1, out_dtype)
    got = got.cpu()
    got = got.numpy().view(np.uint32) if out_dtype == "fp32" else got.view(torch.int16).numpy().view(np.uint16)
    want = want.view(np.uint32) if out_dtype == "fp32" else want
    return got, want, int(err.item())


def test_pooled_multi_hot_beyond_4gib(pdm, dev, big_tables):
    g = big_tables["g"]
    B = 513
    lens = np.clip(g.poisson(6, 3 * B), 0, 40)
    got, want, err = _lookup(pdm, dev, big_tables, lens, lambda n, k: g.integers(0, n, k))
    assert err == 0
    mism = got != want
    assert not mism.any(), f"{mism.sum()} mismatches, first at {np.argwhere(mism)[:3].tolist()}"


def test_pooled_single_hot_beyond_4gib(pdm, dev, big_tables):
    """Bags of at most one id take the single-hot kernel."""
    g = big_tables["g"]
    B = 4099
    lens = (g.random(3 * B) < 0.95).astype(np.int64)
    for out_dtype in ("fp32", "fp16"):
        got, want, err = _lookup(pdm, dev, big_tables, lens, lambda n, k: g.integers(0, n, k), out_dtype)
        assert err == 0
        assert np.array_equal(got, want), out_dtype


def test_seq_gather_and_tokenizer_item_table_beyond_4gib(pdm, dev):
    """The S-token gather (and the fused gather + tokenizer) on a 10 M x 256 bf16 item table (5.12 GB):
    the last rows start past byte 2^32."""
    from oracle import onetrans as ot
    g = np.random.default_rng(77)
    item_rows, dims = 10_000_000, (256, 64, 64)
    small_rows = (1000, 2000)
    item = torch.empty((item_rows, 256), dtype=torch.bfloat16, device=dev)
    assert item_rows * 512 > 4 * GIB
    B, L = 37, [24, 8, 16]
    ids_p, offs = [], []
    for m in (30, 6, 12):
        ln = np.clip(g.poisson(m, B), 0, 48)
        it = _ids(g, item_rows, int(ln.sum()) + 1)[1:]
        ids_p.append(it)
        offs.append(o.offsets_np(ln))
    uniq = np.unique(np.concatenate(ids_p + [np.array([0], np.int64)]))
    payload = torch.from_numpy(g.normal(0, 0.5, (uniq.size, 256)).astype(np.float32)).to(torch.bfloat16)
    item.index_copy_(0, torch.from_numpy(uniq).to(dev), payload.to(dev))
    small = [torch.from_numpy(g.normal(0, 0.5, (r, d)).astype(np.float32)).to(torch.bfloat16)
             for r, d in zip(small_rows, dims[1:])]
    real = [[it, it % small_rows[0], (it * 7) % small_rows[1]] for it in ids_p]
    compact = [[np.searchsorted(uniq, it).astype(np.int64), r[1], r[2]] for it, r in zip(ids_p, real)]
    tabs_d = [item] + [t.to(dev) for t in small]
    ids_d = [[torch.from_numpy(a).to(dev) for a in row] for row in real]
    offs_d = [torch.from_numpy(a).to(dev) for a in offs]
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out, mask = pdm.ops.seq_gather_raw(tabs_d, ids_d, offs_d, L, err_flag=err)
    torch.cuda.synchronize()
    host = [o.table_bytes(payload).view(np.uint16).reshape(uniq.size, 256)] + \
        [o.table_bytes(t).view(np.uint16).reshape(t.shape) for t in small]
    want, wmask = o.seq_gather(host, compact, offs, L)
    assert int(err.item()) == 0
    assert np.array_equal(mask.cpu().numpy(), wmask)
    assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), want)
    del out
    # fused gather + tokenizer (raw 384 -> d 256) reads the same rows
    ws = [ot.random_tokenizer_weights(384, 256, max(L), seed=p) for p in range(3)]
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()} for w in ws]
    tok, tmask = pdm.ops.seq_tokenize_raw(tabs_d, ids_d, offs_d, L, wd)
    torch.cuda.synchronize()
    # the tokenizer tests' per-element bound on the compact host tables (same rows, compact ids)
    from test_gpu_tokenizer import _check
    _check(tok.cpu(), host, compact, offs, L, ws, 0, 0, tmask)
    del item, tabs_d
    torch.cuda.empty_cache()
