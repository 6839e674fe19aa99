"""GPU parity of the pooled TBE backward with the fused optimizer against the C oracle.

Row ids are compared exactly; row gradients within 1e-6 of the sum of |terms| (the kernel adds a
run's terms in lookup order, and a run that crosses a 64-entry chunk as per-chunk partial sums);
weights and optimizer state within rtol 1e-5 (fp32, the stated tolerance) after several steps.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as o

pytestmark = pytest.mark.gpu


def _tables(g, tables, specs, B, lengths=None, mean_len=10.0, max_len=50, min_len=0, zipf=None, pad=None,
            pad_frac=0.0, stride_extra=0):
    """tables: [(rows, dim)]; specs: [(table, pooling)].  Returns slots (oracle naming), flat fp32 weights,
    indices, offsets, grad [B, total + stride_extra]."""
    offs, off = [], 0
    for rows, dim in tables:
        off = (off + 255) // 256 * 256
        offs.append(off)
        off += rows * dim * 4
    flat = np.zeros(max(off // 4, 4), dtype=np.float32)
    for (rows, dim), wo in zip(tables, offs):
        flat[wo // 4: wo // 4 + rows * dim] = g.uniform(-0.01, 0.01, rows * dim).astype(np.float32)
    slots, col = [], 0
    for ti, pooling in specs:
        rows, dim = tables[ti]
        slots.append(dict(rows=rows, weights_offset=offs[ti], dim=dim, dtype="fp32", pooling=pooling, row_bytes=0,
                          out_offset=col))
        col += dim
    ls_all, ids_all = [], []
    for ti, _ in specs:
        rows = tables[ti][0]
        ls = np.clip(g.poisson(mean_len, B), min_len, max_len) if lengths is None else np.full(B, lengths)
        n = int(ls.sum())
        if zipf is not None:
            ids = (g.zipf(zipf, n) - 1) % rows
        else:
            ids = g.integers(0, rows, n)
        if pad is not None and pad_frac > 0:
            ids[g.random(n) < pad_frac] = pad
        ls_all.append(ls)
        ids_all.append(ids)
    offsets = o.offsets_np(np.concatenate(ls_all))
    indices = np.concatenate(ids_all).astype(np.int64)
    grad = g.normal(0, 1, (B, col + stride_extra)).astype(np.float32)
    return slots, flat, indices, offsets, grad


def _plan(pdm, dev, slots):
    L = pdm._lib
    pools = {"sum": L.PDM_POOL_SUM, "mean": L.PDM_POOL_MEAN}
    return pdm.ops.TbePlan([dict(s, dtype=L.PDM_F32, pooling=pools[s["pooling"]]) for s in slots], dev)


def _sparse(pdm, dev, slots, indices, offsets, B, grad, padding_idx=-1, index_dtype=np.int64):
    plan = _plan(pdm, dev, slots)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    ids, rows, nu = pdm.ops.tbe_backward_sparse_grad_raw(
        plan, torch.from_numpy(indices.astype(index_dtype)).to(dev), torch.from_numpy(offsets).to(dev), B,
        torch.from_numpy(grad).to(dev), padding_idx=padding_idx, err_flag=err)
    torch.cuda.synchronize()
    u = int(nu.item())
    out = ids[:u].cpu().numpy(), rows[:u].cpu().numpy(), int(err.item())
    plan.release()
    return out


def _exact_rows(slots, indices, offsets, B, grad, padding_idx, ids):
    """Row gradients summed in float64 (numpy), at the given row ids."""
    row_off, total = o.row_space(slots)
    D = max(s["dim"] for s in slots)
    acc = np.zeros((total, D), np.float64)
    for t, s in enumerate(slots):
        lo, hi = offsets[t * B], offsets[(t + 1) * B]
        idx = indices[lo:hi].astype(np.int64)
        bag = np.repeat(np.arange(B), np.diff(offsets[t * B:(t + 1) * B + 1]))
        keep = (idx >= 0) & (idx < s["rows"])
        if padding_idx >= 0:
            keep &= idx != padding_idx
        cnt = np.bincount(bag[keep], minlength=B)
        sc = 1.0 / np.maximum(cnt[bag[keep]], 1) if s["pooling"] == "mean" else np.ones(int(keep.sum()))
        cols = grad[:, s["out_offset"]:s["out_offset"] + s["dim"]].astype(np.float64)
        np.add.at(acc, row_off[t] + idx[keep], np.pad(cols[bag[keep]] * sc[:, None], ((0, 0), (0, D - s["dim"]))))
    return acc[ids]


def _check_sparse(slots, indices, offsets, B, grad, got_ids, got_rows, padding_idx=-1):
    """Row ids exactly as the oracle's; row gradients within 1e-6 of the sum of |terms| of the exact (float64)
    sums (the kernel adds a run in lookup order within 64-entry chunks, then the chunk sums in order)."""
    want_ids, want_rows, bad = o.tbe_backward(slots, indices, offsets, B, grad, padding_idx=padding_idx)
    np.testing.assert_array_equal(got_ids, want_ids)
    _, absum, _ = o.tbe_backward(slots, indices, offsets, B, np.abs(grad), padding_idx=padding_idx)
    exact = _exact_rows(slots, indices, offsets, B, grad, padding_idx, got_ids)[:, :got_rows.shape[1]]
    err = np.abs(got_rows.astype(np.float64) - exact)
    assert np.all(err <= 1e-6 * absum + 1e-30), f"max err {err.max()} at {np.unravel_index(err.argmax(), err.shape)}"
    return bad


@pytest.mark.parametrize("pooling", ["sum", "mean"])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_sparse_grad_matches_oracle(pdm, dev, pooling, index_dtype):
    g = np.random.default_rng(21)
    tables = [(5000, 64), (3000, 64), (700, 64)]
    specs = [(0, pooling), (1, pooling), (2, pooling)]
    B = 512
    slots, _, idx, offsets, grad = _tables(g, tables, specs, B)
    ids, rows, err = _sparse(pdm, dev, slots, idx, offsets, B, grad, index_dtype=index_dtype)
    assert err == 0
    _check_sparse(slots, idx, offsets, B, grad, ids, rows)


@pytest.mark.parametrize("dim", [4, 12, 32, 128, 256, 512, 1024])
def test_sparse_grad_dims(pdm, dev, dim):
    g = np.random.default_rng(dim)
    tables = [(400, dim), (90, dim)]
    specs = [(0, "sum"), (1, "mean"), (0, "mean")]  # table 0 read by two slots
    B = 96
    slots, _, idx, offsets, grad = _tables(g, tables, specs, B, mean_len=6.0, max_len=20, stride_extra=4)
    ids, rows, _ = _sparse(pdm, dev, slots, idx, offsets, B, grad)
    _check_sparse(slots, idx, offsets, B, grad, ids, rows)


def test_sparse_grad_hot_rows(pdm, dev):
    # Zipf ids: runs of thousands of entries cross many 64-entry chunks
    g = np.random.default_rng(5)
    tables = [(10000, 128), (2000, 128)]
    specs = [(0, "sum"), (1, "mean")]
    B = 4096
    slots, _, idx, offsets, grad = _tables(g, tables, specs, B, mean_len=8.0, zipf=1.2)
    ids, rows, _ = _sparse(pdm, dev, slots, idx, offsets, B, grad)
    _check_sparse(slots, idx, offsets, B, grad, ids, rows)


def test_sparse_grad_single_row(pdm, dev):
    g = np.random.default_rng(6)
    slots, _, idx, offsets, grad = _tables(g, [(50, 64)], [(0, "sum")], 2000, lengths=10)
    idx[:] = 7
    ids, rows, _ = _sparse(pdm, dev, slots, idx, offsets, 2000, grad)
    assert ids.tolist() == [7]
    _check_sparse(slots, idx, offsets, 2000, grad, ids, rows)


@pytest.mark.parametrize("optimizer", [None, o.ADAM])
def test_very_long_run(pdm, dev, optimizer):
    # ~540k lookups of one row: the run covers ~8,400 chunks, folded over two levels of 64
    g = np.random.default_rng(12)
    B = 60_000
    slots, flat, idx, offsets, grad = _tables(g, [(5000, 32)], [(0, "sum")], B, lengths=10)
    idx[g.random(idx.size) < 0.9] = 7
    if optimizer is None:
        ids, rows, _ = _sparse(pdm, dev, slots, idx, offsets, B, grad)
        _check_sparse(slots, idx, offsets, B, grad, ids, rows)
        return
    plan = _plan(pdm, dev, slots)
    w = torch.from_numpy(flat).to(dev)
    m1, m2 = torch.zeros_like(w), torch.zeros_like(w)
    pdm.ops.tbe_backward_fused_raw(plan, w, m1, m2, torch.from_numpy(idx).to(dev), torch.from_numpy(offsets).to(dev),
                                   B, torch.from_numpy(grad).to(dev))
    wm1, wm2 = np.zeros_like(flat), np.zeros_like(flat)
    o.tbe_backward(slots, idx, offsets, B, grad, optimizer=o.ADAM, weights=flat, m1=wm1, m2=wm2)
    _, absum, _ = o.tbe_backward(slots, idx, offsets, B, np.abs(grad))
    ids, _, _ = o.tbe_backward(slots, idx, offsets, B, grad)
    gmag = np.zeros_like(flat)
    for k, a_ in zip(ids, absum):
        gmag[k * 32:(k + 1) * 32] = a_
    _close(w.cpu().numpy(), flat, "weights")
    _close(m1.cpu().numpy(), wm1, "m", gmag)
    plan.release()


def test_sparse_grad_padding_invalid_empty(pdm, dev):
    g = np.random.default_rng(8)
    slots, _, idx, offsets, grad = _tables(g, [(300, 32), (40, 32)], [(0, "mean"), (1, "sum")], 200,
                                           mean_len=3.0, pad=0, pad_frac=0.3)
    idx[5] = 300       # out of range for table 0
    idx[-1] = -2       # negative
    ids, rows, err = _sparse(pdm, dev, slots, idx, offsets, 200, grad, padding_idx=0)
    assert err == 1
    bad = _check_sparse(slots, idx, offsets, 200, grad, ids, rows, padding_idx=0)
    assert bad == 2
    assert 0 not in ids.tolist()  # padding rows get no gradient


def test_sparse_grad_empty_batch(pdm, dev):
    slots = [dict(rows=10, weights_offset=0, dim=8, dtype="fp32", pooling="sum", row_bytes=0, out_offset=0)]
    for B, n in ((0, 0), (4, 0)):
        idx = np.zeros(n, dtype=np.int64)
        offsets = np.zeros(B + 1, dtype=np.int64)
        ids, rows, err = _sparse(pdm, dev, slots, idx, offsets, B, np.zeros((B, 8), np.float32))
        assert ids.size == 0 and err == 0


def test_plan_row_space_matches_oracle(pdm, dev):
    slots = [dict(rows=10, weights_offset=0, dim=8, dtype="fp32", pooling="sum", row_bytes=0, out_offset=0),
             dict(rows=5, weights_offset=512, dim=16, dtype="fp32", pooling="sum", row_bytes=0, out_offset=8),
             dict(rows=10, weights_offset=0, dim=8, dtype="fp32", pooling="mean", row_bytes=0, out_offset=24),
             dict(rows=7, weights_offset=1024, dim=8, dtype="fp32", pooling="sum", row_bytes=0, out_offset=32),
             dict(rows=0, weights_offset=1024, dim=8, dtype="fp32", pooling="sum", row_bytes=0, out_offset=40)]
    plan = _plan(pdm, dev, slots)
    want, total = o.row_space(slots)
    assert plan.row_offsets == want and plan.total_rows == total
    plan.release()


def _fused_steps(pdm, dev, tables, specs, B, optimizer, steps=2, seed=0, wd=1e-5, wd_mode=0, index_dtype=np.int64,
                 padding_idx=-1, **kw):
    g = np.random.default_rng(seed)
    slots, flat, _, _, _ = _tables(g, tables, specs, 1, **kw)
    _, total = o.row_space(slots)
    plan = _plan(pdm, dev, slots)
    adam = optimizer == o.ADAM
    m1 = np.zeros_like(flat) if adam else np.zeros(max(total, 1), dtype=np.float32)
    m2 = np.zeros_like(flat)
    w_d, m1_d, m2_d = (torch.from_numpy(a.copy()).to(dev) for a in (flat, m1, m2))
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    hp = dict(lr=0.01, eps=1e-8, beta1=0.9, beta2=0.999, weight_decay=wd)
    row_off, _ = o.row_space(slots)
    gmag = np.zeros_like(flat)                 # per element: sum over steps of the row's sum |terms|
    rmag = np.zeros(max(total, 1), np.float64)  # per row id: sum over steps of mean_d (sum |terms|)^2
    for step in range(1, steps + 1):
        _, _, idx, offsets, grad = _tables(g, tables, specs, B, **kw)
        ids, absum, _ = o.tbe_backward(slots, idx.astype(index_dtype), offsets, B, np.abs(grad),
                                       padding_idx=padding_idx)
        bases = sorted({(r, i) for i, r in enumerate(row_off)})
        starts = np.array([r for r, _ in bases])
        for k, a in zip(ids.tolist(), absum):
            t = bases[int(np.searchsorted(starts, k, side="right")) - 1][1]
            D = slots[t]["dim"]
            e0 = slots[t]["weights_offset"] // 4 + (k - row_off[t]) * D
            gmag[e0:e0 + D] += a[:D]
            rmag[k] += float(np.mean(a[:D].astype(np.float64) ** 2))
        pdm.ops.tbe_backward_fused_raw(plan, w_d, m1_d, m2_d if adam else None,
                                       torch.from_numpy(idx.astype(index_dtype)).to(dev),
                                       torch.from_numpy(offsets).to(dev), B, torch.from_numpy(grad).to(dev),
                                       optimizer=pdm._lib.PDM_OPT_ADAM if adam else pdm._lib.PDM_OPT_ROWWISE_ADAGRAD,
                                       learning_rate=hp["lr"], eps=hp["eps"], beta1=hp["beta1"], beta2=hp["beta2"],
                                       weight_decay=wd, weight_decay_mode=wd_mode, step=step,
                                       padding_idx=padding_idx, err_flag=err)
        o.tbe_backward(slots, idx.astype(index_dtype), offsets, B, grad, padding_idx=padding_idx,
                       optimizer=optimizer, weights=flat, m1=m1, m2=m2, wd_mode=wd_mode, step=step, **hp)
    torch.cuda.synchronize()
    got = w_d.cpu().numpy(), m1_d.cpu().numpy(), m2_d.cpu().numpy()
    plan.release()
    return got, (flat, m1, m2), int(err.item()), (gmag, rmag)


def _close(got, want, what, mag=None):
    """rtol 1e-5 (fp32); where the value derives from a gradient sum, also 1e-6 of the sum of |terms|
    (the order of an fp32 sum over a long run of lookups is not the oracle's sequential one)."""
    tol = 1e-5 * np.abs(want) + 1e-7
    if mag is not None:
        tol = tol + 1e-6 * mag
    bad = np.abs(got.astype(np.float64) - want) > tol
    assert not bad.any(), f"{what}: {bad.sum()} elements off, first {np.argwhere(bad)[:3].ravel().tolist()}, " \
                          f"got {got[bad][:3]}, want {want[bad][:3]}"


def test_fused_adam_ebc_config(pdm, dev):
    # 8 tables x 100,000 x 64 fp32, batch 2048, Poisson(10) bags clipped to [0, 50], uniform ids;
    # the reference's embedding defaults: lr 1e-2, eps 1e-8, weight decay 1e-5
    tables = [(100_000, 64)] * 8
    specs = [(t, "sum") for t in range(8)]
    (w, m1, m2), (ww, wm1, wm2), err, (gmag, _) = _fused_steps(pdm, dev, tables, specs, 2048, o.ADAM, steps=3)
    assert err == 0
    _close(w, ww, "weights")
    _close(m1, wm1, "m", gmag)
    _close(m2, wm2, "v", 2 * gmag * gmag)
    assert np.mean(w.view(np.uint32) == ww.view(np.uint32)) > 0.999


@pytest.mark.parametrize("wd_mode", [0, 1])
def test_fused_rowwise_adagrad(pdm, dev, wd_mode):
    tables = [(20_000, 64), (5_000, 128), (3_000, 128)]
    specs = [(0, "sum"), (1, "mean"), (2, "sum"), (1, "sum")]
    (w, m1, _), (ww, wm1, _), err, (_, rmag) = _fused_steps(pdm, dev, tables, specs, 1024, o.ROWWISE_ADAGRAD,
                                                            steps=3, wd=0.01, wd_mode=wd_mode)
    assert err == 0
    _close(w, ww, "weights")
    _close(m1, wm1, "row state", 2 * rmag)


@pytest.mark.parametrize("optimizer", [o.ADAM, o.ROWWISE_ADAGRAD])
def test_fused_hot_rows_mixed_dims(pdm, dev, optimizer):
    tables = [(8000, 32), (3000, 128), (500, 4), (900, 12), (400, 512)]
    specs = [(0, "sum"), (1, "mean"), (2, "sum"), (0, "mean"), (3, "sum"), (4, "mean")]
    (w, m1, m2), (ww, wm1, wm2), err, (gmag, rmag) = _fused_steps(
        pdm, dev, tables, specs, 2048, optimizer, steps=3, zipf=1.15, mean_len=6.0, wd=0.01, wd_mode=1,
        index_dtype=np.int32, padding_idx=0, pad=0, pad_frac=0.1, stride_extra=8)
    assert err == 0
    _close(w, ww, "weights")
    if optimizer == o.ADAM:
        _close(m1, wm1, "m", gmag)
        _close(m2, wm2, "v", 2 * gmag * gmag)
    else:
        _close(m1, wm1, "row state", 2 * rmag)


def test_fused_deterministic(pdm, dev):
    g = np.random.default_rng(2)
    tables = [(3000, 64)]
    slots, flat, idx, offsets, grad = _tables(g, tables, [(0, "sum")], 8192, zipf=1.3)
    plan = _plan(pdm, dev, slots)
    outs = []
    for _ in range(2):
        w = torch.from_numpy(flat).to(dev)
        m1, m2 = torch.zeros_like(w), torch.zeros_like(w)
        pdm.ops.tbe_backward_fused_raw(plan, w, m1, m2, torch.from_numpy(idx).to(dev),
                                       torch.from_numpy(offsets).to(dev), 8192, torch.from_numpy(grad).to(dev))
        outs.append((w.cpu().numpy().view(np.uint32), m2.cpu().numpy().view(np.uint32)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    plan.release()


def test_fused_invalid_entries(pdm, dev):
    g = np.random.default_rng(13)
    tables = [(600, 16)]
    slots, flat, idx, offsets, grad = _tables(g, tables, [(0, "mean")], 64, mean_len=5.0, min_len=1)
    idx[3] = 600
    offsets = offsets.copy()
    offsets[-1] = offsets[-1] + 5  # the last bag ends past num_indices: skipped
    plan = _plan(pdm, dev, slots)
    w = torch.from_numpy(flat).to(dev)
    m1, m2 = torch.zeros_like(w), torch.zeros_like(w)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    pdm.ops.tbe_backward_fused_raw(plan, w, m1, m2, torch.from_numpy(idx).to(dev), torch.from_numpy(offsets).to(dev),
                                   64, torch.from_numpy(grad).to(dev), err_flag=err)
    wm1, wm2 = np.zeros_like(flat), np.zeros_like(flat)
    _, _, bad = o.tbe_backward(slots, idx, offsets, 64, grad, optimizer=o.ADAM, weights=flat, m1=wm1, m2=wm2)
    assert bad == 2 and int(err.item()) == 1
    _close(w.cpu().numpy(), flat, "weights")
    plan.release()


def test_backward_rejects_unsupported(pdm, dev):
    L = pdm._lib
    slots = [dict(rows=10, weights_offset=0, dim=8, dtype=L.PDM_BF16, pooling=L.PDM_POOL_SUM, row_bytes=0,
                  out_offset=0)]
    plan = pdm.ops.TbePlan(slots, dev)
    w = torch.zeros(80, device=dev)
    idx = torch.zeros(4, dtype=torch.int64, device=dev)
    off = torch.tensor([0, 2, 4], dtype=torch.int64, device=dev)
    grad = torch.zeros(2, 8, device=dev)
    with pytest.raises(L.PdmError):
        pdm.ops.tbe_backward_fused_raw(plan, w, w.clone(), w.clone(), idx, off, 2, grad)
    plan.release()
    slots[0]["dtype"] = L.PDM_F32
    plan = pdm.ops.TbePlan(slots, dev)
    with pytest.raises(L.PdmError):  # Adam step must be >= 1
        pdm.ops.tbe_backward_fused_raw(plan, w, w.clone(), w.clone(), idx, off, 2, grad, step=0)
    with pytest.raises(L.PdmError):  # too small a workspace
        pdm.ops.tbe_backward_fused_raw(plan, w, w.clone(), w.clone(), idx, off, 2, grad,
                                       workspace=torch.empty(256, dtype=torch.uint8, device=dev))
    plan.release()


def test_large_batch_multi_tile(pdm, dev):
    # ~1.6 M lookups: several hundred sort tiles, multi-pass scans
    g = np.random.default_rng(31)
    tables = [(200_000, 32)] * 4
    specs = [(t, "sum") for t in range(4)]
    slots, _, idx, offsets, grad = _tables(g, tables, specs, 40_000)
    ids, rows, _ = _sparse(pdm, dev, slots, idx, offsets, 40_000, grad)
    _check_sparse(slots, idx, offsets, 40_000, grad, ids, rows)
