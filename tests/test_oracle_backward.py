"""Pins the C oracle's pooled backward and fused optimizers (CPU only).

* row gradients: torch autograd of ``F.embedding_bag`` in float64 (sum, mean, padding id, empty
  bags, two slots reading one table);
* Adam: ``torch.optim.AdamW`` (decoupled decay, the form FBGEMM's ADAM applies) with a large
  decay so a coupled-L2 mistake fails, and ``torch.optim.Adam`` without decay;
* row-wise Adagrad: ``torch.optim.Adagrad`` where the row-wise rule reduces to it: dim-1 tables,
  and rows whose elements and gradients are all equal (a sum instead of a mean over the row fails);
* sparse update, row space numbering and skipped entries by brute force.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as o


def _problem(g, tables, slot_specs, B, mean_len=4.0, max_len=12, pad=None, pad_frac=0.0, cover=False):
    """tables: [(rows, dim)]; slot_specs: [(table index, "sum" | "mean")].
    Returns slots, weights (flat fp32), per-table numpy weights, indices, offsets, grad."""
    offs, off = [], 0
    for rows, dim in tables:
        off = (off + 255) // 256 * 256
        offs.append(off)
        off += rows * dim * 4
    flat = np.zeros(max(off // 4, 1), dtype=np.float32)
    for (rows, dim), wo in zip(tables, offs):
        flat[wo // 4: wo // 4 + rows * dim] = g.uniform(-0.5, 0.5, rows * dim).astype(np.float32)
    slots, col = [], 0
    for ti, pooling in slot_specs:
        rows, dim = tables[ti]
        slots.append(dict(rows=rows, weights_offset=offs[ti], dim=dim, dtype="fp32", pooling=pooling,
                          row_bytes=0, out_offset=col))
        col += dim
    lengths, idx = [], []
    for ti, _ in slot_specs:
        rows = tables[ti][0]
        ls = np.minimum(g.poisson(mean_len, B), max_len)
        ids = g.integers(0, rows, int(ls.sum()))
        if cover:  # every row looked up at least once by this slot
            assert ids.size >= rows
            ids[:rows] = g.permutation(rows)
            g.shuffle(ids)
        if pad is not None and pad_frac > 0:
            ids[g.random(ids.size) < pad_frac] = pad
        lengths.append(ls)
        idx.append(ids)
    offsets = o.offsets_np(np.concatenate(lengths))
    indices = np.concatenate(idx).astype(np.int64)
    grad = g.normal(0, 1, (B, col)).astype(np.float32)
    return slots, flat, offs, indices, offsets, grad


def _torch_grads(tables, slot_specs, slots, flat, offs, indices, offsets, grad, B, pad, dtype=torch.float64):
    ws = [torch.tensor(flat[wo // 4: wo // 4 + r * d].reshape(r, d), dtype=dtype, requires_grad=True)
          for (r, d), wo in zip(tables, offs)]
    loss = 0
    for t, (ti, pooling) in enumerate(slot_specs):
        lo, hi = offsets[t * B], offsets[(t + 1) * B]
        ids = torch.from_numpy(indices[lo:hi])
        bag = torch.from_numpy(offsets[t * B:(t + 1) * B] - lo)
        out = F.embedding_bag(ids, ws[ti], bag, mode=pooling, padding_idx=pad)
        s = slots[t]
        loss = loss + (out * torch.from_numpy(grad[:, s["out_offset"]:s["out_offset"] + s["dim"]]).to(dtype)).sum()
    loss.backward()
    return [w.grad.numpy() for w in ws]


def _dense_from_sparse(tables, slots, slot_specs, ids, rows_g):
    row_off, _ = o.row_space(slots)
    out = [np.zeros((r, d), dtype=np.float64) for r, d in tables]
    first = {}
    for t, (ti, _) in enumerate(slot_specs):
        first.setdefault(ti, row_off[t])
    for k, gr in zip(ids, rows_g):
        for ti, base in first.items():
            if base <= k < base + tables[ti][0]:
                out[ti][k - base] = gr
    return out


@pytest.mark.parametrize("pad", [None, 0])
def test_row_gradients_match_embedding_bag_autograd(pad):
    g = np.random.default_rng(11)
    tables = [(60, 8), (25, 8), (200, 8)]
    specs = [(0, "sum"), (1, "mean"), (0, "mean"), (2, "sum")]  # table 0 read by two slots
    B = 37
    slots, flat, offs, idx, offsets, grad = _problem(g, tables, specs, B, pad=pad, pad_frac=0.2 if pad is not None else 0)
    ids, rows_g, bad = o.tbe_backward(slots, idx, offsets, B, grad, padding_idx=-1 if pad is None else pad)
    assert bad == 0
    assert np.all(np.diff(ids) > 0)
    want = _torch_grads(tables, specs, slots, flat, offs, idx, offsets, grad, B, pad)
    got = _dense_from_sparse(tables, slots, specs, ids, rows_g)
    for w, gt in zip(want, got):
        np.testing.assert_allclose(gt, w, rtol=1e-5, atol=1e-5)
    # the distinct ids are exactly the looked-up (non-padding) rows
    row_off, _ = o.row_space(slots)
    touched = set()
    for t in range(len(specs)):
        for i in range(offsets[t * B], offsets[(t + 1) * B]):
            if pad is None or idx[i] != pad:
                touched.add(row_off[t] + int(idx[i]))
    assert set(ids.tolist()) == touched


def test_row_space_numbering():
    slots = [dict(rows=10, weights_offset=0, dim=8, dtype="fp32", pooling="sum", out_offset=0),
             dict(rows=5, weights_offset=512, dim=16, dtype="fp32", pooling="sum", out_offset=8),
             dict(rows=10, weights_offset=0, dim=8, dtype="fp32", pooling="mean", out_offset=24),
             dict(rows=7, weights_offset=1024, dim=8, dtype="fp32", pooling="sum", out_offset=32),
             dict(rows=0, weights_offset=1024, dim=8, dtype="fp32", pooling="sum", out_offset=40)]
    row_off, total = o.row_space(slots)
    # dim-8 group first (tables at 0 and 1024, the empty table distinct), then dim 16
    assert row_off == [0, 17, 0, 10, 17] and total == 22


@pytest.mark.parametrize("wd,torch_cls", [(0.05, torch.optim.AdamW), (0.0, torch.optim.Adam)])
def test_adam_matches_torch(wd, torch_cls):
    g = np.random.default_rng(5)
    tables, specs, B = [(50, 8)], [(0, "sum"), (0, "mean")], 30
    # betas exact in fp32 (FBGEMM takes fp32 betas; torch keeps 0.999 in double, 1.3e-5 apart in 1 - b2)
    lr, eps, b1, b2 = 0.01, 1e-8, 0.875, 1.0 - 2.0 ** -10
    slots, flat, offs, _, _, _ = _problem(g, tables, specs, B, mean_len=5.0)
    W = torch.nn.Parameter(torch.tensor(flat[:50 * 8].reshape(50, 8)))
    opt = torch_cls([W], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    m1 = np.zeros_like(flat)
    m2 = np.zeros_like(flat)
    for step in range(1, 4):
        _, _, _, idx, offsets, grad = _problem(g, tables, specs, B, mean_len=5.0, cover=True)
        gw = _torch_grads(tables, specs, slots, W.detach().numpy().ravel().copy(), offs, idx, offsets, grad, B,
                          None, dtype=torch.float32)[0]
        W.grad = torch.from_numpy(gw)
        opt.step()
        o.tbe_backward(slots, idx, offsets, B, grad, optimizer=o.ADAM, weights=flat, m1=m1, m2=m2, lr=lr,
                       eps=eps, beta1=b1, beta2=b2, weight_decay=wd, step=step)
    st = opt.state[W]
    np.testing.assert_allclose(flat[:400].reshape(50, 8), W.detach().numpy(), rtol=1e-5, atol=1e-7)
    # m and v are sums of terms up to |g| ~ 3: a few fp32 ulps of those where they cancel
    np.testing.assert_allclose(m1[:400].reshape(50, 8), st["exp_avg"].numpy(), rtol=1e-5, atol=2e-7)
    np.testing.assert_allclose(m2[:400].reshape(50, 8), st["exp_avg_sq"].numpy(), rtol=1e-5, atol=2e-7)


def _adagrad_run(tables, B, wd, wd_mode, equal_rows, steps=3, seed=9):
    g = np.random.default_rng(seed)
    specs = [(0, "sum")]
    rows, D = tables[0]
    slots, flat, offs, _, _, _ = _problem(g, tables, specs, B, mean_len=5.0)
    if equal_rows:
        flat[:rows * D] = np.repeat(flat[:rows * D].reshape(rows, D)[:, :1], D, axis=1).ravel()
    W = torch.nn.Parameter(torch.tensor(flat[:rows * D].reshape(rows, D)[:, :1].copy()))
    opt = torch.optim.Adagrad([W], lr=0.05, eps=1e-8, weight_decay=wd if wd_mode == o.WD_L2 else 0.0)
    state = np.zeros(rows, dtype=np.float32)
    for step in range(steps):
        _, _, _, idx, offsets, grad = _problem(g, tables, specs, B, mean_len=5.0, cover=True)
        if equal_rows:
            grad = np.repeat(grad[:, :1], D, axis=1)
        gw = _torch_grads([(rows, 1)], specs, [dict(slots[0], dim=1)], W.detach().numpy().ravel().copy(), [0],
                          idx, offsets, np.ascontiguousarray(grad[:, :1]), B, None, dtype=torch.float32)[0]
        W.grad = torch.from_numpy(gw)
        opt.step()
        o.tbe_backward(slots, idx, offsets, B, grad, optimizer=o.ROWWISE_ADAGRAD, weights=flat, m1=state,
                       lr=0.05, eps=1e-8, weight_decay=wd, wd_mode=wd_mode)
    return flat[:rows * D].reshape(rows, D), state, W.detach().numpy(), opt.state[W]["sum"].numpy()


@pytest.mark.parametrize("wd,wd_mode", [(0.0, 0), (0.1, 1), (0.1, 0)])
def test_rowwise_adagrad_dim1_matches_torch_adagrad(wd, wd_mode):
    w, state, tw, tsum = _adagrad_run([(40, 1)], 12, wd, wd_mode, equal_rows=False)
    np.testing.assert_allclose(w, tw, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(state, tsum[:, 0], rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("wd_mode", [0, 1])
def test_rowwise_adagrad_uniform_rows_match_torch_adagrad(wd_mode):
    # every element and gradient of a row equal: mean over the row = the element's square
    w, state, tw, tsum = _adagrad_run([(40, 4)], 12, 0.1, wd_mode, equal_rows=True)
    np.testing.assert_allclose(w, np.repeat(tw, 4, axis=1), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(state, tsum[:, 0], rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("optimizer", [o.ADAM, o.ROWWISE_ADAGRAD])
def test_only_looked_up_rows_change(optimizer):
    g = np.random.default_rng(3)
    tables, specs, B = [(500, 8), (300, 8)], [(0, "sum"), (1, "mean")], 16
    slots, flat, offs, idx, offsets, grad = _problem(g, tables, specs, B, mean_len=3.0)
    row_off, total = o.row_space(slots)
    before = flat.copy()
    m1 = np.zeros_like(flat) if optimizer == o.ADAM else np.zeros(total, dtype=np.float32)
    m2 = np.zeros_like(flat)
    ids, _, _ = o.tbe_backward(slots, idx, offsets, B, grad, optimizer=optimizer, weights=flat, m1=m1, m2=m2,
                               weight_decay=0.01, wd_mode=o.WD_L2)
    changed = set()
    for t, (ti, _) in enumerate(specs):
        rows = flat[offs[ti] // 4: offs[ti] // 4 + tables[ti][0] * 8].reshape(-1, 8)
        rows0 = before[offs[ti] // 4: offs[ti] // 4 + tables[ti][0] * 8].reshape(-1, 8)
        for r in np.nonzero(np.any(rows != rows0, axis=1))[0]:
            changed.add(row_off[t] + int(r))
    assert changed == set(ids.tolist())
    if optimizer == o.ROWWISE_ADAGRAD:
        assert set(np.nonzero(m1)[0].tolist()) == set(ids.tolist())


def test_skipped_entries_are_counted():
    g = np.random.default_rng(4)
    slots, flat, offs, idx, offsets, grad = _problem(g, [(20, 4)], [(0, "sum")], 6, mean_len=4.0)
    idx = idx.copy()
    idx[0] = 20  # out of range
    idx[1] = -3
    ids_ok, _, _ = o.tbe_backward(slots, np.delete(idx, [0, 1]), np.maximum(offsets - 2, 0), 6, grad)
    ids, _, bad = o.tbe_backward(slots, idx, offsets, 6, grad)
    assert bad == 2
    bad_off = offsets.copy()
    bad_off[3] = bad_off[4] + 1  # bag 2 ends before it starts
    _, _, bad2 = o.tbe_backward(slots, idx, bad_off, 6, grad)
    assert bad2 >= 3
    del ids_ok, ids


def test_adam_first_step_closed_form():
    # zero state, step 1, no decay: m/bc1 = g, v/bc2 = g^2, so w' = w - lr g / (|g| + eps)
    g = np.random.default_rng(8)
    slots, flat, offs, idx, offsets, grad = _problem(g, [(1000, 4)], [(0, "sum")], 40, mean_len=2.0)
    before = flat.copy()
    m1 = np.zeros_like(flat)
    m2 = np.zeros_like(flat)
    ids, rows_g, _ = o.tbe_backward(slots, idx, offsets, 40, grad, optimizer=o.ADAM, weights=flat, m1=m1, m2=m2,
                                    lr=0.01, eps=1e-8)
    for k, gr in zip(ids, rows_g):
        want = before[k * 4:(k + 1) * 4] - 0.01 * gr / (np.abs(gr) + 1e-8)
        np.testing.assert_allclose(flat[k * 4:(k + 1) * 4], want, rtol=1e-6, atol=1e-9)
    assert math.isfinite(float(flat.sum()))


# ---- S-token gather backward ------------------------------------------------------------

def _seq_problem(g, B=7, pools=((6, 5.0), (4, 2.0)), tables=((40, 8), (25, 4))):
    ids, offs = [], []
    for L, mean in pools:
        ln = np.minimum(g.poisson(mean, B), 2 * L)
        n = int(ln.sum())
        ids.append([g.integers(0, r, n) for r, _ in tables])
        offs.append(o.offsets_np(ln))
    max_len = [L for L, _ in pools]
    slots, off, col = [], 0, 0
    for r, d in tables:
        slots.append(dict(rows=r, weights_offset=off, dim=d, dtype="fp32", pooling="sum", row_bytes=0, out_offset=col))
        off += r * d * 4
        col += d
    return ids, offs, max_len, slots


@pytest.mark.parametrize("pad_mode,align", [("row0", "right"), ("zero", "right"), ("row0", "left")])
def test_seq_token_ids_match_the_forward_oracle(pad_mode, align):
    g = np.random.default_rng(40)
    ids, offs, max_len, slots = _seq_problem(g)
    tabs = [g.integers(1, 1 << 15, (s["rows"], s["dim"]), dtype=np.uint16) for s in slots]
    want, mask = o.seq_gather(tabs, ids, offs, max_len, pad_mode={"row0": 0, "zero": 1}[pad_mode],
                              align={"right": 0, "left": 1}[align])
    tok = o.seq_token_ids(ids, offs, max_len, pad_mode, align)
    got = np.concatenate([np.where((tok[f] == o.SEQ_PAD)[..., None], 0, tabs[f][np.where(tok[f] == o.SEQ_PAD, 0, tok[f])])
                          for f in range(len(tabs))], axis=-1)
    assert np.array_equal(got, want)


def test_seq_gather_backward_matches_embedding_autograd():
    # the reference's path: ids left padded with 0 to L (dataset.py:604-626), EC lookup, per-pool concat of
    # the features (onetrans.py:515-520) and concat of the pools (:553-558)
    g = np.random.default_rng(41)
    ids, offs, max_len, slots = _seq_problem(g)
    B, S, Dt = 7, sum(max_len), sum(s["dim"] for s in slots)
    W = [torch.tensor(g.uniform(-1, 1, (s["rows"], s["dim"])), requires_grad=True) for s in slots]
    pools = []
    for p, L in enumerate(max_len):
        feats = []
        for f in range(len(slots)):
            padded = torch.zeros(B, L, dtype=torch.long)
            for b in range(B):
                seq = ids[p][f][offs[p][b]:offs[p][b + 1]][-L:]
                if len(seq):
                    padded[b, L - len(seq):] = torch.from_numpy(seq)
            feats.append(F.embedding(padded, W[f]))
        pools.append(torch.cat(feats, dim=-1))
    out = torch.cat(pools, dim=1)
    G = g.normal(0, 1, (B, S, Dt)).astype(np.float32)
    (out * torch.from_numpy(G).double()).sum().backward()
    rids, rows, bad = o.seq_gather_backward(slots, ids, offs, max_len, G)
    assert bad == 0
    row_off, _ = o.row_space(slots)
    for f, s in enumerate(slots):
        dense = np.zeros((s["rows"], s["dim"]))
        for k, r in zip(rids, rows):
            if row_off[f] <= k < row_off[f] + s["rows"]:
                dense[k - row_off[f]] = r[:s["dim"]]
        np.testing.assert_allclose(dense, W[f].grad.numpy(), rtol=1e-5, atol=1e-5)
