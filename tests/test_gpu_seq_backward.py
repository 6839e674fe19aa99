"""GPU parity of the S-token gather backward with the fused optimizer (pdm_seq_gather_backward_fused) and of
the fused EmbeddingCollection / SequenceGather modules, against the C oracle (``seq_gather_backward``: the
forward's slot placement restated, every slot a one-id bag of the pooled backward oracle)."""
import numpy as np
import pytest
import torch
from torch.distributed.optim import _apply_optimizer_in_backward

from oracle import oracle as o

pytestmark = pytest.mark.gpu


def _tables(g, specs):
    slots, off, col = [], 0, 0
    for r, d in specs:
        off = (off + 255) // 256 * 256
        slots.append(dict(rows=r, weights_offset=off, dim=d, dtype="fp32", pooling="sum", row_bytes=0, out_offset=col))
        off += r * d * 4
        col += d
    flat = g.uniform(-0.01, 0.01, off // 4).astype(np.float32)
    return slots, flat


def _pools(g, B, pools, specs, zipf=None):
    ids, offs = [], []
    for L, mean in pools:
        ln = g.poisson(mean, B)
        n = int(ln.sum())
        if zipf:
            items = (g.zipf(zipf, n) - 1) % specs[0][0]
        else:
            items = g.integers(0, specs[0][0], n)
        ids.append([items] + [items % r for r, _ in specs[1:]])
        offs.append(o.offsets_np(ln))
    return ids, offs


def _run(pdm, dev, specs, pools, B, optimizer, pad_mode="row0", align="right", steps=2, zipf=None, bad_id=False,
         ids_fn=None):
    L = pdm._lib
    g = np.random.default_rng(17)
    slots, flat = _tables(g, specs)
    plan = pdm.ops.TbePlan([dict(s, dtype=L.PDM_F32, pooling=L.PDM_POOL_SUM) for s in slots], dev)
    _, total = o.row_space(slots)
    adam = optimizer == o.ADAM
    m1 = np.zeros_like(flat) if adam else np.zeros(total, np.float32)
    m2 = np.zeros_like(flat)
    w_d, m1_d, m2_d = (torch.from_numpy(a.copy()).to(dev) for a in (flat, m1, m2))
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    max_len = [L_ for L_, _ in pools]
    S, Dt = sum(max_len), sum(d for _, d in specs)
    hp = dict(lr=0.01, eps=1e-8, beta1=0.9, beta2=0.999, weight_decay=1e-5)
    pm = {"row0": L.PDM_PAD_ROW0, "zero": L.PDM_PAD_ZERO}[pad_mode]
    al = {"right": L.PDM_ALIGN_RIGHT, "left": L.PDM_ALIGN_LEFT}[align]
    bad = 0
    for step in range(1, steps + 1):
        ids, offs = _pools(g, B, pools, specs, zipf)
        if ids_fn is not None:
            ids = ids_fn(g, ids)
        if bad_id:
            ids[0][1][3] = specs[1][0] + 5
        G = g.normal(0, 1, (B, S, Dt)).astype(np.float32)
        pdm.ops.seq_gather_backward_fused_raw(
            plan, w_d, m1_d, m2_d if adam else None, [r for r, _ in specs], [d for _, d in specs],
            [[torch.from_numpy(a).to(dev) for a in row] for row in ids], [torch.from_numpy(x).to(dev) for x in offs],
            max_len, torch.from_numpy(G).to(dev), pad_mode=pm, align=al,
            optimizer=L.PDM_OPT_ADAM if adam else L.PDM_OPT_ROWWISE_ADAGRAD, learning_rate=hp["lr"], eps=hp["eps"],
            weight_decay=hp["weight_decay"], weight_decay_mode=L.PDM_WD_L2, step=step, err_flag=err)
        _, _, b = o.seq_gather_backward(slots, ids, offs, max_len, G, pad_mode, align, optimizer=optimizer,
                                        weights=flat, m1=m1, m2=m2, wd_mode=o.WD_L2, step=step, **hp)
        bad += b
    torch.cuda.synchronize()
    got = w_d.cpu().numpy(), m1_d.cpu().numpy(), m2_d.cpu().numpy(), int(err.item())
    plan.release()
    return got, (flat, m1, m2, bad)


def _close(got, want, what, rtol=1e-5, atol=1e-7):
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol, err_msg=what)


@pytest.mark.parametrize("pad_mode,align", [("row0", "right"), ("zero", "right"), ("row0", "left")])
@pytest.mark.parametrize("optimizer", [o.ADAM, o.ROWWISE_ADAGRAD])
def test_seq_backward_matches_oracle(pdm, dev, pad_mode, align, optimizer):
    specs = [(5000, 32), (500, 16), (800, 16)]
    (w, m1, m2, err), (ww, wm1, wm2, bad) = _run(pdm, dev, specs, [(24, 12.0), (16, 20.0)], 64, optimizer,
                                                 pad_mode, align)
    assert err == 0 and bad == 0
    _close(w, ww, "weights")
    _close(m1, wm1, "state 1", atol=1e-6)
    if optimizer == o.ADAM:
        _close(m2, wm2, "state 2", atol=1e-6)


def test_seq_backward_hot_rows_and_invalid_ids(pdm, dev):
    # Zipf items: long runs of one row (and row 0 from every left-padding slot) across chunks
    specs = [(3000, 64), (300, 32)]
    (w, m1, m2, err), (ww, wm1, wm2, bad) = _run(pdm, dev, specs, [(64, 40.0), (32, 10.0)], 256, o.ADAM,
                                                 zipf=1.3, bad_id=True)
    assert err == 1 and bad == 2
    _close(w, ww, "weights")


@pytest.mark.parametrize("optimizer", [o.ADAM, o.ROWWISE_ADAGRAD])
def test_seq_backward_row0_only_when_looked_up(pdm, dev, optimizer):
    """Row 0 of a table takes the update only when some slot looks it up.  ZERO padding with every id >= 1:
    row 0 and its state keep their bits exactly.  ROW0 padding with a tenth of the events forced to id 0:
    row 0's gradient adds padding slots and events (the oracle's row-0 sum), matching the oracle."""
    specs = [(700, 32), (90, 16), (60, 16)]

    def no_zero(g, ids):
        return [[1 + a % (r - 1) for a, (r, _) in zip(row, specs)] for row in ids]

    def some_zero(g, ids):
        out = []
        for row in ids:
            z = g.random(row[0].size) < 0.1
            out.append([np.where(z, 0, a) for a in row])
        return out

    (w, m1, m2, err), (ww, wm1, wm2, bad) = _run(pdm, dev, specs, [(24, 12.0), (16, 20.0)], 64, optimizer,
                                                 "zero", "right", ids_fn=no_zero)
    assert err == 0 and bad == 0
    _close(w, ww, "weights")
    g0 = np.random.default_rng(17)
    slots, flat0 = _tables(g0, specs)
    for sl in slots:
        r0 = slice(sl["weights_offset"] // 4, sl["weights_offset"] // 4 + sl["dim"])
        assert np.array_equal(w[r0], flat0[r0]), "row 0 changed without a lookup"
        if optimizer == o.ADAM:
            assert not m1[r0].any() and not m2[r0].any()
    (w, m1, m2, err), (ww, wm1, wm2, bad) = _run(pdm, dev, specs, [(24, 12.0), (16, 20.0)], 64, optimizer,
                                                 "row0", "right", ids_fn=some_zero)
    assert err == 0 and bad == 0
    _close(w, ww, "weights")
    _close(m1, wm1, "state 1", atol=1e-6)
    if optimizer == o.ADAM:
        _close(m2, wm2, "state 2", atol=1e-6)


def _seq_module(pdm, dev, optim_cls, kw):
    cfgs = [pdm.EmbeddingConfig(3000, 32, "item", pdm.DataType.FP32, ["lp_item", "sk_item"]),
            pdm.EmbeddingConfig(400, 16, "artist", pdm.DataType.FP32, ["lp_artist", "sk_artist"])]
    ec = pdm.EmbeddingCollection(cfgs, device=dev)
    for p in ec.parameters():
        _apply_optimizer_in_backward(optim_cls, [p], kw)
    sg = pdm.SequenceGather(ec, {"lp": ["lp_item", "lp_artist"], "sk": ["sk_item", "sk_artist"]},
                            {"lp": 20, "sk": 12})
    return ec, sg


@pytest.mark.parametrize("adam", [True, False])
def test_sequence_gather_module_fused(pdm, dev, adam):
    kw = {"lr": 0.02, "eps": 1e-8, "weight_decay": 1e-5}
    if not adam:
        kw["weight_decay_mode"] = pdm.WeightDecayMode.L2
    ec, sg = _seq_module(pdm, dev, torch.optim.Adam if adam else pdm.RowWiseAdagrad, kw)
    fo = ec.fused_optimizer
    slots = [dict(rows=t.num_embeddings, weights_offset=ec._store.offsets[i], dim=t.embedding_dim, dtype="fp32",
                  pooling="sum", row_bytes=0, out_offset=[0, 32][i]) for i, t in enumerate(ec._tables)]
    flat = ec._store.flat.cpu().numpy().view(np.float32).copy()
    m1 = np.zeros_like(flat) if adam else np.zeros(3400, np.float32)
    m2 = np.zeros_like(flat)
    g = np.random.default_rng(3)
    B = 32
    for step in range(1, 3):
        batch, ids, offs = {}, [], []
        for pool, mean in (("lp", 15.0), ("sk", 6.0)):
            ln = g.poisson(mean, B)
            it = g.integers(0, 3000, int(ln.sum()))
            ar = it % 400
            batch[f"{pool}_item"], batch[f"{pool}_artist"] = torch.from_numpy(it).to(dev), torch.from_numpy(ar).to(dev)
            batch[f"{pool}_item__lengths"] = torch.from_numpy(ln).to(dev)
            batch[f"{pool}_artist__lengths"] = torch.from_numpy(ln).to(dev)
            ids.append([it, ar])
            offs.append(o.offsets_np(ln))
        tokens, mask = sg(batch)
        G = g.normal(0, 1, tuple(tokens.shape)).astype(np.float32)
        (tokens * torch.from_numpy(G).to(dev)).sum().backward()
        o.seq_gather_backward(slots, ids, offs, [20, 12], G, optimizer=o.ADAM if adam else o.ROWWISE_ADAGRAD,
                              weights=flat, m1=m1, m2=m2, lr=0.02, eps=1e-8, weight_decay=1e-5,
                              wd_mode=o.WD_L2 if not adam else 0, step=step,
                              row_off=[fo.state_offset["item"], fo.state_offset["artist"]] if not adam else None)
    torch.cuda.synchronize()
    _close(ec._store.flat.cpu().numpy().view(np.float32), flat, "weights")
    _close(fo.momentum1.cpu().numpy(), m1, "state 1", atol=1e-6)
    assert all(p.grad is None for p in ec.parameters())


def test_embedding_collection_forward_fused(pdm, dev):
    cfgs = [pdm.EmbeddingConfig(700, 16, "t0", pdm.DataType.FP32, ["a", "b"]),
            pdm.EmbeddingConfig(90, 32, "t1", pdm.DataType.FP32, ["c"])]
    ec = pdm.EmbeddingCollection(cfgs, device=dev)
    for p in ec.parameters():
        _apply_optimizer_in_backward(torch.optim.Adam, [p], {"lr": 0.01})
    g = np.random.default_rng(9)
    B = 40
    lens = g.integers(0, 5, 3 * B)
    vals = np.concatenate([g.integers(0, r, int(lens[k * B:(k + 1) * B].sum())) for k, r in enumerate((700, 700, 90))])
    kjt = pdm.KeyedJaggedTensor.from_lengths_sync(["a", "b", "c"], torch.from_numpy(vals).to(dev),
                                                  torch.from_numpy(lens).to(dev))
    flat = ec._store.flat.cpu().numpy().view(np.float32).copy()
    out = ec(kjt)
    grads = {k: g.normal(0, 1, tuple(out[k].values().shape)).astype(np.float32) for k in ("a", "b", "c")}
    loss = sum((out[k].values() * torch.from_numpy(grads[k]).to(dev)).sum() for k in ("a", "b", "c"))
    loss.backward()
    # oracle: every id a one-id bag of its feature's slot, features padded to the longest with empty bags
    ns = [int(lens[k * B:(k + 1) * B].sum()) for k in range(3)]
    bags = max(ns)
    dims = [16, 16, 32]
    G = np.zeros((bags, sum(dims)), np.float32)
    col = 0
    for k, key in enumerate(("a", "b", "c")):
        G[:ns[k], col:col + dims[k]] = grads[key]
        col += dims[k]
    lengths = np.concatenate([(np.arange(bags) < n).astype(np.int64) for n in ns])
    slots = [dict(rows=700, weights_offset=ec._store.offsets[0], dim=16, dtype="fp32", pooling="sum", row_bytes=0,
                  out_offset=0),
             dict(rows=700, weights_offset=ec._store.offsets[0], dim=16, dtype="fp32", pooling="sum", row_bytes=0,
                  out_offset=16),
             dict(rows=90, weights_offset=ec._store.offsets[1], dim=32, dtype="fp32", pooling="sum", row_bytes=0,
                  out_offset=32)]
    m1, m2 = np.zeros_like(flat), np.zeros_like(flat)
    o.tbe_backward(slots, vals, o.offsets_np(lengths), bags, G, optimizer=o.ADAM, weights=flat, m1=m1, m2=m2,
                   lr=0.01, eps=1e-8, step=1)
    torch.cuda.synchronize()
    _close(ec._store.flat.cpu().numpy().view(np.float32), flat, "weights")
