"""The fused-optimizer EmbeddingBagCollection driven the reference's way: weights tagged with
``_apply_optimizer_in_backward`` (distributed/wrapper.py:151-174), ``loss.backward()`` updates the tables in
place; checked against the C oracle over several steps."""
import numpy as np
import pytest
import torch
from torch.distributed.optim import _apply_optimizer_in_backward

from oracle import oracle as o

pytestmark = pytest.mark.gpu


def _build(pdm, dev):
    cfgs = [pdm.EmbeddingBagConfig(500, 64, "t0", pdm.DataType.FP32, ["a", "b"], pdm.PoolingType.SUM),
            pdm.EmbeddingBagConfig(300, 32, "t1", pdm.DataType.FP32, ["c"], pdm.PoolingType.MEAN)]
    return pdm.EmbeddingBagCollection(cfgs, device=dev)


def _oracle_slots(pdm, ebc):
    L = pdm._lib
    return [dict(s, dtype="fp32", pooling="sum" if s["pooling"] == L.PDM_POOL_SUM else "mean") for s in ebc._slots]


def _batch(g, B, rows=(500, 500, 300)):
    lens = g.integers(0, 9, 3 * B)
    vals = np.concatenate([g.integers(0, r, int(lens[k * B:(k + 1) * B].sum())) for k, r in enumerate(rows)])
    return lens, vals


def _run_steps(pdm, dev, ebc, optimizer, steps, lr_per_step=None, **hp):
    g = np.random.default_rng(7)
    slots = _oracle_slots(pdm, ebc)
    flat = ebc._store.flat.cpu().numpy().view(np.float32).copy()
    _, total = o.row_space(slots)
    m1 = np.zeros_like(flat) if optimizer == o.ADAM else np.zeros(total, np.float32)
    m2 = np.zeros_like(flat)
    B = 64
    for step in range(1, steps + 1):
        if lr_per_step is not None:
            ebc.fused_optimizer.param_groups[0]["lr"] = lr_per_step[step - 1]
            hp["lr"] = lr_per_step[step - 1]
        lens, vals = _batch(g, B)
        G = g.normal(0, 1, (B, 64 + 64 + 32)).astype(np.float32)
        kjt = pdm.KeyedJaggedTensor.from_lengths_sync(["a", "b", "c"], torch.from_numpy(vals).to(dev),
                                                      torch.from_numpy(lens).to(dev))
        kt = ebc(kjt)
        loss = (kt.values() * torch.from_numpy(G).to(dev)).sum()
        loss.backward()
        o.tbe_backward(slots, vals, o.offsets_np(lens), B, G, optimizer=optimizer, weights=flat, m1=m1, m2=m2,
                       step=step, **hp)
    torch.cuda.synchronize()
    return flat, m1, m2


def _close(got, want, what):
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-7, err_msg=what)


def test_fused_adam_via_apply_optimizer_in_backward(pdm, dev):
    ebc = _build(pdm, dev)
    kw = {"lr": 0.01, "eps": 1e-8, "weight_decay": 1e-5}
    for p in ebc.parameters():
        _apply_optimizer_in_backward(torch.optim.Adam, [p], kw)
    fo = ebc.fused_optimizer
    assert fo is not None and fo.optim_type == pdm.EmbOptimType.ADAM
    flat, m1, m2 = _run_steps(pdm, dev, ebc, o.ADAM, 3, lr=0.01, eps=1e-8, beta1=0.9, beta2=0.999,
                              weight_decay=1e-5)
    _close(ebc._store.flat.cpu().numpy().view(np.float32), flat, "weights")
    _close(fo.momentum1.cpu().numpy(), m1, "momentum1")
    _close(fo.momentum2.cpu().numpy(), m2, "momentum2")
    assert all(p.grad is None for p in ebc.parameters())
    assert fo.iter == 3
    sd = fo.state_dict()
    assert sd["state"]["t0"]["momentum1"].shape == (500, 64) and sd["state"]["t1"]["momentum2"].shape == (300, 32)


def test_fused_rowwise_adagrad_and_lr_schedule(pdm, dev):
    ebc = _build(pdm, dev)
    kw = {"lr": 0.05, "eps": 1e-8, "weight_decay": 1e-5, "weight_decay_mode": pdm.WeightDecayMode.L2}
    for p in ebc.parameters():
        _apply_optimizer_in_backward(pdm.RowWiseAdagrad, [p], kw)
    fo = ebc.fused_optimizer
    assert fo.optim_type == pdm.EmbOptimType.EXACT_ROWWISE_ADAGRAD
    # sparse warm-up style: the trainer changes param_groups[0]["lr"] between steps
    flat, m1, _ = _run_steps(pdm, dev, ebc, o.ROWWISE_ADAGRAD, 3, lr_per_step=[0.005, 0.02, 0.05], eps=1e-8,
                             weight_decay=1e-5, wd_mode=o.WD_L2)
    _close(ebc._store.flat.cpu().numpy().view(np.float32), flat, "weights")
    _close(fo.momentum1.cpu().numpy(), m1, "row state")
    assert fo.state_dict()["state"]["t1"]["sum"].shape == (300,)


def test_no_grad_forward_does_not_update(pdm, dev):
    ebc = _build(pdm, dev)
    for p in ebc.parameters():
        _apply_optimizer_in_backward(torch.optim.Adam, [p], {"lr": 0.01})
    before = ebc._store.flat.clone()
    g = np.random.default_rng(1)
    lens, vals = _batch(g, 32)
    kjt = pdm.KeyedJaggedTensor.from_lengths_sync(["a", "b", "c"], torch.from_numpy(vals).to(dev),
                                                  torch.from_numpy(lens).to(dev))
    with torch.no_grad():
        out = ebc(kjt).values()
    assert not out.requires_grad
    assert torch.equal(before, ebc._store.flat)
    # an untagged collection whose tables require gradients fails loudly at the backward instead of
    # silently training nothing; with frozen tables it is the plain lookup
    plain = _build(pdm, dev)
    out = plain(kjt).values()
    assert plain.fused_optimizer is None and out.requires_grad
    with pytest.raises(NotImplementedError, match="in-backward optimizer"):
        out.sum().backward()
    for p in plain.parameters():
        p.requires_grad_(False)
    assert not plain(kjt).values().requires_grad


def test_torchrec_embeddings_trains_through_fused_optimizer(pdm, dev):
    """TorchRecEmbeddings (embedding.py:72-174 of the reference) tagged like the reference's wrapper: the pooled
    features (padding id 0 filtered) and the unpooled ones update their tables in loss.backward(), matching the
    oracle's fused Adam on the same bags."""
    g = np.random.default_rng(12)
    specs = [pdm.EmbeddingTableConfig("hist", ["h1", "h2"], 400, 32, "mean"),
             pdm.EmbeddingTableConfig("item", ["item", "seq"], 300, 16, "none")]
    emb = pdm.TorchRecEmbeddings(specs, device=dev, scalar_feature_names={"item"})
    kw = {"lr": 0.02, "eps": 1e-8, "weight_decay": 0.0}
    for p in emb.parameters():
        _apply_optimizer_in_backward(torch.optim.Adam, [p], kw)
    B, L = 24, 6
    h1, h2 = g.integers(0, 400, (B, L)), g.integers(0, 400, (B, L))
    h1[g.random((B, L)) < 0.4] = 0
    h1[3] = 0
    item, seq = g.integers(0, 300, B), g.integers(0, 300, (B, 5))
    feats = {k: torch.from_numpy(v).to(dev) for k, v in dict(h1=h1, h2=h2, item=item, seq=seq).items()}
    hist0 = emb.ebc._store.flat.cpu().numpy().view(np.float32).copy()
    row0 = hist0[:32].copy()
    item0 = emb.ec._store.flat.cpu().numpy().view(np.float32).copy()
    G = {k: g.normal(0, 1, s).astype(np.float32) for k, s in
         (("h1", (B, 32)), ("h2", (B, 32)), ("item", (B, 16)), ("seq", (B, 5, 16)))}
    out = emb(feats, padding_idx=0)
    loss = sum((out[k] * torch.from_numpy(v).to(dev)).sum() for k, v in G.items())
    loss.backward()
    torch.cuda.synchronize()
    hp = dict(optimizer=o.ADAM, lr=0.02, eps=1e-8, beta1=0.9, beta2=0.999, weight_decay=0.0, step=1)
    # pooled: two slots (h1, h2) over the one hist table, mean pooling, padding id 0 filtered
    slots = [dict(rows=400, weights_offset=0, dim=32, dtype="fp32", pooling="mean", row_bytes=0, out_offset=0),
             dict(rows=400, weights_offset=0, dim=32, dtype="fp32", pooling="mean", row_bytes=0, out_offset=32)]
    vals = np.concatenate([h1.reshape(-1), h2.reshape(-1)])
    offs = o.offsets_np(np.full(2 * B, L))
    m1, m2 = np.zeros_like(hist0), np.zeros_like(hist0)
    o.tbe_backward(slots, vals, offs, B, np.concatenate([G["h1"], G["h2"]], 1), padding_idx=0, weights=hist0,
                   m1=m1, m2=m2, **hp)
    _close(emb.ebc._store.flat.cpu().numpy().view(np.float32), hist0, "pooled table")
    assert np.array_equal(emb.ebc._store.flat.cpu().numpy().view(np.float32)[:32], row0)  # padding row 0 untouched
    # unpooled: one-id bags of item (B) and seq (B * 5) on the item table, as side-by-side slots
    n = B * 5
    slots = [dict(rows=300, weights_offset=0, dim=16, dtype="fp32", pooling="sum", row_bytes=0, out_offset=c)
             for c in (0, 16)]
    vals = np.concatenate([item, seq.reshape(-1)])
    lens = np.concatenate([(np.arange(n) < B), np.ones(n, bool)]).astype(np.int64)
    grad = np.zeros((n, 32), np.float32)
    grad[:B, :16] = G["item"]
    grad[:, 16:] = G["seq"].reshape(n, 16)
    m1, m2 = np.zeros_like(item0), np.zeros_like(item0)
    o.tbe_backward(slots, vals, o.offsets_np(lens), n, grad, weights=item0, m1=m1, m2=m2, **hp)
    _close(emb.ec._store.flat.cpu().numpy().view(np.float32), item0, "unpooled table")
