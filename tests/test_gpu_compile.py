"""The compile and trace paths the reference relies on: it compiles every OneTransBlock with
``torch.compile(block, fullgraph=False, dynamic=True)`` (primus_dlrm/models/onetrans.py:382-390) and
TorchRec's pipeline runs ``torch.fx.symbolic_trace`` over the model's ``forward(batch)``
(primus_dlrm/models/base.py:15-39).

* ``torch.library.opcheck`` on every ``pdm::`` op (schema, fake kernel, autograd registration, AOT dispatch).
* The drop-in modules under ``torch.compile(fullgraph=True, dynamic=True)`` with no graph break
  (``torch._dynamo.explain``) and outputs equal to eager, bit for bit (the compiled graph calls the same
  kernels on the same inputs).
* Training through the compiled lookups: the fused optimizer update is the ops' registered backward, so
  compiled ``loss.backward()`` updates the tables exactly as eager does, learning-rate changes included.
* An FX trace of a model forward with the embedding modules as leaves (as TorchRec's tracer treats its
  embedding modules) runs the same kernels.
"""
import copy

import numpy as np
import pytest
import torch
from torch.distributed.optim import _apply_optimizer_in_backward

from oracle import onetrans as ot

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _fresh_dynamo():
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def _explain(fn, *args, **kwargs):
    ex = torch._dynamo.explain(fn)(*args, **kwargs)
    print(f"graphs {ex.graph_count}, graph breaks {ex.graph_break_count}", flush=True)
    for b in ex.break_reasons:
        print("  break:", b.reason, flush=True)
    return ex


def _block(pdm, dev, D=128, F=512, n_ns=4, H=2, seed=3):
    blk = pdm.OneTransBlock(D, H, n_ns, ffn_mult=F // D).to(dev).eval()
    w = ot.random_weights(D, F, n_ns, std=0.05, seed=seed, norm_std=0.1)
    with torch.no_grad():
        blk.norm1.weight.copy_(w["norm1"])
        blk.attn.s_qkv.weight.copy_(w["s_qkv"])
        blk.attn.ns_qkv_weight.copy_(w["ns_qkv"])
        blk.attn.out_proj.weight.copy_(w["out"])
        blk.norm2.weight.copy_(w["norm2"])
        blk.ffn.s_w1.weight.copy_(w["s_w1"])
        blk.ffn.s_w2.weight.copy_(w["s_w2"])
        blk.ffn.ns_w1.copy_(w["ns_w1"])
        blk.ffn.ns_w2.copy_(w["ns_w2"])
    return blk


def _block_args(pdm, dev, B, kv, q_len, n_ns, D, seed):
    x = torch.randn(B, kv, D, generator=torch.Generator().manual_seed(seed)).to(dev)
    return x, pdm.build_pyramid_mask(q_len, kv, dev), q_len, kv - n_ns


# ---------------------------------------------------------------------------
# opcheck
# ---------------------------------------------------------------------------

def _opcheck(op, args):
    print(f"opcheck {op}", flush=True)
    res = torch.library.opcheck(op, args)
    bad = {k: v for k, v in res.items() if v != "SUCCESS"}
    assert not bad, bad


def _collections(pdm, dev, tag=None):
    bag_cfgs = [pdm.EmbeddingBagConfig(300, 32, "b0", pdm.DataType.FP32, ["a", "b"], pdm.PoolingType.SUM),
                pdm.EmbeddingBagConfig(200, 16, "b1", pdm.DataType.FP32, ["c"], pdm.PoolingType.MEAN)]
    ec_cfgs = [pdm.EmbeddingConfig(400, 32, "item", pdm.DataType.FP32, ["lp_item", "sk_item", "cand"]),
               pdm.EmbeddingConfig(90, 16, "artist", pdm.DataType.FP32, ["lp_artist", "sk_artist"])]
    torch.manual_seed(11)
    ebc = pdm.EmbeddingBagCollection(bag_cfgs, device=dev)
    ec = pdm.EmbeddingCollection(ec_cfgs, device=dev)
    if tag is not None:
        for p in list(ebc.parameters()) + list(ec.parameters()):
            _apply_optimizer_in_backward(tag[0], [p], tag[1])
    sg = pdm.SequenceGather(ec, {"lp": ["lp_item", "lp_artist"], "sk": ["sk_item", "sk_artist"]},
                            {"lp": 12, "sk": 6})
    return ebc, ec, sg


def _kjt_inputs(dev, B, seed, rows=(300, 300, 200)):
    g = np.random.default_rng(seed)
    lens = g.integers(0, 7, len(rows) * B)
    vals = np.concatenate([g.integers(0, r, int(lens[k * B:(k + 1) * B].sum())) for k, r in enumerate(rows)])
    return torch.from_numpy(vals).to(dev), torch.from_numpy(lens).to(dev)


def _seq_batch(dev, B, seed):
    g = np.random.default_rng(seed)
    batch = {}
    for pool, mean in (("lp", 8.0), ("sk", 3.0)):
        ln = g.poisson(mean, B)
        it = g.integers(0, 400, int(ln.sum()))
        batch[f"{pool}_item"], batch[f"{pool}_artist"] = torch.from_numpy(it), torch.from_numpy(it % 90)
        batch[f"{pool}_item__lengths"] = batch[f"{pool}_artist__lengths"] = torch.from_numpy(ln)
    return {k: v.to(dev) for k, v in batch.items()}


def test_opcheck_lookup_ops(pdm, dev):
    ebc, ec, sg = _collections(pdm, dev)
    vals, lens = _kjt_inputs(dev, 9, 1)
    offs = torch.nn.functional.pad(lens.cumsum(0), (1, 0))
    frozen = [w.detach() for w in (ebc.embedding_bags["b0"].weight, ebc.embedding_bags["b1"].weight)]
    plan = ebc._get_plan()
    for code, padding in ((0, -1), (1, 5)):
        _opcheck(torch.ops.pdm.tbe_pooled_fwd.default,
                 (ebc._store.flat, frozen, vals, offs, plan.plan_id, plan.num_slots, ebc._total_dim, code, padding,
                  ebc._owner_id))
    _opcheck(torch.ops.pdm.kjt_permute.default, (vals, offs, 3, 9, [2, 0, 0]))
    ec_tabs = [w.detach() for w in (ec.embeddings["item"].weight, ec.embeddings["artist"].weight)]
    ids = [vals[:20].clone(), (vals[20:31] % 90).clone()]
    _opcheck(torch.ops.pdm.ec_lookup.default, (ec._store.flat, ec_tabs, ids, [0, 1], ec._owner_id))
    batch = _seq_batch(dev, 7, 2)
    seq_ids = [batch[f] for f in ("lp_item", "lp_artist", "sk_item", "sk_artist")]
    seq_offs = [torch.nn.functional.pad(batch[f"{p}_item__lengths"].cumsum(0), (1, 0)) for p in ("lp", "sk")]
    _opcheck(torch.ops.pdm.seq_gather_fwd.default,
             (ec._store.flat, ec_tabs, seq_ids, seq_offs, [12, 6], sg.pad_mode, sg.align, sg._owner_id))
    keys = [torch.randint(0, 1 << 40, (33,), device=dev), torch.tensor([7], device=dev),
            torch.randint(-50, 50, (33,), device=dev)]
    _opcheck(torch.ops.pdm.cross_hash_fwd.default, (keys, 1000003, 5))


def test_opcheck_fused_update_ops(pdm, dev):
    """The mutating update ops (the lookups' backward) declare exactly the collection buffer as mutated."""
    ebc, ec, sg = _collections(pdm, dev, tag=(torch.optim.Adam, {"lr": 0.01}))
    vals, lens = _kjt_inputs(dev, 9, 3)
    offs = torch.nn.functional.pad(lens.cumsum(0), (1, 0))
    grad = torch.randn(9, ebc._total_dim, device=dev)
    _opcheck(torch.ops.pdm.tbe_fused_update.default, (ebc._store.flat, vals, offs, grad, 3, -1, ebc._owner_id))
    ids = [vals[:20].clone(), (vals[20:31] % 90).clone()]
    grads = [torch.randn(20, 32, device=dev), torch.randn(11, 16, device=dev)]
    _opcheck(torch.ops.pdm.ec_fused_update.default, (ec._store.flat, ids, grads, [0, 1], ec._owner_id))
    batch = _seq_batch(dev, 7, 4)
    seq_ids = [batch[f] for f in ("lp_item", "lp_artist", "sk_item", "sk_artist")]
    seq_offs = [torch.nn.functional.pad(batch[f"{p}_item__lengths"].cumsum(0), (1, 0)) for p in ("lp", "sk")]
    g_out = torch.randn(7, 18, 48, device=dev)
    _opcheck(torch.ops.pdm.seq_fused_update.default,
             (ec._store.flat, seq_ids, seq_offs, [12, 6], g_out, sg._owner_id))


def test_opcheck_block_and_tokenizer_ops(pdm, dev):
    blk = _block(pdm, dev)
    x, _, q_len, _ = _block_args(pdm, dev, 3, 24, 14, 4, 128, 5)
    bf = lambda t: t.detach().to(torch.bfloat16).contiguous()  # noqa: E731
    _opcheck(torch.ops.pdm.onetrans_block_fwd.default,
             (x, blk.norm1.weight.detach().float(), bf(blk.attn.s_qkv.weight), bf(blk.attn.ns_qkv_weight),
              bf(blk.attn.out_proj.weight), blk.norm2.weight.detach().float(), bf(blk.ffn.s_w1.weight),
              bf(blk.ffn.s_w2.weight), bf(blk.ffn.ns_w1), bf(blk.ffn.ns_w2), 2, q_len))
    stack = pdm.OneTransStack(128, 2, 4, 3, schedule=[20, 12, 4]).to(dev).eval()
    x = torch.randn(2, 24, 128, device=dev)
    _opcheck(torch.ops.pdm.onetrans_stack_fwd.default,
             (x, [t for blk in stack.blocks for t in blk.kernel_weights()], 2, [20, 12, 4]))
    tables = [pdm.EmbeddingConfig(500, 128, "item", pdm.DataType.BF16, ["lp_item"]),
              pdm.EmbeddingConfig(60, 64, "artist", pdm.DataType.BF16, ["lp_artist"])]
    ec = pdm.EmbeddingCollection(tables, device=dev)
    tok = pdm.SequentialTokenizer(192, 128, max_len=16).to(dev)
    w1, b1, w2, b2, pos = tok.kernel_weights()
    g = np.random.default_rng(8)
    ln = g.integers(0, 12, 5)
    it = torch.from_numpy(g.integers(0, 500, int(ln.sum()))).to(dev)
    off = torch.nn.functional.pad(torch.from_numpy(ln).to(dev).cumsum(0), (1, 0))
    tabs = [ec.embeddings["item"].weight.detach(), ec.embeddings["artist"].weight.detach()]
    _opcheck(torch.ops.pdm.seq_tokenize_fwd.default,
             (tabs, [it, it % 60], [off], [10], [w1], [b1], [w2], [b2], [pos], pdm._lib.PDM_PAD_ROW0,
              pdm._lib.PDM_ALIGN_RIGHT))


# ---------------------------------------------------------------------------
# OneTransBlock / OneTransStack
# ---------------------------------------------------------------------------

def test_block_compiles_fullgraph_dynamic(pdm, dev):
    blk = _block(pdm, dev)
    args = _block_args(pdm, dev, 4, 40, 24, 4, 128, 1)
    ex = _explain(blk, *args)
    assert ex.graph_break_count == 0 and ex.graph_count == 1
    torch._dynamo.reset()
    cblk = torch.compile(blk, fullgraph=True, dynamic=True)
    with torch.no_grad():
        for B, kv, q_len, seed in ((4, 40, 24, 1), (7, 33, 33, 2), (2, 50, 10, 3)):
            print(f"compiled block B={B} kv={kv} q_len={q_len}", flush=True)
            a = _block_args(pdm, dev, B, kv, q_len, 4, 128, seed)
            got, want = cblk(*a), blk(*a)
            torch.cuda.synchronize()
            assert got.shape == (B, q_len, 128) and torch.equal(got, want)


def test_block_compiled_like_the_reference(pdm, dev):
    """The reference's backbone loop (onetrans.py:568-582) over blocks compiled as OneTransModel.apply_compile
    does (fullgraph=False, dynamic=True): the same output as OneTransStack's one-call stack."""
    D, n_ns = 128, 4
    schedule = [36, 20, 8]
    stack = pdm.OneTransStack(D, 2, n_ns, 3, schedule=schedule).to(dev).eval()
    for i, blk in enumerate(stack.blocks):
        blk.load_state_dict(_block(pdm, dev, seed=20 + i).state_dict())
    compiled = [torch.compile(blk, fullgraph=False, dynamic=True) for blk in stack.blocks]
    with torch.no_grad():
        for B in (3, 6):
            x = torch.randn(B, 36 + n_ns, D, device=dev)
            want = stack(x)
            h = x
            for blk, q_s in zip(compiled, schedule):
                q_len, kv_len = q_s + n_ns, h.shape[1]
                h = blk(h, mask=pdm.build_pyramid_mask(q_len, kv_len, dev), q_len=q_len, n_s_tokens=kv_len - n_ns)
            torch.cuda.synchronize()
            assert torch.equal(h, want)


def test_stack_compiles_fullgraph(pdm, dev):
    D, n_ns = 128, 4
    stack = pdm.OneTransStack(D, 2, n_ns, 3, schedule=[36, 20, 8]).to(dev).eval()
    x = torch.randn(5, 36 + n_ns, D, device=dev)
    ex = _explain(stack, x)
    assert ex.graph_break_count == 0
    torch._dynamo.reset()
    cstack = torch.compile(stack, fullgraph=True, dynamic=True)
    with torch.no_grad():
        for B in (5, 9):
            xb = torch.randn(B, 36 + n_ns, D, device=dev)
            assert torch.equal(cstack(xb), stack(xb))


def test_block_rejects_bf16_residual_stream(pdm, dev):
    """A bf16 residual stream (the reference without positional embeddings) is rejected with a TypeError that
    names the reason, eagerly and under torch.compile."""
    blk = _block(pdm, dev)
    x, mask, q_len, n_s = _block_args(pdm, dev, 2, 20, 20, 4, 128, 4)
    with pytest.raises(TypeError, match="must be fp32"):
        blk(x.to(torch.bfloat16), mask, q_len, n_s)
    with pytest.raises(Exception, match="must be fp32"):
        torch.compile(blk, dynamic=True)(x.to(torch.bfloat16), mask, q_len, n_s)


# ---------------------------------------------------------------------------
# Lookups: inference and training through the compiled modules
# ---------------------------------------------------------------------------

def test_ebc_compiles_inference(pdm, dev):
    ebc, _, _ = _collections(pdm, dev)
    for p in ebc.parameters():
        p.requires_grad_(False)

    def run(kjt):
        return ebc(kjt).values()

    vals, lens = _kjt_inputs(dev, 16, 5)
    kjt = pdm.KeyedJaggedTensor.from_lengths_sync(["a", "b", "c"], vals, lens)
    ex = _explain(run, kjt)
    assert ex.graph_break_count == 0
    # keys in another order: the permute op runs inside the graph
    vals2, lens2 = _kjt_inputs(dev, 16, 6, rows=(200, 300, 300))
    kjt2 = pdm.KeyedJaggedTensor.from_lengths_sync(["c", "a", "b"], vals2, lens2)
    ex = _explain(run, kjt2)
    assert ex.graph_break_count == 0
    torch._dynamo.reset()
    crun = torch.compile(run, fullgraph=True, dynamic=True)
    for k in (kjt, kjt2):
        assert torch.equal(crun(k), run(k))


def _train(fwd, fos, batches, lrs, seed):
    """Forward + backward per batch with a random linear loss; ``fos`` are the fused optimizers whose
    learning rate follows ``lrs``."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    for batch, lr in zip(batches, lrs):
        for fo in fos():
            fo.param_groups[0]["lr"] = lr
        r = fwd(batch, padding_idx=0)
        loss = sum((r[k].float() * torch.randn(r[k].shape, generator=gen).to(r[k].device)).sum() for k in sorted(r))
        loss.backward()
    torch.cuda.synchronize()


def test_torchrec_embeddings_trains_compiled(pdm, dev):
    """TorchRecEmbeddings (the reference's tensor-in/tensor-out wrapper) compiled fullgraph: forward and the
    fused-optimizer backward match eager over three steps with a changing learning rate."""
    specs = [pdm.EmbeddingTableConfig("hist", ["h1", "h2"], 400, 32, "mean"),
             pdm.EmbeddingTableConfig("item", ["item", "seq"], 300, 16, "none")]
    torch.manual_seed(2)
    eager = pdm.TorchRecEmbeddings(specs, device=dev, scalar_feature_names={"item"})
    comp = copy.deepcopy(eager)
    assert comp.ebc._owner_id != eager.ebc._owner_id and comp.ebc._plan is not eager.ebc._plan
    assert torch.equal(comp.ebc._store.flat, eager.ebc._store.flat)
    for m in (eager, comp):
        for p in m.parameters():
            _apply_optimizer_in_backward(torch.optim.Adam, [p], {"lr": 0.02})
    g = np.random.default_rng(4)
    B, L = 24, 6
    batches = []
    for _ in range(3):
        h1 = g.integers(0, 400, (B, L))
        h1[g.random((B, L)) < 0.3] = 0
        batches.append({k: torch.from_numpy(v).to(dev) for k, v in
                        dict(h1=h1, h2=g.integers(0, 400, (B, L)), item=g.integers(0, 300, B),
                             seq=g.integers(0, 300, (B, 5))).items()})
    ex = _explain(comp, batches[0])
    assert ex.graph_break_count == 0
    torch._dynamo.reset()
    cfwd = torch.compile(comp, fullgraph=True, dynamic=True)
    with torch.no_grad():
        want, got = comp(batches[0]), cfwd(batches[0])
        assert all(torch.equal(got[k], want[k]) for k in want)
    lrs = [0.02, 0.005, 0.03]
    init = (comp.ebc._store.flat.clone(), comp.ec._store.flat.clone())
    _train(eager, lambda: (eager.ebc.fused_optimizer, eager.ec.fused_optimizer), batches, lrs, 9)
    _train(cfwd, lambda: (comp.ebc.fused_optimizer, comp.ec.fused_optimizer), batches, lrs, 9)
    for a, b, what in ((eager.ebc._store.flat, comp.ebc._store.flat, "pooled tables"),
                       (eager.ec._store.flat, comp.ec._store.flat, "unpooled tables"),
                       (eager.ebc.fused_optimizer.momentum1, comp.ebc.fused_optimizer.momentum1, "pooled m1"),
                       (eager.ec.fused_optimizer.momentum2, comp.ec.fused_optimizer.momentum2, "unpooled m2")):
        print(what, flush=True)
        f32 = lambda t: t.view(torch.float32) if t.dtype == torch.uint8 else t  # noqa: E731
        torch.testing.assert_close(f32(b), f32(a), rtol=1e-6, atol=1e-9, msg=what)
    assert not torch.equal(init[0], comp.ebc._store.flat) and not torch.equal(init[1], comp.ec._store.flat)
    assert eager.ebc.fused_optimizer.iter == comp.ebc.fused_optimizer.iter == 3


def test_sequence_gather_trains_compiled(pdm, dev):
    _, _, sg_e = _collections(pdm, dev, tag=(torch.optim.Adam, {"lr": 0.01}))
    _, _, sg_c = _collections(pdm, dev, tag=(torch.optim.Adam, {"lr": 0.01}))
    assert torch.equal(sg_e.ec._store.flat, sg_c.ec._store.flat)
    batches = [_seq_batch(dev, 10, 20 + i) for i in range(2)]
    ex = _explain(sg_c, batches[0])
    assert ex.graph_break_count == 0
    torch._dynamo.reset()
    csg = torch.compile(sg_c, fullgraph=True, dynamic=True)
    with torch.no_grad():
        a, ma = csg(batches[1])
        b, mb = sg_c(batches[1])
    assert torch.equal(a, b) and torch.equal(ma, mb)
    gen = [torch.Generator(device="cpu").manual_seed(1) for _ in range(2)]
    for step in range(2):
        for fwd, gg in ((sg_e, gen[0]), (csg, gen[1])):
            tok, _ = fwd(batches[step])
            (tok * torch.randn(tok.shape, generator=gg).to(dev)).sum().backward()
    torch.cuda.synchronize()
    torch.testing.assert_close(sg_c.ec._store.flat.view(torch.float32), sg_e.ec._store.flat.view(torch.float32),
                               rtol=1e-6, atol=1e-9)


def test_untagged_tables_raise_at_compiled_backward(pdm, dev):
    ebc, _, _ = _collections(pdm, dev)
    vals, lens = _kjt_inputs(dev, 8, 7)
    kjt = pdm.KeyedJaggedTensor.from_lengths_sync(["a", "b", "c"], vals, lens)
    out = torch.compile(lambda k: ebc(k).values(), fullgraph=True, dynamic=True)(kjt)
    assert out.requires_grad
    with pytest.raises(NotImplementedError, match="in-backward optimizer"):
        out.sum().backward()


# ---------------------------------------------------------------------------
# FX symbolic trace of a model forward(batch)
# ---------------------------------------------------------------------------

def test_fx_trace_model_forward_with_leaf_lookups(pdm, dev):
    """A model in the reference's shape: forward(batch) -> tokens from the S-token gather, then the pyramid
    stack with the default schedule (pyramid_schedule is wrapped, as the reference wraps it).  Traced by an FX
    tracer that keeps the embedding modules as leaves; the GraphModule calls the stack op directly and
    reproduces the eager output."""
    D, n_ns = 128, 4
    _, ec, sg = _collections(pdm, dev)

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.sg = sg
            self.proj = torch.nn.Linear(48, D).to(dev)
            self.ns = torch.nn.Parameter(torch.randn(n_ns, D, device=dev) * 0.1)
            self.stack = pdm.OneTransStack(D, 2, n_ns, 3)

        def forward(self, batch):
            raw, _ = self.sg(batch)
            s_tok = self.proj(raw)
            x = torch.cat([s_tok, self.ns.expand(s_tok.shape[0], -1, -1)], dim=1)
            return self.stack(x)

    model = Model().to(dev).eval()
    for p in ec.parameters():
        p.requires_grad_(False)

    class LeafTracer(torch.fx.Tracer):
        def is_leaf_module(self, m, qualname):
            return isinstance(m, (pdm.SequenceGather, pdm.EmbeddingCollection, pdm.EmbeddingBagCollection)) or \
                super().is_leaf_module(m, qualname)

    graph = LeafTracer().trace(model)
    gm = torch.fx.GraphModule(model, graph)
    targets = [str(n.target) for n in graph.nodes if n.op in ("call_function", "call_module")]
    print(targets, flush=True)
    assert "sg" in targets and sum("onetrans_stack_fwd" in t for t in targets) == 1
    with torch.no_grad():
        for seed in (30, 31):
            batch = _seq_batch(dev, 6, seed)
            assert torch.equal(gm(batch), model(batch))
