"""GPU parity of the fused S-token gather + SequentialTokenizer (pdm_seq_tokenize_fwd) against the oracle
(``onetrans.seq_tokenize``: the pinned sequence gather, then the autocast tokenizer of
primus_dlrm/models/onetrans.py:238-257 per pool).

Tolerance (bf16 autocast): the kernel and the oracle sum in different orders, so a value can land on the
other side of a bf16 rounding boundary, in the output or in a hidden unit (which moves an output by at most
one ulp of that unit times |w2|).  Every element must satisfy |got - want| <= 2^-7 (|y| + |h| . |w2|^T)
(y: the token before pos, h: the hidden row), fewer than 2% of them may differ at all, and the relative
error norm must stay below 2e-2.  The mask is bit-exact, and padding slots at one position are bitwise
equal across samples (their MLP row is computed once per pool)."""
import numpy as np
import pytest
import torch

from oracle import onetrans as ot
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def _inputs(g, B, pools, specs, dtype, bad_id=False):
    tabs = []
    for r, d in specs:
        w = g.normal(0, 0.5, (r, d)).astype(np.float32)
        tabs.append(o.f32_to_bf16_bits(w).reshape(r, d) if dtype == "bf16" else w)
    ids, offs = [], []
    for L, mean in pools:
        ln = g.poisson(mean, B) if B else np.zeros(0, np.int64)
        n = int(ln.sum())
        items = g.integers(0, specs[0][0], n)
        ids.append([items] + [items % r for r, _ in specs[1:]])
        offs.append(o.offsets_np(ln))
    if bad_id:
        ids[0][-1][len(ids[0][-1]) - 1] = specs[-1][0] + 3
    return tabs, ids, offs


def _dev_tables(tabs, dev):
    out = []
    for t in tabs:
        if t.dtype == np.uint16:
            out.append(torch.from_numpy(t.view(np.int16)).view(torch.bfloat16).to(dev))
        else:
            out.append(torch.from_numpy(t).to(dev))
    return out


def _check(got, tabs, ids, offs, max_len, ws, pad_mode, align, mask=None):
    want, wmask = ot.seq_tokenize(tabs, ids, offs, max_len, ws, pad_mode=pad_mode, align=align)
    raw, _ = o.seq_gather(tabs, ids, offs, max_len, pad_mode=pad_mode, align=align)
    if raw.dtype == np.uint16:
        raw = (raw.astype(np.uint32) << 16).view(np.float32)
    raw = torch.from_numpy(np.ascontiguousarray(raw))
    if mask is not None:
        assert np.array_equal(mask.cpu().numpy(), wmask)
    num = ot._Num("autocast")
    s0 = 0
    for p, L in enumerate(max_len):
        if L == 0:
            continue
        w = ws[p]
        h = num.round(torch.nn.functional.gelu(ot._lin_bias(raw[:, s0:s0 + L], w["w1"], w["b1"], num)))
        y = ot._lin_bias(h, w["w2"], w["b2"], num)
        mag = y.abs() + h.abs() @ w["w2"].abs().T
        g_p, w_p = got[:, s0:s0 + L], want[:, s0:s0 + L]
        diff = (g_p - w_p).abs()
        assert bool((diff <= 2.0 ** -7 * mag + 1e-6).all()), f"pool {p}: max excess {(diff - 2.0 ** -7 * mag).max()}"
        assert (diff > 0).float().mean().item() < 0.02
        rel = ((g_p - w_p).norm() / w_p.norm().clamp_min(1e-30)).item()
        assert rel < 2e-2, rel
        # padding slots: one MLP row per pool, so equal bits at equal positions
        pm = wmask[:, s0:s0 + L] == 0
        for l in range(L):
            bs = np.nonzero(pm[:, l])[0]
            if len(bs) > 1:
                assert torch.equal(g_p[bs, l], g_p[bs[:1], l].expand(len(bs), -1))
        s0 += L


CASES = [
    # name, specs [(rows, dim)], pools [(max_len, mean)], d, dtype, pad, align, pos
    ("k384_d256_bf16", [(3000, 256), (300, 64), (500, 64)], [(48, 30), (16, 12), (32, 20)], 256, "bf16", 0, 0, True),
    ("k128_d128_fp32", [(400, 64), (90, 64)], [(20, 8), (9, 12)], 128, "fp32", 0, 0, True),
    ("k192_d256_zero_left", [(700, 128), (60, 64)], [(24, 10), (40, 30)], 256, "bf16", 1, 1, True),
    ("k256_d128_nopos", [(512, 256)], [(33, 20)], 128, "bf16", 0, 0, False),
    ("k384_d128_fp32_zero", [(800, 128), (300, 128), (200, 128)], [(12, 6), (20, 25)], 128, "fp32", 1, 0, True),
    # the reference's large OneTrans config: item / artist / album of dim 64 per event, d_model 384
    ("k192_d384_reference_large", [(2000, 64), (300, 64), (500, 64)], [(40, 25), (24, 10), (32, 16)], 384, "bf16",
     0, 0, True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_tokenize_matches_oracle(pdm, dev, case):
    name, specs, pools, d, dtype, pad_mode, align, use_pos = case
    g = np.random.default_rng(len(name))
    B = 37
    K = sum(dm for _, dm in specs)
    tabs, ids, offs = _inputs(g, B, pools, specs, dtype)
    max_len = [L for L, _ in pools]
    ws = [ot.random_tokenizer_weights(K, d, L + 3, seed=i, pos=use_pos) for i, (L, _) in enumerate(pools)]
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) if v is not None else None
           for k, v in w.items()} for w in ws]
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out, mask = pdm.ops.seq_tokenize_raw(_dev_tables(tabs, dev), [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
                                         [torch.from_numpy(x).to(dev) for x in offs], max_len, wd,
                                         pad_mode=pad_mode, align=align, err_flag=err)
    torch.cuda.synchronize()
    assert err.item() == 0
    _check(out.cpu(), tabs, ids, offs, max_len, ws, pad_mode, align, mask)


def test_many_passes_and_long_pools(pdm, dev):
    """~45k real tokens: hundreds of passes over the persistent workgroups, pools longer than a pass."""
    g = np.random.default_rng(5)
    specs, pools, d = [(20000, 256), (2000, 64), (3000, 64)], [(200, 150), (64, 40), (128, 80)], 256
    B = 160
    tabs, ids, offs = _inputs(g, B, pools, specs, "bf16")
    max_len = [L for L, _ in pools]
    ws = [ot.random_tokenizer_weights(384, d, 256, seed=10 + i) for i in range(3)]
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()} for w in ws]
    out, mask = pdm.ops.seq_tokenize_raw(_dev_tables(tabs, dev), [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
                                         [torch.from_numpy(x).to(dev) for x in offs], max_len, wd)
    torch.cuda.synchronize()
    _check(out.cpu(), tabs, ids, offs, max_len, ws, 0, 0, mask)


def test_writes_into_block_input_rows(pdm, dev):
    """out = the leading S rows of a [B, S + n_ns, d] buffer: NS rows untouched; a second call reuses the
    workspace (no initialisation needed)."""
    g = np.random.default_rng(9)
    specs, pools, d, n_ns = [(300, 64), (40, 64)], [(10, 5), (6, 4)], 128, 3
    B = 11
    tabs, ids, offs = _inputs(g, B, pools, specs, "bf16")
    max_len = [10, 6]
    ws = [ot.random_tokenizer_weights(128, d, 16, seed=i) for i in range(2)]
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()} for w in ws]
    buf = torch.full((B, 16 + n_ns, d), 7.0, device=dev)
    work = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    args = (_dev_tables(tabs, dev), [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
            [torch.from_numpy(x).to(dev) for x in offs], max_len, wd)
    out, mask = pdm.ops.seq_tokenize_raw(*args, out=buf, workspace=work)
    first = buf.clone()
    pdm.ops.seq_tokenize_raw(*args, out=buf, workspace=work)
    torch.cuda.synchronize()
    assert torch.equal(first, buf)
    assert bool((buf[:, 16:] == 7.0).all())
    _check(buf[:, :16].cpu(), tabs, ids, offs, max_len, ws, 0, 0, mask)


def test_captured_in_a_graph(pdm, dev):
    """The padding fill runs on the library's second stream beside the MLP (fork after the scan, join at the
    end); under HIP graph capture both streams' kernels become nodes of the graph.  Every replay, with eager
    calls on other inputs in between, must give the eager output bit for bit."""
    g = np.random.default_rng(21)
    specs, pools, d = [(900, 256), (90, 64), (120, 64)], [(64, 40), (24, 12), (40, 20)], 256
    B = 200
    args = []
    for seed in (0, 1):
        tabs, ids, offs = _inputs(np.random.default_rng(seed), B, pools, specs, "bf16")
        args.append((_dev_tables(tabs, dev), [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
                     [torch.from_numpy(x).to(dev) for x in offs]))
    max_len = [L for L, _ in pools]
    ws = [ot.random_tokenizer_weights(384, d, 64, seed=30 + i) for i in range(3)]
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()} for w in ws]
    out = torch.empty(B, sum(max_len), d, device=dev)
    other = torch.empty_like(out)
    work = pdm.ops.seq_tokenize_workspace(*args[0], max_len, d)
    work2 = torch.empty_like(work)
    pdm.ops.seq_tokenize_raw(*args[0], max_len, wd, out=out, workspace=work)  # eager first: the side stream exists
    torch.cuda.synchronize()
    want = out.clone()
    out.fill_(-1.0)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            pdm.ops.seq_tokenize_raw(*args[0], max_len, wd, out=out, workspace=work)
    torch.cuda.synchronize()
    for r in range(3):
        out.fill_(-1.0)
        pdm.ops.seq_tokenize_raw(*args[1], max_len, wd, out=other, workspace=work2)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}"


_FIRST_CALL_CAPTURED = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, {root!r})
import __graft_entry__
pdm = __graft_entry__.pdm_import()
from oracle import onetrans as ot
dev = torch.device("cuda:0")
g = np.random.default_rng(3)
B, specs, pools, d = 90, [(500, 256), (60, 64), (80, 64)], [(40, 25), (16, 8), (24, 12)], 256
tabs = [torch.from_numpy(g.normal(0, 0.5, (r, c)).astype(np.float32)).to(torch.bfloat16).to(dev) for r, c in specs]
ids, offs = [], []
for L, mean in pools:
    ln = g.poisson(mean, B)
    it = g.integers(0, specs[0][0], int(ln.sum()))
    ids.append([torch.from_numpy(a).to(dev) for a in [it] + [it % r for r, _ in specs[1:]]])
    offs.append(torch.from_numpy(np.concatenate([[0], np.cumsum(ln)]).astype(np.int64)).to(dev))
max_len = [L for L, _ in pools]
ws = [ot.random_tokenizer_weights(384, d, 48, seed=40 + i) for i in range(3)]
wd = [{{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()}} for w in ws]
out = torch.empty(B, sum(max_len), d, device=dev)
work = pdm.ops.seq_tokenize_workspace(tabs, ids, offs, max_len, d)
stream = torch.cuda.Stream()
stream.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(stream):
    with torch.cuda.graph(graph, stream=stream):  # the library's first tokenizer call: inside the capture
        pdm.ops.seq_tokenize_raw(tabs, ids, offs, max_len, wd, out=out, workspace=work)
torch.cuda.synchronize()
out.fill_(-1.0)
graph.replay()
torch.cuda.synchronize()
captured = out.clone()
eager = torch.empty_like(out)
for _ in range(2):  # eager calls: the first makes the second stream, both use it
    pdm.ops.seq_tokenize_raw(tabs, ids, offs, max_len, wd, out=eager, workspace=work)
    torch.cuda.synchronize()
    assert torch.equal(eager, captured)
graph.replay()
torch.cuda.synchronize()
assert torch.equal(out, captured)
print("FIRST_CALL_CAPTURED_OK")
"""


def test_first_call_inside_a_capture(dev):
    """In a fresh process whose first tokenizer call is captured into a graph (before the library has its
    second stream, which is made outside captures only), the call runs on the capturing stream alone; the
    eager calls after it make the second stream and give the graph's output bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED.format(root=root)], capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0 and "FIRST_CALL_CAPTURED_OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]


def test_bad_ids_and_offsets_raise_the_flag(pdm, dev):
    g = np.random.default_rng(4)
    specs, pools, d = [(100, 64), (30, 64)], [(8, 5)], 128
    B = 6
    tabs, ids, offs = _inputs(g, B, pools, specs, "bf16", bad_id=True)
    ws = [ot.random_tokenizer_weights(128, d, 8, seed=1)]
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()} for w in ws]
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out, mask = pdm.ops.seq_tokenize_raw(_dev_tables(tabs, dev), [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
                                         [torch.from_numpy(x).to(dev) for x in offs], [8], wd, err_flag=err)
    torch.cuda.synchronize()
    assert err.item() == 1
    # the bad id's feature reads zeros, as in the gather
    _check(out.cpu(), tabs, ids, offs, [8], ws, 0, 0, mask)
    # offsets past the ids: the sample counts as empty and the flag is raised
    bad_offs = [offs[0].copy()]
    bad_offs[0][-1] = len(ids[0][0]) + 4
    err.zero_()
    out2, mask2 = pdm.ops.seq_tokenize_raw(_dev_tables(tabs, dev),
                                           [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
                                           [torch.from_numpy(x).to(dev) for x in bad_offs], [8], wd, err_flag=err)
    torch.cuda.synchronize()
    assert err.item() == 1
    assert int(mask2[-1].sum().item()) == 0


def test_empty_batch_and_empty_pool(pdm, dev):
    g = np.random.default_rng(3)
    specs, d = [(50, 64), (20, 64)], 128
    ws = [ot.random_tokenizer_weights(128, d, 8, seed=i) for i in range(2)]
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()} for w in ws]
    tabs, ids, offs = _inputs(g, 0, [(8, 3), (0, 2)], specs, "bf16")
    out, mask = pdm.ops.seq_tokenize_raw(_dev_tables(tabs, dev), [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
                                         [torch.from_numpy(x).to(dev) for x in offs], [8, 0], wd)
    assert out.shape == (0, 8, d)
    tabs, ids, offs = _inputs(g, 5, [(8, 3), (0, 2)], specs, "bf16")
    wd[1] = {k: None for k in wd[1]}
    out, mask = pdm.ops.seq_tokenize_raw(_dev_tables(tabs, dev), [[torch.from_numpy(a).to(dev) for a in r] for r in ids],
                                         [torch.from_numpy(x).to(dev) for x in offs], [8, 0], [wd[0], wd[1]])
    torch.cuda.synchronize()
    _check(out.cpu(), tabs, ids, offs, [8, 0], ws, 0, 0, mask)


def test_unsupported_width_is_an_error(pdm, dev):
    tabs = [torch.zeros(10, 72, dtype=torch.bfloat16, device=dev)]
    ids = [[torch.zeros(3, dtype=torch.int64, device=dev)]]
    offs = [torch.tensor([0, 3], dtype=torch.int64, device=dev)]
    w = ot.random_tokenizer_weights(72, 128, 4)
    wd = [{k: (v.to(torch.bfloat16) if k != "pos" else v).contiguous().to(dev) for k, v in w.items()}]
    with pytest.raises(pdm._lib.PdmError):
        pdm.ops.seq_tokenize_raw(tabs, ids, offs, [4], wd)


def _module_weights(tok):
    """The oracle's weight dict from a SequentialTokenizer module (fp32 parameters; the oracle rounds to bf16)."""
    return {"w1": tok.proj[0].weight.detach().cpu(), "b1": tok.proj[0].bias.detach().cpu(),
            "w2": tok.proj[2].weight.detach().cpu(), "b2": tok.proj[2].bias.detach().cpu(),
            "pos": None if tok.pos_emb is None else tok.pos_emb.weight.detach().cpu()}


@pytest.mark.parametrize("raw_dtype", [torch.float32, torch.bfloat16])
def test_sequential_tokenizer_module(pdm, dev, raw_dtype):
    """SequentialTokenizer.forward(raw) (onetrans.py:250-257) against the oracle on the module's parameters."""
    torch.manual_seed(3)
    tok = pdm.SequentialTokenizer(384, 256, max_len=64).to(dev)
    raw = torch.randn(5, 37, 384, device=dev).to(raw_dtype)
    got = tok(raw)
    assert got.dtype == torch.float32 and got.shape == (5, 37, 256)
    w = _module_weights(tok)
    num = ot._Num("autocast")
    rawc = raw.float().cpu()
    want = ot.sequential_tokenizer(rawc, w)
    h = num.round(torch.nn.functional.gelu(ot._lin_bias(rawc, w["w1"], w["b1"], num)))
    y = ot._lin_bias(h, w["w2"], w["b2"], num)
    mag = y.abs() + h.abs() @ num.round(w["w2"]).abs().T
    diff = (got.cpu() - want).abs()
    assert bool((diff <= 2.0 ** -7 * mag + 1e-6).all())
    assert (diff > 0).float().mean().item() < 0.02


def test_fused_sequence_tokenizer_module(pdm, dev):
    """FusedSequenceTokenizer (gather + per-pool tokenizers fused) equals SequenceGather followed by the
    SequentialTokenizer modules bit for bit (the same kernel arithmetic per token), and the oracle within
    the bf16 tolerance."""
    g = np.random.default_rng(21)
    tables = [pdm.EmbeddingConfig(1000, 128, "item", pdm.DataType.BF16, ["lp_item", "like_item"]),
              pdm.EmbeddingConfig(100, 64, "artist", pdm.DataType.BF16, ["lp_artist", "like_artist"])]
    ec = pdm.EmbeddingCollection(tables, device=dev)
    B = 23
    lens_lp, lens_like = g.integers(0, 30, B), g.integers(0, 9, B)
    lp_items, like_items = g.integers(0, 1000, lens_lp.sum()), g.integers(0, 1000, lens_like.sum())
    batch = {"lp_item": lp_items, "lp_artist": lp_items % 100, "like_item": like_items,
             "like_artist": like_items % 100, "lp_item__lengths": lens_lp, "like_item__lengths": lens_like}
    batch = {k: torch.from_numpy(np.asarray(v)).to(dev) for k, v in batch.items()}
    sg = pdm.SequenceGather(ec, {"lp": ["lp_item", "lp_artist"], "like": ["like_item", "like_artist"]},
                            {"lp": 24, "like": 8})
    torch.manual_seed(5)
    toks = torch.nn.ModuleDict({"lp": pdm.SequentialTokenizer(192, 128, max_len=32),
                                "like": pdm.SequentialTokenizer(192, 128, max_len=32, use_pos_embed=False)}).to(dev)
    fused = pdm.FusedSequenceTokenizer(sg, toks)
    with torch.no_grad():
        tokens, mask = fused(batch)
        raw, mask2 = sg(batch)
        want = torch.cat([toks["lp"](raw[:, :24]), toks["like"](raw[:, 24:])], dim=1)
    torch.cuda.synchronize()
    assert torch.equal(mask, mask2)
    assert torch.equal(tokens, want)
    # and the oracle, through the C gather and the torch restatement
    tabs = [o.table_bytes(ec.embeddings[n].weight.detach().cpu()).view(np.uint16).reshape(r, d)
            for n, r, d in (("item", 1000, 128), ("artist", 100, 64))]
    ids = [[lp_items, lp_items % 100], [like_items, like_items % 100]]
    offs = [o.offsets_np(lens_lp), o.offsets_np(lens_like)]
    _check(tokens.cpu(), tabs, ids, offs, [24, 8], [_module_weights(toks["lp"]), _module_weights(toks["like"])],
           0, 0, mask.to(torch.uint8))
