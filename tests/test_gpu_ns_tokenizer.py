"""GPU parity of the NS tokens (pdm_ns_tokenize_fwd: the NS input rows of onetrans.py:522-532 through the
AutoSplitTokenizer of onetrans.py:260-276) against the oracle (``onetrans.ns_tokenize``), and of the
AutoSplitTokenizer / FusedNSTokenizer modules.

Tolerance (bf16 autocast), as for the sequential tokenizer: every element within 2^-7 (|y| + |h| . |W2|^T)
(y: the output, h: the hidden row), fewer than 2 % of elements different at all, rel-L2 below 2e-2."""
import numpy as np
import pytest
import torch

from oracle import onetrans as ot
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def _parts(g, B, scalar, dense_dims, dtype, bad=False):
    tabs = []
    for r, d in scalar:
        w = g.normal(0, 0.5, (r, d)).astype(np.float32)
        tabs.append(o.f32_to_bf16_bits(w).reshape(r, d) if dtype == "bf16" else w)
    ids = [g.integers(0, r, B) for r, _ in scalar]
    if bad and ids:
        ids[-1][B // 2] = scalar[-1][0] + 2
    dense = [g.normal(0, 1, (B, d)).astype(np.float32) for d in dense_dims]
    return tabs, ids, dense


def _dev(tabs, ids, dense, dev):
    dt = [torch.from_numpy(t.view(np.int16)).view(torch.bfloat16).to(dev) if t.dtype == np.uint16
          else torch.from_numpy(t).to(dev) for t in tabs]
    return dt, [torch.from_numpy(i).to(dev) for i in ids], [torch.from_numpy(x).to(dev) for x in dense]


def _check(got, tabs, ids, dense, w, n_ns):
    want = ot.ns_tokenize(tabs, ids, dense, w, n_ns)
    B = want.shape[0]
    parts = []
    for t, i in zip(tabs, ids):
        t = (t.astype(np.uint32) << 16).view(np.float32) if t.dtype == np.uint16 else t
        ok = (i >= 0) & (i < t.shape[0])
        rows = t[np.where(ok, i, 0)].copy()
        rows[~ok] = 0
        parts.append(torch.from_numpy(rows))
    parts += [torch.from_numpy(x) for x in dense]
    num = ot._Num("autocast")
    h = num.round(torch.nn.functional.gelu(ot._lin_bias(torch.cat(parts, 1), w["w1"], w["b1"], num)))
    mag = (want.reshape(B, -1).abs() + h.abs() @ num.round(w["w2"]).abs().T).view_as(want)
    diff = (got - want).abs()
    assert bool((diff <= 2.0 ** -7 * mag + 1e-6).all()), float((diff - 2.0 ** -7 * mag).max())
    assert (diff > 0).float().mean().item() < 0.02
    assert ((got - want).norm() / want.norm()).item() < 2e-2


@pytest.mark.parametrize("case", [
    # scalar tables [(rows, dim)], dense dims, d, n_ns, table dtype, B
    ([(5000, 64), (3000, 64), (800, 64), (1200, 64)], [64, 6, 6, 64], 256, 16, "bf16", 37),
    ([(700, 32), (90, 64)], [2, 32], 128, 4, "fp32", 200),
    ([], [130], 64, 2, "bf16", 5),
    ([(100, 128)], [], 64, 4, "bf16", 129),
    ([(5000, 64), (3000, 64), (800, 64), (1200, 64)], [64, 6, 6, 64], 384, 16, "bf16", 21),
], ids=["reference_shape_k396_n4096", "fp32_k130_n512", "dense_only", "scalar_only_b129",
        "reference_large_k396_n6144"])
def test_ns_tokenize_matches_oracle(pdm, dev, case):
    scalar, dense_dims, d, n_ns, dtype, B = case
    g = np.random.default_rng(B)
    tabs, ids, dense = _parts(g, B, scalar, dense_dims, dtype)
    K = sum(dm for _, dm in scalar) + sum(dense_dims)
    w = ot.random_autosplit_weights(K, d * n_ns, seed=K)
    wb = {k: v.to(torch.bfloat16).contiguous().to(dev) for k, v in w.items()}
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out = pdm.ops.ns_tokenize_raw(*_dev(tabs, ids, dense, dev), wb["w1"], wb["b1"], wb["w2"], wb["b2"], n_ns,
                                  err_flag=err)
    torch.cuda.synchronize()
    assert err.item() == 0 and out.shape == (B, n_ns, d)
    _check(out.cpu(), tabs, ids, dense, w, n_ns)


def test_ns_tokens_into_block_input_and_bad_ids(pdm, dev):
    """out = the NS rows of a [B, S + n_ns, d] block input (S rows untouched); an id outside its table reads
    zeros and raises the flag."""
    g = np.random.default_rng(8)
    scalar, dense_dims, d, n_ns, B, S = [(300, 64), (50, 64)], [6], 128, 4, 20, 7
    tabs, ids, dense = _parts(g, B, scalar, dense_dims, "bf16", bad=True)
    w = ot.random_autosplit_weights(134, d * n_ns, seed=1)
    wb = {k: v.to(torch.bfloat16).contiguous().to(dev) for k, v in w.items()}
    x = torch.full((B, S + n_ns, d), 3.0, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    pdm.ops.ns_tokenize_raw(*_dev(tabs, ids, dense, dev), wb["w1"], wb["b1"], wb["w2"], wb["b2"], n_ns,
                            out=x[:, S:], err_flag=err)
    torch.cuda.synchronize()
    assert err.item() == 1
    assert bool((x[:, :S] == 3.0).all())
    _check(x[:, S:].cpu(), tabs, ids, dense, w, n_ns)


def test_autosplit_and_fused_ns_modules(pdm, dev):
    """AutoSplitTokenizer.forward(ns_features) matches the oracle on the module's parameters, and
    FusedNSTokenizer (scalar lookups fused) equals it bit for bit on the same NS input."""
    g = np.random.default_rng(12)
    tables = [pdm.EmbeddingConfig(400, 64, "uid", pdm.DataType.BF16, ["uid"]),
              pdm.EmbeddingConfig(900, 64, "item", pdm.DataType.BF16, ["item"])]
    ec = pdm.EmbeddingCollection(tables, device=dev)
    B, d, n_ns = 50, 128, 8
    torch.manual_seed(2)
    tok = pdm.AutoSplitTokenizer(64 + 64 + 6 + 64, d, n_ns).to(dev)
    batch = {"uid": torch.from_numpy(g.integers(0, 400, B)).to(dev),
             "item": torch.from_numpy(g.integers(0, 900, B)).to(dev)}
    dense = [torch.randn(B, 6, device=dev), torch.randn(B, 64, device=dev)]
    fused = pdm.FusedNSTokenizer(ec, ["uid", "item"], tok)
    with torch.no_grad():
        got = fused(batch, dense)
        feats = torch.cat([ec.embeddings["uid"].weight[batch["uid"]].float(),
                           ec.embeddings["item"].weight[batch["item"]].float()] + dense, dim=1)
        want_mod = tok(feats)
    torch.cuda.synchronize()
    assert torch.equal(got, want_mod)
    w = {"w1": tok.proj[0].weight.detach().cpu(), "b1": tok.proj[0].bias.detach().cpu(),
         "w2": tok.proj[2].weight.detach().cpu(), "b2": tok.proj[2].bias.detach().cpu()}
    want = ot.autosplit_tokenizer(feats.cpu(), w, n_ns)
    num = ot._Num("autocast")
    h = num.round(torch.nn.functional.gelu(ot._lin_bias(feats.cpu(), w["w1"], w["b1"], num)))
    mag = (want.reshape(B, -1).abs() + h.abs() @ num.round(w["w2"]).abs().T).view_as(want)
    diff = (got.cpu() - want).abs()
    assert bool((diff <= 2.0 ** -7 * mag + 1e-6).all())
