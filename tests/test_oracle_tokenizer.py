"""Pins the tokenizer oracle (oracle/onetrans.py: sequential_tokenizer, seq_tokenize).

* autocast rounding points: against torch's own CPU autocast(bf16) running the
  SequentialTokenizer's layers (nn.Linear, nn.GELU, nn.Linear, nn.Embedding;
  primus_dlrm/models/onetrans.py:243-256), which decides where bf16 rounding
  happens independently of the oracle's explicit ``round`` calls;
* fp64 mode: against the same layers in float64;
* seq_tokenize: the gather it composes is the pinned sequence gather; the
  padding slots of a pool share one raw row, so their tokens minus pos[l] are
  one row; real slots match the tokenizer applied to the gathered rows.
"""
import numpy as np
import pytest
import torch

from oracle import onetrans as ot
from oracle import oracle as orc


def _module(K, d, w):
    m = torch.nn.Sequential(torch.nn.Linear(K, d), torch.nn.GELU(), torch.nn.Linear(d, d))
    pe = torch.nn.Embedding(w["pos"].shape[0], d)
    with torch.no_grad():
        m[0].weight.copy_(w["w1"])
        m[0].bias.copy_(w["b1"])
        m[2].weight.copy_(w["w2"])
        m[2].bias.copy_(w["b2"])
        pe.weight.copy_(w["pos"])
    return m, pe


@pytest.mark.parametrize("K,d", [(384, 256), (192, 128)])
def test_autocast_rounding_points_match_torch_autocast(K, d):
    L = 40
    w = ot.random_tokenizer_weights(K, d, 64, seed=K + d)
    raw = ot._bf16(torch.randn(3, L, K, generator=torch.Generator().manual_seed(5)))
    m, pe = _module(K, d, w)
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        ref = m(raw) + pe(torch.arange(L))
    assert ref.dtype == torch.float32
    got = ot.sequential_tokenizer(raw, w)
    diff = (got - ref).abs()
    # accumulation order may move a value across a bf16 rounding boundary: a few one-ulp differences, in
    # the output or in a hidden unit (which moves the output by at most one ulp of that unit times |w2|)
    num = ot._Num("autocast")
    h = num.round(torch.nn.functional.gelu(ot._lin_bias(raw, w["w1"], w["b1"], num)))
    mag = (got - w["pos"][:L]).abs() + h.abs() @ w["w2"].abs().T
    assert (diff > 0).float().mean().item() < 0.01
    assert bool((diff <= 2.0 ** -7 * mag).all())
    # the double-rounded alternative (bias added after rounding the product) is far from torch's autocast
    u_alt = ot._bf16(ot._bf16(num.round(raw) @ w["w1"].T) + w["b1"])
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        u_ref = m[0](raw).float()
    u_or = ot._lin_bias(raw, w["w1"], w["b1"], num)
    assert ((u_or != u_ref).float().mean() < 0.01) and ((u_alt != u_ref).float().mean() > 0.1)


def test_fp64_mode_matches_float64_layers():
    K, d, L = 256, 128, 17
    w = ot.random_tokenizer_weights(K, d, 32, seed=2)
    raw = torch.randn(2, L, K, dtype=torch.float64)
    m, pe = _module(K, d, w)
    m, pe = m.double(), pe.double()
    with torch.no_grad():
        ref = m(raw) + pe(torch.arange(L))
    got = ot.sequential_tokenizer(raw, w, mode="fp64")
    assert torch.allclose(got, ref, rtol=0, atol=1e-12)


def test_no_pos_embedding():
    K, d = 128, 128
    w = ot.random_tokenizer_weights(K, d, 8, seed=3, pos=False)
    raw = ot._bf16(torch.randn(2, 8, K))
    got = ot.sequential_tokenizer(raw, w)
    w2 = dict(w, pos=torch.zeros(8, d))
    assert torch.equal(got, ot.sequential_tokenizer(raw, w2))


@pytest.mark.parametrize("pad_mode,align", [(0, 0), (1, 0), (0, 1)])
def test_seq_tokenize_composes_gather_and_tokenizer(pad_mode, align):
    g = np.random.default_rng(11)
    B, max_len = 5, [6, 4]
    tabs = [orc.f32_to_bf16_bits(g.normal(0, 0.5, (50, 64)).astype(np.float32)).reshape(50, 64),
            orc.f32_to_bf16_bits(g.normal(0, 0.5, (20, 64)).astype(np.float32)).reshape(20, 64)]
    ids, offs = [], []
    for mean in (4, 2):
        ln = g.poisson(mean, B)
        it = g.integers(0, 50, int(ln.sum()))
        ids.append([it, it % 20])
        offs.append(orc.offsets_np(ln))
    ws = [ot.random_tokenizer_weights(128, 128, 8, seed=p) for p in range(2)]
    tok, mask = ot.seq_tokenize(tabs, ids, offs, max_len, ws, pad_mode=pad_mode, align=align)
    raw, wmask = orc.seq_gather(tabs, ids, offs, max_len, pad_mode=pad_mode, align=align)
    assert np.array_equal(mask, wmask)
    rawf = torch.from_numpy((raw.astype(np.uint32) << 16).view(np.float32))
    s0 = 0
    for p, L in enumerate(max_len):
        want = ot.sequential_tokenizer(rawf[:, s0:s0 + L], ws[p])
        assert torch.equal(tok[:, s0:s0 + L], want)
        # without positions, every padding slot of the pool is one row
        nopos = ot.sequential_tokenizer(rawf[:, s0:s0 + L], dict(ws[p], pos=None))
        pads = [(b, l) for b in range(B) for l in range(L) if mask[b, s0 + l] == 0]
        rows = {tuple(nopos[b, l].tolist()) for b, l in pads}
        assert len(pads) > 0 and len(rows) == 1
        s0 += L


def test_autosplit_rounding_points_match_torch_autocast():
    """AutoSplitTokenizer (onetrans.py:260-276) under torch's CPU autocast vs the oracle's rounding points."""
    K, d, n_ns = 130, 64, 4
    N = d * n_ns
    w = ot.random_autosplit_weights(K, N, seed=4)
    x = torch.randn(9, K, generator=torch.Generator().manual_seed(2))
    m = torch.nn.Sequential(torch.nn.Linear(K, N), torch.nn.GELU(), torch.nn.Linear(N, N))
    with torch.no_grad():
        m[0].weight.copy_(w["w1"])
        m[0].bias.copy_(w["b1"])
        m[2].weight.copy_(w["w2"])
        m[2].bias.copy_(w["b2"])
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        ref = m(x).view(-1, n_ns, d)
    assert ref.dtype == torch.bfloat16
    got = ot.autosplit_tokenizer(x, w, n_ns)
    num = ot._Num("autocast")
    h = num.round(torch.nn.functional.gelu(ot._lin_bias(x, w["w1"], w["b1"], num)))
    mag = (got.reshape(9, N).abs() + h.abs() @ w["w2"].abs().T).view(9, n_ns, d)
    diff = (got - ref.float()).abs()
    assert (diff > 0).float().mean().item() < 0.01
    assert bool((diff <= 2.0 ** -7 * mag).all())
    # fp64 mode = the float64 layers
    m64 = m.double()
    with torch.no_grad():
        r64 = m64(x.double()).view(-1, n_ns, d)
    assert torch.allclose(ot.autosplit_tokenizer(x.double(), w, n_ns, mode="fp64"), r64, rtol=0, atol=1e-12)


def test_ns_tokenize_concatenates_scalar_rows_then_dense():
    """_build_ns_raw order (onetrans.py:522-532): scalar rows in feature order, then dense parts; an id outside
    a table gives a zero row."""
    g = np.random.default_rng(1)
    t0 = g.normal(0, 1, (10, 8)).astype(np.float32)
    t1 = g.normal(0, 1, (5, 16)).astype(np.float32)
    ids = [np.array([3, 9, 0]), np.array([4, 7, 1])]  # 7 is outside t1
    dense = [g.normal(0, 1, (3, 6)).astype(np.float32)]
    w = ot.random_autosplit_weights(30, 64, seed=2)
    got = ot.ns_tokenize([t0, t1], ids, dense, w, 2, mode="fp64")
    raw = np.concatenate([t0[[3, 9, 0]], np.stack([t1[4], np.zeros(16, np.float32), t1[1]]), dense[0]], axis=1)
    want = ot.autosplit_tokenizer(torch.from_numpy(raw).double(), w, 2, mode="fp64")
    assert torch.equal(got, want)
