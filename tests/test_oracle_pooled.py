"""Pins the C oracle's pooled lookup, conversions and int8 rowwise decode
against library routines, closed forms and brute force (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import oracle as o


def _rng(seed=0):
    return np.random.default_rng(seed)


# ---- conversions: pinned by numpy / torch rounding -----------------------------

def _special_f32():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05, 6.0975552e-05,
            5.9604645e-08, 2.9802322e-08, 2.98023259e-08, 1e-10, np.inf, -np.inf, 3.0e38, 1.17549435e-38,
            1e-40, 0.5 + 2 ** -12, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11]
    return np.array(vals, dtype=np.float32)


def test_f32_to_f16_matches_numpy():
    g = _rng(1)
    x = np.concatenate([_special_f32(), g.normal(0, 1, 4000).astype(np.float32),
                        (g.normal(0, 1, 2000) * 1e-5).astype(np.float32),
                        (g.normal(0, 1, 2000) * 3e4).astype(np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = o.f32_to_f16_bits(x)
    assert np.array_equal(got, want)


def test_f32_to_bf16_matches_torch():
    g = _rng(2)
    x = np.concatenate([_special_f32(), g.normal(0, 1, 4000).astype(np.float32),
                        g.uniform(-3e38, 3e38, 1000).astype(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = o.f32_to_bf16_bits(x)
    assert np.array_equal(got, want)


def test_f16_to_f32_matches_numpy():
    h = np.arange(0, 65536, 7, dtype=np.uint16)
    h = h[(h & 0x7c00) != 0x7c00]  # finite values
    got = o.f16_bits_to_f32(h)
    assert np.array_equal(got, h.view(np.float16).astype(np.float32))


# ---- pooled lookup -------------------------------------------------------------

@pytest.mark.parametrize("mode", ["sum", "mean"])
@pytest.mark.parametrize("dim", [4, 64, 132])
def test_pooled_fp32_bitexact_vs_torch_embedding_bag(mode, dim):
    g = _rng(3)
    rows, B = 777, 257
    W = g.uniform(-0.01, 0.01, (rows, dim)).astype(np.float32)
    lengths = np.clip(g.poisson(10, B), 0, 50)
    idx = g.integers(0, rows, lengths.sum())
    off = o.offsets_np(lengths)
    ref = torch.nn.functional.embedding_bag(torch.from_numpy(idx), torch.from_numpy(W), torch.from_numpy(off),
                                            mode=mode, include_last_offset=True).numpy()
    got = o.tbe_pooled_from_tables([W], [mode], idx, off, B)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_pooled_bf16_fp16_tables_bitexact_vs_upcast_embedding_bag():
    g = _rng(4)
    rows, B, D = 500, 128, 128
    idx = g.integers(0, rows, 1000)
    off = np.sort(np.concatenate([[0, 1000], g.integers(0, 1000, B - 1)])).astype(np.int64)
    for dt in (torch.bfloat16, torch.float16):
        W = torch.from_numpy(g.normal(0, 0.02, (rows, D)).astype(np.float32)).to(dt)
        ref = torch.nn.functional.embedding_bag(torch.from_numpy(idx), W.float(), torch.from_numpy(off),
                                                mode="sum", include_last_offset=True).numpy()
        got = o.tbe_pooled_from_tables([W], ["sum"], idx, off, B)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_pooled_matches_reference_masked_formula_with_padding():
    """sharded_embedding.py:220-227: sum = sum(mask * e), mean = sum / clamp(count, 1), mask = ids != pad."""
    g = _rng(5)
    rows, B, L, D = 300, 64, 12, 16
    W = g.normal(0, 1, (rows, D)).astype(np.float32)
    ids = g.integers(0, rows, (B, L))
    ids[g.random((B, L)) < 0.4] = 0
    ids[3] = 0  # an all-padding bag
    e = torch.from_numpy(W)[torch.from_numpy(ids)]
    mask = (torch.from_numpy(ids) != 0).unsqueeze(-1).float()
    ref_sum = (e.double() * mask.double()).sum(-2).numpy()
    ref_mean = ref_sum / np.maximum(mask.sum(-2).double().numpy(), 1)
    off = np.arange(0, B * L + 1, L, dtype=np.int64)
    for mode, ref in (("sum", ref_sum), ("mean", ref_mean)):
        got = o.tbe_pooled_from_tables([W], [mode], ids.reshape(-1), off, B, padding_idx=0)
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
        assert np.all(got[3] == 0)


def test_pooled_fp64_bruteforce_and_edge_cases():
    g = _rng(6)
    rows, D = 40, 8
    W = g.normal(0, 1, (rows, D)).astype(np.float32)
    lengths = np.array([0, 1, 5, 0, 50, 2])
    B = lengths.size
    idx = g.integers(0, rows, lengths.sum()).astype(np.int32)  # 32-bit indices
    off = o.offsets_np(lengths)
    got = o.tbe_pooled_from_tables([W], ["mean"], idx, off, B)
    for b in range(B):
        seg = idx[off[b]:off[b + 1]]
        want = W[seg].astype(np.float64).sum(0) / max(len(seg), 1)
        np.testing.assert_allclose(got[b], want, rtol=1e-5, atol=1e-6)
    assert np.all(got[0] == 0) and np.all(got[3] == 0)


def test_pooled_single_hot_is_row_copy_and_multi_table_layout():
    g = _rng(7)
    tabs = [g.normal(0, 1, (r, d)).astype(np.float32) for r, d in ((50, 8), (70, 16), (30, 4))]
    B = 20
    idx = np.concatenate([g.integers(0, t.shape[0], B) for t in tabs])
    off = np.arange(3 * B + 1, dtype=np.int64)
    got = o.tbe_pooled_from_tables(tabs, ["sum", "mean", "sum"], idx, off, B)
    want = np.concatenate([tabs[t][idx[t * B:(t + 1) * B]] for t in range(3)], axis=1)
    assert np.array_equal(got, want)


def test_pooled_invalid_entries_are_skipped_and_counted():
    W = np.arange(40, dtype=np.float32).reshape(10, 4)
    idx = np.array([1, 99, -3, 2, 5], dtype=np.int64)
    off = np.array([0, 3, 5], dtype=np.int64)
    flat = W.view(np.uint8).reshape(-1)
    slots = [dict(rows=10, weights_offset=0, dim=4, dtype="fp32", pooling="mean", out_offset=0)]
    out, bad = o.tbe_pooled(flat, slots, idx, off, 2, return_bad=True)
    assert bad == 2
    assert np.array_equal(out[0], W[1])  # invalid ids neither added nor counted
    assert np.allclose(out[1], (W[2] + W[5]) / 2)
    # non-monotone offsets: the bag is empty and counted as bad (plus the two invalid ids of bag 0)
    out, bad = o.tbe_pooled(flat, slots, idx, np.array([0, 4, 2]), 2, return_bad=True)
    assert bad == 3 and np.all(out[1] == 0)


def test_pooled_fp16_bf16_outputs_round_like_numpy_and_torch():
    g = _rng(8)
    W = g.normal(0, 3, (64, 32)).astype(np.float32)
    idx = g.integers(0, 64, 200)
    off = np.linspace(0, 200, 11).astype(np.int64)
    f32 = o.tbe_pooled_from_tables([W], ["mean"], idx, off, 10)
    f16 = o.tbe_pooled_from_tables([W], ["mean"], idx, off, 10, out_dtype="fp16")
    bf16 = o.tbe_pooled_from_tables([W], ["mean"], idx, off, 10, out_dtype="bf16")
    assert np.array_equal(f16, f32.astype(np.float16).view(np.uint16))
    assert np.array_equal(bf16, torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


# ---- int8 rowwise ---------------------------------------------------------------

def _pack_for_torch(q, D):
    rows = q.shape[0]
    sb = q[:, :4].copy().view(np.float16).astype(np.float32)
    return np.concatenate([q[:, 4:4 + D], sb.view(np.uint8).reshape(rows, 8)], axis=1)


def test_int8_sum_bitexact_vs_torch_quantized_embedding_bag():
    """Decode q*scale + bias (two fp32 roundings) and sequential accumulation match
    torch's quantized::embedding_bag_byte_rowwise_offsets on the same rows."""
    g = _rng(9)
    rows, D, B = 500, 128, 200
    q = o.int8_quantize(g.normal(0, 0.05, (rows, D)).astype(np.float32))
    lengths = np.clip(g.poisson(20, B), 1, 100)
    idx = g.integers(0, rows, lengths.sum())
    off = o.offsets_np(lengths)
    ref = torch.ops.quantized.embedding_bag_byte_rowwise_offsets(
        torch.from_numpy(_pack_for_torch(q, D)), torch.from_numpy(idx), torch.from_numpy(off), False, 0, False,
        None, None, True).numpy()
    got = o.tbe_pooled_from_tables([q], ["sum"], idx, off, B, dims=[D])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # mean = fl(sum / count), then fp16 rounding
    mean = o.tbe_pooled_from_tables([q], ["mean"], idx, off, B, dims=[D], out_dtype="fp16")
    want = (ref / lengths[:, None].astype(np.float32)).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(mean, want)


def test_int8_quantizer_closed_forms():
    g = _rng(10)
    D = 128
    x = g.normal(0, 0.05, (300, D)).astype(np.float32)
    x[0] = 0.125  # constant row: range 0 -> scale 1, q = 0, decodes to bias exactly
    x[1] = np.linspace(-1, 1, D)
    q = o.int8_quantize(x)
    sb = q[:, :4].copy().view(np.float16)
    scale, bias = sb[:, 0].astype(np.float32), sb[:, 1].astype(np.float32)
    assert scale[0] == 1.0 and bias[0] == 0.125 and np.all(q[0, 4:] == 0)
    assert np.array_equal(sb[:, 1], x.min(1).astype(np.float16))  # bias = fp16(min)
    dec = o.int8_decode(q, D)
    err = np.abs(dec - x)
    # |x - decode| <= scale/2 plus the bias rounding and fp16 scale rounding slack
    assert np.all(err <= scale[:, None] * 0.5 + np.abs(x.min(1) - bias)[:, None] + 1e-6)
    assert q[1, 4:].max() == 255 or q[1, 4:].max() == 254
    assert np.all(q[2:, 4:].max(1) >= 254)  # max element lands at the top code
    # every code is the nearest grid point: no neighbouring code decodes closer to x
    codes = q[:, 4:].astype(np.int64)
    for dq in (-1, 1):
        nb = np.clip(codes + dq, 0, 255)
        dec_nb = nb.astype(np.float32) * scale[:, None] + bias[:, None]
        assert np.all(np.abs(dec - x) <= np.abs(dec_nb - x) + 1e-7 * np.abs(x))
    # codes are monotone in x within a row
    for r in range(2, 40):
        order = np.argsort(x[r], kind="stable")
        assert np.all(np.diff(codes[r, order]) >= 0)


def test_int8_quantizer_rounds_half_to_even_on_exact_ties():
    """A row whose grid is exact (bias 0, scale 2^-8: min 0, max 255/256) puts x = (k + 1/2) / 256 exactly halfway
    between two codes: the quantizer keeps the even one (round half to even), whatever the parity of k."""
    D = 64
    k = np.arange(D, dtype=np.float32) * 3 + 1  # codes 1, 4, 7, ... both parities
    x = ((k + 0.5) / 256.0).astype(np.float32)
    x[0], x[-1] = 0.0, 255.0 / 256.0  # pin min and max
    q = o.int8_quantize(x[None, :])
    sb = q[:, :4].copy().view(np.float16)
    assert float(sb[0, 0]) == 2.0 ** -8 and float(sb[0, 1]) == 0.0
    codes = q[0, 4:].astype(np.int64)
    tie = (k[1:-1] + 0.5).astype(np.float64)
    want = np.where(np.floor(tie) % 2 == 0, np.floor(tie), np.ceil(tie))
    assert np.array_equal(codes[1:-1], want.astype(np.int64))
    assert codes[0] == 0 and codes[-1] == 255
