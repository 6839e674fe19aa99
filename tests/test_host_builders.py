"""Host-side pieces of the path, on the CPU:

* ``build_unpooled_kjt`` / ``build_kjt`` (primus_dlrm/models/embedding.py:207-232,
  primus_dlrm/data/pipeline_batch.py:70-100): hand-worked cases, then seeded cases against the
  reference's loop (keys in feature order, missing features skipped, dense rows as bags of L ids,
  ``<key>__lengths`` marking jagged features, ``feature_to_batch_key`` renames) with TorchRec's
  ``from_lengths_sync`` offsets (a cumulative sum with a leading 0);
* ``pyramid_schedule`` of the package (primus_dlrm/models/onetrans.py:50-59) against the reference's own
  invariants (tests/test_model.py:322-326) and hand-computed schedules, including round-half-even ties;
* the seeded generators the five workloads are built from (synthetic.py): the Zipf log-log slope, the
  rank -> row map being a bijection, Poisson means and clip bounds, the log-uniform row range.
"""
import math

import numpy as np
import pytest
import torch


# ---- KJT builders ----------------------------------------------------------------------

def _kjt_parts(kjt):
    return kjt.keys(), kjt.values().tolist(), kjt.lengths().tolist(), kjt.offsets().tolist(), kjt.stride()


def test_build_unpooled_kjt_hand_worked(pdm):
    feats = {"a": torch.tensor([[1, 2, 3], [4, 5, 6]]), "s": torch.tensor([7, 8]), "unused": torch.tensor([9, 9])}
    kjt = pdm.kjt.build_unpooled_kjt(feats, ["s", "missing", "a"])
    keys, values, lengths, offsets, stride = _kjt_parts(kjt)
    assert keys == ["s", "a"] and stride == 2
    assert values == [7, 8, 1, 2, 3, 4, 5, 6]
    assert lengths == [1, 1, 3, 3] and offsets == [0, 1, 2, 5, 8]
    assert kjt.lengths().dtype == torch.int32 and kjt.values().dtype == torch.int64
    empty = pdm.kjt.build_unpooled_kjt(feats, ["missing"])
    assert empty.keys() == [] and empty.values().numel() == 0


def test_build_kjt_hand_worked(pdm):
    batch = {"seq": torch.tensor([10, 11, 12, 13]), "seq__lengths": torch.tensor([3, 0, 1], dtype=torch.int32),
             "user": torch.tensor([5, 6, 7]), "hist": torch.tensor([[1, 2], [3, 4], [5, 6]])}
    kjt = pdm.kjt.build_kjt(batch, ["user", "history", "seq"], {"history": "hist"})
    keys, values, lengths, offsets, stride = _kjt_parts(kjt)
    assert keys == ["user", "history", "seq"] and stride == 3
    assert values == [5, 6, 7, 1, 2, 3, 4, 5, 6, 10, 11, 12, 13]
    assert lengths == [1, 1, 1, 2, 2, 2, 3, 0, 1]
    assert offsets == [0, 1, 2, 3, 5, 7, 9, 12, 12, 13]


def _reference_build_kjt(tensors, feat_order, feat_to_key):
    """The loop of pipeline_batch.py:70-100 (and, without lengths keys, embedding.py:207-232), with
    KJT.from_lengths_sync's offsets."""
    keys, vals, lens = [], [], []
    for feat in feat_order:
        key = feat_to_key.get(feat, feat)
        if key not in tensors:
            continue
        ids = tensors[key]
        keys.append(feat)
        if key + "__lengths" in tensors:
            vals.append(ids)
            lens.append(tensors[key + "__lengths"])
        else:
            B = ids.shape[0]
            flat = ids.reshape(-1)
            vals.append(flat)
            lens.append(torch.full((B,), flat.shape[0] // B, dtype=torch.int32))
    values = torch.cat(vals)
    lengths = torch.cat(lens)
    offsets = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(lengths.to(torch.int64), 0)])
    return keys, values, lengths, offsets


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_build_kjt_matches_reference_loop(pdm, seed):
    g = torch.Generator().manual_seed(seed)
    B = 17
    tensors, order = {}, []
    for i in range(6):
        name = f"f{i}"
        kind = i % 3
        if kind == 0:  # scalar feature
            tensors[name] = torch.randint(0, 1000, (B,), generator=g)
        elif kind == 1:  # dense [B, L]
            tensors[name] = torch.randint(0, 1000, (B, 3 + i), generator=g)
        else:  # jagged
            ln = torch.randint(0, 9, (B,), generator=g, dtype=torch.int32)
            tensors[name] = torch.randint(0, 1000, (int(ln.sum()),), generator=g)
            tensors[name + "__lengths"] = ln
        order.append(name)
    order = order[::-1] + ["absent"]
    rename = {"g5": "f5"}
    order[0] = "g5"
    keys, values, lengths, offsets = _reference_build_kjt(tensors, order, rename)
    kjt = pdm.kjt.build_kjt(tensors, order, rename)
    assert kjt.keys() == keys
    assert torch.equal(kjt.values(), values)
    assert torch.equal(kjt.lengths(), lengths.to(torch.int32))
    assert torch.equal(kjt.offsets(), offsets)
    assert kjt.stride() == B
    # without lengths keys build_kjt is the unpooled builder
    dense = {k: v for k, v in tensors.items() if not k.endswith("__lengths") and v.shape[0] == B}
    order_d = [k for k in order if k in dense]
    ref = _reference_build_kjt(dense, order_d, {})
    got = pdm.kjt.build_unpooled_kjt(dense, order_d)
    assert got.keys() == ref[0] and torch.equal(got.values(), ref[1]) and torch.equal(got.offsets(), ref[3])


# ---- pyramid schedule --------------------------------------------------------------------

def test_pyramid_schedule_reference_invariants(pdm):
    s = pdm.pyramid_schedule(300, 8, 4)  # tests/test_model.py:322-326
    assert s[0] == 300 and s[-1] == 8 and all(s[i] >= s[i + 1] for i in range(len(s) - 1))


@pytest.mark.parametrize("args,want", [
    ((384, 16, 4), [384, 261, 139, 16]),   # 384 - l*368/3: 261.33, 138.67
    ((384, 16, 1), [16]),                  # one layer keeps only the NS count
    ((10, 2, 3), [10, 6, 2]),
    ((11, 2, 3), [11, 6, 2]),              # 6.5 rounds half to even
    ((13, 2, 3), [13, 8, 2]),              # 7.5 rounds half to even
    ((1500, 16, 8), [1500, 1288, 1076, 864, 652, 440, 228, 16]),
    ((8, 16, 3), [16, 16, 16]),            # floor at the NS count
])
def test_pyramid_schedule_values(pdm, args, want):
    assert pdm.pyramid_schedule(*args) == want


def test_pyramid_schedule_closed_form(pdm):
    for l_s in (64, 300, 384, 1500):
        for l_ns in (0, 8, 16):
            for n in range(2, 9):
                s = pdm.pyramid_schedule(l_s, l_ns, n)
                for layer, q in enumerate(s):
                    exact = l_s - layer * (l_s - l_ns) / (n - 1)
                    assert abs(q - max(exact, l_ns)) <= 0.5 + 1e-9
                assert s[0] == max(l_s, l_ns) and s[-1] == l_ns


def test_pyramid_mask_product_matches_bruteforce(pdm):
    for q, kv in ((5, 5), (3, 7), (1, 4), (80, 144)):
        m = pdm.build_pyramid_mask(q, kv, torch.device("cpu"))
        want = torch.tensor([[j <= i + kv - q for j in range(kv)] for i in range(q)])
        assert torch.equal(m, want)


def test_block_rejects_masks_other_than_the_pyramid(pdm):
    """The kernels always apply the bottom-right pyramid mask, so the block refuses any other mask before it
    launches anything (the checks run on the host, so CPU tensors reach them)."""
    from primus_dlrm_amd.onetrans import check_pyramid_mask
    q, kv, n_ns = 6, 10, 2
    blk = pdm.OneTransBlock(16, 2, n_ns).eval()
    x = torch.zeros(1, kv, 16)
    good = torch.tensor([[j <= i + kv - q for j in range(kv)] for i in range(q)])  # not made by the builder
    check_pyramid_mask(good, q, kv)  # equal values pass, and the tensor is tagged
    assert good._pdm_pyramid == (q, kv, good._version)
    good[0, 0] = True  # an in-place change bumps the version: compared again, still the pyramid mask
    check_pyramid_mask(good, q, kv)
    wrong = [
        torch.ones(q, kv, dtype=torch.bool),                                  # no mask at all
        torch.tensor([[j <= i for j in range(kv)] for i in range(q)]),        # top-left causal
        good.float(),                                                          # additive / float masks
        pdm.build_pyramid_mask(q, kv + 1, torch.device("cpu")),               # another shape
    ]
    flipped = pdm.build_pyramid_mask(q, kv, torch.device("cpu"))
    flipped[q - 1, 0] = False  # modified after it was built: the tag no longer applies
    wrong.append(flipped)
    for m in wrong:
        with pytest.raises(ValueError):
            blk(x, m, q, kv - n_ns)
    with torch.inference_mode():
        inf = pdm.build_pyramid_mask(q, kv, torch.device("cpu"))  # no version counter: compared each call
        check_pyramid_mask(inf, q, kv)
        inf[0, kv - 1] = True
        with pytest.raises(ValueError):
            check_pyramid_mask(inf, q, kv)


# ---- synthetic generators ------------------------------------------------------------------

def test_zipf_rank_to_row_is_a_bijection(pdm):
    syn = pdm.synthetic
    for rows in (1, 2, 97, 1000, 65_536, 1_000_003):
        r = np.arange(1, rows + 1, dtype=np.int64)
        mapped = (r * syn.ZIPF_SCATTER) % rows
        assert np.unique(mapped).size == rows and mapped.min() == 0 and mapped.max() == rows - 1
    # every table size of the workloads is coprime with the multiplier
    for rows in syn.single_hot_bf16(batch=8).rows + [5_000_000, 10_000_000, 100_000]:
        assert math.gcd(rows, syn.ZIPF_SCATTER) == 1


@pytest.mark.parametrize("alpha", [1.05, 1.1, 1.2])
def test_zipf_log_log_slope(pdm, alpha):
    """The rank frequencies fall as rank^-alpha: fit log f(r) against log r over ranks 10..1000."""
    syn = pdm.synthetic
    rows, n = 1_000_000, 4_000_000
    g = np.random.Generator(np.random.PCG64(5))
    u_rows = syn.zipf_rows(g, n, rows, alpha)
    # invert the scatter map to recover ranks: rank = row * P^-1 mod rows (rank rows maps to row 0)
    inv = pow(syn.ZIPF_SCATTER, -1, rows)
    ranks = u_rows * inv % rows  # both factors < 2^20: no overflow
    ranks[ranks == 0] = rows
    counts = np.bincount(ranks, minlength=rows + 1)
    r = np.arange(10, 1001)
    slope = np.polyfit(np.log(r), np.log(counts[r]), 1)[0]
    assert abs(slope + alpha) < 0.05, slope
    assert ranks.min() >= 1 and ranks.max() <= rows


def test_zipf_alpha_one_and_tiny_tables(pdm):
    syn = pdm.synthetic
    g = np.random.Generator(np.random.PCG64(6))
    for rows in (1, 2, 3):
        v = syn.zipf_rows(g, 1000, rows, 1.1)
        assert v.min() >= 0 and v.max() < rows
    v = syn.zipf_rows(g, 100_000, 1000, 1.0)
    assert v.min() >= 0 and v.max() < 1000
    with pytest.raises(ValueError):
        syn.zipf_rows(g, 10, 0, 1.1)


def test_poisson_lengths_mean_and_clip(pdm):
    syn = pdm.synthetic
    g = np.random.Generator(np.random.PCG64(7))
    for mean, lo, hi in ((10, 0, 50), (20, 1, 100), (150, 0, 256), (40, 0, 256), (80, 0, 256)):
        ln = syn.poisson_lengths(g, 200_000, mean, lo, hi)
        assert ln.min() >= lo and ln.max() <= hi and ln.dtype == np.int64
        assert abs(ln.mean() - mean) < 0.05 * math.sqrt(mean) + 0.02
    # the clip binds: Poisson(20) with lo=1 moves the zeros up; Poisson(10) clipped at 5 piles up at 5
    ln = syn.poisson_lengths(g, 100_000, 10, 0, 5)
    assert ln.max() == 5 and (ln == 5).mean() > 0.9


def test_workload_generators(pdm):
    syn = pdm.synthetic
    w = syn.single_hot_bf16(batch=64)
    assert len(w.rows) == 26 and all(1000 <= r <= 40_000_000 for r in w.rows)
    # log-uniform: ln(rows) spread over most of [ln 1e3, ln 4e7]
    lr = np.log(w.rows)
    assert lr.max() - lr.min() > 0.6 * (math.log(4e7) - math.log(1e3))
    assert np.array_equal(w.offsets, np.arange(26 * 64 + 1))
    for t in range(26):
        ids = w.indices[t * 64:(t + 1) * 64]
        assert ids.min() >= 0 and ids.max() < w.rows[t]
    # deterministic from the seed
    assert np.array_equal(syn.single_hot_bf16(batch=64).indices, w.indices)
    e = syn.ebc_fp32(batch=512)
    assert e.offsets.size == 8 * 512 + 1 and e.indices.max() < 100_000
    i8 = syn.int8_mean(batch=256, rows=50_000, tables=4)
    lens = np.diff(i8.offsets)
    assert lens.min() >= 1 and lens.max() <= 100
    s = syn.seq_gather(batch=64, item_rows=10_000, artist_rows=100, album_rows=200)
    for p in range(3):
        items, artists, albums = s.ids[p]
        assert np.array_equal(artists, syn.item_to_artist(items, 100))
        assert np.array_equal(albums, syn.item_to_album(items, 200))
        assert np.diff(s.offsets[p]).max() <= 256
