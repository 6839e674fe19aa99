"""Pins the C oracle's jagged -> padded S-token gather against a brute-force
restatement of the reference's host padding (primus_dlrm/data/dataset.py:604-626),
its per-event concat (onetrans.py:515-520) and pool concat (onetrans.py:553-558)."""
import numpy as np
import pytest

from oracle import oracle as o


def _reference_style(tables, ids, offsets, L):
    """dataset.py pad_and_lookup: keep the last L items, left pad with 0, then
    look every feature up (id 0 -> row 0) and concat features, then pools."""
    B = offsets[0].size - 1
    pools = []
    for p in range(len(offsets)):
        per_b = []
        for b in range(B):
            feats = []
            for f, tab in enumerate(tables):
                items = ids[p][f][offsets[p][b]:offsets[p][b + 1]][-L[p]:] if L[p] > 0 else ids[p][f][:0]
                padded = np.zeros(L[p], dtype=np.int64)
                n = len(items)
                if n > 0:
                    padded[L[p] - n:] = items
                feats.append(tab[padded])
            per_b.append(np.concatenate(feats, axis=-1))
        pools.append(np.stack(per_b))
    return np.concatenate(pools, axis=1)


def _case(seed, B=7, means=(5, 2, 9), L=(6, 3, 8), dims=(8, 4, 4), rows=(50, 9, 13)):
    g = np.random.default_rng(seed)
    tables = [g.integers(0, 65535, (r, d)).astype(np.uint16) for r, d in zip(rows, dims)]
    ids, offs = [], []
    for p, m in enumerate(means):
        ln = np.clip(g.poisson(m, B), 0, 3 * max(L))
        ln[0] = 0
        items = g.integers(1, rows[0], ln.sum())
        ids.append([items, items % rows[1], (items * 7) % rows[2]])
        offs.append(o.offsets_np(ln))
    return tables, ids, offs, list(L)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_seq_gather_right_row0_matches_reference_padding(seed):
    tables, ids, offs, L = _case(seed)
    out, mask = o.seq_gather(tables, ids, offs, L, pad_mode=0, align=0)
    want = _reference_style(tables, ids, offs, L)
    assert np.array_equal(out, want)
    # mask: 1 exactly on the last min(len, L) slots of each pool
    s0 = 0
    for p, Lp in enumerate(L):
        ln = np.diff(offs[p])
        n = np.minimum(ln, Lp)
        for b in range(len(ln)):
            row = mask[b, s0:s0 + Lp]
            assert row.sum() == n[b] and (n[b] == 0 or row[Lp - n[b]:].all())
        s0 += Lp


def test_seq_gather_zero_pad_and_left_align():
    tables, ids, offs, L = _case(3)
    right, mask_r = o.seq_gather(tables, ids, offs, L, pad_mode=1, align=0)
    left, mask_l = o.seq_gather(tables, ids, offs, L, pad_mode=1, align=1)
    assert np.all(right[mask_r == 0] == 0) and np.all(left[mask_l == 0] == 0)
    assert mask_r.sum() == mask_l.sum()
    # left alignment is the right-aligned row with each pool's valid block moved to the front
    s0 = 0
    for Lp in L:
        for b in range(right.shape[0]):
            r = right[b, s0:s0 + Lp][mask_r[b, s0:s0 + Lp] == 1]
            l = left[b, s0:s0 + Lp][mask_l[b, s0:s0 + Lp] == 1]
            assert np.array_equal(r, l)
        s0 += Lp


def test_seq_gather_bad_ids_write_zeros_and_count():
    tables, ids, offs, L = _case(4)
    ids[1][2] = ids[1][2].copy()
    if ids[1][2].size:
        ids[1][2][-1] = 10 ** 9
    out, mask, bad = o.seq_gather(tables, ids, offs, L, return_bad=True)
    assert bad == (1 if ids[1][2].size else 0)
