"""Pins the KJT oracle (CPU): the padding filter against the reference's own torch expression of
_build_pooled_kjt (primus_dlrm/models/embedding.py:186-194: mask = ids != padding_idx, lengths =
mask.sum(1), values = ids[mask], concatenated in feature order), the permutation by key-wise brute force."""
import numpy as np
import pytest
import torch

from oracle import oracle as o


@pytest.mark.parametrize("pad", [0, -1, 7])
def test_kjt_from_dense_matches_reference_expression(pad):
    g = np.random.default_rng(pad + 5)
    mats = [g.integers(0, 12, (9, L)) for L in (1, 5, 20, 0, 3)]
    values, lengths, offsets = o.kjt_from_dense(mats, pad)
    tv, tl = [], []
    for m in mats:
        ids = torch.from_numpy(m)
        mask = ids != pad if pad >= 0 else torch.ones_like(ids, dtype=torch.bool)
        tl.append(mask.sum(dim=1).to(torch.int32))
        tv.append(ids[mask])
    assert np.array_equal(values, torch.cat(tv).numpy())
    assert np.array_equal(lengths, torch.cat(tl).numpy())
    assert offsets[0] == 0 and offsets[-1] == values.size and np.array_equal(np.diff(offsets), lengths)


def test_kjt_permute_brute_force():
    g = np.random.default_rng(3)
    K, B = 4, 6
    lengths = g.integers(0, 5, K * B)
    offsets = o.offsets_np(lengths)
    values = g.integers(0, 1000, int(lengths.sum()))
    perm = [2, 0, 2, 3]
    v, ln, off = o.kjt_permute(values, offsets, K, B, perm)
    for k_out, k_in in enumerate(perm):
        for b in range(B):
            got = v[off[k_out * B + b]:off[k_out * B + b + 1]]
            want = values[offsets[k_in * B + b]:offsets[k_in * B + b + 1]]
            assert np.array_equal(got, want)
    assert ln.sum() == v.size
