"""GPU parity of the cross-feature ids (pdm_cross_hash_fwd, through the C ABI
and the hashing drop-in) against the CPU oracle: bit-exact for every key count
2..8, broadcast keys, extreme key values, table sizes up to 2^64 - 1 and salts,
plus the reference's golden vectors (tests/test_cross_features.py)."""
import ctypes

import numpy as np
import pytest
import torch

from test_oracle_cross_hash import GOLDEN

pytestmark = pytest.mark.gpu


def _u64(t):
    return [int(v) & (2**64 - 1) for v in t]


@pytest.mark.parametrize("n_keys", range(2, 9))
@pytest.mark.parametrize("n", [1, 255, 257, 70_001])
def test_cross_hash_matches_oracle(pdm, orc, dev, n_keys, n):
    rng = np.random.default_rng(n_keys * 1000 + n)
    keys = [rng.integers(-2**63, 2**63 - 1, n, dtype=np.int64, endpoint=True) for _ in range(n_keys)]
    keys[0][: min(n, 4)] = [0, -1, 2**63 - 1, -2**63][: min(n, 4)]
    for table, salt in ((1000, 0), (2**62 + 3, 5), (2**64 - 1, 2**63 + 9), (1, 0), (100_000_000, 3)):
        got = pdm.ops.cross_hash_raw([torch.from_numpy(k).to(dev) for k in keys], table, salt)
        want = orc.cross_hash(keys, table, salt)
        assert _u64(got.cpu().numpy()) == _u64(want), (n_keys, n, table, salt)


def test_broadcast_keys(pdm, orc, dev):
    rng = np.random.default_rng(3)
    a = rng.integers(0, 1 << 40, 10_000, dtype=np.int64)
    for pos in range(3):
        keys = [a, a[::-1].copy(), np.array([12345], dtype=np.int64)]
        keys[pos], keys[2] = keys[2], keys[pos]
        got = pdm.ops.cross_hash_raw([torch.from_numpy(k).to(dev) for k in keys], 24_000_000, 0)
        want = orc.cross_hash(keys, 24_000_000, 0)
        assert (got.cpu().numpy() == want).all()


@pytest.mark.parametrize("keys,table,salt,want", GOLDEN)
def test_golden_vectors_through_dropin(pdm, dev, keys, table, salt, want):
    t = [torch.tensor([k], dtype=torch.int64, device=dev) for k in keys]
    assert pdm.hashing.cross_hash_nway(t, table, salt).tolist() == [want]
    if len(keys) == 2:
        assert pdm.hashing.cross_hash_int64(t[0], t[1], table, salt).tolist() == [want]


def test_dropin_batch_scalar_broadcast_and_errors(pdm, orc, dev):
    a = torch.tensor([1, 2, 3, 4], dtype=torch.int64, device=dev)
    got = pdm.hashing.cross_hash_batch(a, 7, 1000)
    want = orc.cross_hash([a.cpu().numpy(), np.array([7])], 1000)
    assert (got.cpu().numpy() == want).all()
    with pytest.raises(AssertionError):
        pdm.hashing.cross_hash_nway([a], 1000)
    with pytest.raises(ValueError):
        pdm.ops.cross_hash_raw([a, a[:3]], 1000)
    with pytest.raises(ValueError):
        pdm.ops.cross_hash_raw([a, a], 0)
    with pytest.raises(RuntimeError, match="GPU only"):
        pdm.ops.cross_hash_raw([a.cpu(), a.cpu()], 10)


def test_empty_input(pdm, dev):
    e = torch.empty(0, dtype=torch.int64, device=dev)
    assert pdm.ops.cross_hash_raw([e, e], 10).numel() == 0
