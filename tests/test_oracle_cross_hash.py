"""Pins the CPU oracle of the cross-feature ids (oracle_cross_hash / oracle_xxh64)
against the reference's golden vectors (tests/test_cross_features.py), the
installed xxhash library's XXH64 over every input length 0..79 and a few longer
ones, and the invariants the reference tests state (range, order, salt,
broadcast).  CPU only."""
import struct

import numpy as np
import pytest

# (keys, table_size, salt, expected) from the reference's golden-vector tests:
# tests/test_cross_features.py:31-35 (2-way), :100-103 (3- and 4-way), :123 (order)
GOLDEN = [
    ((1, 2), 1000, 0, 524),
    ((1, 2), 1 << 30, 0, 1056167084),
    ((42, 7), 1_000_000, 0, 924376),
    ((0, 0), 1000, 0, 434),
    ((-1, -1), 1000, 0, 28),
    ((1, 2, 3), 1000, 0, 706),
    ((1, 2, 3), 1 << 30, 0, 633392634),
    ((42, 7, 15), 1_000_000, 0, 847584),
    ((1, 2, 3, 4), 1000, 0, 45),
    ((3, 2, 1), 1000, 0, 313),
]


@pytest.mark.parametrize("keys,table,salt,want", GOLDEN)
def test_golden_vectors(orc, keys, table, salt, want):
    got = orc.cross_hash([np.array([k]) for k in keys], table, salt)
    assert got.tolist() == [want]


def test_xxh64_matches_library_every_length(orc):
    xxhash = pytest.importorskip("xxhash")
    rng = np.random.default_rng(0)
    for length in list(range(80)) + [100, 255, 256, 257, 1000]:
        for seed in (0, 1, 5, 2**63 + 7, 2**64 - 1):
            data = rng.integers(0, 256, length, dtype=np.uint8).tobytes()
            assert orc.xxh64(data, seed) == xxhash.xxh64(data, seed=seed).intdigest(), (length, seed)


def test_cross_hash_matches_library_random_keys(orc):
    xxhash = pytest.importorskip("xxhash")
    rng = np.random.default_rng(1)
    for n_keys in range(2, 9):
        keys = [rng.integers(-2**63, 2**63 - 1, 200, dtype=np.int64, endpoint=True) for _ in range(n_keys)]
        for table in (1, 7, 1000, 100_000_000, 2**62 + 3, 2**64 - 1):
            for salt in (0, 5, 2**63 + 9):
                got = orc.cross_hash(keys, table, salt)
                pack = struct.Struct(f"<{n_keys}q").pack
                want = [xxhash.xxh64(pack(*[int(k[i]) for k in keys]), seed=salt).intdigest() % table
                        for i in range(200)]
                assert [int(v) & (2**64 - 1) for v in got] == want, (n_keys, table, salt)


def test_range_order_salt_broadcast(orc):
    a = np.array([0, 1, 123, 1 << 40], dtype=np.int64)
    b = np.array([0, 2, 456, 1 << 30], dtype=np.int64)
    for table in (1, 7, 1024, 1_000_000):  # test_cross_features.py:38-45
        h = orc.cross_hash([a, b], table)
        assert ((h >= 0) & (h < table)).all()
    assert orc.cross_hash([np.array([1]), np.array([2])], 1000)[0] != orc.cross_hash(
        [np.array([2]), np.array([1])], 1000)[0]  # :48-53
    assert orc.cross_hash([np.array([1]), np.array([2])], 1000, 0)[0] != orc.cross_hash(
        [np.array([1]), np.array([2])], 1000, 5)[0]  # :56-59
    # broadcast of a length-1 key equals the explicit repeat (:78-91)
    arr = np.array([1, 2, 3, 4], dtype=np.int64)
    assert (orc.cross_hash([arr, np.array([7])], 1000) == orc.cross_hash([arr, np.full(4, 7)], 1000)).all()
    # table_size 1: every id is 0
    assert (orc.cross_hash([arr, arr], 1) == 0).all()
