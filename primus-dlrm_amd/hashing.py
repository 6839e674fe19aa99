"""Cross-feature ids on the GPU: drop-in for primus_dlrm/data/hashing.py.

``cross_hash_nway`` / ``cross_hash_int64`` / ``cross_hash_batch`` keep the
reference's names, argument meaning and wire format (xxHash64 with
seed = salt over the little-endian int64 keys, remainder by table_size;
primus_dlrm/data/hashing.py:23-52, 55-69, 72-112).  They take int64 CUDA
tensors of keys (one value per row, or one value broadcast to every row) and
return an int64 CUDA tensor of row ids, computed by ``pdm_cross_hash_fwd``.
Scalar Python ints are accepted as broadcast keys of a batch whose length is
set by the tensor keys; a call with only scalar keys hashes one row.
"""
from __future__ import annotations

from typing import Optional, Sequence, Union

import torch

from . import ops

Key = Union[int, torch.Tensor]

__all__ = ["cross_hash_nway", "cross_hash_int64", "cross_hash_batch"]


def _as_tensors(keys: Sequence[Key], device: Optional[torch.device]):
    dev = device
    for k in keys:
        if isinstance(k, torch.Tensor):
            dev = k.device if dev is None else dev
    if dev is None:
        raise RuntimeError("cross hash runs on the GPU: pass a CUDA tensor key or device=")
    return [k if isinstance(k, torch.Tensor) else torch.tensor([int(k)], dtype=torch.int64, device=dev)
            for k in keys]


def cross_hash_nway(keys: Sequence[Key], table_size: int, salt: int = 0,
                    device: Optional[torch.device] = None) -> torch.Tensor:
    """Row ids ``xxh64(pack("<nq", keys...), seed=salt) % table_size`` (hashing.py:23-52).

    The reference requires at least two keys (AssertionError otherwise); so does this."""
    assert len(keys) >= 2, f"cross_hash_nway needs >=2 keys, got {len(keys)}"
    return torch.ops.pdm.cross_hash_fwd(_as_tensors(keys, device), int(table_size), int(salt))


def cross_hash_int64(feat_a: Key, feat_b: Key, table_size: int, salt: int = 0,
                     device: Optional[torch.device] = None) -> torch.Tensor:
    """2-way wrapper with the same wire format as ``cross_hash_nway([a, b], ...)`` (hashing.py:55-69)."""
    return cross_hash_nway([feat_a, feat_b], table_size, salt, device)


def cross_hash_batch(arr_a: Key, arr_b: Key, table_size: int, salt: int = 0,
                     device: Optional[torch.device] = None) -> torch.Tensor:
    """Element-wise 2-way hash of two int64 key arrays; a length-1 array broadcasts (hashing.py:72-112)."""
    return cross_hash_nway([arr_a, arr_b], table_size, salt, device)
