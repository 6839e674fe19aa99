"""Jagged containers with the TorchRec surface the lookup path uses.

``KeyedJaggedTensor`` mirrors the constructor and accessors the reference
calls (``KeyedJaggedTensor.from_lengths_sync(keys, values, lengths)`` at
primus_dlrm/models/embedding.py:200,228 and pipeline_batch.py:97;
``keys() / values() / lengths() / offsets() / stride()``).  Layout is
TorchRec's: ``values`` holds the ids of every (key, sample) bag key-major,
``lengths`` is ``[len(keys) * stride]``.  Offsets are computed on the device
with a cumulative sum, so building one never synchronises the host.

``KeyedTensor`` (pooled output, ``kt[key] -> [B, D]``, embedding.py:154) and
``JaggedTensor`` (unpooled output, ``jt.values() -> [sum len, D]``,
embedding.py:161-172) are the matching result types.  Objects from a real
TorchRec install are accepted wherever a KJT is expected (duck typing on
``keys() / values() / lengths() / offsets() / stride()``).
"""
from __future__ import annotations

from typing import Dict, List, Optional

import torch


def _offsets_from_lengths(lengths: torch.Tensor) -> torch.Tensor:
    out = torch.zeros(lengths.numel() + 1, dtype=torch.int64, device=lengths.device)
    if lengths.numel():
        torch.cumsum(lengths.reshape(-1).to(torch.int64), 0, out=out[1:])
    return out


class KeyedJaggedTensor:
    """Key-major jagged ids: bag (key k, sample b) is
    ``values[offsets[k*stride+b] : offsets[k*stride+b+1]]``."""

    def __init__(self, keys: List[str], values: torch.Tensor, weights: Optional[torch.Tensor] = None,
                 lengths: Optional[torch.Tensor] = None, offsets: Optional[torch.Tensor] = None,
                 stride: Optional[int] = None):
        if lengths is None and offsets is None:
            raise ValueError("KeyedJaggedTensor needs lengths or offsets")
        self._keys = list(keys)
        self._values = values
        self._weights = weights
        self._lengths = lengths
        self._offsets = offsets
        n = (lengths.numel() if lengths is not None else offsets.numel() - 1)
        if stride is None:
            stride = n // len(self._keys) if self._keys else 0
        if self._keys and stride * len(self._keys) != n:
            raise ValueError(f"{n} lengths do not split into {len(self._keys)} keys")
        self._stride = int(stride)

    @staticmethod
    def from_lengths_sync(keys: List[str], values: torch.Tensor, lengths: torch.Tensor,
                          weights: Optional[torch.Tensor] = None, stride: Optional[int] = None
                          ) -> "KeyedJaggedTensor":
        return KeyedJaggedTensor(keys, values, weights=weights, lengths=lengths, stride=stride)

    @staticmethod
    def from_offsets_sync(keys: List[str], values: torch.Tensor, offsets: torch.Tensor,
                          weights: Optional[torch.Tensor] = None, stride: Optional[int] = None
                          ) -> "KeyedJaggedTensor":
        return KeyedJaggedTensor(keys, values, weights=weights, offsets=offsets, stride=stride)

    def keys(self) -> List[str]:
        return self._keys

    def values(self) -> torch.Tensor:
        return self._values

    def weights_or_none(self) -> Optional[torch.Tensor]:
        return self._weights

    def stride(self) -> int:
        return self._stride

    def lengths(self) -> torch.Tensor:
        if self._lengths is None:
            self._lengths = (self._offsets[1:] - self._offsets[:-1]).to(torch.int32)
        return self._lengths

    def offsets(self) -> torch.Tensor:
        if self._offsets is None:
            self._offsets = _offsets_from_lengths(self._lengths)
        return self._offsets

    def device(self) -> torch.device:
        return self._values.device

    def __repr__(self) -> str:
        return f"KeyedJaggedTensor(keys={self._keys}, stride={self._stride}, values={tuple(self._values.shape)})"


class KeyedTensor:
    """Pooled output: ``values`` is ``[B, sum(length_per_key)]``; ``kt[key]`` is
    the column slice of that key."""

    def __init__(self, keys: List[str], length_per_key: List[int], values: torch.Tensor, key_dim: int = 1):
        self._keys = list(keys)
        self._length_per_key = list(length_per_key)
        self._values = values
        self._key_dim = key_dim
        self._starts = {}
        off = 0
        for k, n in zip(self._keys, self._length_per_key):
            self._starts[k] = (off, n)
            off += n

    def keys(self) -> List[str]:
        return self._keys

    def values(self) -> torch.Tensor:
        return self._values

    def length_per_key(self) -> List[int]:
        return self._length_per_key

    def offset_per_key(self) -> List[int]:
        out = [0]
        for n in self._length_per_key:
            out.append(out[-1] + n)
        return out

    def key_dim(self) -> int:
        return self._key_dim

    def __getitem__(self, key: str) -> torch.Tensor:
        off, n = self._starts[key]
        return self._values.narrow(self._key_dim, off, n)

    def to_dict(self) -> Dict[str, torch.Tensor]:
        return {k: self[k] for k in self._keys}


class JaggedTensor:
    """Unpooled output of one key: ``values`` is ``[sum(lengths), D]``."""

    def __init__(self, values: torch.Tensor, lengths: Optional[torch.Tensor] = None,
                 offsets: Optional[torch.Tensor] = None):
        self._values = values
        self._lengths = lengths
        self._offsets = offsets

    def values(self) -> torch.Tensor:
        return self._values

    def lengths(self) -> torch.Tensor:
        if self._lengths is None:
            self._lengths = (self._offsets[1:] - self._offsets[:-1]).to(torch.int32)
        return self._lengths

    def offsets(self) -> torch.Tensor:
        if self._offsets is None:
            self._offsets = _offsets_from_lengths(self._lengths)
        return self._offsets
