"""Jagged containers with the TorchRec surface the lookup path uses.

``KeyedJaggedTensor`` mirrors the constructor and accessors the reference
calls (``KeyedJaggedTensor.from_lengths_sync(keys, values, lengths)`` at
primus_dlrm/models/embedding.py:200,228 and pipeline_batch.py:97;
``keys() / values() / lengths() / offsets() / stride()``).  Layout is
TorchRec's: ``values`` holds the ids of every (key, sample) bag key-major,
``lengths`` is ``[len(keys) * stride]``.  Offsets are computed on the device
with a cumulative sum, so building one never synchronises the host.

``build_pooled_kjt`` / ``build_unpooled_kjt`` / ``build_kjt`` mirror the reference's builders
(embedding.py:177-232, data/pipeline_batch.py:70-100) and ``KeyedJaggedTensor.permute`` TorchRec's; on the GPU
the padding filter and the permutation run in the library's kernels without a host sync, so ``values()`` of
such a KJT is a buffer of the known capacity whose first ``offsets()[-1]`` entries are the ids.

``KeyedTensor`` (pooled output, ``kt[key] -> [B, D]``, embedding.py:154) and
``JaggedTensor`` (unpooled output, ``jt.values() -> [sum len, D]``,
embedding.py:161-172) are the matching result types.  Objects from a real
TorchRec install are accepted wherever a KJT is expected (duck typing on
``keys() / values() / lengths() / offsets() / stride()``).
"""
from __future__ import annotations

from typing import Dict, List, Optional

import torch


def mask_as_bool(mask: torch.Tensor) -> torch.Tensor:
    """The kernels' uint8 0/1 mask as bool: a free reinterpretation eagerly; a conversion inside a compiled graph
    (Inductor does not lower a uint8 -> bool view)."""
    return mask.bool() if torch.compiler.is_compiling() else mask.view(torch.bool)


def _offsets_from_lengths(lengths: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.pad(lengths.reshape(-1).to(torch.int64).cumsum(0), (1, 0))


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

    def permute(self, indices: List[int]) -> "KeyedJaggedTensor":
        """Output key k is key ``indices[k]`` (TorchRec's KJT.permute); keys may repeat or be dropped.
        On the GPU one kernel pass, no host sync."""
        if self._values.device.type != "cuda":
            raise RuntimeError("KeyedJaggedTensor.permute runs on the GPU only")
        from . import ops  # noqa: F401  (registers pdm::kjt_permute)
        v, lengths, offsets = torch.ops.pdm.kjt_permute(self._values, self.offsets().to(torch.int64).contiguous(),
                                                        len(self._keys), self._stride, list(indices))
        return KeyedJaggedTensor([self._keys[i] for i in indices], v, lengths=lengths, offsets=offsets,
                                 stride=self._stride)

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


def build_pooled_kjt(features: Dict[str, torch.Tensor], feature_order: List[str],
                     padding_idx: int) -> KeyedJaggedTensor:
    """``_build_pooled_kjt`` (primus_dlrm/models/embedding.py:177-204): per feature present in
    ``feature_order``, the ids of each row of ``features[name]`` ([B, L]) that differ from ``padding_idx``,
    in row order; lengths int32.  On the GPU: ``pdm_kjt_from_dense``, no host sync."""
    names = [n for n in feature_order if n in features]
    if not names:
        return KeyedJaggedTensor([], torch.empty(0, dtype=torch.long), lengths=torch.empty(0, dtype=torch.int32))
    mats = [features[n] if features[n].dim() == 2 else features[n].reshape(features[n].shape[0], -1) for n in names]
    if mats[0].device.type != "cuda":
        raise RuntimeError("build_pooled_kjt runs on the GPU only")
    from . import ops
    dt = torch.int64 if any(m.dtype == torch.int64 for m in mats) else mats[0].dtype
    values, lengths, offsets = ops.kjt_from_dense_raw([m.to(dt) for m in mats], padding_idx)
    return KeyedJaggedTensor(names, values, lengths=lengths, offsets=offsets, stride=mats[0].shape[0])


def build_unpooled_kjt(features: Dict[str, torch.Tensor], feature_order: List[str]) -> KeyedJaggedTensor:
    """``_build_unpooled_kjt`` (embedding.py:207-232): every id of ``features[name]`` ([B] or [B, L]), each row
    a bag of L ids (no filter; the sizes are known, so nothing synchronises)."""
    names, vals, lens = [], [], []
    for n in feature_order:
        if n not in features:
            continue
        ids = features[n]
        B = ids.shape[0]
        flat = ids.reshape(-1)
        names.append(n)
        vals.append(flat.to(torch.int64))
        lens.append(torch.full((B,), flat.shape[0] // max(B, 1), dtype=torch.int32, device=ids.device))
    if not names:
        return KeyedJaggedTensor([], torch.empty(0, dtype=torch.long), lengths=torch.empty(0, dtype=torch.int32))
    return KeyedJaggedTensor(names, torch.cat(vals), lengths=torch.cat(lens))


def build_kjt(tensors: Dict[str, torch.Tensor], feature_order: List[str],
              feature_to_batch_key: Optional[Dict[str, str]] = None) -> KeyedJaggedTensor:
    """``build_kjt`` (primus_dlrm/data/pipeline_batch.py:70-100): a feature with ``<key>__lengths`` in the
    batch is jagged (its flat ids and lengths are taken as they are), any other is a dense [B, L] matrix of
    bags of L ids."""
    fk = feature_to_batch_key or {}
    names, vals, lens = [], [], []
    for feat in feature_order:
        key = fk.get(feat, feat)
        if key not in tensors:
            continue
        ids = tensors[key]
        names.append(feat)
        if key + "__lengths" in tensors:
            vals.append(ids.reshape(-1).to(torch.int64))
            lens.append(tensors[key + "__lengths"].to(torch.int32))
        else:
            B = ids.shape[0]
            flat = ids.reshape(-1)
            vals.append(flat.to(torch.int64))
            lens.append(torch.full((B,), flat.shape[0] // max(B, 1), dtype=torch.int32, device=ids.device))
    if not names:
        return KeyedJaggedTensor([], torch.empty(0, dtype=torch.long), lengths=torch.empty(0, dtype=torch.int32))
    return KeyedJaggedTensor(names, torch.cat(vals), lengths=torch.cat(lens))
