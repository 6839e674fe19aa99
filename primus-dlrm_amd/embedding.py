"""Drop-in embedding modules over the gfx950 lookup kernels.

* ``EmbeddingBagCollection``  — TorchRec EBC surface: ``EmbeddingBagCollection(tables=[EmbeddingBagConfig],
  device)``, ``forward(KeyedJaggedTensor) -> KeyedTensor`` (reference call sites:
  primus_dlrm/models/embedding.py:50-57,118-120,151; primus_dlrm/models/dlrm.py:147).
  State dict keys ``embedding_bags.<table>.weight`` as in TorchRec.
* ``EmbeddingCollection``     — TorchRec EC surface: ``forward(KJT) -> Dict[str, JaggedTensor]``
  (embedding.py:60-66,122-124,161; onetrans.py:496).  Keys ``embeddings.<table>.weight``.
* ``SequenceGather``          — jagged ids of the behaviour pools -> padded S-token rows ``[B, S, sum D]``
  plus mask, on the device (replaces EC lookup + view + cat at onetrans.py:501-520,553-558 and the
  host padding at data/dataset.py:604-636).
* ``TorchRecEmbeddings``      — the reference's tensor-in/tensor-out wrapper (embedding.py:72-174):
  ``forward({feat: ids[B] | ids[B, L]}, padding_idx=0) -> {feat: [B, D] | [B, L, D]}``.

Every table of a collection lives in ONE device allocation (rows of table t start at a 256-byte
aligned byte offset); the per-table ``weight`` parameters are typed views of it, so one pointer plus
per-table offsets describe all tables to the kernels.
"""
from __future__ import annotations

import enum
import itertools
import math
import weakref
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn

from . import _lib as L
from . import ops
from .kjt import JaggedTensor, KeyedJaggedTensor, KeyedTensor, mask_as_bool
from .optim import FusedEmbeddingOptimizer, _optimizer_tag


class PoolingType(enum.Enum):
    SUM = "SUM"
    MEAN = "MEAN"
    NONE = "NONE"


class DataType(enum.Enum):
    FP32 = "FP32"
    FP16 = "FP16"
    BF16 = "BF16"
    INT8 = "INT8"  # rowwise: [fp16 scale][fp16 bias][dim x uint8] per row


_DT_TORCH = {DataType.FP32: torch.float32, DataType.FP16: torch.float16, DataType.BF16: torch.bfloat16}
_DT_PDM = {DataType.FP32: L.PDM_F32, DataType.FP16: L.PDM_F16, DataType.BF16: L.PDM_BF16,
           DataType.INT8: L.PDM_I8_SB_F16}
_POOL_PDM = {PoolingType.SUM: L.PDM_POOL_SUM, PoolingType.MEAN: L.PDM_POOL_MEAN}


@dataclass
class EmbeddingBagConfig:
    """Mirrors torchrec.EmbeddingBagConfig as the reference builds it (embedding.py:50-57)."""
    num_embeddings: int
    embedding_dim: int
    name: str = ""
    data_type: DataType = DataType.FP32
    feature_names: List[str] = field(default_factory=list)
    pooling: PoolingType = PoolingType.SUM
    init_fn: Optional[Callable[[torch.Tensor], None]] = None
    row_bytes: int = 0  # INT8 only: row stride (0 = 4 + dim rounded up to 4)


@dataclass
class EmbeddingConfig:
    """Mirrors torchrec.EmbeddingConfig (embedding.py:60-66)."""
    num_embeddings: int
    embedding_dim: int
    name: str = ""
    data_type: DataType = DataType.FP32
    feature_names: List[str] = field(default_factory=list)
    init_fn: Optional[Callable[[torch.Tensor], None]] = None
    pooling: PoolingType = PoolingType.NONE


@dataclass
class EmbeddingTableConfig:
    """Mirrors primus_dlrm.config.EmbeddingTableConfig (config.py:101-113)."""
    name: str = ""
    features: List[str] = field(default_factory=list)
    num_embeddings: int = 0
    embedding_dim: int = 0
    pooling: str = "none"


def _row_bytes(cfg) -> int:
    if cfg.data_type == DataType.INT8:
        rb = cfg.row_bytes if getattr(cfg, "row_bytes", 0) else (4 + cfg.embedding_dim + 3) & ~3
        if rb < 4 + cfg.embedding_dim or rb % 4:
            raise ValueError(f"table {cfg.name}: bad INT8 row_bytes {rb}")
        return rb
    return cfg.embedding_dim * torch.tensor([], dtype=_DT_TORCH[cfg.data_type]).element_size()


def _default_init(w: torch.Tensor) -> None:
    # TorchRec's default table init: U(-sqrt(1/rows), sqrt(1/rows)).
    bound = math.sqrt(1.0 / max(w.shape[0], 1))
    w.uniform_(-bound, bound)


_IN_BACKWARD_TAGS = ("_optimizer_classes", "_optimizer_kwargs", "_in_backward_optimizers")


class _TableWeight(nn.Module):
    def __init__(self, weight: torch.Tensor, previous: Optional[torch.Tensor] = None):
        super().__init__()
        # float tables require grad like TorchRec's, so _apply_optimizer_in_backward can tag them; their
        # gradient never materialises (the lookup's backward updates the rows in place)
        self.weight = nn.Parameter(weight, requires_grad=weight.is_floating_point())
        if previous is not None:  # keep in-backward optimizer tags across .to() / .cuda()
            for k in _IN_BACKWARD_TAGS:
                if hasattr(previous, k):
                    setattr(self.weight, k, getattr(previous, k))


def _collection_fused_optimizer(module) -> Optional[FusedEmbeddingOptimizer]:
    """The in-backward optimizer the tables of ``module`` (a collection with ``_tables`` and ``_store``) were
    tagged with by ``torch.distributed.optim._apply_optimizer_in_backward`` (None when untagged), created on
    first use and rebuilt when the tags or the device change."""
    tables, store = module._tables, module._store
    tags = [_optimizer_tag(store.weight(t.name)) for t in tables]
    if all(tg is None for tg in tags):
        return None
    if any(tg is None for tg in tags) or any(tg[0] is not tags[0][0] or tg[1] != tags[0][1] for tg in tags):
        raise NotImplementedError("every table of the collection needs the same in-backward optimizer")
    key = (tags[0][0], tuple(sorted((k, repr(v)) for k, v in tags[0][1].items())), store.flat.device)
    if module._fused is None or module._fused_key != key:
        fo = FusedEmbeddingOptimizer(
            tags[0][0], tags[0][1], store.total_bytes, store.flat.device, [t.name for t in tables],
            {t.name: t.num_embeddings for t in tables}, {t.name: t.embedding_dim for t in tables},
            {t.name: store.offsets[i] for i, t in enumerate(tables)})
        fo.param_groups[0]["params"] = [store.weight(t.name) for t in tables]
        module._fused, module._fused_key = fo, key
        module._fused_plans = {}
    return module._fused


_OWNERS: Dict[int, "weakref.ReferenceType"] = {}
_OWNER_IDS = itertools.count(1)


def _register_owner(module: nn.Module) -> int:
    """A process-wide id for ``module``.  The lookup ops carry it (an op's arguments are tensors and scalars)
    so their backward finds the module's fused optimizer and plans."""
    oid = next(_OWNER_IDS)
    _OWNERS[oid] = weakref.ref(module)
    weakref.finalize(module, _OWNERS.pop, oid, None)
    return oid


def _owner(oid: int):
    ref = _OWNERS.get(oid)
    module = ref() if ref is not None else None
    if module is None:
        raise RuntimeError(f"the embedding module of this lookup (owner {oid}) no longer exists")
    return module


class _LookupModule(nn.Module):
    """What the collections and the S-token gather share: an owner id, re-issued for copies, and lookup
    plans built eagerly whenever the tables move to a GPU, so a compiled forward only reads them."""

    _PLAN_ATTRS: Dict[str, Callable] = {}

    def _build_plans(self) -> None:
        pass

    def _refresh_plans(self) -> None:
        for name, empty in self._PLAN_ATTRS.items():
            old = getattr(self, name, None)
            for plan in (old.values() if isinstance(old, dict) else [old]):
                if plan is not None:
                    plan.release()
            setattr(self, name, empty())
        if self._tables_device().type == "cuda":
            self._build_plans()

    def _tables_device(self) -> torch.device:
        return self._store.flat.device

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        self._refresh_plans()
        return self

    def __getstate__(self):
        # plans hold device handles: a copy builds its own
        state = self.__dict__.copy()
        for name, empty in self._PLAN_ATTRS.items():
            state[name] = empty()
        return state

    def __setstate__(self, state):
        super().__setstate__(state)
        self._owner_id = _register_owner(self)
        self._refresh_plans()


class _FlatTables(nn.Module):
    """All tables of a collection in one uint8 device buffer, exposed as typed
    per-table ``weight`` views under ``<prefix>.<table>.weight``."""

    ALIGN = 256

    def __init__(self, configs: Sequence, prefix: str, device: torch.device, init_chunk_rows: int = 1 << 20):
        super().__init__()
        self._configs = list(configs)
        self._prefix = prefix
        self.offsets: List[int] = []
        off = 0
        for cfg in self._configs:
            off = (off + self.ALIGN - 1) // self.ALIGN * self.ALIGN
            self.offsets.append(off)
            off += cfg.num_embeddings * _row_bytes(cfg)
        self.total_bytes = max(off, 1)
        flat = torch.empty(self.total_bytes, dtype=torch.uint8, device=device)
        self.register_buffer("_flat", flat, persistent=False)
        setattr(self, prefix, nn.ModuleDict())
        self._make_views()
        self._initialise(init_chunk_rows)

    def _view(self, i: int) -> torch.Tensor:
        cfg = self._configs[i]
        rb = _row_bytes(cfg)
        raw = self._flat.narrow(0, self.offsets[i], cfg.num_embeddings * rb)
        if cfg.data_type == DataType.INT8:
            return raw.view(cfg.num_embeddings, rb)
        return raw.view(_DT_TORCH[cfg.data_type]).view(cfg.num_embeddings, cfg.embedding_dim)

    def _make_views(self) -> None:
        md = getattr(self, self._prefix)
        for i, cfg in enumerate(self._configs):
            prev = md[cfg.name].weight if cfg.name in md else None
            md[cfg.name] = _TableWeight(self._view(i), prev)

    @torch.no_grad()
    def _initialise(self, chunk: int) -> None:
        for i, cfg in enumerate(self._configs):
            init = cfg.init_fn or _default_init
            w = self._view(i)
            rows = cfg.num_embeddings
            if rows == 0:
                continue
            if cfg.data_type == DataType.FP32 and cfg.init_fn is not None:
                init(w)
                continue
            for r0 in range(0, rows, chunk):
                n = min(chunk, rows - r0)
                tmp = torch.empty((n, cfg.embedding_dim), dtype=torch.float32, device=w.device)
                if cfg.init_fn is None:
                    bound = math.sqrt(1.0 / rows)
                    tmp.uniform_(-bound, bound)
                else:
                    init(tmp)
                if cfg.data_type == DataType.INT8:
                    if w.device.type == "cuda":
                        w[r0:r0 + n].copy_(ops.int8_rowwise_quantize(tmp, _row_bytes(cfg)))
                    else:
                        w[r0:r0 + n].zero_()  # CPU construction: quantize after moving to the GPU
                else:
                    w[r0:r0 + n].copy_(tmp)

    def _apply(self, fn, recurse=True):
        # Keep the per-table parameters views of the (moved) flat buffer.
        self._flat = fn(self._flat)
        self._make_views()
        return self

    @property
    def flat(self) -> torch.Tensor:
        return self._flat

    def weight(self, name: str) -> torch.Tensor:
        return getattr(self, self._prefix)[name].weight


def _kjt_slot_offsets(kjt, order: List[str]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Returns (values, offsets) with bags laid out key-major in ``order``.

    Zero copy when the KJT already holds exactly ``order``; otherwise the keys are permuted on the device
    (pdm_kjt_permute, no host sync; TorchRec permutes the KJT the same way before its lookup)."""
    keys = list(kjt.keys())
    values = kjt.values()
    B = kjt.stride()
    offsets = kjt.offsets().to(torch.int64)
    if keys == order:
        return values, offsets
    pos = {k: i for i, k in enumerate(keys)}
    missing = [k for k in order if k not in pos]
    if missing:
        raise KeyError(f"KeyedJaggedTensor lacks features {missing}")
    v, _, o = torch.ops.pdm.kjt_permute(values, offsets.contiguous(), len(keys), B, [pos[k] for k in order])
    return v, o


class EmbeddingBagCollection(_LookupModule):
    """Pooled lookups of several tables in one table-batched launch per
    (dtype, dim) group.  Output ``KeyedTensor`` columns follow table order,
    then feature order inside a table (TorchRec's order)."""

    _PLAN_ATTRS = {"_plan": lambda: None, "_fused_plans": dict}

    def __init__(self, tables: List[EmbeddingBagConfig], device: Optional[torch.device] = None,
                 output_dtype: torch.dtype = torch.float32, is_weighted: bool = False):
        super().__init__()
        if is_weighted:
            raise NotImplementedError("per-sample weights are not on this path")
        if device is None:
            device = torch.device("cuda")
        device = torch.device(device)
        names = [t.name for t in tables]
        if len(set(names)) != len(names):
            raise ValueError("table names must be unique")
        for t in tables:
            if t.pooling not in (PoolingType.SUM, PoolingType.MEAN):
                raise ValueError(f"table {t.name}: EmbeddingBagCollection needs SUM or MEAN pooling")
            if t.embedding_dim % 4:
                raise ValueError(f"table {t.name}: embedding_dim must be a multiple of 4")
        self._tables = list(tables)
        self._output_dtype = output_dtype
        self._store = _FlatTables(tables, "embedding_bags", device)
        self._feature_names: List[str] = []
        self._dims: List[int] = []
        self._slots: List[dict] = []
        col = 0
        for i, t in enumerate(tables):
            for f in t.feature_names:
                self._feature_names.append(f)
                self._dims.append(t.embedding_dim)
                self._slots.append(dict(rows=t.num_embeddings, weights_offset=self._store.offsets[i],
                                        dim=t.embedding_dim, dtype=_DT_PDM[t.data_type],
                                        pooling=_POOL_PDM[t.pooling], row_bytes=_row_bytes(t), out_offset=col))
                col += t.embedding_dim
        self._total_dim = col
        self._plan: Optional[ops.TbePlan] = None
        self._fused: Optional[FusedEmbeddingOptimizer] = None
        self._fused_key = None
        self._fused_plans: Dict[str, ops.TbePlan] = {}
        self._owner_id = _register_owner(self)
        self._refresh_plans()

    # TorchRec-style accessors
    @property
    def embedding_bags(self) -> nn.ModuleDict:
        return self._store.embedding_bags

    def embedding_bag_configs(self) -> List[EmbeddingBagConfig]:
        return self._tables

    def feature_names(self) -> List[str]:
        return self._feature_names

    def state_dict(self, *args, **kwargs):
        sd = super().state_dict(*args, **kwargs)
        prefix = kwargs.get("prefix", args[1] if len(args) > 1 else "")
        return {k.replace(prefix + "_store.", prefix, 1): v for k, v in sd.items()}

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        with torch.no_grad():
            for t in self._tables:
                key = f"embedding_bags.{t.name}.weight"
                if key in state_dict:
                    self._store.weight(t.name).copy_(state_dict[key])
                elif strict:
                    raise KeyError(f"missing key {key}")
        return None

    def _build_plans(self) -> None:
        self._plan = ops.TbePlan(self._slots, self._tables_device())

    def _get_plan(self) -> ops.TbePlan:
        if self._plan is None:
            raise RuntimeError("the collection's tables are not on a GPU")
        return self._plan

    def pooled(self, values: torch.Tensor, offsets: torch.Tensor, batch_size: int,
               padding_idx: int = -1, err_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Raw table-batched call: ``offsets`` is ``[T*B+1]`` over this
        collection's feature order; returns ``[B, sum D]``."""
        return ops.tbe_pooled_raw(self._get_plan(), self._store.flat, values, offsets, batch_size,
                                  self._output_dtype, padding_idx, err_flag=err_flag)

    @property
    def fused_optimizer(self) -> Optional[FusedEmbeddingOptimizer]:
        """The in-backward optimizer the table weights were tagged with by
        ``torch.distributed.optim._apply_optimizer_in_backward`` (None when untagged); TorchRec's sharded
        model exposes the same as ``model.fused_optimizer`` (dist_trainer.py:298)."""
        return _collection_fused_optimizer(self)

    def _fused_plan(self) -> ops.TbePlan:
        """The lookup plan with its row-wise state offsets pointed at the fused optimizer's state."""
        plan = self._get_plan()
        if self._fused_plans.get("ebc") is not plan:
            fo = self._fused
            plan.set_state_offsets([fo.state_offset[t.name] for t in self._tables for _ in t.feature_names])
            self._fused_plans["ebc"] = plan
        return plan

    def pooled_lookup(self, values: torch.Tensor, offsets: torch.Tensor, padding_idx: int = -1) -> torch.Tensor:
        """Table-batched pooled lookup ``[B, sum D]`` over this collection's feature order (``offsets`` is
        ``[T*B+1]``), with autograd: when gradients are enabled and the tables require them, the backward
        is the fused backward + optimizer update of the tables' in-backward optimizer (pdm::tbe_fused_update)."""
        plan = self._get_plan()
        code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[self._output_dtype]
        tables = [self._store.weight(t.name) for t in self._tables]
        return torch.ops.pdm.tbe_pooled_fwd(self._store.flat, tables, values, offsets, plan.plan_id, plan.num_slots,
                                            self._total_dim, code, int(padding_idx), self._owner_id)

    def forward(self, features) -> KeyedTensor:
        values, offsets = _kjt_slot_offsets(features, self._feature_names)
        return KeyedTensor(self._feature_names, self._dims, self.pooled_lookup(values, offsets))


_NO_OPTIMIZER = ("the embedding tables have no in-backward optimizer: tag their weights with "
                 "torch.distributed.optim._apply_optimizer_in_backward(torch.optim.Adam or RowWiseAdagrad, ...) "
                 "as the reference's wrapper does (primus_dlrm/distributed/wrapper.py:151-174), or set "
                 "requires_grad=False on them; the lookup's backward is the fused update and produces no "
                 "weight gradient")


def _fused_optimizer_of(module) -> FusedEmbeddingOptimizer:
    fo = module.fused_optimizer
    if fo is None:
        raise NotImplementedError(_NO_OPTIMIZER)
    return fo


# The lookups' backward is the owner's fused backward + optimizer update: the table rows change in place and
# no weight gradient is produced, as with TorchRec's fused TBE.  Each update is an op that declares the
# collection buffer mutated, so a compiled backward keeps it and orders it.  The buffer is kept on the
# autograd context as an attribute, not a saved tensor: several lookups of one collection in one graph each
# update it, which a saved tensor's version check would reject.

@torch.library.custom_op("pdm::tbe_fused_update", mutates_args=("flat",))
def tbe_fused_update(flat: torch.Tensor, indices: torch.Tensor, offsets: torch.Tensor, grad_out: torch.Tensor,
                     num_slots: int, padding_idx: int, owner_id: int) -> None:
    """Fused backward + update of an EmbeddingBagCollection's pooled lookup (pdm_tbe_backward_fused); ids equal
    to ``padding_idx`` receive no update."""
    ebc = _owner(owner_id)
    fo = _fused_optimizer_of(ebc)
    batch = (offsets.numel() - 1) // num_slots
    fo.apply(ebc._fused_plan(), flat, indices.contiguous(), offsets.contiguous(), batch,
             grad_out.float().contiguous(), padding_idx=padding_idx)


@tbe_fused_update.register_fake
def _(flat, indices, offsets, grad_out, num_slots, padding_idx, owner_id):
    return None


def _pooled_setup(ctx, inputs, output):
    flat, tables, indices, offsets, _plan_id, num_slots, _total_dim, _code, padding_idx, owner_id = inputs
    ctx.flat = flat
    ctx.save_for_backward(indices, offsets)
    ctx.n_tables, ctx.num_slots, ctx.padding_idx, ctx.owner_id = len(tables), num_slots, padding_idx, owner_id


def _pooled_backward(ctx, grad_out):
    indices, offsets = ctx.saved_tensors
    torch.ops.pdm.tbe_fused_update(ctx.flat, indices, offsets, grad_out, ctx.num_slots, ctx.padding_idx,
                                   ctx.owner_id)
    return (None, [None] * ctx.n_tables) + (None,) * 8


ops.tbe_pooled_fwd.register_autograd(_pooled_backward, setup_context=_pooled_setup)


class EmbeddingCollection(_LookupModule):
    """Unpooled lookups: every id of feature f becomes row ``weight[id]`` of
    f's table, bit-exact (a one-id bag summed in fp32 and written in the
    table's dtype is the stored value)."""

    _PLAN_ATTRS = {"_plans": dict, "_fused_plans": dict}

    def __init__(self, tables: List[EmbeddingConfig], device: Optional[torch.device] = None):
        super().__init__()
        if device is None:
            device = torch.device("cuda")
        device = torch.device(device)
        for t in tables:
            if t.data_type == DataType.INT8:
                raise ValueError("EmbeddingCollection tables must be FP32, FP16 or BF16")
            if t.embedding_dim % 4:
                raise ValueError(f"table {t.name}: embedding_dim must be a multiple of 4")
        self._tables = list(tables)
        self._store = _FlatTables(tables, "embeddings", device)
        self._feature_names: List[str] = []
        self._feature_table: Dict[str, int] = {}
        for i, t in enumerate(tables):
            for f in t.feature_names:
                self._feature_names.append(f)
                self._feature_table[f] = i
        self._plans: Dict[int, ops.TbePlan] = {}
        self._fused: Optional[FusedEmbeddingOptimizer] = None
        self._fused_key = None
        self._fused_plans: Dict[str, ops.TbePlan] = {}
        self._owner_id = _register_owner(self)
        self._refresh_plans()

    @property
    def fused_optimizer(self) -> Optional[FusedEmbeddingOptimizer]:
        """The in-backward optimizer of the collection's tables (see EmbeddingBagCollection.fused_optimizer);
        the S-token gather over these tables updates them through it."""
        return _collection_fused_optimizer(self)

    @property
    def embeddings(self) -> nn.ModuleDict:
        return self._store.embeddings

    def embedding_configs(self) -> List[EmbeddingConfig]:
        return self._tables

    def feature_names(self) -> List[str]:
        return self._feature_names

    def table_of(self, feature: str) -> torch.Tensor:
        return self._store.weight(self._tables[self._feature_table[feature]].name)

    def state_dict(self, *args, **kwargs):
        sd = super().state_dict(*args, **kwargs)
        prefix = kwargs.get("prefix", args[1] if len(args) > 1 else "")
        return {k.replace(prefix + "_store.", prefix, 1): v for k, v in sd.items()}

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        with torch.no_grad():
            for t in self._tables:
                key = f"embeddings.{t.name}.weight"
                if key in state_dict:
                    self._store.weight(t.name).copy_(state_dict[key])
                elif strict:
                    raise KeyError(f"missing key {key}")
        return None

    def _build_plans(self) -> None:
        for ti, t in enumerate(self._tables):
            self._plans[ti] = ops.TbePlan([dict(rows=t.num_embeddings, weights_offset=self._store.offsets[ti],
                                                dim=t.embedding_dim, dtype=_DT_PDM[t.data_type],
                                                pooling=L.PDM_POOL_SUM, row_bytes=_row_bytes(t),
                                                out_offset=0)], self._tables_device())

    def _gather_table(self, ti: int, ids: torch.Tensor) -> torch.Tensor:
        """``weight[ids]`` of table ``ti`` for a flat id vector: ``[n, D]`` (one-id bags)."""
        if ti not in self._plans:
            raise RuntimeError("the collection's tables are not on a GPU")
        ids = ids.reshape(-1).contiguous()
        n = ids.numel()
        offsets = torch.arange(n + 1, dtype=torch.int64, device=ids.device)
        return ops.tbe_pooled_raw(self._plans[ti], self._store.flat, ids, offsets, n,
                                  _DT_TORCH[self._tables[ti].data_type])

    def gather(self, feature: str, ids: torch.Tensor) -> torch.Tensor:
        """``weight[ids]`` for a flat id vector of ``feature``: ``[n, D]``."""
        return self._gather_table(self._feature_table[feature], ids)

    def _fused_plan(self, table_index: Sequence[int]) -> ops.TbePlan:
        """One slot per looked-up feature (its table ``table_index[k]``, sum, the feature's column) with the
        optimizer's state offsets."""
        key = f"ec:{tuple(table_index)}"
        if key not in self._fused_plans:
            slots, col = [], 0
            for ti in table_index:
                t = self._tables[ti]
                slots.append(dict(rows=t.num_embeddings, weights_offset=self._store.offsets[ti], dim=t.embedding_dim,
                                  dtype=_DT_PDM[t.data_type], pooling=L.PDM_POOL_SUM, row_bytes=_row_bytes(t),
                                  out_offset=col))
                col += t.embedding_dim
            plan = ops.TbePlan(slots, self._store.flat.device)
            plan.set_state_offsets([self._fused.state_offset[self._tables[ti].name] for ti in table_index])
            self._fused_plans[key] = plan
        return self._fused_plans[key]

    def lookup(self, names: Sequence[str], ids: Sequence[torch.Tensor]) -> List[torch.Tensor]:
        """``weight[ids]`` ``[n_f, D_f]`` per feature, with autograd: when gradients are enabled and the tables
        require them, the backward is the fused update of the tables' in-backward optimizer."""
        if not names:
            return []
        segs = [i.reshape(-1) for i in ids]
        tables = [self._store.weight(t.name) for t in self._tables]
        return list(torch.ops.pdm.ec_lookup(self._store.flat, tables, segs,
                                            [self._feature_table[n] for n in names], self._owner_id))

    def forward(self, features) -> Dict[str, JaggedTensor]:
        keys = list(features.keys())
        B = features.stride()
        offsets = features.offsets().to(torch.int64)
        bounds = offsets.view(-1)[:: B] if B > 0 else offsets[:1]
        starts = bounds.tolist()  # per-key value ranges: one host sync, as TorchRec's length_per_key()
        values = features.values()
        names, segs, seg_offs = [], [], []
        for k, name in enumerate(keys):
            if name not in self._feature_table:
                continue
            lo, hi = starts[k], starts[k + 1]
            names.append(name)
            segs.append(values[lo:hi])
            seg_offs.append(offsets[k * B:(k + 1) * B + 1] - lo)
        rows = self.lookup(names, segs)
        return {n: JaggedTensor(r, offsets=o) for n, r, o in zip(names, rows, seg_offs)}


@torch.library.custom_op("pdm::ec_lookup", mutates_args=())
def ec_lookup(flat: torch.Tensor, tables: List[torch.Tensor], ids: List[torch.Tensor], table_index: List[int],
              owner_id: int) -> List[torch.Tensor]:
    """``tables[table_index[k]][ids[k]]`` per looked-up feature k, read from the collection buffer ``flat``."""
    ec = _owner(owner_id)
    return [ec._gather_table(ti, seg) for ti, seg in zip(table_index, ids)]


@ec_lookup.register_fake
def _(flat, tables, ids, table_index, owner_id):
    return [tables[ti].new_empty((seg.shape[0], tables[ti].shape[1])) for ti, seg in zip(table_index, ids)]


@torch.library.custom_op("pdm::ec_fused_update", mutates_args=("flat",))
def ec_fused_update(flat: torch.Tensor, ids: List[torch.Tensor], grads: List[torch.Tensor], table_index: List[int],
                    owner_id: int) -> None:
    """Fused backward + update of an EmbeddingCollection's unpooled lookups (pdm_tbe_backward_fused): every id
    of feature k is a one-id bag of slot k; the features' bag counts are padded to the largest with empty
    bags, and the output gradients are laid side by side in one [max n_k, sum D] buffer."""
    ec = _owner(owner_id)
    fo = _fused_optimizer_of(ec)
    dev = flat.device
    ns = [int(seg.numel()) for seg in ids]
    dims = [ec._tables[ti].embedding_dim for ti in table_index]
    bags = max(ns)
    g_all = torch.zeros((bags, sum(dims)), dtype=torch.float32, device=dev)
    col = 0
    for gr, n, d in zip(grads, ns, dims):
        g_all[:n, col:col + d] = gr
        col += d
    ar = torch.arange(bags, device=dev)
    lengths = torch.cat([(ar < n).to(torch.int64) for n in ns])
    offsets = torch.nn.functional.pad(lengths.cumsum(0), (1, 0))
    fo.apply(ec._fused_plan(table_index), flat, torch.cat([seg.contiguous() for seg in ids]), offsets, bags, g_all)


@ec_fused_update.register_fake
def _(flat, ids, grads, table_index, owner_id):
    return None


def _ec_setup(ctx, inputs, output):
    flat, tables, ids, table_index, owner_id = inputs
    ctx.flat = flat
    ctx.save_for_backward(*ids)
    ctx.n_tables, ctx.table_index, ctx.owner_id = len(tables), list(table_index), owner_id


def _ec_backward(ctx, grads):
    ids = list(ctx.saved_tensors)
    torch.ops.pdm.ec_fused_update(ctx.flat, ids, [g.contiguous() for g in grads], ctx.table_index, ctx.owner_id)
    return None, [None] * ctx.n_tables, [None] * len(ids), None, None


ec_lookup.register_autograd(_ec_backward, setup_context=_ec_setup)


class SequenceGather(_LookupModule):
    """Jagged behaviour-pool ids -> padded S-token rows on the device.

    ``sequence_groups`` maps a pool name to its features (concat order per
    event, e.g. ``{"hist_lp": ["hist_lp_item", "hist_lp_artist", "hist_lp_album"], ...}``,
    reference: configs/bench_onetrans_v6.yaml:33-35, onetrans.py:515-520).
    Feature ``f`` is looked up in ``tables[feature_table[f]]`` (an
    ``EmbeddingCollection``'s tables).  Pools are laid out along the sequence
    in ``sequence_groups`` order, each padded to ``max_len[pool]``.

    ``pad_mode="row0"`` with ``align="right"`` reproduces the reference
    exactly (left padding with id 0, whose lookup is table row 0);
    ``pad_mode="zero"`` writes zero rows instead.
    """

    def __init__(self, ec: EmbeddingCollection, sequence_groups: Dict[str, List[str]],
                 max_len: Dict[str, int] | int, pad_mode: str = "row0", align: str = "right"):
        super().__init__()
        self.ec = ec
        self.groups = {g: list(fs) for g, fs in sequence_groups.items()}
        nfeat = {len(fs) for fs in self.groups.values()}
        if len(nfeat) != 1:
            raise ValueError("every pool must list the same number of features")
        self.max_len = {g: (max_len if isinstance(max_len, int) else int(max_len[g])) for g in self.groups}
        self.pad_mode = {"row0": L.PDM_PAD_ROW0, "zero": L.PDM_PAD_ZERO}[pad_mode]
        self.align = {"right": L.PDM_ALIGN_RIGHT, "left": L.PDM_ALIGN_LEFT}[align]
        first = next(iter(self.groups.values()))
        # the k-th feature of every pool must use the same table as the first pool's
        for fs in self.groups.values():
            for a, b in zip(fs, first):
                if self.ec._feature_table[a] != self.ec._feature_table[b]:
                    raise ValueError("the k-th feature of every pool must share one table")
        self._feature_tables = [ec._feature_table[f] for f in first]
        self._owner_id = _register_owner(self)

    def _tables_device(self) -> torch.device:
        return self.ec._store.flat.device

    def slot_ranges(self) -> Dict[str, Tuple[int, int]]:
        out, s = {}, 0
        for g in self.groups:
            out[g] = (s, self.max_len[g])
            s += self.max_len[g]
        return out

    def forward(self, batch: Dict[str, torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
        """``batch[f]`` is the flat int64 id vector of feature f and
        ``batch[f + "__lengths"]`` its per-sample lengths (the pipeline-batch
        convention of primus_dlrm/data/synthetic.py:224-228); every feature of
        a pool shares its lengths.  Returns (tokens ``[B, S, sum D]``,
        mask bool ``[B, S]``)."""
        tables = [self.ec._store.weight(self.ec._tables[ti].name) for ti in self._feature_tables]
        ids, offsets, max_len = [], [], []
        for g, fs in self.groups.items():
            lengths = batch[fs[0] + "__lengths"]
            offsets.append(torch.nn.functional.pad(lengths.reshape(-1).to(torch.int64).cumsum(0), (1, 0)))
            ids.extend(batch[f].reshape(-1).to(torch.int64).contiguous() for f in fs)
            max_len.append(self.max_len[g])
        out, mask = torch.ops.pdm.seq_gather_fwd(self.ec._store.flat, tables, ids, offsets, max_len, self.pad_mode,
                                                 self.align, self._owner_id)
        return out, mask_as_bool(mask)

    def _fused_plan(self) -> ops.TbePlan:
        """One slot per feature (fp32 table, sum, column of the feature) with the EC optimizer's state offsets."""
        ec = self.ec
        fo = ec._fused
        key = f"seq:{id(self)}:{ec._store.flat.device}"
        if key not in ec._fused_plans:
            slots, col = [], 0
            for ti in self._feature_tables:
                t = ec._tables[ti]
                slots.append(dict(rows=t.num_embeddings, weights_offset=ec._store.offsets[ti], dim=t.embedding_dim,
                                  dtype=_DT_PDM[t.data_type], pooling=L.PDM_POOL_SUM, row_bytes=_row_bytes(t),
                                  out_offset=col))
                col += t.embedding_dim
            plan = ops.TbePlan(slots, ec._store.flat.device)
            plan.set_state_offsets([fo.state_offset[ec._tables[ti].name] for ti in self._feature_tables])
            ec._fused_plans[key] = plan
        return ec._fused_plans[key]


@torch.library.custom_op("pdm::seq_fused_update", mutates_args=("flat",))
def seq_fused_update(flat: torch.Tensor, ids: List[torch.Tensor], offsets: List[torch.Tensor], max_len: List[int],
                     grad_out: torch.Tensor, owner_id: int) -> None:
    """Fused backward + update of a SequenceGather's tables (pdm_seq_gather_backward_fused); ``ids`` is
    pool-major as for pdm::seq_gather_fwd."""
    sg = _owner(owner_id)
    ec = sg.ec
    fo = _fused_optimizer_of(ec)
    tabs = [ec._tables[ti] for ti in sg._feature_tables]
    F = len(tabs)
    grid = [ids[p * F:(p + 1) * F] for p in range(len(offsets))]
    fo.apply_seq(sg._fused_plan(), flat, [t.num_embeddings for t in tabs], [t.embedding_dim for t in tabs], grid,
                 offsets, max_len, grad_out.float().contiguous(), sg.pad_mode, sg.align)


@seq_fused_update.register_fake
def _(flat, ids, offsets, max_len, grad_out, owner_id):
    return None


def _seq_setup(ctx, inputs, output):
    flat, tables, ids, offsets, max_len, _pad_mode, _align, owner_id = inputs
    ctx.flat = flat
    ctx.save_for_backward(*ids, *offsets)
    ctx.n_tables, ctx.n_ids, ctx.max_len, ctx.owner_id = len(tables), len(ids), list(max_len), owner_id
    ctx.set_materialize_grads(False)


def _seq_backward(ctx, grad_out, _grad_mask):
    saved = ctx.saved_tensors
    ids, offsets = list(saved[:ctx.n_ids]), list(saved[ctx.n_ids:])
    if grad_out is not None:
        torch.ops.pdm.seq_fused_update(ctx.flat, ids, offsets, ctx.max_len, grad_out, ctx.owner_id)
    return None, [None] * ctx.n_tables, [None] * len(ids), [None] * len(offsets), None, None, None, None


ops.seq_gather_fwd.register_autograd(_seq_backward, setup_context=_seq_setup)


class TorchRecEmbeddings(nn.Module):
    """Tensor-in / tensor-out lookup wrapper with the reference's constructor
    and forward (primus_dlrm/models/embedding.py:72-174).

    Pooled features: ``[B, L] -> [B, D]`` with ids equal to ``padding_idx``
    skipped on the device (the reference removes them with boolean indexing
    and a host sync in _build_pooled_kjt, embedding.py:179-204; here no sync).
    Unpooled: ``[B] -> [B, D]``, ``[B, L] -> [B, L, D]``.
    """

    _POOLING = {"sum": PoolingType.SUM, "mean": PoolingType.MEAN}

    def __init__(self, table_specs: List[EmbeddingTableConfig], device: Optional[torch.device] = None,
                 embedding_init: str = "uniform", scalar_feature_names: Optional[set] = None,
                 data_type: DataType = DataType.FP32):
        super().__init__()
        if device is None:
            device = torch.device("cuda")
        init_fn = None
        if embedding_init == "normal":
            def init_fn(w: torch.Tensor) -> None:
                nn.init.normal_(w, mean=0.0, std=1.0)
        pooled, unpooled = [], []
        self._pooled_features: List[str] = []
        self._unpooled_features: List[str] = []
        self._feature_dims: Dict[str, int] = {}
        for spec in table_specs:
            for feat in spec.features:
                self._feature_dims[feat] = spec.embedding_dim
            if spec.pooling in self._POOLING:
                pooled.append(EmbeddingBagConfig(spec.num_embeddings, spec.embedding_dim, spec.name, data_type,
                                                 list(spec.features), self._POOLING[spec.pooling], init_fn))
                self._pooled_features.extend(spec.features)
            else:
                unpooled.append(EmbeddingConfig(spec.num_embeddings, spec.embedding_dim, spec.name, data_type,
                                                list(spec.features), init_fn))
                self._unpooled_features.extend(spec.features)
        self._pooled_set = set(self._pooled_features)
        self._unpooled_set = set(self._unpooled_features)
        self._scalar_features = (set(scalar_feature_names) & self._unpooled_set) if scalar_feature_names else set()
        self.ebc = EmbeddingBagCollection(pooled, device) if pooled else None
        self.ec = EmbeddingCollection(unpooled, device) if unpooled else None

    def forward(self, features: Dict[str, torch.Tensor], padding_idx: int = 0) -> Dict[str, torch.Tensor]:
        results: Dict[str, torch.Tensor] = {}
        if self.ebc is not None:
            present = [f for f in self._pooled_features if f in features]
            if present:
                if len(present) != len(self._pooled_features):
                    raise KeyError(f"pooled lookup needs every pooled feature, missing "
                                   f"{sorted(self._pooled_set - set(present))}")
                B = features[present[0]].shape[0]
                vals, offs, base = [], [], 0
                for f in present:
                    ids = features[f]
                    if ids.dim() == 1:
                        ids = ids.unsqueeze(1)
                    if ids.shape[0] != B:
                        raise ValueError("pooled features must share the batch size")
                    Lf = ids.shape[1]
                    vals.append(ids.reshape(-1))
                    offs.append(torch.arange(B, device=ids.device, dtype=torch.int64) * Lf + base)
                    base += B * Lf
                offs.append(torch.full((1,), base, dtype=torch.int64, device=vals[0].device))
                values = torch.cat(vals) if len(vals) > 1 else vals[0].contiguous()
                if values.dtype not in (torch.int32, torch.int64):
                    values = values.to(torch.int64)
                out = self.ebc.pooled_lookup(values, torch.cat(offs), padding_idx)
                col = 0
                for f in self._pooled_features:
                    D = self._feature_dims[f]
                    results[f] = out[:, col:col + D]
                    col += D
        if self.ec is not None:
            present = [f for f in self._unpooled_features if f in features]
            for f, rows in zip(present, self.ec.lookup(present, [features[f] for f in present])):
                D = self._feature_dims[f]
                B = features[f].shape[0]
                results[f] = rows.view(B, D) if f in self._scalar_features else rows.view(B, -1, D)
        return results
