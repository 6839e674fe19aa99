"""PyTorch custom ops over the C ABI (include/pdm.h).

Each op validates shapes, dtypes and devices on the host, then enqueues the
HIP kernels of libpdm.so on torch's current stream.  Ops are registered with
``torch.library.custom_op`` and carry fake (meta) kernels, so FX tracing and
``torch.compile(dynamic=True, fullgraph=True)`` see them as single opaque nodes
(the reference compiles its blocks that way: primus_dlrm/models/onetrans.py:382-390).
The lookup ops also take the per-table weight views and the id of the module
that owns them: the views make autograd record the lookup when the tables
require gradients, and the backward registered for the op (in embedding.py)
runs the owner's fused optimizer update as an op that mutates the tables.

There is no CPU implementation: called with CPU tensors these ops raise.
"""
from __future__ import annotations

import ctypes
import itertools
import threading
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib as L

TORCH_TO_PDM = {torch.float32: L.PDM_F32, torch.float16: L.PDM_F16, torch.bfloat16: L.PDM_BF16}
PDM_TO_TORCH = {v: k for k, v in TORCH_TO_PDM.items()}


def _require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"pdm ops run on the GPU only; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# Pooled TBE
# ---------------------------------------------------------------------------

class TbePlan:
    """A pdm_tbe_plan: per-slot table metadata resident on one device.

    ``slots`` are dicts with keys rows, weights_offset, dim, dtype (pdm
    dtype), pooling (pdm pooling), row_bytes, out_offset.  A slot is one
    pooled output (one feature); several slots may share a table.
    """

    _registry: Dict[int, "TbePlan"] = {}
    _ids = itertools.count(1)
    _lock = threading.Lock()

    def __init__(self, slots: Sequence[dict], device: torch.device):
        if not slots:
            raise ValueError("a TBE plan needs at least one table slot")
        arr = (L.TableDesc * len(slots))()
        for i, s in enumerate(slots):
            arr[i] = L.TableDesc(int(s["rows"]), int(s["weights_offset"]), int(s["dim"]), int(s["dtype"]),
                                 int(s["pooling"]), int(s.get("row_bytes", 0)), int(s["out_offset"]), 0)
        handle = ctypes.c_void_p()
        with torch.cuda.device(device):
            L.check(L.lib().pdm_tbe_plan_create(arr, len(slots), ctypes.byref(handle)), "pdm_tbe_plan_create")
        self.handle = handle
        self.device = torch.device(device)
        self.num_slots = len(slots)
        self.dims = [int(s["dim"]) for s in slots]
        self.fp32_extent = max(int(s["weights_offset"]) + int(s["rows"]) * 4 * int(s["dim"]) for s in slots)
        self.total_dim = int(L.lib().pdm_tbe_plan_total_dim(handle))
        self.total_rows = int(L.lib().pdm_tbe_plan_total_rows(handle))
        self.row_offsets = [int(L.lib().pdm_tbe_plan_row_offset(handle, i)) for i in range(len(slots))]
        with TbePlan._lock:
            self.plan_id = next(TbePlan._ids)
            TbePlan._registry[self.plan_id] = self

    def set_state_offsets(self, offsets: Sequence[int]) -> None:
        """Row-wise optimizer state index of row 0 of each slot's table (pdm_tbe_plan_set_state_offsets)."""
        if len(offsets) != self.num_slots:
            raise ValueError("one state offset per slot")
        arr = (ctypes.c_int64 * self.num_slots)(*[int(v) for v in offsets])
        with torch.cuda.device(self.device):
            L.check(L.lib().pdm_tbe_plan_set_state_offsets(self.handle, arr), "pdm_tbe_plan_set_state_offsets")

    def release(self) -> None:
        if self.handle is not None and self.handle.value:
            with TbePlan._lock:
                TbePlan._registry.pop(self.plan_id, None)
            L.lib().pdm_tbe_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    @staticmethod
    def get(plan_id: int) -> "TbePlan":
        try:
            return TbePlan._registry[plan_id]
        except KeyError:
            raise RuntimeError(f"TBE plan {plan_id} does not exist (released?)") from None


def tbe_pooled_raw(plan: TbePlan, weights: torch.Tensor, indices: torch.Tensor, offsets: torch.Tensor,
                   batch_size: int, out_dtype: torch.dtype = torch.float32, padding_idx: int = -1,
                   out: Optional[torch.Tensor] = None, err_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Launches pdm_tbe_pooled_fwd; returns ``out`` ([B, total_dim])."""
    dev = _require_cuda(weights, indices, offsets, out, err_flag)
    if indices.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"indices must be int32 or int64, got {indices.dtype}")
    if offsets.dtype != torch.int64:
        raise TypeError(f"offsets must be int64, got {offsets.dtype}")
    if not (weights.is_contiguous() and indices.is_contiguous() and offsets.is_contiguous()):
        raise ValueError("weights, indices and offsets must be contiguous")
    if offsets.numel() != plan.num_slots * batch_size + 1:
        raise ValueError(f"offsets has {offsets.numel()} entries, expected T*B+1 = "
                         f"{plan.num_slots * batch_size + 1}")
    if out_dtype not in TORCH_TO_PDM:
        raise TypeError(f"unsupported output dtype {out_dtype}")
    if out is None:
        out = torch.empty((batch_size, plan.total_dim), dtype=out_dtype, device=dev)
    elif out.dim() != 2 or out.shape[0] != batch_size or out.stride(1) != 1 or out.dtype != out_dtype:
        raise ValueError("out must be [B, >=total_dim] with unit column stride and the requested dtype")
    if out.shape[1] < plan.total_dim:
        raise ValueError("out has fewer columns than the plan writes")
    if err_flag is not None and (err_flag.dtype != torch.int32 or err_flag.numel() < 1):
        raise ValueError("err_flag must be an int32 tensor with at least one element")
    status = L.lib().pdm_tbe_pooled_fwd(
        plan.handle, weights.data_ptr(), indices.data_ptr() if indices.numel() else None,
        32 if indices.dtype == torch.int32 else 64, indices.numel(), offsets.data_ptr(), batch_size,
        padding_idx, out.data_ptr(), TORCH_TO_PDM[out_dtype], out.stride(0), _ptr(err_flag),
        L.stream_ptr(dev))
    L.check(status, "pdm_tbe_pooled_fwd")
    return out


def tbe_backward_workspace(plan: TbePlan, num_indices: int, batch_size: int, device=None) -> torch.Tensor:
    """Device workspace for pdm_tbe_backward_fused / _sparse_grad over ``num_indices`` lookups in
    ``batch_size`` bags per slot."""
    n = int(L.lib().pdm_tbe_backward_workspace_size(plan.handle, int(num_indices), int(batch_size)))
    if n < 0:
        raise ValueError("bad plan or num_indices")
    return torch.empty(n, dtype=torch.uint8, device=device if device is not None else plan.device)


def _check_bwd_inputs(plan: TbePlan, indices, offsets, batch_size, grad_out, workspace):
    if indices.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"indices must be int32 or int64, got {indices.dtype}")
    if offsets.dtype != torch.int64:
        raise TypeError(f"offsets must be int64, got {offsets.dtype}")
    if not (indices.is_contiguous() and offsets.is_contiguous()):
        raise ValueError("indices and offsets must be contiguous")
    if offsets.numel() != plan.num_slots * batch_size + 1:
        raise ValueError(f"offsets has {offsets.numel()} entries, expected T*B+1 = "
                         f"{plan.num_slots * batch_size + 1}")
    if grad_out.dtype != torch.float32 or grad_out.dim() != 2 or grad_out.shape[0] != batch_size \
            or (grad_out.numel() and grad_out.stride(1) != 1) or grad_out.shape[1] < plan.total_dim:
        raise ValueError("grad_out must be float32 [B, >= total_dim] with unit column stride")
    if workspace is None:
        workspace = tbe_backward_workspace(plan, indices.numel(), batch_size, grad_out.device)
    if workspace.dtype != torch.uint8 or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 tensor")
    return workspace


def tbe_backward_fused_raw(plan: TbePlan, weights: torch.Tensor, momentum1: torch.Tensor,
                           momentum2: Optional[torch.Tensor], indices: torch.Tensor, offsets: torch.Tensor,
                           batch_size: int, grad_out: torch.Tensor, optimizer: int = L.PDM_OPT_ADAM,
                           learning_rate: float = 0.01, eps: float = 1e-8, beta1: float = 0.9,
                           beta2: float = 0.999, weight_decay: float = 0.0, weight_decay_mode: int = L.PDM_WD_NONE,
                           step: int = 1, padding_idx: int = -1, workspace: Optional[torch.Tensor] = None,
                           err_flag: Optional[torch.Tensor] = None) -> None:
    """Launches pdm_tbe_backward_fused: updates ``weights`` (the plan's fp32 table buffer) and the
    optimizer state in place from d(loss)/d(pooled output) ``grad_out`` [B, >= total_dim]."""
    dev = _require_cuda(weights, momentum1, momentum2, indices, offsets, grad_out, workspace, err_flag)
    workspace = _check_bwd_inputs(plan, indices, offsets, batch_size, grad_out, workspace)
    for name, t in (("weights", weights), ("momentum1", momentum1), ("momentum2", momentum2)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if momentum1.dtype != torch.float32 or (momentum2 is not None and momentum2.dtype != torch.float32):
        raise TypeError("optimizer state must be float32")

    def nbytes(t):
        return t.numel() * t.element_size()

    if nbytes(weights) < plan.fp32_extent:
        raise ValueError("weights is smaller than the plan's fp32 tables")
    if optimizer == L.PDM_OPT_ADAM:
        if momentum2 is None or nbytes(momentum1) < plan.fp32_extent or nbytes(momentum2) < plan.fp32_extent:
            raise ValueError("Adam state must be laid out like the weights (as many bytes)")
    elif momentum1.numel() < plan.total_rows:
        raise ValueError(f"row-wise state needs {plan.total_rows} entries (one per row id)")
    if err_flag is not None and (err_flag.dtype != torch.int32 or err_flag.numel() < 1):
        raise ValueError("err_flag must be an int32 tensor with at least one element")
    opt = L.OptimParams(int(optimizer), int(weight_decay_mode), float(learning_rate), float(eps), float(beta1),
                        float(beta2), float(weight_decay), 0, int(step))
    status = L.lib().pdm_tbe_backward_fused(
        plan.handle, weights.data_ptr(), momentum1.data_ptr(), _ptr(momentum2),
        indices.data_ptr() if indices.numel() else None, 32 if indices.dtype == torch.int32 else 64,
        indices.numel(), offsets.data_ptr(), batch_size, padding_idx, grad_out.data_ptr(), grad_out.stride(0),
        ctypes.byref(opt), workspace.data_ptr(), workspace.numel(), _ptr(err_flag), L.stream_ptr(dev))
    L.check(status, "pdm_tbe_backward_fused")


def tbe_backward_sparse_grad_raw(plan: TbePlan, indices: torch.Tensor, offsets: torch.Tensor, batch_size: int,
                                 grad_out: torch.Tensor, padding_idx: int = -1,
                                 workspace: Optional[torch.Tensor] = None,
                                 err_flag: Optional[torch.Tensor] = None):
    """Launches pdm_tbe_backward_sparse_grad; returns (row_ids [N] int64, grad_rows [N, D] float32,
    num_unique int64 scalar tensor): the first num_unique entries are the distinct row ids (ascending)
    and their gradients."""
    dev = _require_cuda(indices, offsets, grad_out, workspace, err_flag)
    workspace = _check_bwd_inputs(plan, indices, offsets, batch_size, grad_out, workspace)
    n = max(indices.numel(), 1)
    if len(set(plan.dims)) != 1:
        raise ValueError("the sparse gradient needs one dim across the plan")
    D = plan.dims[0]
    row_ids = torch.empty(n, dtype=torch.int64, device=dev)
    grad_rows = torch.empty((n, D), dtype=torch.float32, device=dev)
    num_unique = torch.empty((), dtype=torch.int64, device=dev)
    status = L.lib().pdm_tbe_backward_sparse_grad(
        plan.handle, indices.data_ptr() if indices.numel() else None, 32 if indices.dtype == torch.int32 else 64,
        indices.numel(), offsets.data_ptr(), batch_size, padding_idx, grad_out.data_ptr(), grad_out.stride(0),
        row_ids.data_ptr(), grad_rows.data_ptr(), num_unique.data_ptr(), workspace.data_ptr(), workspace.numel(),
        _ptr(err_flag), L.stream_ptr(dev))
    L.check(status, "pdm_tbe_backward_sparse_grad")
    return row_ids, grad_rows, num_unique


# ---------------------------------------------------------------------------
# KeyedJaggedTensor construction
# ---------------------------------------------------------------------------

def kjt_from_dense_raw(features: Sequence[torch.Tensor], padding_idx: int = -1):
    """Dense [B, L_f] id matrices (one dtype, int32 or int64) -> (values, lengths int32 [F*B], offsets int64
    [F*B+1]) with every id equal to ``padding_idx`` removed (pdm_kjt_from_dense).  ``values`` has the inputs'
    total id count as capacity; its first ``offsets[-1]`` entries are the kept ids."""
    if not features:
        raise ValueError("need at least one feature")
    if len(features) > L.PDM_KJT_MAX_FEATURES:
        raise ValueError(f"at most {L.PDM_KJT_MAX_FEATURES} features")
    dev = _require_cuda(*features)
    dt = features[0].dtype
    if dt not in (torch.int32, torch.int64):
        raise TypeError("ids must be int32 or int64")
    B = features[0].shape[0]
    feats = []
    for t in features:
        if t.dtype != dt or t.dim() != 2 or t.shape[0] != B:
            raise ValueError("features must be [B, L_f] tensors of one dtype and one B")
        feats.append(t.contiguous())
    F = len(feats)
    cap = sum(t.numel() for t in feats)
    values = torch.empty(max(cap, 1), dtype=dt, device=dev)
    lengths = torch.empty(F * B, dtype=torch.int32, device=dev)
    offsets = torch.empty(F * B + 1, dtype=torch.int64, device=dev)
    ws = torch.empty(int(L.lib().pdm_kjt_workspace_size(F * B)), dtype=torch.uint8, device=dev)
    ids_arr = (ctypes.c_void_p * F)(*[t.data_ptr() if t.numel() else None for t in feats])
    len_arr = (ctypes.c_int32 * F)(*[t.shape[1] for t in feats])
    L.check(L.lib().pdm_kjt_from_dense(ids_arr, len_arr, F, B, 32 if dt == torch.int32 else 64, int(padding_idx),
                                       values.data_ptr(), lengths.data_ptr(), offsets.data_ptr(), ws.data_ptr(),
                                       ws.numel(), L.stream_ptr(dev)), "pdm_kjt_from_dense")
    return values[:cap], lengths, offsets


def kjt_permute_raw(values: torch.Tensor, offsets: torch.Tensor, num_keys: int, batch_size: int,
                    perm: Sequence[int]):
    """Key permutation of a KJT on the device (pdm_kjt_permute): output key k is input key perm[k].
    Returns (values with the input's capacity, lengths int32, offsets int64)."""
    dev = _require_cuda(values, offsets)
    if values.dtype not in (torch.int32, torch.int64):
        raise TypeError("values must be int32 or int64")
    if offsets.dtype != torch.int64 or offsets.numel() != num_keys * batch_size + 1 or not offsets.is_contiguous():
        raise ValueError("offsets must be contiguous int64 [num_keys * B + 1]")
    if len(perm) > L.PDM_KJT_MAX_FEATURES:
        raise ValueError(f"at most {L.PDM_KJT_MAX_FEATURES} output keys")
    values = values.contiguous()
    K = len(perm)
    out_v = torch.empty(max(values.numel(), 1), dtype=values.dtype, device=dev)
    out_l = torch.empty(K * batch_size, dtype=torch.int32, device=dev)
    out_o = torch.empty(K * batch_size + 1, dtype=torch.int64, device=dev)
    ws = torch.empty(int(L.lib().pdm_kjt_workspace_size(K * batch_size)), dtype=torch.uint8, device=dev)
    perm_arr = (ctypes.c_int32 * max(K, 1))(*[int(p) for p in perm])
    L.check(L.lib().pdm_kjt_permute(values.data_ptr() if values.numel() else None,
                                    32 if values.dtype == torch.int32 else 64, offsets.data_ptr(), num_keys,
                                    batch_size, perm_arr, K, out_v.data_ptr(), out_l.data_ptr(), out_o.data_ptr(),
                                    ws.data_ptr(), ws.numel(), L.stream_ptr(dev)), "pdm_kjt_permute")
    return (out_v if values.numel() else out_v[:0]), out_l, out_o


@torch.library.custom_op("pdm::kjt_permute", mutates_args=())
def kjt_permute(values: torch.Tensor, offsets: torch.Tensor, num_keys: int, batch_size: int,
                perm: List[int]) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    v, lengths, offs = kjt_permute_raw(values, offsets, num_keys, batch_size, perm)
    return (v if v._base is None else v.clone()), lengths, offs


@kjt_permute.register_fake
def _(values, offsets, num_keys, batch_size, perm):
    K = len(perm)
    return (values.new_empty(values.shape), offsets.new_empty(K * batch_size, dtype=torch.int32),
            offsets.new_empty(K * batch_size + 1, dtype=torch.int64))


_DTYPE_CODES = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


@torch.library.custom_op("pdm::tbe_pooled_fwd", mutates_args=())
def tbe_pooled_fwd(weights: torch.Tensor, tables: List[torch.Tensor], indices: torch.Tensor, offsets: torch.Tensor,
                   plan_id: int, num_slots: int, total_dim: int, out_dtype_code: int, padding_idx: int,
                   owner_id: int) -> torch.Tensor:
    """Pooled lookup over the collection buffer ``weights`` (``tables``: its per-table views, not read here;
    ``owner_id``: the collection, used by the backward)."""
    plan = TbePlan.get(plan_id)
    batch = (offsets.numel() - 1) // num_slots
    return tbe_pooled_raw(plan, weights, indices.contiguous(), offsets.contiguous(), batch,
                          _DTYPE_CODES[out_dtype_code], padding_idx)


@tbe_pooled_fwd.register_fake
def _(weights, tables, indices, offsets, plan_id, num_slots, total_dim, out_dtype_code, padding_idx, owner_id):
    batch = (offsets.shape[0] - 1) // num_slots
    return weights.new_empty((batch, total_dim), dtype=_DTYPE_CODES[out_dtype_code])


def int8_rowwise_quantize(src: torch.Tensor, row_bytes: int = 0) -> torch.Tensor:
    """fp32 [rows, dim] -> uint8 [rows, row_bytes] int8-rowwise rows
    ([fp16 scale][fp16 bias][dim x uint8], padded to row_bytes)."""
    dev = _require_cuda(src)
    if src.dtype != torch.float32 or src.dim() != 2 or not src.is_contiguous():
        raise ValueError("src must be a contiguous fp32 [rows, dim] tensor")
    rows, dim = src.shape
    if row_bytes == 0:
        row_bytes = (4 + dim + 3) & ~3
    dst = torch.empty((rows, row_bytes), dtype=torch.uint8, device=dev)
    L.check(L.lib().pdm_int8_rowwise_quantize(src.data_ptr(), rows, dim, dst.data_ptr(), row_bytes,
                                              L.stream_ptr(dev)), "pdm_int8_rowwise_quantize")
    return dst


# ---------------------------------------------------------------------------
# Jagged -> padded S-token gather
# ---------------------------------------------------------------------------

def _seq_desc(tables: Sequence[torch.Tensor], ids: Sequence[Sequence[torch.Tensor]], offsets: Sequence[torch.Tensor],
              max_len: Sequence[int], pad_mode: int, align: int, err_flag: Optional[torch.Tensor]):
    """Validates a sequence gather's inputs; returns (desc, device, B, S, table / id / offset pointer arrays)."""
    P, F = len(offsets), len(tables)
    if not (1 <= P <= L.PDM_SEQ_MAX_POOLS and 1 <= F <= L.PDM_SEQ_MAX_FEATURES):
        raise ValueError(f"need 1..{L.PDM_SEQ_MAX_POOLS} pools and 1..{L.PDM_SEQ_MAX_FEATURES} features")
    if len(ids) != P or any(len(r) != F for r in ids) or len(max_len) != P:
        raise ValueError("ids must be [pools][features] and max_len one per pool")
    flat_ids = [t for row in ids for t in row]
    dev = _require_cuda(*tables, *flat_ids, *offsets, err_flag)
    dtype = tables[0].dtype
    if dtype not in TORCH_TO_PDM:
        raise TypeError(f"unsupported table dtype {dtype}")
    B = offsets[0].numel() - 1
    desc = L.SeqDesc()
    desc.num_pools, desc.num_features = P, F
    desc.dtype, desc.pad_mode, desc.align = TORCH_TO_PDM[dtype], pad_mode, align
    desc.batch_size = B
    for f, t in enumerate(tables):
        if t.dtype != dtype or t.dim() != 2 or not t.is_contiguous():
            raise ValueError("tables must be contiguous 2-D tensors of one dtype")
        desc.dim[f] = t.shape[1]
        desc.rows[f] = t.shape[0]
    for p in range(P):
        o = offsets[p]
        if o.dtype != torch.int64 or o.dim() != 1 or o.numel() != B + 1 or not o.is_contiguous():
            raise ValueError("offsets must be contiguous int64 [B+1], the same B for every pool")
        n = ids[p][0].numel()
        for t in ids[p]:
            if t.dtype != torch.int64 or t.dim() != 1 or not t.is_contiguous() or t.numel() != n:
                raise ValueError("ids of one pool must be contiguous int64 vectors of equal length")
        desc.num_ids[p] = n
        if int(max_len[p]) < 0:
            raise ValueError("max_len must be >= 0")
        desc.max_len[p] = int(max_len[p])
    S = sum(int(m) for m in max_len)
    tab_arr = (ctypes.c_void_p * F)(*[t.data_ptr() for t in tables])
    ids_arr = (ctypes.c_void_p * (P * F))(*[t.data_ptr() if t.numel() else None for t in flat_ids])
    off_arr = (ctypes.c_void_p * P)(*[o.data_ptr() for o in offsets])
    return desc, dev, B, S, tab_arr, ids_arr, off_arr


def seq_gather_raw(tables: Sequence[torch.Tensor], ids: Sequence[Sequence[torch.Tensor]],
                   offsets: Sequence[torch.Tensor], max_len: Sequence[int], pad_mode: int = L.PDM_PAD_ROW0,
                   align: int = L.PDM_ALIGN_RIGHT, want_mask: bool = True,
                   err_flag: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """tables[f]: [rows_f, dim_f]; ids[p][f]: int64 [n_p]; offsets[p]: int64 [B+1].
    Returns out [B, sum(max_len), sum(dim)] and mask uint8 [B, sum(max_len)]."""
    desc, dev, B, S, tab_arr, ids_arr, off_arr = _seq_desc(tables, ids, offsets, max_len, pad_mode, align, err_flag)
    Dtot = sum(t.shape[1] for t in tables)
    out = torch.empty((B, S, Dtot), dtype=tables[0].dtype, device=dev)
    mask = torch.empty((B, S), dtype=torch.uint8, device=dev) if want_mask else None
    status = L.lib().pdm_seq_gather_fwd(ctypes.byref(desc), tab_arr, ids_arr, off_arr, out.data_ptr(),
                                        _ptr(mask), _ptr(err_flag), L.stream_ptr(dev))
    L.check(status, "pdm_seq_gather_fwd")
    return out, mask


def seq_tokenize_workspace(tables: Sequence[torch.Tensor], ids: Sequence[Sequence[torch.Tensor]],
                           offsets: Sequence[torch.Tensor], max_len: Sequence[int], d_model: int) -> torch.Tensor:
    """A workspace for :func:`seq_tokenize_raw` on inputs of these shapes."""
    desc, dev = _seq_desc(tables, ids, offsets, max_len, L.PDM_PAD_ROW0, L.PDM_ALIGN_RIGHT, None)[:2]
    need = int(L.lib().pdm_seq_tokenize_workspace_size(ctypes.byref(desc), d_model))
    if need < 0:
        raise L.PdmError(L.PDM_ERR_INVALID, "pdm_seq_tokenize_workspace_size", L.last_error())
    return torch.empty(max(need, 1), dtype=torch.uint8, device=dev)


def seq_tokenize_raw(tables: Sequence[torch.Tensor], ids: Sequence[Sequence[torch.Tensor]],
                     offsets: Sequence[torch.Tensor], max_len: Sequence[int], weights: Sequence[dict],
                     pad_mode: int = L.PDM_PAD_ROW0, align: int = L.PDM_ALIGN_RIGHT, want_mask: bool = True,
                     out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                     err_flag: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """The S-token gather fused with one SequentialTokenizer per pool (C ABI ``pdm_seq_tokenize_fwd``).

    tables / ids / offsets / max_len as :func:`seq_gather_raw` (bf16 or fp32 tables).  ``weights[p]`` holds
    ``w1`` [d, K] / ``b1`` [d] / ``w2`` [d, d] / ``b2`` [d] (bf16) and ``pos`` (fp32 [>= max_len[p], d] or
    None).  ``out`` may be a float32 view [B, >= S, d] whose rows are contiguous (e.g. the leading S-token
    rows of the block input); by default a new [B, S, d] tensor.  Returns (out, mask)."""
    desc, dev, B, S, tab_arr, ids_arr, off_arr = _seq_desc(tables, ids, offsets, max_len, pad_mode, align, err_flag)
    P = len(offsets)
    if len(weights) != P:
        raise ValueError("one tokenizer weight dict per pool")
    d = None
    warr = (L.TokenizerWeights * P)()
    keep = []
    for p, w in enumerate(weights):
        if int(max_len[p]) == 0:
            continue
        w1, b1, w2, b2, pos = w["w1"], w["b1"], w["w2"], w["b2"], w.get("pos")
        d = w1.shape[0] if d is None else d
        for t, shape in ((w1, (d, None)), (b1, (d,)), (w2, (d, d)), (b2, (d,))):
            if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != dev or t.dim() != len(shape) or \
                    any(e is not None and e != g for e, g in zip(shape, t.shape)):
                raise ValueError("tokenizer weights must be contiguous bf16 w1 [d, K], b1 [d], w2 [d, d], b2 [d] "
                                 "on the tables' device")
        if pos is not None and (pos.dtype != torch.float32 or not pos.is_contiguous() or pos.device != dev or
                                pos.dim() != 2 or pos.shape[1] != d):
            raise ValueError("pos must be a contiguous float32 [rows, d] tensor on the tables' device")
        warr[p] = L.TokenizerWeights(w1.data_ptr(), b1.data_ptr(), w2.data_ptr(), b2.data_ptr(),
                                     None if pos is None else pos.data_ptr(), 0 if pos is None else pos.shape[0])
        keep.append(w)
    if d is None:
        d = int(out.shape[-1]) if out is not None else 256
    if out is None:
        out = torch.empty((B, S, d), dtype=torch.float32, device=dev)
    elif (out.dtype != torch.float32 or out.device != dev or out.dim() != 3 or out.shape[0] != B or
          out.shape[1] < S or out.shape[2] != d or out.stride(2) != 1 or out.stride(1) != d):
        raise ValueError("out must be float32 [B, >= S, d] with contiguous rows on the tables' device")
    mask = torch.empty((B, S), dtype=torch.uint8, device=dev) if want_mask else None
    lib = L.lib()
    need = int(lib.pdm_seq_tokenize_workspace_size(ctypes.byref(desc), d))
    if need < 0:
        raise L.PdmError(L.PDM_ERR_INVALID, "pdm_seq_tokenize_workspace_size", L.last_error())
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    status = lib.pdm_seq_tokenize_fwd(ctypes.byref(desc), tab_arr, ids_arr, off_arr, warr, d, out.data_ptr(),
                                      out.stride(0) if B > 0 else S * d, _ptr(mask), workspace.data_ptr(),
                                      workspace.numel(), _ptr(err_flag), L.stream_ptr(dev))
    L.check(status, "pdm_seq_tokenize_fwd")
    return out, mask


def seq_gather_backward_fused_raw(plan: TbePlan, weights: torch.Tensor, momentum1: torch.Tensor,
                                  momentum2: Optional[torch.Tensor], table_rows: Sequence[int],
                                  table_dims: Sequence[int], ids: Sequence[Sequence[torch.Tensor]],
                                  offsets: Sequence[torch.Tensor], max_len: Sequence[int], grad_out: torch.Tensor,
                                  pad_mode: int = L.PDM_PAD_ROW0, align: int = L.PDM_ALIGN_RIGHT,
                                  optimizer: int = L.PDM_OPT_ADAM, learning_rate: float = 0.01, eps: float = 1e-8,
                                  beta1: float = 0.9, beta2: float = 0.999, weight_decay: float = 0.0,
                                  weight_decay_mode: int = L.PDM_WD_NONE, step: int = 1,
                                  workspace: Optional[torch.Tensor] = None,
                                  err_flag: Optional[torch.Tensor] = None) -> None:
    """Launches pdm_seq_gather_backward_fused: the S-token gather's backward with the fused update of the
    feature tables (``plan``: one fp32 slot per feature, sum pooling, out_offset = column of the feature).
    ``grad_out``: fp32 [B, sum(max_len), sum(dims)] gradient of the gathered tokens."""
    P, F = len(offsets), len(table_dims)
    flat_ids = [t for row in ids for t in row]
    dev = _require_cuda(weights, momentum1, momentum2, grad_out, *flat_ids, *offsets, workspace, err_flag)
    if not (1 <= P <= L.PDM_SEQ_MAX_POOLS and 1 <= F <= L.PDM_SEQ_MAX_FEATURES) or len(ids) != P \
            or any(len(r) != F for r in ids) or len(max_len) != P:
        raise ValueError("ids must be [pools][features] and max_len one per pool")
    B = offsets[0].numel() - 1
    S = sum(int(m) for m in max_len)
    Dtot = sum(int(d) for d in table_dims)
    if grad_out.dtype != torch.float32 or tuple(grad_out.shape) != (B, S, Dtot) or not grad_out.is_contiguous():
        raise ValueError(f"grad_out must be contiguous float32 [{B}, {S}, {Dtot}]")
    desc = L.SeqDesc()
    desc.num_pools, desc.num_features = P, F
    desc.dtype, desc.pad_mode, desc.align = L.PDM_F32, pad_mode, align
    desc.batch_size = B
    for f in range(F):
        desc.dim[f] = int(table_dims[f])
        desc.rows[f] = int(table_rows[f])
    for p in range(P):
        o = offsets[p]
        if o.dtype != torch.int64 or o.numel() != B + 1 or not o.is_contiguous():
            raise ValueError("offsets must be contiguous int64 [B+1], the same B for every pool")
        n = ids[p][0].numel()
        for t in ids[p]:
            if t.dtype != torch.int64 or not t.is_contiguous() or t.numel() != n:
                raise ValueError("ids of one pool must be contiguous int64 vectors of equal length")
        desc.num_ids[p] = n
        desc.max_len[p] = int(max_len[p])
    ntok = B * S
    if workspace is None:
        workspace = tbe_backward_workspace(plan, F * ntok, ntok, dev)
    for name, t in (("weights", weights), ("momentum1", momentum1), ("momentum2", momentum2)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if weights.numel() * weights.element_size() < plan.fp32_extent:
        raise ValueError("weights is smaller than the plan's fp32 tables")
    opt = L.OptimParams(int(optimizer), int(weight_decay_mode), float(learning_rate), float(eps), float(beta1),
                        float(beta2), float(weight_decay), 0, int(step))
    ids_arr = (ctypes.c_void_p * (P * F))(*[t.data_ptr() if t.numel() else None for t in flat_ids])
    off_arr = (ctypes.c_void_p * P)(*[o.data_ptr() for o in offsets])
    status = L.lib().pdm_seq_gather_backward_fused(
        plan.handle, ctypes.byref(desc), weights.data_ptr(), momentum1.data_ptr(), _ptr(momentum2), ids_arr, off_arr,
        grad_out.data_ptr(), ctypes.byref(opt), workspace.data_ptr(), workspace.numel(), _ptr(err_flag),
        L.stream_ptr(dev))
    L.check(status, "pdm_seq_gather_backward_fused")


@torch.library.custom_op("pdm::seq_gather_fwd", mutates_args=())
def seq_gather_fwd(flat: torch.Tensor, tables: List[torch.Tensor], ids: List[torch.Tensor],
                   offsets: List[torch.Tensor], max_len: List[int], pad_mode: int, align: int,
                   owner_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """S-token gather from ``tables`` (views of the collection buffer ``flat``, which the backward updates);
    ``ids`` is pool-major, ``len(tables)`` features per pool."""
    F = len(tables)
    grid = [ids[p * F:(p + 1) * F] for p in range(len(offsets))]
    out, mask = seq_gather_raw(tables, grid, offsets, max_len, pad_mode, align, want_mask=True)
    return out, mask


@seq_gather_fwd.register_fake
def _(flat, tables, ids, offsets, max_len, pad_mode, align, owner_id):
    B = offsets[0].shape[0] - 1
    S = sum(max_len)
    D = sum(t.shape[1] for t in tables)
    return (tables[0].new_empty((B, S, D)), tables[0].new_empty((B, S), dtype=torch.uint8))


@torch.library.custom_op("pdm::seq_tokenize_fwd", mutates_args=())
def seq_tokenize_fwd(tables: List[torch.Tensor], ids: List[torch.Tensor], offsets: List[torch.Tensor],
                     max_len: List[int], w1: List[torch.Tensor], b1: List[torch.Tensor], w2: List[torch.Tensor],
                     b2: List[torch.Tensor], pos: List[Optional[torch.Tensor]], pad_mode: int,
                     align: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """S-token gather fused with one SequentialTokenizer per pool (bf16 weights, fp32 positions or None);
    ``ids`` is pool-major as for ``seq_gather_fwd``.  Returns (fp32 tokens [B, S, d], mask uint8 [B, S])."""
    F = len(tables)
    grid = [ids[p * F:(p + 1) * F] for p in range(len(offsets))]
    weights = [dict(w1=w1[p], b1=b1[p], w2=w2[p], b2=b2[p], pos=pos[p]) for p in range(len(offsets))]
    return seq_tokenize_raw(tables, grid, offsets, max_len, weights, pad_mode, align, want_mask=True)


@seq_tokenize_fwd.register_fake
def _(tables, ids, offsets, max_len, w1, b1, w2, b2, pos, pad_mode, align):
    B = offsets[0].shape[0] - 1
    S = sum(max_len)
    d = w1[0].shape[0]
    return (tables[0].new_empty((B, S, d), dtype=torch.float32), tables[0].new_empty((B, S), dtype=torch.uint8))


def ns_tokenize_raw(tables: Sequence[torch.Tensor], ids: Sequence[torch.Tensor], dense: Sequence[torch.Tensor],
                    w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor, b2: torch.Tensor, n_ns: int,
                    out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                    err_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """NS tokens (C ABI ``pdm_ns_tokenize_fwd``): the NS input rows (``tables[j][ids[j]]`` for the scalar features,
    then the fp32 ``dense`` parts [B, dim], in that order) through AutoSplitTokenizer's Linear + bias, GELU,
    Linear + bias (``w1`` [N, K], ``b1`` [N], ``w2`` [N, N], ``b2`` [N] bf16; N = n_ns * d).  Returns fp32
    [B, n_ns, d]; ``out`` may be a float32 view [B, n_ns, d] with contiguous rows (e.g. the block input's NS
    rows)."""
    if len(tables) != len(ids) or len(tables) > L.PDM_NS_MAX_PARTS or len(dense) > L.PDM_NS_MAX_PARTS:
        raise ValueError("one ids vector per scalar table, at most 8 scalar tables and 8 dense parts")
    dev = _require_cuda(*tables, *ids, *dense, w1, b1, w2, b2, err_flag)
    N, K = int(w1.shape[0]), int(w1.shape[1]) if w1.dim() == 2 else -1
    if N % n_ns:
        raise ValueError("w1 rows must be n_ns * d_model")
    d = N // n_ns
    for t, shape in ((w1, (N, K)), (b1, (N,)), (w2, (N, N)), (b2, (N,))):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or tuple(t.shape) != shape:
            raise ValueError("w1 [N, K], b1 [N], w2 [N, N], b2 [N] must be contiguous bf16")
    B = ids[0].numel() if ids else dense[0].shape[0]
    desc = L.NsDesc()
    desc.num_scalar, desc.num_dense, desc.n_out, desc.batch_size = len(tables), len(dense), N, B
    desc.table_dtype = TORCH_TO_PDM[tables[0].dtype] if tables else L.PDM_F32
    ksum = 0
    for j, (t, i) in enumerate(zip(tables, ids)):
        if t.dim() != 2 or not t.is_contiguous() or t.dtype != tables[0].dtype or t.dtype not in (torch.float32,
                                                                                                 torch.bfloat16):
            raise ValueError("scalar tables must be contiguous 2-D fp32 or bf16 tensors of one dtype")
        if i.dtype != torch.int64 or i.numel() != B or not i.is_contiguous():
            raise ValueError("ids must be contiguous int64 vectors of one length (one id per sample)")
        desc.scalar_dim[j], desc.scalar_rows[j] = t.shape[1], t.shape[0]
        ksum += t.shape[1]
    strides = (ctypes.c_int64 * max(len(dense), 1))()
    for j, x in enumerate(dense):
        if x.dtype != torch.float32 or x.dim() != 2 or x.shape[0] != B or x.stride(1) != 1:
            raise ValueError("dense parts must be fp32 [B, dim] with contiguous rows")
        desc.dense_dim[j] = x.shape[1]
        strides[j] = x.stride(0)
        ksum += x.shape[1]
    if ksum != K:
        raise ValueError(f"w1 has {K} columns but the NS parts are {ksum} wide")
    if out is None:
        out = torch.empty((B, n_ns, d), dtype=torch.float32, device=dev)
    elif (out.dtype != torch.float32 or out.device != dev or tuple(out.shape) != (B, n_ns, d) or
          out.stride(2) != 1 or out.stride(1) != d):
        raise ValueError("out must be float32 [B, n_ns, d] with contiguous sample rows")
    lib = L.lib()
    need = int(lib.pdm_ns_tokenize_workspace_size(ctypes.byref(desc)))
    if need < 0:
        raise L.PdmError(L.PDM_ERR_INVALID, "pdm_ns_tokenize_workspace_size", L.last_error())
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    tab_arr = (ctypes.c_void_p * max(len(tables), 1))(*[t.data_ptr() for t in tables])
    ids_arr = (ctypes.c_void_p * max(len(ids), 1))(*[i.data_ptr() for i in ids])
    den_arr = (ctypes.c_void_p * max(len(dense), 1))(*[x.data_ptr() for x in dense])
    status = lib.pdm_ns_tokenize_fwd(ctypes.byref(desc), tab_arr, ids_arr, den_arr, strides, w1.data_ptr(),
                                     b1.data_ptr(), w2.data_ptr(), b2.data_ptr(), out.data_ptr(),
                                     out.stride(0) if B > 0 else N, workspace.data_ptr(), workspace.numel(),
                                     _ptr(err_flag), L.stream_ptr(dev))
    L.check(status, "pdm_ns_tokenize_fwd")
    return out


# ---------------------------------------------------------------------------
# OneTrans block
# ---------------------------------------------------------------------------

def onetrans_workspace_layout(B: int, kv: int, q_len: int, D: int, F: int) -> Dict[str, Tuple[int, int]]:
    """Byte (offset, size) of each region of the block workspace, as laid out by
    pdm_onetrans_block_fwd: q (Q tail rows [B, q_len, D] bf16, later the
    attention output), k ([B, kv, D] bf16), vt (V transposed per head [B, D/64,
    64, kv_ld] bf16, kv_ld = kv rounded up to 64).  d_model 128 and 256 run
    fused kernels; other widths also hold h (normalised rows [B, kv, D] bf16)
    and g (GELU of the FFN-up GEMM [B, q_len, F] bf16)."""
    a = lambda v: (v + 255) // 256 * 256  # noqa: E731
    kv_ld = (kv + 63) // 64 * 64
    sizes = [("q", B * q_len * D * 2), ("k", B * kv * D * 2), ("vt", B * D * kv_ld * 2)]
    if D not in (128, 256):
        sizes += [("h", B * kv * D * 2), ("g", B * q_len * F * 2)]
    out, off = {}, 0
    for name, n in sizes:
        out[name] = (off, n)
        off = a(off + n)
    out["total"] = (off, 0)
    return out


def onetrans_block_raw(x: torch.Tensor, w: Dict[str, torch.Tensor], n_heads: int, q_len: int,
                       out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None
                       ) -> torch.Tensor:
    """x: fp32 [B, kv, D]; w: norm1_w/norm2_w fp32 [D], the GEMM weights bf16
    in nn.Linear layout.  Returns fp32 [B, q_len, D].  ``workspace`` (uint8,
    at least pdm_onetrans_block_workspace_size bytes) is allocated when not
    given."""
    names = ("norm1_w", "s_qkv_w", "ns_qkv_w", "out_w", "norm2_w", "s_w1", "s_w2", "ns_w1", "ns_w2")
    dev = _require_cuda(x, *[w[k] for k in names])
    if x.dtype != torch.float32 or x.dim() != 3 or not x.is_contiguous():
        raise ValueError("x must be a contiguous fp32 [B, kv_len, D] tensor")
    B, kv, D = x.shape
    n_ns = w["ns_qkv_w"].shape[0]
    Fd = w["s_w1"].shape[0]
    shapes = {"norm1_w": (D,), "s_qkv_w": (3 * D, D), "ns_qkv_w": (n_ns, 3 * D, D), "out_w": (D, D),
              "norm2_w": (D,), "s_w1": (Fd, D), "s_w2": (D, Fd), "ns_w1": (n_ns, Fd, D), "ns_w2": (n_ns, D, Fd)}
    for k in names:
        t = w[k]
        want = torch.float32 if k.startswith("norm") else torch.bfloat16
        if tuple(t.shape) != shapes[k] or t.dtype != want or not t.is_contiguous():
            raise ValueError(f"{k}: expected contiguous {want} {shapes[k]}, got {t.dtype} {tuple(t.shape)}")
    if not (n_ns <= q_len <= kv):
        raise ValueError(f"need n_ns <= q_len <= kv_len, got n_ns={n_ns} q_len={q_len} kv_len={kv}")
    desc = L.BlockDesc(B, D, n_heads, n_ns, Fd, kv, q_len, 0)
    ws_bytes = int(L.lib().pdm_onetrans_block_workspace_size(ctypes.byref(desc)))
    if ws_bytes < 0:
        raise L.PdmError(ws_bytes, "pdm_onetrans_block_workspace_size", L.last_error())
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    elif workspace.dtype != torch.uint8 or workspace.numel() < ws_bytes or workspace.device != dev:
        raise ValueError(f"workspace must be a uint8 tensor of >= {ws_bytes} bytes on {dev}")
    ws = workspace
    if out is None:
        out = torch.empty((B, q_len, D), dtype=torch.float32, device=dev)
    bw = L.BlockWeights(*[w[k].data_ptr() for k in names])
    status = L.lib().pdm_onetrans_block_fwd(ctypes.byref(desc), x.data_ptr(), ctypes.byref(bw), out.data_ptr(),
                                            ws.data_ptr(), ws_bytes, L.stream_ptr(dev))
    L.check(status, "pdm_onetrans_block_fwd")
    return out


@torch.library.custom_op("pdm::onetrans_block_fwd", mutates_args=())
def onetrans_block_fwd(x: torch.Tensor, norm1_w: torch.Tensor, s_qkv_w: torch.Tensor, ns_qkv_w: torch.Tensor,
                       out_w: torch.Tensor, norm2_w: torch.Tensor, s_w1: torch.Tensor, s_w2: torch.Tensor,
                       ns_w1: torch.Tensor, ns_w2: torch.Tensor, n_heads: int, q_len: int) -> torch.Tensor:
    w = dict(norm1_w=norm1_w, s_qkv_w=s_qkv_w, ns_qkv_w=ns_qkv_w, out_w=out_w, norm2_w=norm2_w,
             s_w1=s_w1, s_w2=s_w2, ns_w1=ns_w1, ns_w2=ns_w2)
    return onetrans_block_raw(x, w, n_heads, q_len)


@onetrans_block_fwd.register_fake
def _(x, norm1_w, s_qkv_w, ns_qkv_w, out_w, norm2_w, s_w1, s_w2, ns_w1, ns_w2, n_heads, q_len):
    return x.new_empty((x.shape[0], q_len, x.shape[2]))


_BLOCK_WEIGHT_NAMES = ("norm1_w", "s_qkv_w", "ns_qkv_w", "out_w", "norm2_w", "s_w1", "s_w2", "ns_w1", "ns_w2")


def onetrans_stack_workspace_bytes(B: int, kv: int, D: int, F: int, n_ns: int, n_heads: int,
                                   q_s: Sequence[int]) -> int:
    """pdm_onetrans_stack_workspace_size for a stack whose layer 0 sees ``kv`` tokens."""
    desc = L.BlockDesc(B, D, n_heads, n_ns, F, kv, int(q_s[0]) + n_ns if len(q_s) else n_ns, 0)
    qs = (ctypes.c_int32 * max(len(q_s), 1))(*[int(q) for q in q_s])
    n = int(L.lib().pdm_onetrans_stack_workspace_size(ctypes.byref(desc), qs, len(q_s)))
    if n < 0:
        raise L.PdmError(n, "pdm_onetrans_stack_workspace_size", L.last_error())
    return n


def onetrans_stack_raw(x: torch.Tensor, layers: Sequence[Dict[str, torch.Tensor]], n_heads: int,
                       q_s: Sequence[int], out: Optional[torch.Tensor] = None,
                       workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The block loop in one call (pdm_onetrans_stack_fwd): layer l keeps ``q_s[l] + n_ns`` tokens of the
    previous layer's output.  ``layers[l]`` holds the weights of block l as for ``onetrans_block_raw``.
    Returns fp32 [B, q_s[-1] + n_ns, D]."""
    n = len(layers)
    if n != len(q_s) or not 1 <= n <= L.PDM_STACK_MAX_LAYERS:
        raise ValueError(f"need one schedule entry per layer and 1..{L.PDM_STACK_MAX_LAYERS} layers")
    dev = _require_cuda(x, *[w[k] for w in layers for k in _BLOCK_WEIGHT_NAMES])
    if x.dtype != torch.float32 or x.dim() != 3 or not x.is_contiguous():
        raise ValueError("x must be a contiguous fp32 [B, kv_len, D] tensor")
    B, kv, D = x.shape
    n_ns = layers[0]["ns_qkv_w"].shape[0]
    Fd = layers[0]["s_w1"].shape[0]
    shapes = {"norm1_w": (D,), "s_qkv_w": (3 * D, D), "ns_qkv_w": (n_ns, 3 * D, D), "out_w": (D, D),
              "norm2_w": (D,), "s_w1": (Fd, D), "s_w2": (D, Fd), "ns_w1": (n_ns, Fd, D), "ns_w2": (n_ns, D, Fd)}
    for w in layers:
        for k in _BLOCK_WEIGHT_NAMES:
            t = w[k]
            want = torch.float32 if k.startswith("norm") else torch.bfloat16
            if tuple(t.shape) != shapes[k] or t.dtype != want or not t.is_contiguous():
                raise ValueError(f"{k}: expected contiguous {want} {shapes[k]}, got {t.dtype} {tuple(t.shape)}")
    kv_l = kv
    for q in q_s:
        if q < 0 or q + n_ns > kv_l:
            raise ValueError(f"schedule {list(q_s)}: each layer keeps n_ns <= q + n_ns <= its kv_len")
        kv_l = q + n_ns
    desc = L.BlockDesc(B, D, n_heads, n_ns, Fd, kv, int(q_s[0]) + n_ns, 0)
    qs = (ctypes.c_int32 * n)(*[int(q) for q in q_s])
    ws_bytes = onetrans_stack_workspace_bytes(B, kv, D, Fd, n_ns, n_heads, q_s)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    elif workspace.dtype != torch.uint8 or workspace.numel() < ws_bytes or workspace.device != dev:
        raise ValueError(f"workspace must be a uint8 tensor of >= {ws_bytes} bytes on {dev}")
    if out is None:
        out = torch.empty((B, int(q_s[-1]) + n_ns, D), dtype=torch.float32, device=dev)
    bw = (L.BlockWeights * n)(*[L.BlockWeights(*[w[k].data_ptr() for k in _BLOCK_WEIGHT_NAMES]) for w in layers])
    status = L.lib().pdm_onetrans_stack_fwd(ctypes.byref(desc), qs, n, x.data_ptr(), bw, out.data_ptr(),
                                            workspace.data_ptr(), ws_bytes, L.stream_ptr(dev))
    L.check(status, "pdm_onetrans_stack_fwd")
    return out


@torch.library.custom_op("pdm::onetrans_stack_fwd", mutates_args=())
def onetrans_stack_fwd(x: torch.Tensor, weights: List[torch.Tensor], n_heads: int, q_s: List[int]) -> torch.Tensor:
    """``weights``: the nine block weights of every layer in turn (the order of pdm_block_weights)."""
    k = len(_BLOCK_WEIGHT_NAMES)
    layers = [dict(zip(_BLOCK_WEIGHT_NAMES, weights[i * k:(i + 1) * k])) for i in range(len(weights) // k)]
    return onetrans_stack_raw(x, layers, n_heads, q_s)


@onetrans_stack_fwd.register_fake
def _(x, weights, n_heads, q_s):
    return x.new_empty((x.shape[0], q_s[-1] + weights[2].shape[0], x.shape[2]))


# ---------------------------------------------------------------------------
# Cross-feature ids (xxHash64)
# ---------------------------------------------------------------------------

def cross_hash_raw(keys: Sequence[torch.Tensor], table_size: int, salt: int = 0,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``out[i] = xxh64(le int64 keys[0][i] .. keys[n-1][i], seed=salt) % table_size`` on the GPU.

    Each key is an int64 device tensor of N values, or of one value broadcast
    to every row (primus_dlrm/data/hashing.py:23-52 n-way, :72-112 batch)."""
    n_keys = len(keys)
    if not 2 <= n_keys <= L.PDM_CROSS_MAX_KEYS:
        raise ValueError(f"cross hash needs 2..{L.PDM_CROSS_MAX_KEYS} keys, got {n_keys}")
    if table_size < 1:
        raise ValueError("table_size must be >= 1")
    ks = [k.reshape(-1) for k in keys]
    dev = _require_cuda(*ks)
    for k in ks:
        if k.dtype != torch.int64:
            raise TypeError(f"keys must be int64, got {k.dtype}")
    n = max(k.numel() for k in ks)
    strides = []
    for k in ks:
        if k.numel() == n:
            strides.append(1)
        elif k.numel() == 1:
            strides.append(0)
        else:
            raise ValueError("key tensors must have one length (or length 1)")
    ks = [k.contiguous() for k in ks]
    if out is None:
        out = torch.empty(n, dtype=torch.int64, device=dev)
    elif out.dtype != torch.int64 or out.numel() != n or not out.is_contiguous() or out.device != dev:
        raise ValueError("out must be a contiguous int64 tensor of N rows on the keys' device")
    ptrs = (ctypes.c_void_p * n_keys)(*[k.data_ptr() for k in ks])
    st = (ctypes.c_int64 * n_keys)(*strides)
    with torch.cuda.device(dev):
        L.check(L.lib().pdm_cross_hash_fwd(ptrs, st, n_keys, n, table_size, salt & (2**64 - 1), _ptr(out),
                                           L.stream_ptr(dev)), "pdm_cross_hash_fwd")
    return out


@torch.library.custom_op("pdm::cross_hash_fwd", mutates_args=())
def cross_hash_fwd(keys: List[torch.Tensor], table_size: int, salt: int) -> torch.Tensor:
    return cross_hash_raw(keys, table_size, salt)


@cross_hash_fwd.register_fake
def _(keys, table_size, salt):
    n = max(k.numel() for k in keys)
    return keys[0].new_empty(n, dtype=torch.int64)
