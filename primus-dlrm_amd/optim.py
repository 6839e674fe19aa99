"""Embedding optimizers applied inside the pooled-lookup backward.

The reference tags every embedding weight with ``_apply_optimizer_in_backward(optim_cls, [p], kwargs)``
(primus_dlrm/distributed/wrapper.py:151-174): ``torch.optim.Adam`` by default, or
``torchrec.optim.RowWiseAdagrad`` with ``weight_decay_mode=WeightDecayMode.L2``; TorchRec then runs FBGEMM's
fused backward (ADAM / EXACT_ROWWISE_ADAGRAD) and exposes ``model.fused_optimizer``, whose ``param_groups`` lr
the trainer's sparse warm-up drives (primus_dlrm/training/dist_trainer.py:298,316-325).

Here :class:`FusedEmbeddingOptimizer` is that object for one collection of this package
(``EmbeddingBagCollection``, or ``EmbeddingCollection`` whose tables the S-token gather reads): it reads the
tags, owns the optimizer state (laid out for the C ABI's ``pdm_tbe_backward_fused`` /
``pdm_seq_gather_backward_fused``) and launches the fused backward with the current ``param_groups[0]["lr"]``.

* ``torch.optim.Adam`` -> FBGEMM ADAM: ``m = b1 m + (1-b1) g``, ``v = b2 v + (1-b2) g^2``,
  ``w -= lr ((m / (1-b1^t)) / (sqrt(v / (1-b2^t)) + eps) + wd w)`` (weight decay applied decoupled, inside
  the learning rate, as FBGEMM does).
* :class:`RowWiseAdagrad` -> EXACT_ROWWISE_ADAGRAD: one accumulator per row,
  ``G += mean_d((g + wd w)^2)`` (L2) and ``w -= lr / (sqrt(G) + eps) (g + wd w)``.
"""
from __future__ import annotations

import enum
from typing import Any, Dict, Iterable, List, Optional

import torch

from . import _lib as L


class WeightDecayMode(enum.IntEnum):
    """Mirrors fbgemm_gpu's WeightDecayMode (the values the reference passes)."""
    NONE = 0
    L2 = 1
    DECOUPLED = 2


class EmbOptimType(enum.Enum):
    """Mirrors fbgemm_gpu's EmbOptimType for the two optimizers on this path."""
    ADAM = "adam"
    EXACT_ROWWISE_ADAGRAD = "exact_row_wise_adagrad"


class RowWiseAdagrad(torch.optim.Optimizer):
    """Constructor surface of torchrec.optim.RowWiseAdagrad (the reference passes lr, eps, weight_decay and
    weight_decay_mode).  Under :func:`torch.distributed.optim._apply_optimizer_in_backward` on an
    EmbeddingBagCollection of this package the update runs fused in the backward; ``step`` here is the same
    rule on a dense ``.grad`` (one accumulator per row of a 2-D parameter)."""

    def __init__(self, params: Iterable, lr: float = 1e-2, lr_decay: float = 0.0, weight_decay: float = 0.0,
                 initial_accumulator_value: float = 0.0, eps: float = 1e-10, *, maximize: bool = False,
                 weight_decay_mode: Any = WeightDecayMode.L2, **unused):
        if lr_decay != 0.0 or maximize:
            raise NotImplementedError("lr_decay and maximize are not supported")
        defaults = dict(lr=lr, eps=eps, weight_decay=weight_decay, initial_accumulator_value=initial_accumulator_value,
                        weight_decay_mode=int(getattr(weight_decay_mode, "value", weight_decay_mode)))
        super().__init__(params, defaults)

    @torch.no_grad()
    def step(self, closure=None):
        loss = closure() if closure is not None else None
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                g = p.grad if p.dim() > 1 else p.grad.unsqueeze(1)
                w = p if p.dim() > 1 else p.unsqueeze(1)
                st = self.state[p]
                if "sum" not in st:
                    st["sum"] = torch.full((w.shape[0],), group["initial_accumulator_value"], dtype=torch.float32,
                                           device=p.device)
                if group["weight_decay_mode"] == WeightDecayMode.L2 and group["weight_decay"]:
                    g = g + group["weight_decay"] * w
                st["sum"].add_((g.float() * g.float()).mean(dim=1))
                mult = group["lr"] / (st["sum"].sqrt() + group["eps"])
                w.sub_((mult.unsqueeze(1) * g).to(w.dtype))
        return loss


def _optimizer_tag(p: torch.Tensor):
    classes = getattr(p, "_optimizer_classes", None)
    kwargs = getattr(p, "_optimizer_kwargs", None)
    if not classes:
        return None
    if len(classes) != 1:
        raise NotImplementedError("one in-backward optimizer per embedding weight is supported")
    return classes[0], dict(kwargs[0])


class FusedEmbeddingOptimizer:
    """The fused optimizer of one collection: hyper-parameters, state and step count.

    ``momentum1`` / ``momentum2`` are fp32 device tensors laid out as the C ABI expects (Adam: like the fp32
    weights buffer; row-wise Adagrad: one entry per row of the collection, tables in collection order, so every
    plan over these tables addresses the same state through ``state_offset``)."""

    def __init__(self, optimizer_class, kwargs: Dict[str, Any], weights_bytes: int, device: torch.device,
                 table_names: List[str], table_rows: Dict[str, int], table_dims: Dict[str, int],
                 table_offsets: Dict[str, int]):
        name = getattr(optimizer_class, "__name__", str(optimizer_class))
        if optimizer_class is torch.optim.Adam or name == "Adam":
            self.optim_type = EmbOptimType.ADAM
            betas = kwargs.get("betas", (0.9, 0.999))
            self.beta1, self.beta2 = float(betas[0]), float(betas[1])
            self.weight_decay_mode = WeightDecayMode.DECOUPLED
            if kwargs.get("amsgrad", False):
                raise NotImplementedError("amsgrad is not supported by the fused Adam")
            eps_default = 1e-8
        elif name == "RowWiseAdagrad":
            self.optim_type = EmbOptimType.EXACT_ROWWISE_ADAGRAD
            self.beta1, self.beta2 = 0.9, 0.999
            mode = kwargs.get("weight_decay_mode", WeightDecayMode.L2)
            self.weight_decay_mode = WeightDecayMode(int(getattr(mode, "value", mode)))
            if self.weight_decay_mode == WeightDecayMode.DECOUPLED:
                raise NotImplementedError("row-wise Adagrad supports weight_decay_mode NONE or L2")
            eps_default = 1e-10
        else:
            raise NotImplementedError(f"no fused embedding optimizer for {name} (Adam and RowWiseAdagrad are)")
        self.eps = float(kwargs.get("eps", eps_default))
        self.weight_decay = float(kwargs.get("weight_decay", 0.0))
        self.param_groups = [{"lr": float(kwargs.get("lr", 1e-2)), "params": []}]
        self.iter = 0
        self._names = list(table_names)
        self._rows, self._dims, self._offsets = table_rows, table_dims, table_offsets
        self.state_offset: Dict[str, int] = {}
        r = 0
        for n in self._names:
            self.state_offset[n] = r
            r += table_rows[n]
        adam = self.optim_type == EmbOptimType.ADAM
        n1 = (weights_bytes + 3) // 4 if adam else max(r, 1)
        self.momentum1 = torch.zeros(n1, dtype=torch.float32, device=device)
        self.momentum2 = torch.zeros(n1, dtype=torch.float32, device=device) if adam else None
        self._workspace: Optional[torch.Tensor] = None

    # torch.optim-like surface (the update itself happens in the backward)
    def step(self, closure=None):
        return closure() if closure is not None else None

    def zero_grad(self, set_to_none: bool = True) -> None:
        return None

    def _table_state(self, name: str) -> Dict[str, torch.Tensor]:
        rows, dim = self._rows[name], self._dims[name]
        if self.optim_type == EmbOptimType.ADAM:
            e0 = self._offsets[name] // 4
            return {"momentum1": self.momentum1[e0:e0 + rows * dim].view(rows, dim),
                    "momentum2": self.momentum2[e0:e0 + rows * dim].view(rows, dim)}
        r0 = self.state_offset[name]
        return {"sum": self.momentum1[r0:r0 + rows]}

    def state_dict(self) -> Dict[str, Any]:
        return {"state": {n: {k: v.clone() for k, v in self._table_state(n).items()} for n in self._names},
                "param_groups": [{"lr": self.param_groups[0]["lr"]}], "iter": self.iter}

    def load_state_dict(self, sd: Dict[str, Any]) -> None:
        with torch.no_grad():
            for n, st in sd["state"].items():
                dst = self._table_state(n)
                for k, v in st.items():
                    dst[k].copy_(v)
        self.param_groups[0]["lr"] = float(sd["param_groups"][0]["lr"])
        self.iter = int(sd.get("iter", self.iter))

    def _hyper(self) -> Dict[str, Any]:
        adam = self.optim_type == EmbOptimType.ADAM
        return dict(optimizer=L.PDM_OPT_ADAM if adam else L.PDM_OPT_ROWWISE_ADAGRAD,
                    learning_rate=self.param_groups[0]["lr"], eps=self.eps, beta1=self.beta1, beta2=self.beta2,
                    weight_decay=self.weight_decay,
                    weight_decay_mode=L.PDM_WD_L2 if self.weight_decay_mode == WeightDecayMode.L2 else L.PDM_WD_NONE,
                    step=self.iter)

    def _ws(self, plan, num_lookups: int, num_bags: int, device) -> torch.Tensor:
        need = int(L.lib().pdm_tbe_backward_workspace_size(plan.handle, num_lookups, num_bags))
        if self._workspace is None or self._workspace.numel() < need:
            self._workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
        return self._workspace

    def apply(self, plan, weights_flat: torch.Tensor, values: torch.Tensor, offsets: torch.Tensor, batch_size: int,
              grad_out: torch.Tensor, padding_idx: int = -1) -> None:
        """The fused backward + update of one pooled batch (called from the autograd backward); ``plan``'s
        state offsets must be this optimizer's (``state_offset``)."""
        from . import ops

        self.iter += 1
        ops.tbe_backward_fused_raw(plan, weights_flat, self.momentum1, self.momentum2, values, offsets, batch_size,
                                   grad_out, padding_idx=padding_idx,
                                   workspace=self._ws(plan, values.numel(), batch_size, weights_flat.device),
                                   **self._hyper())

    def apply_seq(self, plan, weights_flat: torch.Tensor, table_rows, table_dims, ids, offsets, max_len,
                  grad_out: torch.Tensor, pad_mode: int, align: int) -> None:
        """The fused backward + update of one S-token gather (called from the autograd backward)."""
        from . import ops

        self.iter += 1
        B = offsets[0].numel() - 1
        ntok = B * sum(int(m) for m in max_len)
        ops.seq_gather_backward_fused_raw(
            plan, weights_flat, self.momentum1, self.momentum2, table_rows, table_dims, ids, offsets, max_len,
            grad_out, pad_mode=pad_mode, align=align,
            workspace=self._ws(plan, ntok * len(table_dims), ntok, weights_flat.device), **self._hyper())
