"""OneTrans interaction block with the reference's module surface.

``OneTransBlock(d_model, n_heads, n_ns_tokens, ffn_mult=4, dropout=0.0, attention_impl=...)``
and ``forward(x, mask, q_len, n_s_tokens) -> [B, q_len, D]`` follow
primus_dlrm/models/onetrans.py:207-231; parameter names and shapes
(``norm1.weight``, ``attn.s_qkv.weight``, ``attn.ns_qkv_weight``,
``attn.out_proj.weight``, ``norm2.weight``, ``ffn.s_w1.weight``,
``ffn.s_w2.weight``, ``ffn.ns_w1``, ``ffn.ns_w2``; :77,111-113,180-184,214-218)
match so reference state dicts load unchanged.  Forward runs the fused gfx950
kernels in the numerics the reference gets under ``autocast(bf16)``
(primus_dlrm/training/dist_trainer.py:471): bf16 GEMM operands with fp32
accumulation, fp32 RMSNorm, exact-erf GELU, fp32 residual stream.

``pyramid_schedule`` and ``build_pyramid_mask`` restate onetrans.py:50-67.

``SequentialTokenizer(raw_dim, d_model, max_len, use_pos_embed)`` follows
onetrans.py:238-257 (``proj.0`` / ``proj.2`` Linear layers, ``pos_emb``); its
forward and ``FusedSequenceTokenizer`` (the S-token construction of
onetrans.py:553-558 straight from the sequence ids) run the fused gather +
tokenizer kernel with the same autocast numerics.  ``AutoSplitTokenizer(ns_input_dim,
d_model, n_ns_tokens)`` follows onetrans.py:260-276; ``FusedNSTokenizer`` builds the
NS input of onetrans.py:522-532 (scalar-feature rows, then dense parts) on the
device and runs it.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn

from . import _lib as L
from . import ops
from .kjt import mask_as_bool


def pyramid_schedule(l_s: int, l_ns: int, n_layers: int) -> List[int]:
    """S-token queries kept per layer, shrinking linearly from l_s to l_ns
    (onetrans.py:50-59; Python's round-half-even, floor at l_ns)."""
    if n_layers == 1:
        return [l_ns]
    out = []
    for layer in range(n_layers):
        q = l_s - layer * (l_s - l_ns) / (n_layers - 1)
        out.append(max(int(round(q)), l_ns))
    return out


# symbolic tracing records calls to the schedule as one node (its Python loop needs concrete ints), as the
# reference's @torch.fx.wrap does (onetrans.py:49)
torch.fx.wrap("pyramid_schedule")


def _in_graph(*tensors) -> bool:
    """True inside torch.compile tracing or torch.fx symbolic tracing (where tensors are proxies)."""
    return torch.compiler.is_compiling() or any(isinstance(t, torch.fx.Proxy) for t in tensors)


def _bf16_copies(module: nn.Module, params: Sequence[torch.Tensor]) -> tuple:
    """bf16 copies of ``params``: autocast's casts of fp32 weights for every matmul.  Eagerly they are made once
    per parameter version and kept on ``module``; inside a traced or compiled graph they are graph ops."""
    if _in_graph(*params):
        return tuple(p.detach().to(torch.bfloat16).contiguous() for p in params)
    key = tuple((p.data_ptr(), p._version, p.device) for p in params)
    cache = module.__dict__.get("_bf16_cache")
    if cache is None or cache[0] != key:
        cache = (key, tuple(p.detach().to(torch.bfloat16).contiguous() for p in params))
        module.__dict__["_bf16_cache"] = cache
    return cache[1]


def _check_stream(x: torch.Tensor) -> None:
    if x.dtype != torch.float32:
        raise TypeError("the residual stream x must be fp32: the reference's stream under autocast when the "
                        "S-tokens carry positional embeddings (use_pos_embed=True); a bf16 stream "
                        "(use_pos_embed=False) rounds the RMSNorm outputs and residual sums to bf16, rounding "
                        "points these kernels do not implement")


def build_pyramid_mask(q_len: int, kv_len: int, device: torch.device) -> torch.Tensor:
    """Bottom-right causal mask ``[q_len, kv_len]``: query i sees keys
    j <= i + (kv_len - q_len) (onetrans.py:62-67).  The mask is tagged as the pyramid mask of its shape, so
    ``OneTransBlock.forward`` accepts it without comparing its values (inference tensors, which keep no
    version counter, are compared on every call)."""
    offset = kv_len - q_len
    q_idx = torch.arange(q_len, device=device).unsqueeze(1) + offset
    kv_idx = torch.arange(kv_len, device=device).unsqueeze(0)
    mask = kv_idx <= q_idx
    _tag_pyramid(mask, q_len, kv_len)
    return mask


def _version_of(t: torch.Tensor) -> Optional[int]:
    try:
        return t._version
    except RuntimeError:  # inference tensors keep no version counter
        return None


def _tag_pyramid(mask: torch.Tensor, q_len: int, kv_len: int) -> None:
    version = _version_of(mask)
    if version is not None and not torch.compiler.is_compiling() and not isinstance(mask, torch.fx.Proxy):
        mask._pdm_pyramid = (q_len, kv_len, version)


def check_pyramid_mask(mask: torch.Tensor, q_len: int, kv_len: int) -> None:
    """The kernels apply the pyramid mask (``build_pyramid_mask(q_len, kv_len)``, the only mask the
    reference's backbone passes, onetrans.py:568-582) whatever mask they are given, so any other mask is
    rejected here.  A mask made by ``build_pyramid_mask`` and not modified since passes at once; any other
    tensor is compared with the pyramid mask (one device-to-host sync) and, when equal, tagged so that later
    calls with the same unmodified tensor pass at once."""
    if tuple(mask.shape) != (q_len, kv_len):
        raise ValueError(f"mask must be [q_len, kv_len] = [{q_len}, {kv_len}]")
    if mask.dtype != torch.bool:
        raise ValueError("mask must be a bool mask (True = the query attends to the key), as build_pyramid_mask "
                         "makes it")
    version = _version_of(mask)
    if version is not None and getattr(mask, "_pdm_pyramid", None) == (q_len, kv_len, version):
        return
    if not torch.equal(mask, build_pyramid_mask(q_len, kv_len, mask.device)):
        raise ValueError("only the pyramid mask build_pyramid_mask(q_len, kv_len) is supported: the kernels "
                         "apply the bottom-right causal mask; run the reference's attention for other masks")
    _tag_pyramid(mask, q_len, kv_len)


class RMSNorm(nn.Module):
    """Parameter container with the reference's RMSNorm surface (onetrans.py:74-82)."""

    def __init__(self, d: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps


class MixedAttention(nn.Module):
    """Parameters of the reference MixedAttention (onetrans.py:85-121)."""

    def __init__(self, d_model: int, n_heads: int, n_ns_tokens: int, dropout: float = 0.0,
                 attention_impl: str = "pdm"):
        super().__init__()
        if d_model % n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        self.d_model, self.n_heads, self.d_head, self.n_ns = d_model, n_heads, d_model // n_heads, n_ns_tokens
        self.attention_impl = attention_impl
        self.s_qkv = nn.Linear(d_model, 3 * d_model, bias=False)
        self.ns_qkv_weight = nn.Parameter(torch.empty(n_ns_tokens, 3 * d_model, d_model))
        self.out_proj = nn.Linear(d_model, d_model, bias=False)
        self.attn_drop = dropout
        nn.init.xavier_uniform_(self.s_qkv.weight)
        nn.init.xavier_uniform_(self.out_proj.weight)
        for i in range(n_ns_tokens):
            nn.init.xavier_uniform_(self.ns_qkv_weight.data[i])


class MixedFFN(nn.Module):
    """Parameters of the reference MixedFFN (onetrans.py:172-193)."""

    def __init__(self, d_model: int, ffn_dim: int, n_ns_tokens: int, dropout: float = 0.0):
        super().__init__()
        self.n_ns, self.d_model = n_ns_tokens, d_model
        self.s_w1 = nn.Linear(d_model, ffn_dim, bias=False)
        self.s_w2 = nn.Linear(ffn_dim, d_model, bias=False)
        self.ns_w1 = nn.Parameter(torch.empty(n_ns_tokens, ffn_dim, d_model))
        self.ns_w2 = nn.Parameter(torch.empty(n_ns_tokens, d_model, ffn_dim))
        self.dropout = nn.Dropout(dropout)
        nn.init.xavier_uniform_(self.s_w1.weight)
        nn.init.xavier_uniform_(self.s_w2.weight)
        for i in range(n_ns_tokens):
            nn.init.xavier_uniform_(self.ns_w1.data[i])
            nn.init.xavier_uniform_(self.ns_w2.data[i])


class OneTransBlock(nn.Module):
    """Pre-norm causal block with shared S-token and per-token NS weights.

    Forward only (inference / evaluation); dropout must be inactive.  ``x``
    is the fp32 residual stream ``[B, kv_len, D]`` whose last ``n_ns`` tokens
    are the NS-tokens; ``mask`` must be ``build_pyramid_mask(q_len, kv_len)`` or None
    (``check_pyramid_mask``: other masks raise ``ValueError``; checked eagerly, not inside a compiled graph).
    """

    def __init__(self, d_model: int, n_heads: int, n_ns_tokens: int, ffn_mult: int = 4,
                 dropout: float = 0.0, attention_impl: str = "pdm"):
        super().__init__()
        self.norm1 = RMSNorm(d_model)
        self.attn = MixedAttention(d_model, n_heads, n_ns_tokens, dropout, attention_impl)
        self.norm2 = RMSNorm(d_model)
        self.ffn = MixedFFN(d_model, d_model * ffn_mult, n_ns_tokens, dropout)

    def forward(self, x: torch.Tensor, mask: torch.Tensor, q_len: int, n_s_tokens: int) -> torch.Tensor:
        self._check_eval()
        # under torch.fx symbolic tracing the arguments are proxies: the checks run when the traced graph runs
        # the op (its host-side validation), not here
        fx_tracing = isinstance(x, torch.fx.Proxy)
        if not fx_tracing:
            kv_len = x.shape[1]
            if n_s_tokens != kv_len - self.attn.n_ns:
                raise ValueError(f"n_s_tokens ({n_s_tokens}) must equal kv_len - n_ns ({kv_len - self.attn.n_ns})")
            # (not while compiling: the mask is no graph input, and equating q_len with its size would leave
            # q_len bound to a symbol the compiled graph does not receive)
            if mask is not None and not torch.compiler.is_compiling():
                check_pyramid_mask(mask, q_len, kv_len)
            _check_stream(x)
        return torch.ops.pdm.onetrans_block_fwd(x.contiguous(), *self.kernel_weights(), self.attn.n_heads, q_len)

    def kernel_weights(self) -> Tuple[torch.Tensor, ...]:
        """The nine tensors the kernels take, in pdm_block_weights order: the RMSNorm weights as fp32 and the
        projection weights as autocast's bf16 casts (made once per parameter version)."""
        s_qkv, ns_qkv, out_w, s_w1, s_w2, ns_w1, ns_w2 = _bf16_copies(self, (
            self.attn.s_qkv.weight, self.attn.ns_qkv_weight, self.attn.out_proj.weight,
            self.ffn.s_w1.weight, self.ffn.s_w2.weight, self.ffn.ns_w1, self.ffn.ns_w2))
        return (self.norm1.weight.detach().float().contiguous(), s_qkv, ns_qkv, out_w,
                self.norm2.weight.detach().float().contiguous(), s_w1, s_w2, ns_w1, ns_w2)

    def _check_eval(self) -> None:
        if self.training and (self.attn.attn_drop > 0 or self.ffn.dropout.p > 0):
            raise RuntimeError("OneTransBlock forward kernels do not implement dropout; call .eval()")


class OneTransStack(nn.Module):
    """The block loop of OneTransModel._backbone (onetrans.py:568-582): layer
    l keeps ``schedule[l] + n_ns`` query tokens of the previous output.  The
    whole loop is one call (pdm_onetrans_stack_fwd): the layers share one
    workspace and the inner layers' outputs never leave it."""

    def __init__(self, d_model: int, n_heads: int, n_ns_tokens: int, n_layers: int, ffn_mult: int = 4,
                 schedule: Optional[Sequence[int]] = None):
        super().__init__()
        self.n_ns = n_ns_tokens
        self.schedule = list(schedule) if schedule is not None else None
        self.blocks = nn.ModuleList([OneTransBlock(d_model, n_heads, n_ns_tokens, ffn_mult)
                                     for _ in range(n_layers)])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        L_S = x.shape[1] - self.n_ns
        schedule = self.schedule or pyramid_schedule(L_S, self.n_ns, len(self.blocks))
        if not isinstance(x, torch.fx.Proxy):
            _check_stream(x)
        weights = []
        for block in self.blocks:
            block._check_eval()
            weights.extend(block.kernel_weights())
        return torch.ops.pdm.onetrans_stack_fwd(x.contiguous(), weights, self.blocks[0].attn.n_heads, schedule)


class SequentialTokenizer(nn.Module):
    """Per-position history embeddings -> S-tokens (onetrans.py:238-257): ``proj`` = Linear(raw_dim, d_model),
    GELU, Linear(d_model, d_model), plus ``pos_emb(arange(L))`` when ``use_pos_embed``.

    ``forward(raw)`` takes raw ``[B, L, raw_dim]`` (fp32 or bf16) and returns fp32 ``[B, L, d_model]``: the
    reference's result under ``autocast(bf16)``.  The rows of ``raw`` are fed to the fused kernel as a table
    read in order.  Forward only; raw_dim in {128, 192, 256, 384}, d_model in {128, 256, 384}."""

    def __init__(self, raw_dim: int, d_model: int, max_len: int = 1024, use_pos_embed: bool = True):
        super().__init__()
        self.proj = nn.Sequential(nn.Linear(raw_dim, d_model), nn.GELU(), nn.Linear(d_model, d_model))
        self.pos_emb = nn.Embedding(max_len, d_model) if use_pos_embed else None

    def kernel_weights(self) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
        """(w1, b1, w2, b2) as bf16 (autocast's casts, made once per parameter version) and the fp32 positions."""
        lin1, lin2 = self.proj[0], self.proj[2]
        pos = None if self.pos_emb is None else self.pos_emb.weight.detach().float().contiguous()
        return (*_bf16_copies(self, (lin1.weight, lin1.bias, lin2.weight, lin2.bias)), pos)

    def forward(self, raw: torch.Tensor) -> torch.Tensor:
        if raw.dim() != 3:
            raise ValueError("raw must be [B, L, raw_dim]")
        B, Lq, K = raw.shape
        if raw.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("raw must be fp32 or bf16")
        table = raw.reshape(B * Lq, K).contiguous()
        ids = torch.arange(B * Lq, dtype=torch.int64, device=raw.device)
        offsets = torch.arange(0, B * Lq + 1, max(Lq, 1), dtype=torch.int64, device=raw.device)[:B + 1]
        if Lq == 0:
            offsets = torch.zeros(B + 1, dtype=torch.int64, device=raw.device)
        w1, b1, w2, b2, pos = self.kernel_weights()
        out, _ = torch.ops.pdm.seq_tokenize_fwd([table], [ids], [offsets], [Lq], [w1], [b1], [w2], [b2], [pos],
                                                L.PDM_PAD_ROW0, L.PDM_ALIGN_RIGHT)
        return out


class FusedSequenceTokenizer(nn.Module):
    """The S-tokens of OneTransModel._backbone (onetrans.py:553-558) from the sequence ids: the padded gather of
    ``gather`` (a SequenceGather) and ``tokenizers[pool]`` (SequentialTokenizer modules, e.g. the reference's
    ``seq_tokenizers`` ModuleDict) fused, so the ``[B, S, sum D]`` raw rows never reach memory.

    ``forward(batch)`` takes the SequenceGather batch convention and returns (tokens fp32 ``[B, S, d_model]``,
    mask bool ``[B, S]``); the pools' tokens are concatenated along the sequence in the gather's pool order.
    With ``out`` given (fp32 ``[B, >= S, d_model]`` with contiguous rows, e.g. the leading rows of the block
    input) the tokens are written there.  Forward only."""

    def __init__(self, gather, tokenizers: Dict[str, SequentialTokenizer]):
        super().__init__()
        self.gather = gather
        self.tokenizers = tokenizers if isinstance(tokenizers, nn.ModuleDict) else nn.ModuleDict(tokenizers)
        missing = [g for g in gather.groups if g not in self.tokenizers]
        if missing:
            raise ValueError(f"no tokenizer for pools {missing}")

    def forward(self, batch: Dict[str, torch.Tensor], out: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
        g = self.gather
        ec = g.ec
        tables = [ec._store.weight(ec._tables[ti].name) for ti in g._feature_tables]
        ids, offsets, max_len = [], [], []
        w = {k: [] for k in ("w1", "b1", "w2", "b2", "pos")}
        for name, fs in g.groups.items():
            lengths = batch[fs[0] + "__lengths"]
            offsets.append(torch.nn.functional.pad(lengths.reshape(-1).to(torch.int64).cumsum(0), (1, 0)))
            ids.extend(batch[f].reshape(-1).to(torch.int64).contiguous() for f in fs)
            max_len.append(g.max_len[name])
            for k, t in zip(("w1", "b1", "w2", "b2", "pos"), self.tokenizers[name].kernel_weights()):
                w[k].append(t)
        if out is None:
            tokens, mask = torch.ops.pdm.seq_tokenize_fwd(tables, ids, offsets, max_len, w["w1"], w["b1"], w["w2"],
                                                          w["b2"], w["pos"], g.pad_mode, g.align)
            return tokens, mask_as_bool(mask)
        F = len(tables)
        grid = [ids[p * F:(p + 1) * F] for p in range(len(offsets))]
        weights = [dict(w1=w["w1"][p], b1=w["b1"][p], w2=w["w2"][p], b2=w["b2"][p], pos=w["pos"][p])
                   for p in range(len(offsets))]
        tokens, mask = ops.seq_tokenize_raw(tables, grid, offsets, max_len, weights, g.pad_mode, g.align, out=out)
        return tokens, mask_as_bool(mask)


class AutoSplitTokenizer(nn.Module):
    """NS features -> n_ns tokens (onetrans.py:260-276): ``proj`` = Linear(ns_input_dim, d*n_ns), GELU,
    Linear(d*n_ns, d*n_ns), viewed as [B, n_ns, d].  ``forward(ns_features)`` takes fp32 [B, ns_input_dim] and
    returns fp32 [B, n_ns, d] (the bf16 result of the reference under autocast).  Forward only; d*n_ns a
    multiple of 64."""

    def __init__(self, ns_input_dim: int, d_model: int, n_ns_tokens: int):
        super().__init__()
        out_dim = d_model * n_ns_tokens
        self.proj = nn.Sequential(nn.Linear(ns_input_dim, out_dim), nn.GELU(), nn.Linear(out_dim, out_dim))
        self.n_ns_tokens = n_ns_tokens
        self.d_model = d_model
        self._ws: Optional[torch.Tensor] = None

    def kernel_weights(self) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """(w1, b1, w2, b2) as bf16 (autocast's casts, made once per parameter version)."""
        lin1, lin2 = self.proj[0], self.proj[2]
        return _bf16_copies(self, (lin1.weight, lin1.bias, lin2.weight, lin2.bias))

    def run(self, tables, ids, dense, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        w1, b1, w2, b2 = self.kernel_weights()
        return ops.ns_tokenize_raw(tables, ids, dense, w1, b1, w2, b2, self.n_ns_tokens, out=out)

    def forward(self, ns_features: torch.Tensor) -> torch.Tensor:
        x = ns_features if ns_features.dtype == torch.float32 else ns_features.float()
        return self.run([], [], [x])


class FusedNSTokenizer(nn.Module):
    """The NS tokens of OneTransModel._backbone (onetrans.py:522-532,561-563) with the scalar-feature lookups
    fused: ``forward(batch, dense_parts)`` reads one id per sample of every scalar feature from ``batch`` (the
    EmbeddingCollection ``ec``'s tables, in ``scalar_features`` order), appends the fp32 dense parts (the
    reference's ``dense_projs[name](batch[name])`` or raw features, in config order) and runs ``tokenizer`` (an
    AutoSplitTokenizer).  Returns fp32 [B, n_ns, d]; ``out`` may be the block input's NS rows.  Forward only."""

    def __init__(self, ec, scalar_features: Sequence[str], tokenizer: AutoSplitTokenizer):
        super().__init__()
        self.ec = ec
        self.scalar_features = list(scalar_features)
        self.tokenizer = tokenizer
        self._tables = [ec._feature_table[f] for f in self.scalar_features]

    def forward(self, batch: Dict[str, torch.Tensor], dense_parts: Sequence[torch.Tensor] = (),
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
        ec = self.ec
        tables = [ec._store.weight(ec._tables[ti].name) for ti in self._tables]
        ids = [batch[f].reshape(-1).to(torch.int64).contiguous() for f in self.scalar_features]
        dense = [x if x.dtype == torch.float32 else x.float() for x in dense_parts]
        return self.tokenizer.run(tables, ids, dense, out=out)
