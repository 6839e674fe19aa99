"""CPU oracle of the OneTrans interaction block.  TEST INFRASTRUCTURE ONLY:
used by tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg
as the checker, never by the product package.

Restates primus_dlrm/models/onetrans.py in PyTorch on the CPU:

* ``pyramid_schedule``   onetrans.py:50-59
* ``pyramid_mask``       onetrans.py:62-67  (bottom-right causal: key j <= i + kv - q)
* ``rmsnorm``            onetrans.py:74-82  (fp32, eps 1e-6, ``(x * rms) * w``)
* ``block_forward``      OneTransBlock.forward onetrans.py:220-231 with
                         MixedAttention.forward :124-169 and MixedFFN.forward :195-204
* ``sequential_tokenizer`` SequentialTokenizer.forward onetrans.py:250-257 (Linear, exact GELU,
                         Linear, + pos_emb(arange(L)))
* ``autosplit_tokenizer`` AutoSplitTokenizer.forward onetrans.py:260-276 (Linear, exact GELU, Linear,
                         view [B, n_ns, d])
* ``ns_tokenize``        OneTransModel._build_ns_raw onetrans.py:522-532 (scalar rows, then dense parts)
                         followed by the AutoSplitTokenizer (onetrans.py:561-563)
* ``seq_tokenize``       the S-token construction of OneTransModel._backbone onetrans.py:553-558:
                         per-pool gather (onetrans.py:515-520, the sequence gather of oracle.py),
                         tokenizer, concatenation along the sequence

``mode="autocast"`` reproduces the rounding points the reference has under
``torch.autocast(bf16)`` (primus_dlrm/training/dist_trainer.py:471) with an
fp32 residual stream: every Linear / einsum takes bf16-rounded operands,
accumulates in fp32 and rounds its output to bf16; attention takes bf16
q/k/v, runs the softmax in fp32 and rounds its output to bf16; GELU (exact
erf) runs in fp32 on the bf16 GEMM output and rounds to bf16; RMSNorm and the
residual additions stay fp32.  ``mode="fp64"`` runs the same graph in float64
without any rounding (ground truth).  A Linear with a bias rounds once, after
the bias: bf16(x . W^T + b) with the bias taken as bf16 (the fused GEMM
epilogue of autocast's ``addmm``).  The tokenizer's sum ``tokens + pos_emb``
adds the bf16 tokens to the fp32 position table in fp32 (type promotion).

Weights use the reference's parameter names (onetrans.py:111-113,180-184,214-218):
norm1, s_qkv [3D, D], ns_qkv [NS, 3D, D], out [D, D], norm2, s_w1 [F, D],
s_w2 [D, F], ns_w1 [NS, F, D], ns_w2 [NS, D, F].
"""
from __future__ import annotations

import math
from typing import Dict, List

import torch

WEIGHT_NAMES = ("norm1", "s_qkv", "ns_qkv", "out", "norm2", "s_w1", "s_w2", "ns_w1", "ns_w2")


def pyramid_schedule(l_s: int, l_ns: int, n_layers: int) -> List[int]:
    """onetrans.py:50-59."""
    if n_layers == 1:
        return [l_ns]
    out = []
    for layer in range(n_layers):
        q = l_s - layer * (l_s - l_ns) / (n_layers - 1)
        out.append(max(int(round(q)), l_ns))
    return out


def pyramid_mask(q_len: int, kv_len: int) -> torch.Tensor:
    """onetrans.py:62-67: mask[i, j] = j <= i + (kv_len - q_len)."""
    i = torch.arange(q_len).unsqueeze(1) + (kv_len - q_len)
    j = torch.arange(kv_len).unsqueeze(0)
    return j <= i


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


class _Num:
    """Arithmetic of one mode: ``lin`` is an autocast Linear / einsum."""

    def __init__(self, mode: str):
        if mode not in ("autocast", "fp64"):
            raise ValueError(mode)
        self.mode = mode
        self.dt = torch.float64 if mode == "fp64" else torch.float32

    def round(self, t: torch.Tensor) -> torch.Tensor:
        return _bf16(t) if self.mode == "autocast" else t

    def lin(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """x [..., K] . w[N, K]^T"""
        return self.round(torch.matmul(self.round(x), self.round(w.to(self.dt)).transpose(-1, -2)))


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """onetrans.py:80-82 (x is the fp32 or fp64 residual stream, so ``.to(x.dtype)`` keeps it)."""
    rms = x.pow(2).mean(-1, keepdim=True).add(eps).rsqrt()
    return (x * rms) * w.to(x.dtype)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num: _Num) -> torch.Tensor:
    """Causal bottom-right softmax attention on BSHD tensors, scale 1/sqrt(dh)
    (onetrans.py:148-161; the flash/SDPA default scale)."""
    B, Lq, H, dh = q.shape
    Lk = k.shape[1]
    qt, kt, vt = (num.round(t).transpose(1, 2) for t in (q, k, v))  # [B, H, L, dh]
    s = torch.matmul(qt, kt.transpose(-1, -2)) / math.sqrt(dh)
    s = s.masked_fill(~pyramid_mask(Lq, Lk), float("-inf"))
    p = torch.softmax(s, dim=-1)
    o = torch.matmul(p, vt)
    return num.round(o.transpose(1, 2))  # [B, Lq, H, dh]


def _num(mode) -> _Num:
    return mode if isinstance(mode, _Num) else _Num(mode)


def attention_inputs(x: torch.Tensor, w: Dict[str, torch.Tensor], q_len: int, n_heads: int, mode="autocast"):
    """MixedAttention's projections (onetrans.py:124-146) on RMSNorm1(x) (OneTransBlock.forward :224-225):
    shared S-token QKV Linear on the first kv - n_ns tokens, one QKV matrix per NS-token (the einsum
    "btn,tmn->btm"), Q cut to its last ``q_len`` rows.  Returns (h1, q [B, q_len, H, dh], k, v [B, kv, H, dh])."""
    num = _num(mode)
    x = x.to(num.dt)
    B, kv, D = x.shape
    n_ns = w["ns_qkv"].shape[0]
    n_s = kv - n_ns
    dh = D // n_heads
    h = rmsnorm(x, w["norm1"])
    s_qkv = num.lin(h[:, :n_s], w["s_qkv"]).reshape(B, n_s, 3, n_heads, dh)
    ns_qkv = torch.stack([num.lin(h[:, n_s + t], w["ns_qkv"][t]) for t in range(n_ns)], dim=1) if n_ns else \
        h.new_zeros(B, 0, 3 * D)
    ns_qkv = ns_qkv.reshape(B, n_ns, 3, n_heads, dh)
    q = torch.cat([s_qkv[:, :, 0], ns_qkv[:, :, 0]], dim=1)
    k = torch.cat([s_qkv[:, :, 1], ns_qkv[:, :, 1]], dim=1)
    v = torch.cat([s_qkv[:, :, 2], ns_qkv[:, :, 2]], dim=1)
    return h, q[:, kv - q_len:], k, v


def out_residual(o: torch.Tensor, x_tail: torch.Tensor, w: Dict[str, torch.Tensor], mode="autocast"):
    """z = out_proj(o) + x[:, kv - q_len:] (onetrans.py:169, :226-227) for o [B, q_len, D]."""
    num = _num(mode)
    return num.lin(o.to(num.dt), w["out"]) + x_tail.to(num.dt)


def ffn_residual(z: torch.Tensor, w: Dict[str, torch.Tensor], mode="autocast"):
    """y = z + MixedFFN(RMSNorm2(z), n_s = q_len - n_ns) (onetrans.py:195-204, :229-231): shared
    Linear -> exact GELU -> Linear on the S rows, per-token matrices on the last n_ns rows.
    Returns (y, h2, g) with g the GELU activations [B, q_len, F]."""
    num = _num(mode)
    z = z.to(num.dt)
    n_ns = w["ns_w1"].shape[0]
    h2 = rmsnorm(z, w["norm2"])
    n_s_out = z.shape[1] - n_ns
    gelu = lambda t: num.round(torch.nn.functional.gelu(t))  # noqa: E731  exact erf
    g_s = gelu(num.lin(h2[:, :n_s_out], w["s_w1"]))
    g_ns = [gelu(num.lin(h2[:, n_s_out + t], w["ns_w1"][t])) for t in range(n_ns)]
    s_out = num.lin(g_s, w["s_w2"])
    ns_out = [num.lin(g_ns[t], w["ns_w2"][t]) for t in range(n_ns)]
    y = z + torch.cat([s_out] + [t.unsqueeze(1) for t in ns_out], dim=1)
    g = torch.cat([g_s] + [t.unsqueeze(1) for t in g_ns], dim=1)
    return y, h2, g


def block_forward(x: torch.Tensor, w: Dict[str, torch.Tensor], q_len: int, n_heads: int,
                  mode="autocast", return_parts: bool = False):
    """OneTransBlock.forward (onetrans.py:220-231) for x [B, kv, D]; the last
    ``w['ns_qkv'].shape[0]`` tokens of x are the NS-tokens.  With
    ``return_parts`` also returns the intermediates (h1, q, k, v, o, z, h2, g)."""
    num = _num(mode)
    x = x.to(num.dt)
    B, kv, D = x.shape
    h, q, k, v = attention_inputs(x, w, q_len, n_heads, num)
    o = attention(q, k, v, num).reshape(B, q_len, D)
    z = out_residual(o, x[:, kv - q_len:], w, num)
    y, h2, g = ffn_residual(z, w, num)
    if return_parts:
        return y, dict(h1=h, q=q.reshape(B, q_len, D), k=k.reshape(B, kv, D), v=v.reshape(B, kv, D), o=o, z=z,
                       h2=h2, g=g)
    return y


def stack_forward(x: torch.Tensor, layers: List[Dict[str, torch.Tensor]], schedule: List[int], n_heads: int,
                  mode="autocast") -> torch.Tensor:
    """The block loop of OneTransModel._backbone (onetrans.py:568-582)."""
    n_ns = layers[0]["ns_qkv"].shape[0]
    for w, q_s in zip(layers, schedule):
        x = block_forward(x, w, q_s + n_ns, n_heads, mode)
    return x


def random_weights(D: int, F: int, n_ns: int, std: float = 0.02, seed: int = 0,
                   norm_std: float = 0.0) -> Dict[str, torch.Tensor]:
    """N(0, std) weights (bf16-representable, fp32 storage); RMSNorm weights
    1 + N(0, norm_std) (the reference initialises them to ones, onetrans.py:77)."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *shape: _bf16(torch.randn(*shape, generator=g) * std)  # noqa: E731
    return {
        "norm1": 1.0 + torch.randn(D, generator=g) * norm_std,
        "s_qkv": r(3 * D, D), "ns_qkv": r(n_ns, 3 * D, D), "out": r(D, D),
        "norm2": 1.0 + torch.randn(D, generator=g) * norm_std,
        "s_w1": r(F, D), "s_w2": r(D, F), "ns_w1": r(n_ns, F, D), "ns_w2": r(n_ns, D, F),
    }


def block_flops(B: int, kv: int, q_len: int, D: int, F: int, n_ns: int) -> float:
    """Forward FLOPs of one block by the reference's convention
    (onetrans.py:392-474 without the backward factor): S-token QKV on every kv
    S-token, attention counted full (no causal discount)."""
    n_s = kv - n_ns
    f = 2 * n_s * D * 3 * D + 2 * n_ns * 3 * D * D
    f += 4 * q_len * kv * D
    f += 2 * q_len * D * D
    f += 4 * q_len * D * F
    return float(f) * B


def _lin_bias(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, num: _Num) -> torch.Tensor:
    """autocast ``F.linear(x, w, b)``: bf16 operands, fp32 accumulation, one rounding after the bias."""
    acc = torch.matmul(num.round(x), num.round(w.to(num.dt)).transpose(-1, -2)) + num.round(b.to(num.dt))
    return num.round(acc)


def sequential_tokenizer(raw: torch.Tensor, w: Dict[str, torch.Tensor], mode: str = "autocast") -> torch.Tensor:
    """SequentialTokenizer.forward (onetrans.py:250-257) for raw [B, L, K]:
    proj = Linear(K, d) -> GELU (exact erf) -> Linear(d, d) (:243-247), then
    ``+ pos_emb(arange(L))`` when ``w["pos"]`` is not None (:254-256).  Weights
    use the module's parameter names: ``w1`` / ``b1`` = proj.0, ``w2`` / ``b2`` =
    proj.2, ``pos`` = pos_emb.weight [max_len, d] (fp32)."""
    num = _Num(mode)
    u = _lin_bias(raw.to(num.dt), w["w1"], w["b1"], num)
    h = num.round(torch.nn.functional.gelu(u))
    y = _lin_bias(h, w["w2"], w["b2"], num)
    if w.get("pos") is not None:
        L = raw.shape[1]
        y = y + w["pos"][:L].to(num.dt)
    return y


def seq_tokenize(tables, ids, offsets, max_len: List[int], weights: List[Dict[str, torch.Tensor]],
                 pad_mode: int = 0, align: int = 0, mode: str = "autocast"):
    """S-tokens of OneTransModel._backbone (onetrans.py:553-558): the padded
    per-pool gather (``oracle.seq_gather``: tables as uint16 bf16 bits or
    float32), one SequentialTokenizer per pool, pools concatenated along the
    sequence.  Returns (tokens [B, S, d] float32 (float64 in fp64 mode), mask)."""
    from . import oracle as orc
    import numpy as np

    raw, mask = orc.seq_gather(tables, ids, offsets, max_len, pad_mode=pad_mode, align=align)
    if raw.dtype == np.uint16:
        raw = (raw.astype(np.uint32) << 16).view(np.float32)
    raw = torch.from_numpy(np.ascontiguousarray(raw))
    parts, s0 = [], 0
    for p, L in enumerate(max_len):
        parts.append(sequential_tokenizer(raw[:, s0:s0 + L], weights[p], mode))
        s0 += L
    return torch.cat(parts, dim=1), mask


def random_tokenizer_weights(K: int, d: int, max_len: int, std: float = 0.05, seed: int = 0,
                             pos: bool = True) -> Dict[str, torch.Tensor]:
    """bf16-representable N(0, std) Linear weights and biases (fp32 storage), N(0, 1) fp32 positions."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *shape: _bf16(torch.randn(*shape, generator=g) * std)  # noqa: E731
    return {"w1": r(d, K), "b1": r(d), "w2": r(d, d), "b2": r(d),
            "pos": torch.randn(max_len, d, generator=g) if pos else None}


def autosplit_tokenizer(ns_raw: torch.Tensor, w: Dict[str, torch.Tensor], n_ns: int,
                        mode: str = "autocast") -> torch.Tensor:
    """AutoSplitTokenizer.forward (onetrans.py:260-276) for ns_raw [B, K]: proj = Linear(K, d*n_ns), GELU,
    Linear(d*n_ns, d*n_ns), viewed as [B, n_ns, d] (bf16 values as float32 in autocast mode)."""
    num = _Num(mode)
    h = num.round(torch.nn.functional.gelu(_lin_bias(ns_raw.to(num.dt), w["w1"], w["b1"], num)))
    y = _lin_bias(h, w["w2"], w["b2"], num)
    return y.view(y.shape[0], n_ns, -1)


def ns_tokenize(tables, ids, dense, w: Dict[str, torch.Tensor], n_ns: int, mode: str = "autocast"):
    """NS tokens from the scalar-feature rows ``tables[j][ids[j]]`` (numpy uint16 bf16 bits or float32; an id
    outside the table gives a zero row) and the float32 ``dense`` parts [B, dim], concatenated in that order
    (onetrans.py:522-532), through the AutoSplitTokenizer."""
    import numpy as np

    parts = []
    for t, i in zip(tables, ids):
        t = np.ascontiguousarray(t)
        if t.dtype == np.uint16:
            t = (t.astype(np.uint32) << 16).view(np.float32)
        i = np.asarray(i, dtype=np.int64)
        ok = (i >= 0) & (i < t.shape[0])
        rows = t[np.where(ok, i, 0)].copy()
        rows[~ok] = 0
        parts.append(torch.from_numpy(rows))
    parts += [torch.as_tensor(np.asarray(x, dtype=np.float32)) for x in dense]
    return autosplit_tokenizer(torch.cat(parts, dim=1), w, n_ns, mode)


def random_autosplit_weights(K: int, N: int, std: float = 0.05, seed: int = 0) -> Dict[str, torch.Tensor]:
    """bf16-representable N(0, std) AutoSplitTokenizer weights and biases (fp32 storage)."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *shape: _bf16(torch.randn(*shape, generator=g) * std)  # noqa: E731
    return {"w1": r(N, K), "b1": r(N), "w2": r(N, N), "b2": r(N)}


def term_magnitudes(x: torch.Tensor, w: Dict[str, torch.Tensor], q_len: int, n_heads: int,
                    parts: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """Sum of the absolute terms behind each block intermediate (float64), the scale against which a
    rounding difference is measured: a dot product's result may move by about one bf16 ulp of its
    largest terms when an input moves across a rounding boundary or the summation order changes.

    k, v: |h1| . |W_qkv|^T (shared or per-token rows); o: P . |V| with the softmax probabilities P of the
    bf16 q, k; y (and the update y - x_tail): |o| . |W_out|^T + |g| . |W_2|^T (shared or per-token);
    h2 (when ``parts`` holds z): the out-projection's terms scaled by RMSNorm2's factor and weight;
    g (when ``parts`` holds h2): |h2| . |W_1|^T, the FFN-up terms (GELU's slope is at most 1.13)."""
    B, kv, D = x.shape
    n_ns = w["ns_qkv"].shape[0]
    n_s = kv - n_ns
    dh = D // n_heads
    f = lambda t: t.double().abs()  # noqa: E731
    h1 = f(_bf16(parts["h1"].float()))
    qkv = torch.cat([h1[:, :n_s] @ f(w["s_qkv"]).T] +
                    [(h1[:, n_s + t] @ f(w["ns_qkv"][t]).T).unsqueeze(1) for t in range(n_ns)], dim=1)
    q = parts["q"].double().reshape(B, q_len, n_heads, dh).transpose(1, 2)
    k = parts["k"].double().reshape(B, kv, n_heads, dh).transpose(1, 2)
    v = f(parts["v"]).reshape(B, kv, n_heads, dh).transpose(1, 2)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(dh)
    p = torch.softmax(s.masked_fill(~pyramid_mask(q_len, kv), float("-inf")), dim=-1)
    o = (p @ v).transpose(1, 2).reshape(B, q_len, D)
    n_s_out = q_len - n_ns
    g = f(parts["g"])
    ffn = torch.cat([g[:, :n_s_out] @ f(w["s_w2"]).T] +
                    [(g[:, n_s_out + t] @ f(w["ns_w2"][t]).T).unsqueeze(1) for t in range(n_ns)], dim=1)
    z_terms = f(parts["o"]) @ f(w["out"]).T
    upd = z_terms + ffn
    out = dict(k=qkv[..., D:2 * D], v=qkv[..., 2 * D:], q=qkv[:, kv - q_len:, :D], o=o, y=upd)
    if "z" in parts:
        z = parts["z"].double()
        out["h2"] = z_terms * z.pow(2).mean(-1, keepdim=True).add(1e-6).rsqrt() * f(w["norm2"])
    if "h2" in parts:
        h2 = f(_bf16(parts["h2"].float()))
        out["g"] = torch.cat([h2[:, :n_s_out] @ f(w["s_w1"]).T] +
                             [(h2[:, n_s_out + t] @ f(w["ns_w1"][t]).T).unsqueeze(1) for t in range(n_ns)], dim=1)
    return out
