"""Pins the rounding points of the block oracle's autocast mode (oracle/onetrans.py) against torch's own
CPU ``autocast(bf16)`` running a restatement of the reference block with torch modules: RMSNorm as
written at primus_dlrm/models/onetrans.py:80-82, ``nn.Linear`` for the shared projections, the reference's
``einsum``s for the per-token ones (:137,201-202), ``F.scaled_dot_product_attention`` with the bool pyramid
mask (:156-161) and ``F.gelu`` (:200-201), composed as in OneTransBlock.forward (:220-231).  Autocast decides
where bf16 rounding happens independently of the oracle's explicit ``round`` calls.

Each stage is fed the same inputs on both sides, so a difference belongs to that stage:
  * projections: K and V equal except where fp32 summation order moves a value across a bf16 rounding
    boundary (< 1 % of the values, one ulp);
  * attention: within 2^-7 of the sum of absolute terms P.|V| (torch's CPU flash kernel rounds the
    unnormalised probabilities to bf16 before P.V; the oracle keeps them in fp32);
  * out-projection + residual, FFN + residual: < 1 % of the values differ, by one ulp of the bf16 GEMM output.
Each check is shown to fail for a misplaced rounding point planted in the oracle."""
import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import onetrans as ot

D, FD, H, N_NS = 256, 1024, 4, 16


def _rms(x, w):
    """onetrans.py:80-82."""
    rms = x.float().pow(2).mean(-1, keepdim=True).add(1e-6).rsqrt()
    return (x.float() * rms).to(x.dtype) * w


class _RefStages(nn.Module):
    """The reference block's computation, split at the same points as the oracle's stage functions."""

    def __init__(self, w):
        super().__init__()
        self.w = w
        self.s_qkv = nn.Linear(D, 3 * D, bias=False)
        self.out_proj = nn.Linear(D, D, bias=False)
        self.s_w1 = nn.Linear(D, FD, bias=False)
        self.s_w2 = nn.Linear(FD, D, bias=False)
        with torch.no_grad():
            self.s_qkv.weight.copy_(w["s_qkv"])
            self.out_proj.weight.copy_(w["out"])
            self.s_w1.weight.copy_(w["s_w1"])
            self.s_w2.weight.copy_(w["s_w2"])

    def projections(self, x, q_len):
        B, kv, _ = x.shape
        n_s = kv - N_NS
        normed = _rms(x, self.w["norm1"])
        s_qkv = self.s_qkv(normed[:, :n_s]).reshape(B, n_s, 3, H, D // H)
        ns_qkv = torch.einsum("btn,tmn->btm", normed[:, n_s:], self.w["ns_qkv"]).reshape(B, N_NS, 3, H, D // H)
        q = torch.cat([s_qkv[:, :, 0], ns_qkv[:, :, 0]], 1)[:, kv - q_len:]
        k = torch.cat([s_qkv[:, :, 1], ns_qkv[:, :, 1]], 1)
        v = torch.cat([s_qkv[:, :, 2], ns_qkv[:, :, 2]], 1)
        return q, k, v

    @staticmethod
    def attention(q, k, v):
        mask = ot.pyramid_mask(q.shape[1], k.shape[1])
        o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                           attn_mask=mask[None, None]).transpose(1, 2)
        return o.reshape(q.shape[0], q.shape[1], D)

    def out_residual(self, o, x_tail):
        return self.out_proj(o) + x_tail

    def ffn_residual(self, z):
        n_s_out = z.shape[1] - N_NS
        h2 = _rms(z, self.w["norm2"])
        s_out = self.s_w2(F.gelu(self.s_w1(h2[:, :n_s_out])))
        ns_h = F.gelu(torch.einsum("btn,tmn->btm", h2[:, n_s_out:], self.w["ns_w1"]))
        ns_out = torch.einsum("btm,tnm->btn", ns_h, self.w["ns_w2"])
        return z + torch.cat([s_out, ns_out], 1)


@pytest.fixture(scope="module")
def case():
    w = ot.random_weights(D, FD, N_NS, std=0.02, seed=41, norm_std=0.3)
    x = torch.randn(3, 144, D, generator=torch.Generator().manual_seed(42))
    return w, x, 80, _RefStages(w)


def _auto():
    return torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16)


def _frac_differ(a, b):
    return (a.float() != b.float()).float().mean().item()


def test_projections_round_like_autocast(case, monkeypatch):
    w, x, q_len, ref = case
    with _auto()[0], _auto()[1]:
        q_r, k_r, v_r = ref.projections(x, q_len)
    assert k_r.dtype == torch.bfloat16
    _, parts = ot.block_forward(x, w, q_len, H, return_parts=True)
    mag = ot.term_magnitudes(x, w, q_len, H, parts)
    _, q_o, k_o, v_o = ot.attention_inputs(x, w, q_len, H)
    for name, a, b in (("q", q_r, q_o), ("k", k_r, k_o), ("v", v_r, v_o)):
        a, b = a.reshape(mag[name].shape).double(), b.reshape(mag[name].shape).double()
        assert _frac_differ(a, b) < 0.01
        # one bf16 ulp of the value, plus fp32 summation-order noise of the terms
        assert bool(((a - b).abs() <= 2.0 ** -7 * b.abs() + 2.0 ** -16 * mag[name]).all())
    # planted: RMSNorm output rounded to bf16 before the weight multiply (a bf16 residual stream's rounding)
    rms = ot.rmsnorm
    monkeypatch.setattr(ot, "rmsnorm", lambda t, wt, eps=1e-6: ot._bf16(rms(t, torch.ones_like(wt), eps)) * wt)
    _, _, k_bad, _ = ot.attention_inputs(x, w, q_len, H)
    assert _frac_differ(k_r, k_bad) > 0.05


def test_attention_within_bf16_noise_of_sdpa(case, monkeypatch):
    w, x, q_len, ref = case
    with _auto()[0], _auto()[1]:
        q, k, v = ref.projections(x, q_len)
        o_r = ref.attention(q, k, v)
    assert o_r.dtype == torch.bfloat16
    o_o = ot.attention(q.float(), k.float(), v.float(), ot._Num("autocast")).reshape(o_r.shape)
    assert torch.equal(o_o, ot._bf16(o_o))
    B, kv = k.shape[:2]
    parts = dict(h1=torch.zeros(B, kv, D), q=q.float(), k=k.float(), v=v.float(), o=o_o,
                 g=torch.zeros(B, q_len, FD))
    mag = ot.term_magnitudes(x, w, q_len, H, parts)["o"]
    err = (o_r.double() - o_o.double()).abs()
    assert bool((err <= 2.0 ** -7 * mag).all())
    assert (err.norm() / o_o.double().norm()).item() < 4e-3
    # planted: top-left causal alignment instead of the bottom-right pyramid mask
    monkeypatch.setattr(ot, "pyramid_mask", lambda ql, kl: torch.ones(ql, kl, dtype=torch.bool).tril())
    o_bad = ot.attention(q.float(), k.float(), v.float(), ot._Num("autocast")).reshape(o_r.shape)
    assert not bool(((o_r.double() - o_bad.double()).abs() <= 2.0 ** -7 * mag).all())


def test_out_projection_residual_round_like_autocast(case):
    w, x, q_len, ref = case
    with _auto()[0], _auto()[1]:
        q, k, v = ref.projections(x, q_len)
        o = ref.attention(q, k, v)
        z_r = ref.out_residual(o, x[:, -q_len:])
    assert z_r.dtype == torch.float32
    z_o = ot.out_residual(o.float(), x[:, -q_len:], w)
    assert _frac_differ(z_r, z_o) < 0.01
    # planted: a bf16 residual stream (z rounded)
    assert _frac_differ(z_r, ot._bf16(z_o)) > 0.5


def test_ffn_residual_round_like_autocast(case):
    w, x, q_len, ref = case
    z = x[:, -q_len:] + 0.05 * torch.randn(x.shape[0], q_len, D, generator=torch.Generator().manual_seed(43))
    with _auto()[0], _auto()[1]:
        y_r = ref.ffn_residual(z)
    assert y_r.dtype == torch.float32
    y_o, _, g = ot.ffn_residual(z, w)
    assert torch.equal(g, ot._bf16(g))
    assert _frac_differ(y_r, y_o) < 0.01

    # planted: the FFN GEMM outputs left in fp32 (no rounding after the up or the down projection)
    class NoOutRound(ot._Num):
        def lin(self, a, b):
            return torch.matmul(self.round(a), self.round(b.to(self.dt)).transpose(-1, -2))

    y_bad, _, _ = ot.ffn_residual(z, w, NoOutRound("autocast"))
    assert _frac_differ(y_r, y_bad) > 0.5

    # planted: GELU taken on the fp32 up-projection (rounding moved after the GELU)
    class LateRound(ot._Num):
        def lin(self, a, b):
            out = torch.matmul(self.round(a), self.round(b.to(self.dt)).transpose(-1, -2))
            return out if b.shape[-2] == FD else self.round(out)

    y_late, _, _ = ot.ffn_residual(z, w, LateRound("autocast"))
    assert _frac_differ(y_r, y_late) > 0.02


def test_whole_block_within_bf16_noise_of_autocast(case):
    w, x, q_len, ref = case
    with _auto()[0], _auto()[1]:
        q, k, v = ref.projections(x, q_len)
        o = ref.attention(q, k, v)
        z = ref.out_residual(o, x[:, -q_len:])
        y_r = ref.ffn_residual(z)
    y_o, parts = ot.block_forward(x, w, q_len, H, return_parts=True)
    mag = ot.term_magnitudes(x, w, q_len, H, parts)["y"]
    err = (y_r.double() - y_o.double()).abs()
    x_tail = x[:, -q_len:].double()
    assert bool((err <= 2e-2 * mag).all())
    assert (err > 2.0 ** -7 * mag).float().mean().item() < 0.01
    assert (err.norm() / (y_o.double() - x_tail).norm()).item() < 5e-3
    assert math.isfinite(err.max().item())
