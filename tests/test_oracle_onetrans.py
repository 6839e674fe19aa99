"""Pins the CPU oracle of the OneTrans block (oracle/onetrans.py) against the
reference's own schedule test, library routines (torch rms_norm, scaled dot
product attention, multi-head attention), brute force on tiny inputs and the
invariants of the mixed parameterisation (CPU only)."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import onetrans as ot


def test_pyramid_schedule_reference_invariants():
    # tests/test_model.py:322-326 of the reference
    s = ot.pyramid_schedule(300, 8, 4)
    assert s[0] == 300 and s[-1] == 8 and all(s[i] >= s[i + 1] for i in range(len(s) - 1))
    # (384 - l * 368 / 3) rounded half to even: 384, 261.33, 138.67, 16
    assert ot.pyramid_schedule(384, 16, 4) == [384, 261, 139, 16]
    assert ot.pyramid_schedule(384, 16, 1) == [16]
    assert ot.pyramid_schedule(10, 2, 3) == [10, 6, 2]


def test_pyramid_mask_bruteforce():
    for q, kv in ((5, 5), (3, 7), (1, 4), (6, 9)):
        m = ot.pyramid_mask(q, kv)
        for i in range(q):
            for j in range(kv):
                assert bool(m[i, j]) == (j <= i + kv - q)
        # bottom-right alignment: the last query sees every key, the first sees kv - q + 1
        assert m[-1].all() and int(m[0].sum()) == kv - q + 1


def test_rmsnorm_matches_torch_rms_norm():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(7, 11, 256, generator=g, dtype=torch.float64) * 3
    w = 1 + 0.1 * torch.randn(256, generator=g, dtype=torch.float64)
    want = F.rms_norm(x, (256,), w, eps=1e-6)
    torch.testing.assert_close(ot.rmsnorm(x, w), want, rtol=1e-12, atol=1e-12)


def _bruteforce_attention(q, k, v):
    """Per (b, h, i): softmax over j <= i + kv - q of q.k / sqrt(dh), then sum p v (python loops)."""
    B, Lq, H, dh = q.shape
    Lk = k.shape[1]
    out = torch.zeros_like(q)
    for b in range(B):
        for h in range(H):
            for i in range(Lq):
                keys = [j for j in range(Lk) if j <= i + Lk - Lq]
                sc = [float((q[b, i, h] * k[b, j, h]).sum()) / math.sqrt(dh) for j in keys]
                mx = max(sc)
                e = [math.exp(s - mx) for s in sc]
                tot = sum(e)
                for jj, j in enumerate(keys):
                    out[b, i, h] += e[jj] / tot * v[b, j, h]
    return out


def test_attention_bruteforce_and_sdpa():
    g = torch.Generator().manual_seed(2)
    num = ot._Num("fp64")
    for Lq, Lk in ((6, 6), (3, 8), (1, 5)):
        q = torch.randn(2, Lq, 2, 4, generator=g, dtype=torch.float64)
        k = torch.randn(2, Lk, 2, 4, generator=g, dtype=torch.float64)
        v = torch.randn(2, Lk, 2, 4, generator=g, dtype=torch.float64)
        got = ot.attention(q, k, v, num)
        torch.testing.assert_close(got, _bruteforce_attention(q, k, v), rtol=1e-10, atol=1e-12)
        sdpa = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                              attn_mask=ot.pyramid_mask(Lq, Lk)).transpose(1, 2)
        torch.testing.assert_close(got, sdpa, rtol=1e-10, atol=1e-12)


def _bruteforce_block(x, w, q_len, H):
    """OneTransBlock.forward written with per-(sample, token) loops in float64."""
    x = x.double()
    B, kv, D = x.shape
    n_ns = w["ns_qkv"].shape[0]
    n_s = kv - n_ns
    dh = D // H
    Wd = {k: v.double() for k, v in w.items()}

    def norm(v, wt):
        return v / math.sqrt(float((v * v).mean()) + 1e-6) * wt

    def gelu(t):
        return 0.5 * t * (1 + torch.erf(t / math.sqrt(2)))

    y = torch.zeros(B, q_len, D, dtype=torch.float64)
    for b in range(B):
        qkv = torch.zeros(kv, 3 * D, dtype=torch.float64)
        for t in range(kv):
            Wt = Wd["s_qkv"] if t < n_s else Wd["ns_qkv"][t - n_s]
            qkv[t] = Wt @ norm(x[b, t], Wd["norm1"])
        q = qkv[:, :D].reshape(kv, H, dh)[kv - q_len:]
        k = qkv[:, D:2 * D].reshape(kv, H, dh)
        v = qkv[:, 2 * D:].reshape(kv, H, dh)
        o = _bruteforce_attention(q[None], k[None], v[None])[0].reshape(q_len, D)
        for i in range(q_len):
            z = Wd["out"] @ o[i] + x[b, kv - q_len + i]
            h2 = norm(z, Wd["norm2"])
            if i < q_len - n_ns:
                W1, W2 = Wd["s_w1"], Wd["s_w2"]
            else:
                W1, W2 = Wd["ns_w1"][i - (q_len - n_ns)], Wd["ns_w2"][i - (q_len - n_ns)]
            y[b, i] = z + W2 @ gelu(W1 @ h2)
    return y


@pytest.mark.parametrize("kv,q_len,n_ns", [(7, 7, 2), (9, 5, 3), (6, 2, 2), (5, 5, 0)])
def test_block_fp64_matches_bruteforce(kv, q_len, n_ns):
    D, H, Fd, B = 8, 2, 16, 2
    w = ot.random_weights(D, Fd, n_ns, std=0.5, seed=kv + q_len, norm_std=0.2)
    x = torch.randn(B, kv, D, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    got = ot.block_forward(x, w, q_len, H, mode="fp64")
    torch.testing.assert_close(got, _bruteforce_block(x, w, q_len, H), rtol=1e-10, atol=1e-10)


def test_shared_ns_weights_reduce_to_standard_causal_transformer_block():
    """With every NS weight equal to the shared one, the block is a plain pre-norm causal
    transformer block: attention = torch's multi_head_attention_forward with a bottom-right mask."""
    D, H, Fd, B, kv, q_len, n_ns = 16, 2, 32, 3, 10, 6, 3
    w = ot.random_weights(D, Fd, n_ns, std=0.3, seed=9, norm_std=0.1)
    w = {k: v.double() for k, v in w.items()}
    w["ns_qkv"] = w["s_qkv"].expand(n_ns, -1, -1).clone()
    w["ns_w1"] = w["s_w1"].expand(n_ns, -1, -1).clone()
    w["ns_w2"] = w["s_w2"].expand(n_ns, -1, -1).clone()
    x = torch.randn(B, kv, D, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    got = ot.block_forward(x, w, q_len, H, mode="fp64")
    h = F.rms_norm(x, (D,), w["norm1"], eps=1e-6)
    wq, wk, wv = w["s_qkv"].split(D)
    attn, _ = F.multi_head_attention_forward(
        h[:, kv - q_len:].transpose(0, 1), h.transpose(0, 1), h.transpose(0, 1), D, H, None, None, None, None,
        False, 0.0, w["out"], None, training=False, need_weights=False, attn_mask=~ot.pyramid_mask(q_len, kv),
        use_separate_proj_weight=True, q_proj_weight=wq, k_proj_weight=wk, v_proj_weight=wv)
    z = attn.transpose(0, 1) + x[:, kv - q_len:]
    want = z + F.linear(F.gelu(F.linear(F.rms_norm(z, (D,), w["norm2"], eps=1e-6), w["s_w1"])), w["s_w2"])
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)


def test_autocast_mode_close_to_fp64_and_rounds_like_bf16():
    D, H, Fd, B, kv, q_len, n_ns = 64, 1, 256, 2, 40, 24, 4
    w = ot.random_weights(D, Fd, n_ns, std=0.05, seed=5)
    x = torch.randn(B, kv, D, generator=torch.Generator().manual_seed(6))
    y16, parts = ot.block_forward(x, w, q_len, H, mode="autocast", return_parts=True)
    y64 = ot.block_forward(x, w, q_len, H, mode="fp64")
    d16, d64 = y16.double() - x[:, kv - q_len:].double(), y64 - x[:, kv - q_len:].double()
    rel = (d16 - d64).norm() / d64.norm()
    assert rel < 2e-2, rel
    # GEMM outputs and attention output are bf16 values, residual stream fp32
    for name in ("q", "k", "v", "o", "g"):
        t = parts[name]
        assert torch.equal(t, t.to(torch.bfloat16).float()), name
    assert y16.dtype == torch.float32

    # the 4-layer benchmark stack: B=1024, L_S=384, 16 NS, d 256, FFN 1024, schedule 384/256/128/64
def test_block_flops_reference_convention():
    # the benchmark workload: B=1024, L_S=384, 16 NS, d 256, FFN 1024, schedule 384/256/128/64
    tot, kv = 0.0, 400
    for q_s in (384, 256, 128, 64):
        tot += ot.block_flops(1024, kv, q_s + 16, 256, 1024, 16)
        kv = q_s + 16
    assert abs(tot / 1e9 - 1907.0) < 0.5
