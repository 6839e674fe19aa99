"""GPU parity of the OneTrans block kernels against the CPU oracle
(oracle/onetrans.py, autocast emulation) on the same seeded inputs.

Tolerance (bf16 path): every bf16 intermediate (Q, K, V, attention output,
GELU activations) and the block's update y - x_tail must satisfy
|got - want| <= 2e-2 * max|want| elementwise and ||got - want||_2 <= 1e-2 * ||want||_2.
GEMM and softmax summation orders differ from the oracle's, so bf16
intermediates may round to a neighbouring bf16 value; nothing larger."""
import pytest
import torch

from oracle import onetrans as ot

pytestmark = pytest.mark.gpu

MAX_TOL = 2e-2
L2_TOL = 1e-2


def _close(name, got, want):
    got, want = got.double().cpu(), want.double().cpu()
    assert got.shape == want.shape, (name, got.shape, want.shape)
    assert torch.isfinite(got).all(), f"{name}: non-finite values"
    scale = want.abs().max().item()
    err = (got - want).abs()
    assert err.max().item() <= MAX_TOL * scale, f"{name}: max err {err.max().item():.3e} vs scale {scale:.3e}"
    l2 = ((got - want).norm() / want.norm()).item()
    assert l2 <= L2_TOL, f"{name}: rel l2 {l2:.3e}"
    return l2


def _gpu_weights(w, dev):
    bf = lambda t: t.to(torch.bfloat16).contiguous().to(dev)  # noqa: E731
    return dict(norm1_w=w["norm1"].float().contiguous().to(dev), s_qkv_w=bf(w["s_qkv"]),
                ns_qkv_w=bf(w["ns_qkv"]), out_w=bf(w["out"]), norm2_w=w["norm2"].float().contiguous().to(dev),
                s_w1=bf(w["s_w1"]), s_w2=bf(w["s_w2"]), ns_w1=bf(w["ns_w1"]), ns_w2=bf(w["ns_w2"]))


def _ws_view(ws, layout, name, shape, dtype=torch.bfloat16):
    off, size = layout[name]
    n = 1
    for s in shape:
        n *= s
    return ws[off:off + size].view(dtype)[:n].view(*shape)


def _run_case(pdm, dev, B, kv, q_len, n_ns, D=256, F=1024, seed=0, x_std=1.0, w_std=0.02, norm_std=0.0):
    H = D // 64
    w = ot.random_weights(D, F, n_ns, std=w_std, seed=seed, norm_std=norm_std)
    x = torch.randn(B, kv, D, generator=torch.Generator().manual_seed(seed + 1)) * x_std
    want, parts = ot.block_forward(x, w, q_len, H, mode="autocast", return_parts=True)
    layout = pdm.ops.onetrans_workspace_layout(B, kv, q_len, D, F)
    ws = torch.empty(layout["total"][0], dtype=torch.uint8, device=dev)
    got = pdm.ops.onetrans_block_raw(x.to(dev), _gpu_weights(w, dev), H, q_len, workspace=ws)
    torch.cuda.synchronize()
    # intermediates still held by the workspace: K, V^T, GELU activations, RMSNorm2 rows
    k = _ws_view(ws, layout, "k", (B, kv, D))
    kv_pad = (kv + 31) // 32 * 32
    vt = _ws_view(ws, layout, "vt", (B, H, 64, kv_pad))[..., :kv]
    v = vt.permute(0, 3, 1, 2).reshape(B, kv, D)
    o = _ws_view(ws, layout, "q", (B, q_len, D))
    _close("k", k, parts["k"])
    _close("v", v, parts["v"])
    _close("attention out", o, parts["o"])
    if "g" in layout:  # the unfused path keeps RMSNorm2 rows and GELU activations in the workspace
        g = _ws_view(ws, layout, "g", (B, q_len, F))
        h2 = _ws_view(ws, layout, "h", (B, q_len, D))
        _close("rmsnorm2", h2, parts["h2"].to(torch.bfloat16))
        _close("gelu(ffn up)", g, parts["g"])
    x_tail = x[:, kv - q_len:]
    _close("block update y - x_tail", got.cpu() - x_tail, want - x_tail)
    _close("block output y", got.cpu(), want)
    return got


@pytest.mark.parametrize("B,kv,q_len,n_ns", [
    (3, 40, 40, 4),      # full layer, ragged sizes
    (5, 70, 37, 16),     # pyramid layer: keep a tail
    (2, 33, 16, 16),     # q_len == n_ns: no S-token query
    (130, 48, 48, 2),    # B > one GEMM row tile of NS tokens
    (4, 64, 20, 0),      # no NS tokens
])
def test_block_matches_oracle(pdm, dev, B, kv, q_len, n_ns):
    _run_case(pdm, dev, B, kv, q_len, n_ns, seed=B + kv)


def test_block_d128_ffn384_and_norm_weights(pdm, dev):
    _run_case(pdm, dev, 6, 50, 30, 5, D=128, F=384, seed=7, norm_std=0.3, w_std=0.05)


def test_block_d384_tiled_path(pdm, dev):
    """d_model 384 (the reference's OneTransL width) runs the tiled GEMM path."""
    _run_case(pdm, dev, 5, 45, 21, 3, D=384, F=1536, seed=8, norm_std=0.2)


def test_block_baseline_shape_reduced_batch(pdm, dev):
    """The benchmark's first layer (400 tokens, 16 NS, d 256, FFN 1024) at batch 8."""
    _run_case(pdm, dev, 8, 400, 400, 16, seed=11)


def test_stack_pyramid_matches_oracle(pdm, dev):
    """OneTransStack with an explicit schedule against the oracle's block loop."""
    D, F, n_ns, H, B = 256, 1024, 16, 4, 4
    schedule = [96, 64, 32, 0]
    stack = pdm.OneTransStack(D, H, n_ns, len(schedule), schedule=schedule).to(dev).eval()
    layers = []
    with torch.no_grad():
        for i, blk in enumerate(stack.blocks):
            w = ot.random_weights(D, F, n_ns, std=0.02, seed=100 + i, norm_std=0.1)
            blk.norm1.weight.copy_(w["norm1"])
            blk.attn.s_qkv.weight.copy_(w["s_qkv"])
            blk.attn.ns_qkv_weight.copy_(w["ns_qkv"])
            blk.attn.out_proj.weight.copy_(w["out"])
            blk.norm2.weight.copy_(w["norm2"])
            blk.ffn.s_w1.weight.copy_(w["s_w1"])
            blk.ffn.s_w2.weight.copy_(w["s_w2"])
            blk.ffn.ns_w1.copy_(w["ns_w1"])
            blk.ffn.ns_w2.copy_(w["ns_w2"])
            layers.append(w)
    x = torch.randn(B, 96 + n_ns, D, generator=torch.Generator().manual_seed(5))
    got = stack(x.to(dev))
    want = ot.stack_forward(x, layers, schedule, H)
    assert got.shape == (B, n_ns, D)
    _close("stack output", got.cpu(), want)
    _close("stack update", got.cpu() - x[:, -n_ns:], want - x[:, -n_ns:])


def test_block_rejects_bad_shapes(pdm, dev):
    w = _gpu_weights(ot.random_weights(256, 1024, 2), dev)
    x = torch.zeros(2, 10, 256, device=dev)
    with pytest.raises(ValueError):
        pdm.ops.onetrans_block_raw(x, w, 4, 1)  # q_len < n_ns
    with pytest.raises(pdm._lib.PdmError, match="head dim"):
        pdm.ops.onetrans_block_raw(x, w, 2, 10)  # head dim 128
