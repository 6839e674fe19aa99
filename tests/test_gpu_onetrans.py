"""GPU parity of the OneTrans block kernels against the CPU oracle
(oracle/onetrans.py, autocast mode, whose rounding points are pinned against
torch's CPU autocast) on the same seeded inputs.

Tolerance (bf16 path), per element: every bf16 intermediate (Q, K, V,
attention output, GELU activations) and the block's update y - x_tail
satisfy |got - want| <= 2e-2 * (|want| + terms), where ``terms`` is the sum
of the absolute terms of the dot products that produce the value
(``oracle.onetrans.term_magnitudes``: |h| . |W|^T for a GEMM output, P . |V|
for attention).  That is the bf16 relative tolerance of 2e-2, measured
against the magnitude a rounding difference scales with.  Beyond it, fewer
than 1 % of the elements may differ by more than 2^-7 of that scale (one
bf16 ulp): GEMM and softmax summation orders differ from the oracle's, so a
bf16 value may round to its neighbour, and nothing larger."""
import pytest
import torch

from oracle import onetrans as ot

pytestmark = pytest.mark.gpu

ELEM_TOL = 2e-2
ULP = 2.0 ** -7


def _close(name, got, want, terms=None, tight_frac=0.01):
    got, want = got.double().cpu(), want.double().cpu()
    assert got.shape == want.shape, (name, got.shape, want.shape)
    assert torch.isfinite(got).all(), f"{name}: non-finite values"
    scale = want.abs() if terms is None else want.abs() + terms.double().reshape(want.shape)
    err = (got - want).abs()
    worst = (err / scale.clamp_min(1e-30)).max().item()
    beyond = (err > ULP * scale).double().mean().item()
    print(f"{name}: worst err / (|want| + terms) {worst:.2e}, beyond one ulp {beyond:.2e}", flush=True)
    assert bool((err <= ELEM_TOL * scale).all()), f"{name}: worst err / (|want| + terms) {worst:.3e}"
    assert beyond < tight_frac, f"{name}: {beyond:.3%} of the elements beyond one bf16 ulp"


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


def _check_layer(pdm, dev, x, w, q_len, label=""):
    """Runs one block on the GPU and checks its intermediates and output against the oracle on the same x."""
    B, kv, D = x.shape
    H = D // 64
    F = w["s_w1"].shape[0]
    print(f"block {label} B={B} kv={kv} q_len={q_len} D={D} n_ns={w['ns_qkv'].shape[0]}", flush=True)
    want, parts = ot.block_forward(x, w, q_len, H, mode="autocast", return_parts=True)
    terms = ot.term_magnitudes(x, w, q_len, H, parts)
    layout = pdm.ops.onetrans_workspace_layout(B, kv, q_len, D, F)
    ws = torch.empty(layout["total"][0], dtype=torch.uint8, device=dev)
    got = pdm.ops.onetrans_block_raw(x.to(dev), _gpu_weights(w, dev), H, q_len, workspace=ws)
    torch.cuda.synchronize()
    # intermediates still held by the workspace: K, V^T, the attention output, GELU activations
    k = _ws_view(ws, layout, "k", (B, kv, D))
    kv_ld = (kv + 63) // 64 * 64  # V^T row stride: rows start on 128-byte lines
    vt = _ws_view(ws, layout, "vt", (B, H, 64, kv_ld))[..., :kv]
    v = vt.permute(0, 3, 1, 2).reshape(B, kv, D)
    o = _ws_view(ws, layout, "q", (B, q_len, D))
    _close("k", k, parts["k"], terms["k"])
    _close("v", v, parts["v"], terms["v"])
    _close("attention out", o, parts["o"], terms["o"])
    if "g" in layout:  # the tiled path keeps RMSNorm2 rows and GELU activations in the workspace
        g = _ws_view(ws, layout, "g", (B, q_len, F))
        h2 = _ws_view(ws, layout, "h", (B, q_len, D))
        _close("rmsnorm2", h2, parts["h2"].to(torch.bfloat16), terms["h2"])
        _close("gelu(ffn up)", g, parts["g"], terms["g"])
    x_tail = x[:, kv - q_len:]
    got = got.cpu()
    _close("block update y - x_tail", got - x_tail, want - x_tail, terms["y"])
    return got


def _run_case(pdm, dev, B, kv, q_len, n_ns, D=256, F=1024, seed=0, x_std=1.0, w_std=0.02, norm_std=0.0):
    w = ot.random_weights(D, F, n_ns, std=w_std, seed=seed, norm_std=norm_std)
    x = torch.randn(B, kv, D, generator=torch.Generator().manual_seed(seed + 1)) * x_std
    return _check_layer(pdm, dev, x, w, q_len)


@pytest.mark.parametrize("B,kv,q_len,n_ns", [
    (3, 40, 40, 4),      # full layer, ragged sizes
    (5, 70, 37, 16),     # pyramid layer: keep a tail
    (2, 33, 16, 16),     # q_len == n_ns: no S-token query
    (130, 48, 48, 2),    # B > one GEMM row tile of NS tokens
    (4, 64, 20, 0),      # no NS tokens
    (6, 240, 100, 16),   # 4 query tiles over 240 keys: the 4-wave attention with 8 copy rounds
    (2, 600, 600, 16),   # 19 query tiles over 608 padded keys: 8 waves, Q read from memory, <10,8>
    (3, 500, 300, 16),   # 10 query tiles over 512 padded keys: Q does not fit beside K/V^T in LDS, <10,8>
    (4, 250, 200, 16),   # 7 query tiles over 256 padded keys: the <4,8> instance
])
def test_block_matches_oracle(pdm, dev, B, kv, q_len, n_ns):
    _run_case(pdm, dev, B, kv, q_len, n_ns, seed=B + kv)


def test_block_d128_ffn384_and_norm_weights(pdm, dev):
    _run_case(pdm, dev, 6, 50, 30, 5, D=128, F=384, seed=7, norm_std=0.3, w_std=0.05)


def test_block_d384_tiled_path(pdm, dev):
    """d_model 384 (the reference's OneTransL width) runs the tiled GEMM path."""
    _run_case(pdm, dev, 5, 45, 21, 3, D=384, F=1536, seed=8, norm_std=0.2)


def test_block_d512_tiled_path(pdm, dev):
    """d_model 512 (8 heads) on the tiled GEMM path."""
    _run_case(pdm, dev, 3, 40, 20, 3, D=512, F=2048, seed=9, norm_std=0.2)


def test_block_baseline_shape_reduced_batch(pdm, dev):
    """The 4-layer benchmark's first layer (400 tokens, 16 NS, d 256, FFN 1024) at batch 8."""
    _run_case(pdm, dev, 8, 400, 400, 16, seed=11)


def test_block_batch1024_short_sequence(pdm, dev):
    """Batch 1024 (the benchmark's batch: 48 k rows, hundreds of GEMM row tiles and 4096 attention
    (sample, head) pairs over the persistent grids) at a short sequence of 48 tokens keeping 32."""
    _run_case(pdm, dev, 1024, 48, 32, 16, seed=12, norm_std=0.1)


def test_block_vt_paired_tiles(pdm, dev):
    """Batch 160 with 128 S tokens: 640 S tiles over the Q/K/V projection's 256 workgroups, shares of 2 or 3
    consecutive tiles, so some workgroups write two tiles' V^T as whole lines together and others write a
    tile alone (a share starting at token 64 pairs it with token 96; a share's last tile at token 0 goes
    alone)."""
    _run_case(pdm, dev, 160, 144, 32, 16, seed=14, norm_std=0.1)


def test_block_ffn_ns_last_round(pdm, dev):
    """Batch 1024 keeping 80 of 96 tokens: 640 FFN row tiles of 128 rows, one whole round of 512 resident
    workgroups (256 CUs x 2) on the S tiles and a last round holding the 128 NS tiles (per-token weights)."""
    _run_case(pdm, dev, 1024, 96, 80, 16, seed=15, norm_std=0.1)


def test_block_ns_tiles_cross_tokens(pdm, dev):
    """Batch 1100 with 16 NS tokens: 35 row tiles of 32 samples per NS token (the last partial), 560 NS
    tiles over the Q/K/V projection's persistent grid, so workgroups' shares start and end inside a token's
    tiles and cross from one NS token's weight to the next; 33 S tokens (one full and one single-row tile per
    sample) with the kept tail starting inside the first tile."""
    _run_case(pdm, dev, 1100, 49, 20, 16, seed=13, norm_std=0.1)


@pytest.mark.parametrize("B,kv,q_len,D", [
    (2, 720, 300, 256),    # above the LDS-resident attention's 608 keys: the streaming attention kernel
    (1, 1516, 1516, 256),  # the reference OneTransL's first layer (L_S = 1500 + 16 NS, full causal)
    (3, 1000, 700, 384),   # 6 heads: 18 (sample, head) pairs x 3 query blocks of 256, the last partial
    (2, 650, 650, 384),    # just above 608 keys, full causal, tiled d_model 384 path
])
def test_block_long_sequence_streaming_attention(pdm, dev, B, kv, q_len, D):
    _run_case(pdm, dev, B, kv, q_len, 16, D=D, F=4 * D, seed=kv, norm_std=0.1)


def _load_block(blk, w):
    with torch.no_grad():
        blk.norm1.weight.copy_(w["norm1"])
        blk.attn.s_qkv.weight.copy_(w["s_qkv"])
        blk.attn.ns_qkv_weight.copy_(w["ns_qkv"])
        blk.attn.out_proj.weight.copy_(w["out"])
        blk.norm2.weight.copy_(w["norm2"])
        blk.ffn.s_w1.weight.copy_(w["s_w1"])
        blk.ffn.s_w2.weight.copy_(w["s_w2"])
        blk.ffn.ns_w1.copy_(w["ns_w1"])
        blk.ffn.ns_w2.copy_(w["ns_w2"])


@pytest.mark.parametrize("B,L_S,schedule,D", [
    (16, 384, [384, 256, 128, 64], 256),  # the benchmark's 4-layer pyramid: (kv, q) = (400,400),(400,272),(272,144),(144,80)
    (4, 96, [96, 64, 32, 0], 256),        # down to the NS tokens only
    (2, 984, [984, 656, 328, 0], 384),    # d_model 384, 6 heads: streaming attention at kv 1000 and 672, then LDS
])
def test_stack_pyramid_matches_oracle(pdm, dev, B, L_S, schedule, D):
    """OneTransStack (the block loop of onetrans.py:568-582) with an explicit schedule.  Each layer is
    checked element-wise against the oracle on the GPU's own input to that layer; the stack's output
    equals the chained layers bit for bit, and stays within 1e-2 (relative L2) of the oracle's stack."""
    F, n_ns, H = 4 * D, 16, D // 64
    stack = pdm.OneTransStack(D, H, n_ns, len(schedule), schedule=schedule).to(dev).eval()
    layers = []
    for i, blk in enumerate(stack.blocks):
        w = ot.random_weights(D, F, n_ns, std=0.02, seed=100 + i, norm_std=0.1)
        _load_block(blk, w)
        layers.append(w)
    x = torch.randn(B, L_S + n_ns, D, generator=torch.Generator().manual_seed(5))
    got = stack(x.to(dev)).cpu()
    assert got.shape == (B, schedule[-1] + n_ns, D)
    h = x
    for i, (w, q_s) in enumerate(zip(layers, schedule)):
        h = _check_layer(pdm, dev, h, w, q_s + n_ns, label=f"layer {i}")
    assert torch.equal(got, h)
    want = ot.stack_forward(x, layers, schedule, H)
    drift = ((got.double() - want.double()).norm() / (want.double() - x[:, -got.shape[1]:].double()).norm()).item()
    print(f"stack drift (relative L2 of the update) {drift:.2e}", flush=True)
    assert drift <= 1e-2


def test_stack_default_schedule_is_reference_pyramid(pdm, dev):
    """Without an explicit schedule the stack keeps pyramid_schedule(L_S, n_ns, n_layers) queries."""
    D, n_ns, H = 128, 4, 2
    stack = pdm.OneTransStack(D, H, n_ns, 3).to(dev).eval()
    x = torch.randn(2, 40 + n_ns, D, device=dev)
    assert stack(x).shape == (2, pdm.pyramid_schedule(40, n_ns, 3)[-1] + n_ns, D)


def test_block_rejects_bad_shapes(pdm, dev):
    w = _gpu_weights(ot.random_weights(256, 1024, 2), dev)
    x = torch.zeros(2, 10, 256, device=dev)
    with pytest.raises(ValueError):
        pdm.ops.onetrans_block_raw(x, w, 4, 1)  # q_len < n_ns
    with pytest.raises(pdm._lib.PdmError, match="head dim"):
        pdm.ops.onetrans_block_raw(x, w, 2, 10)  # head dim 128
