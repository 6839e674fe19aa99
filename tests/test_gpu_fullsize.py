"""Parity at the full sizes of the two largest workloads, checked on sampled outputs.

* Quantized-inference TBE at full size: 64 tables x 5,000,000 rows x 128 int8 rowwise (42.2 GB on the device,
  quantized on the device from N(0, 0.05) exactly as the benchmark builds them), the full batch of 16,384 bags
  per table (Poisson(20) lengths in [1, 100], Zipf(1.2) ids), mean pooling, fp16 out.  The whole batch runs in
  one launch; 16 sampled samples (1,024 bags: each table's bag of every sampled sample) are compared bit for
  bit with the oracle on a compact host copy of exactly the rows those bags touch.
* The OneTrans 4-layer stack at B = 1024 (384 S + 16 NS tokens, d_model 256, schedule 384/256/128/64): every
  layer runs on the whole batch on the GPU; for 16 sampled samples the layer's K, V, attention output and
  output are checked against the oracle on the GPU's own input to that layer (samples are independent, so the
  oracle on the sampled rows is exact for them); the stack's output equals the chained layers bit for bit."""
import numpy as np
import pytest
import torch

from oracle import oracle as o
from oracle import onetrans as ot
from test_gpu_onetrans import _close, _gpu_weights, _load_block, _ws_view

pytestmark = pytest.mark.gpu


def test_int8_mean_full_size_sampled_bags(pdm, dev):
    import bench
    import primus_dlrm_amd.synthetic as syn

    w = syn.int8_mean()
    T, B, dim = w.num_tables, w.batch, w.dim
    print(f"int8 TBE full size: {T} tables x {w.rows[0]} rows, B={B}, {w.num_lookups} lookups", flush=True)
    step, _, keep = bench.setup_pooled(pdm, torch, dev, w, 0.05)
    flat, plan, _, _, out = keep
    step()
    torch.cuda.synchronize()
    rb = (4 + dim + 3) & ~3
    base = []
    off = 0
    for r in w.rows:
        off = (off + 255) // 256 * 256
        base.append(off)
        off += r * rb
    sample = np.sort(np.random.default_rng(33).choice(B, 16, replace=False))
    chunks, slots, idx, lens, coff = [], [], [], [], 0
    for t in range(T):
        bags = [w.indices[w.offsets[t * B + b]:w.offsets[t * B + b + 1]] for b in sample]
        uniq = np.unique(np.concatenate(bags))
        view = flat[base[t]:base[t] + w.rows[t] * rb].view(w.rows[t], rb)
        rows = view.index_select(0, torch.from_numpy(uniq).to(dev)).cpu().numpy()
        pad = (-coff) % 256
        if pad:
            chunks.append(np.zeros(pad, np.uint8))
            coff += pad
        slots.append(dict(rows=uniq.size, weights_offset=coff, dim=dim, dtype="int8", pooling="mean",
                          row_bytes=rb, out_offset=t * dim))
        chunks.append(rows.reshape(-1))
        coff += rows.size
        idx.extend(np.searchsorted(uniq, bg) for bg in bags)
        lens.extend(bg.size for bg in bags)
    want = o.tbe_pooled(np.concatenate(chunks), slots, np.concatenate(idx).astype(np.int64), o.offsets_np(lens),
                        len(sample), -1, "fp16")
    got = out[torch.from_numpy(sample).to(dev)].cpu().view(torch.int16).numpy().view(np.uint16)
    mism = got != want
    assert not mism.any(), f"{mism.sum()} of {mism.size} fp16 outputs differ, first at {np.argwhere(mism)[:3].tolist()}"
    del keep, flat, plan, out, step
    torch.cuda.empty_cache()


def _stack_sampled(pdm, dev, D, F, n_ns, B, schedule, n_sample, seed):
    """The full-batch stack on the GPU, layer by layer; each layer's K, V, attention output and update of
    n_sample sampled samples checked against the oracle on the GPU's own input to that layer, then the
    whole stack in one call equal to the chained layers bit for bit."""
    H = D // 64
    layers = [ot.random_weights(D, F, n_ns, std=0.02, seed=seed + i, norm_std=0.1) for i in range(len(schedule))]
    x = torch.randn(B, schedule[0] + n_ns, D, generator=torch.Generator().manual_seed(seed))
    sample = torch.from_numpy(np.sort(np.random.default_rng(seed + 25).choice(B, n_sample, replace=False)))
    h = x
    for i, (w, q_s) in enumerate(zip(layers, schedule)):
        kv, q_len = h.shape[1], q_s + n_ns
        print(f"stack layer {i}: B={B} kv={kv} q_len={q_len} D={D}, {n_sample} sampled samples", flush=True)
        layout = pdm.ops.onetrans_workspace_layout(B, kv, q_len, D, F)
        ws = torch.empty(layout["total"][0], dtype=torch.uint8, device=dev)
        got = pdm.ops.onetrans_block_raw(h.to(dev), _gpu_weights(w, dev), H, q_len, workspace=ws)
        torch.cuda.synchronize()
        hs = h[sample]
        want, parts = ot.block_forward(hs, w, q_len, H, mode="autocast", return_parts=True)
        terms = ot.term_magnitudes(hs, w, q_len, H, parts)
        sd = sample.to(dev)
        k = _ws_view(ws, layout, "k", (B, kv, D))[sd]
        kv_ld = (kv + 63) // 64 * 64
        vt = _ws_view(ws, layout, "vt", (B, H, 64, kv_ld))[sd][..., :kv]
        v = vt.permute(0, 3, 1, 2).reshape(len(sample), kv, D)
        att = _ws_view(ws, layout, "q", (B, q_len, D))[sd]
        _close(f"layer {i} k", k, parts["k"], terms["k"])
        _close(f"layer {i} v", v, parts["v"], terms["v"])
        _close(f"layer {i} attention out", att, parts["o"], terms["o"])
        got = got.cpu()
        tail = hs[:, kv - q_len:]
        _close(f"layer {i} update y - x_tail", got[sample] - tail, want - tail, terms["y"])
        h = got
        del ws
    stack = pdm.OneTransStack(D, H, n_ns, len(schedule), ffn_mult=F // D, schedule=schedule).to(dev).eval()
    for blk, w in zip(stack.blocks, layers):
        _load_block(blk, w)
    with torch.no_grad():
        out = stack(x.to(dev)).cpu()
    assert torch.equal(out, h)
    del stack, out
    torch.cuda.empty_cache()


def test_onetrans_stack_b1024_sampled_samples(pdm, dev):
    """The benchmark's 4-layer stack at B = 1024 (3,200 FFN row tiles per layer at kv 400)."""
    _stack_sampled(pdm, dev, 256, 1024, 16, 1024, [384, 256, 128, 64], 16, 300)


def test_onetransl_stack_b1024_sampled_samples(pdm, dev):
    """The reference's OneTransL shape at B = 1024: d_model 384 (tiled path), 1516 tokens, the 8-layer pyramid
    1500 -> 16; layers 0-5 run the streaming attention (kv 1516 .. 668)."""
    _stack_sampled(pdm, dev, 384, 1536, 16, 1024, [1500, 1288, 1076, 864, 652, 440, 228, 16], 4, 700)
