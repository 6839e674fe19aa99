"""pdm_kjt_from_dense_noalloc (the device KJT build whose scan scratch is a library-owned static device array)
against pdm_kjt_from_dense (the same build with a caller workspace), both called through the C ABI: bit-exact
values, lengths and offsets on two calls in a row, the second with a smaller input, so the second call runs
on a scratch array that still holds the first call's block sums; inputs beyond the stated row limit are
rejected before any device work."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _mats(seed, F, B, L, pad_frac):
    g = np.random.default_rng(seed)
    out = []
    for f in range(F):
        m = g.integers(1, 1 << 40, (B, L + f % 3), dtype=np.int64)
        m[g.random(m.shape) < pad_frac] = 0
        out.append(m)
    return out


def _build(pdm, dev, mats, padding_idx, noalloc):
    L = pdm._lib
    lib = L.lib()
    F, B = len(mats), mats[0].shape[0]
    ids = [torch.from_numpy(m).to(dev) for m in mats]
    cap = sum(m.size for m in mats)
    values = torch.full((cap,), -7, dtype=torch.int64, device=dev)
    lengths = torch.full((F * B,), -7, dtype=torch.int32, device=dev)
    offsets = torch.full((F * B + 1,), -7, dtype=torch.int64, device=dev)
    id_ptrs = (ctypes.c_void_p * F)(*[t.data_ptr() for t in ids])
    row_len = (ctypes.c_int32 * F)(*[m.shape[1] for m in mats])
    stream = L.stream_ptr(dev)
    if noalloc:
        st = lib.pdm_kjt_from_dense_noalloc(id_ptrs, row_len, F, B, 64, padding_idx, values.data_ptr(),
                                            lengths.data_ptr(), offsets.data_ptr(), stream)
    else:
        ws_bytes = int(lib.pdm_kjt_workspace_size(F * B))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        st = lib.pdm_kjt_from_dense(id_ptrs, row_len, F, B, 64, padding_idx, values.data_ptr(), lengths.data_ptr(),
                                    offsets.data_ptr(), ws.data_ptr(), ws_bytes, stream)
    L.check(st, "pdm_kjt_from_dense_noalloc" if noalloc else "pdm_kjt_from_dense")
    torch.cuda.synchronize()
    n = int(offsets[-1].item())
    return values[:n].cpu(), lengths.cpu(), offsets.cpu()


@pytest.mark.parametrize("first,second", [
    ((6, 200_000, 20, 0.3), (3, 5_000, 7, 0.5)),     # 1.2 M rows (1172 scan blocks), then 15 k rows
    ((2, 70_000, 13, 0.0), (1, 3, 5, 0.9)),          # no padding, then a 3-row input
])
def test_noalloc_matches_workspace_entry_point(pdm, dev, first, second):
    for i, (F, B, Lr, pad) in enumerate((first, second)):
        mats = _mats(100 + i + F, F, B, Lr, pad)
        print(f"kjt no-alloc call {i}: F={F} B={B} L={Lr} padding {pad}", flush=True)
        want = _build(pdm, dev, mats, 0, noalloc=False)
        got = _build(pdm, dev, mats, 0, noalloc=True)
        for name, a, b in zip(("values", "lengths", "offsets"), got, want):
            assert torch.equal(a, b), f"call {i}: {name} differ"
        # the reference expression of _build_pooled_kjt (embedding.py:179-204) on the host
        keep = [m[m != 0] for m in mats]
        assert np.array_equal(got[0].numpy(), np.concatenate(keep))
        assert np.array_equal(got[1].numpy(), np.concatenate([(m != 0).sum(1) for m in mats]).astype(np.int32))


def test_noalloc_rejects_inputs_beyond_the_scratch(pdm, dev):
    L = pdm._lib
    lib = L.lib()
    too_many = L.PDM_KJT_NOALLOC_MAX_ROWS // 64 + 1
    st = lib.pdm_kjt_from_dense_noalloc(None, None, 64, too_many, 64, 0, None, None, None, None)
    assert st == L.PDM_ERR_INVALID
    assert "no-allocation limit" in L.last_error()


def test_noalloc_under_graph_capture(pdm, dev):
    """The no-allocation build captured in a HIP graph (torch.cuda.graph) after one eager call on the device
    (the first call on a device looks up the scratch array's address), replayed three times on new ids
    written into the same input buffers, with eager work and synchronisations between the replays: every
    replay matches the workspace entry point on the same ids bit for bit."""
    L = pdm._lib
    lib = L.lib()
    F, B, Lr = 3, 5000, 7
    ids = [torch.zeros((B, Lr + f), dtype=torch.int64, device=dev) for f in range(F)]
    cap = sum(t.numel() for t in ids)
    values = torch.zeros(cap, dtype=torch.int64, device=dev)
    lengths = torch.zeros(F * B, dtype=torch.int32, device=dev)
    offsets = torch.zeros(F * B + 1, dtype=torch.int64, device=dev)
    id_ptrs = (ctypes.c_void_p * F)(*[t.data_ptr() for t in ids])
    row_len = (ctypes.c_int32 * F)(*[t.shape[1] for t in ids])

    def call():
        st = lib.pdm_kjt_from_dense_noalloc(id_ptrs, row_len, F, B, 64, 0, values.data_ptr(), lengths.data_ptr(),
                                            offsets.data_ptr(), L.stream_ptr(dev))
        L.check(st, "pdm_kjt_from_dense_noalloc")

    def fill(seed):
        for f, m in enumerate(_mats(seed, F, B, Lr, 0.4)):
            ids[f].copy_(torch.from_numpy(m))
        torch.cuda.synchronize()
        return [t.cpu().numpy() for t in ids]

    fill(1)
    call()  # eager first call: resolves the scratch address outside the capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(3):
        mats = fill(40 + rep)
        values.fill_(-7)
        lengths.fill_(-7)
        offsets.fill_(-7)
        print(f"kjt no-alloc graph replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        want = _build(pdm, dev, mats, 0, noalloc=False)
        n = int(offsets[-1].item())
        got = (values[:n].cpu(), lengths.cpu(), offsets.cpu())
        for name, a, b in zip(("values", "lengths", "offsets"), got, want):
            assert torch.equal(a, b), f"replay {rep}: {name} differ"
