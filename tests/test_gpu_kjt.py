"""GPU parity of the device KJT construction (pdm_kjt_from_dense, pdm_kjt_permute) with the oracle: bit-exact
values / lengths / offsets; and the EBC fed with a device-built, permuted KJT."""
import numpy as np
import pytest
import torch

from oracle import oracle as o

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("pad", [0, -1, 3])
@pytest.mark.parametrize("lens", [(1,), (5, 20, 1), (64,), (100, 7, 300), (0, 4), (20, 2, 40), (2,)])
def test_kjt_from_dense(pdm, dev, dtype, pad, lens):
    g = np.random.default_rng(sum(lens) + pad)
    B = 257
    mats = [g.integers(0, 8, (B, L)).astype(dtype) for L in lens]
    if lens[0] > 0:
        mats[0][5, :] = max(pad, 0)  # an all-padding row
    v, ln, off = pdm.ops.kjt_from_dense_raw([torch.from_numpy(m).to(dev) for m in mats], pad)
    wv, wl, wo = o.kjt_from_dense(mats, pad)
    off = off.cpu().numpy()
    assert np.array_equal(off, wo)
    assert np.array_equal(ln.cpu().numpy(), wl)
    assert np.array_equal(v.cpu().numpy()[:off[-1]], wv)


def test_kjt_from_dense_large(pdm, dev):
    # 26 features x 65,536 rows x 20 ids, 30 % padding: several hundred scan blocks
    g = np.random.default_rng(1)
    B = 65536
    mats = []
    for f in range(26):
        m = g.integers(1, 1 << 30, (B, 20))
        m[g.random(m.shape) < 0.3] = 0
        mats.append(m)
    v, ln, off = pdm.ops.kjt_from_dense_raw([torch.from_numpy(m).to(dev) for m in mats], 0)
    wv, wl, wo = o.kjt_from_dense(mats, 0)
    off = off.cpu().numpy()
    assert np.array_equal(off, wo) and np.array_equal(v.cpu().numpy()[:off[-1]], wv)


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_kjt_permute(pdm, dev, dtype):
    g = np.random.default_rng(4)
    K, B = 5, 300
    lengths = g.integers(0, 40, K * B)
    lengths[7] = 2000  # one long segment
    offsets = o.offsets_np(lengths)
    values = g.integers(0, 1 << 30, int(lengths.sum())).astype(dtype)
    perm = [3, 0, 0, 4]  # repeat and drop keys
    v, ln, off = pdm.ops.kjt_permute_raw(torch.from_numpy(values).to(dev), torch.from_numpy(offsets).to(dev), K, B,
                                         perm)
    wv, wl, wo = o.kjt_permute(values, offsets, K, B, perm)
    off = off.cpu().numpy()
    assert np.array_equal(off, wo) and np.array_equal(ln.cpu().numpy(), wl)
    assert np.array_equal(v.cpu().numpy()[:off[-1]], wv)


def test_kjt_empty(pdm, dev):
    v, ln, off = pdm.ops.kjt_from_dense_raw([torch.zeros((0, 4), dtype=torch.int64, device=dev)], 0)
    assert off.cpu().tolist() == [0]
    v, ln, off = pdm.ops.kjt_permute_raw(torch.zeros(0, dtype=torch.int64, device=dev),
                                         torch.zeros(1, dtype=torch.int64, device=dev), 1, 0, [0])
    assert off.cpu().tolist() == [0]


def test_ebc_with_device_built_permuted_kjt(pdm, dev):
    from primus_dlrm_amd.kjt import build_pooled_kjt
    g = np.random.default_rng(9)
    cfgs = [pdm.EmbeddingBagConfig(300, 32, "t0", pdm.DataType.FP32, ["a"], pdm.PoolingType.MEAN),
            pdm.EmbeddingBagConfig(200, 16, "t1", pdm.DataType.FP32, ["b"], pdm.PoolingType.SUM)]
    ebc = pdm.EmbeddingBagCollection(cfgs, device=dev)
    B = 50
    a = g.integers(0, 300, (B, 12))
    b = g.integers(0, 200, (B, 7))
    a[g.random(a.shape) < 0.4] = 0
    b[g.random(b.shape) < 0.4] = 0
    # built in the other key order, then permuted by the collection on the device
    kjt = build_pooled_kjt({"a": torch.from_numpy(a).to(dev), "b": torch.from_numpy(b).to(dev)}, ["b", "a"], 0)
    got = ebc(kjt).values().detach().cpu().numpy()
    wv, wl, wo = o.kjt_from_dense([a, b], 0)
    w0, w1 = ebc.embedding_bags["t0"].weight.cpu(), ebc.embedding_bags["t1"].weight.cpu()
    want = o.tbe_pooled_from_tables([w0, w1], ["mean", "sum"], wv, wo, B)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
