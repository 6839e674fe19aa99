"""The dense step of RowWiseAdagrad (CPU): torch.optim.Adagrad on dim-1 rows and on rows whose elements and
gradients are equal, and the C oracle's row-wise rule on a general row."""
import numpy as np
import torch

from oracle import oracle as o


def test_rowwise_adagrad_dense_step_matches_torch_adagrad(pdm):
    g = torch.Generator().manual_seed(0)
    w0 = torch.randn(30, 1, generator=g)
    a, b = torch.nn.Parameter(w0.clone()), torch.nn.Parameter(w0.clone())
    ra = pdm.RowWiseAdagrad([a], lr=0.05, eps=1e-8, weight_decay=0.1, weight_decay_mode=pdm.WeightDecayMode.L2)
    tb = torch.optim.Adagrad([b], lr=0.05, eps=1e-8, weight_decay=0.1)
    for _ in range(3):
        grad = torch.randn(30, 1, generator=g)
        a.grad, b.grad = grad.clone(), grad.clone()
        ra.step()
        tb.step()
    torch.testing.assert_close(a.detach(), b.detach(), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(ra.state[a]["sum"], tb.state[b]["sum"][:, 0], rtol=1e-6, atol=1e-8)


def test_rowwise_adagrad_dense_step_matches_oracle(pdm):
    # one bag per row: the oracle's row gradient is that bag's output gradient
    g = np.random.default_rng(2)
    rows, D = 20, 8
    flat = g.uniform(-0.5, 0.5, rows * D).astype(np.float32)
    slots = [dict(rows=rows, weights_offset=0, dim=D, dtype="fp32", pooling="sum", row_bytes=0, out_offset=0)]
    p = torch.nn.Parameter(torch.from_numpy(flat.copy()).view(rows, D))
    opt = pdm.RowWiseAdagrad([p], lr=0.05, eps=1e-8, weight_decay=0.01, weight_decay_mode=pdm.WeightDecayMode.L2)
    state = np.zeros(rows, np.float32)
    for _ in range(3):
        grad = g.normal(0, 1, (rows, D)).astype(np.float32)
        p.grad = torch.from_numpy(grad.copy())
        opt.step()
        o.tbe_backward(slots, np.arange(rows), np.arange(rows + 1), rows, grad, optimizer=o.ROWWISE_ADAGRAD,
                       weights=flat, m1=state, lr=0.05, eps=1e-8, weight_decay=0.01, wd_mode=o.WD_L2)
    np.testing.assert_allclose(p.detach().numpy().ravel(), flat, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(opt.state[p]["sum"].numpy(), state, rtol=1e-5, atol=1e-9)
