"""Pins oracle/sinkhorn_dense_ref.py (dense sinkhorn_solve / compute_transport_output).

Checks, in float64 on the CPU:
* potentials equal the independent flash oracle (oracle/sinkhorn.py) when C is
  the flash cost -C = QK^T/sqrt(d) (two restatements of one iteration);
* the reference's own invariants (tests/test_sinkhorn_batch.py): batched ==
  per-sample, masked == unpadded slice, padded potentials exactly 0; T_norm rows
  sum to 1 up to the 1e-6 guard;
* early stop halts at the first checked iteration with change < threshold;
* central finite differences agree with the autograd gradients.
"""

import numpy as np
import pytest
import torch

from oracle import sinkhorn as flash
from oracle import sinkhorn_dense_ref as dref

F64 = dict(dtype=torch.float64)


def _case(B, H, N, d=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, N, d, generator=g, dtype=torch.float64) / d ** 0.5
    K = torch.randn(B, H, N, d, generator=g, dtype=torch.float64) / d ** 0.5
    C = -(Q @ K.transpose(-1, -2)) / d ** 0.5
    lmu = torch.log_softmax(torch.randn(B, H, N, generator=g, dtype=torch.float64), -1)
    lnu = torch.log_softmax(torch.randn(B, H, N, generator=g, dtype=torch.float64), -1)
    eps = torch.linspace(0.4, 1.5, H, dtype=torch.float64)
    return Q, K, C, lmu, lnu, eps


def test_potentials_equal_flash_oracle():
    B, H, N, d, Kit = 2, 3, 20, 8, 9
    Q, Kt, C, lmu, lnu, eps = _case(B, H, N, d, seed=1)
    lu, lv = dref.sinkhorn_solve(C, lmu, lnu, eps, K=Kit)
    fo = flash.forward(Q.numpy(), Kt.numpy(), np.zeros((B, H, N, d)), np.zeros((B, H, N, d)), np.zeros((B, N, 3)),
                       np.zeros((H, 68)), None, eps.numpy(), np.zeros(H), lmu.numpy(), lnu.numpy(), K_iter=Kit)
    assert np.max(np.abs(lu.numpy() - fo["log_u"])) < 1e-11
    assert np.max(np.abs(lv.numpy() - fo["log_v"])) < 1e-11


def test_batched_equals_per_sample_and_masked_equals_unpadded():
    B, H, N = 3, 2, 16
    _, _, C, lmu, lnu, eps = _case(B, H, N, seed=2)
    lengths = [16, 11, 5]
    mask = torch.zeros(B, N, **F64)
    for b, n in enumerate(lengths):
        mask[b, :n] = 1
    lu, lv = dref.sinkhorn_solve(C, lmu, lnu, eps, K=6, mask=mask)
    V = torch.randn(B, H, N, 4, **F64)
    G = torch.randn(B, H, N, 4, **F64)
    x = torch.randn(B, N, 3, **F64)
    o, Tn, xc = dref.compute_transport_output(V, G, lu, lv, C, eps, x, mask)
    for b, n in enumerate(lengths):
        lu1, lv1 = dref.sinkhorn_solve(C[b, :, :n, :n], lmu[b, :, :n], lnu[b, :, :n], eps, K=6)
        assert torch.allclose(lu[b, :, :n], lu1, atol=1e-12) and torch.allclose(lv[b, :, :n], lv1, atol=1e-12)
        assert torch.all(lu[b, :, n:] == 0) and torch.all(lv[b, :, n:] == 0)
        o1, Tn1, xc1 = dref.compute_transport_output(V[b, :, :n], G[b, :, :n], lu1, lv1, C[b, :, :n, :n], eps,
                                                     x[b, :n])
        assert torch.allclose(o[b, :n], o1, atol=1e-12)
        assert torch.allclose(Tn[b, :, :n, :n], Tn1, atol=1e-12)
        assert torch.allclose(xc[b, :, :n], xc1, atol=1e-12)
        assert torch.all(o[b, n:] == 0) and torch.all(Tn[b, :, n:] == 0)
        rows = Tn1.sum(-1)
        assert torch.allclose(rows, torch.ones_like(rows), atol=1e-5)


def test_early_stop():
    B, H, N = 1, 2, 12
    _, _, C, lmu, lnu, eps = _case(B, H, N, seed=3)
    full = [dref.sinkhorn_solve(C, lmu, lnu, eps, K=k) for k in range(1, 41)]
    thr = 1e-4
    _, _, done = dref.sinkhorn_solve(C, lmu, lnu, eps, K=40, threshold=thr, check_every=2, return_iters=True)
    # the first even iteration whose change from the previous one is below thr
    want = None
    for k in range(2, 41, 2):
        u1, v1 = full[k - 1]
        u0, v0 = full[k - 2]
        if max(float((u1 - u0).abs().max()), float((v1 - v0).abs().max())) < thr:
            want = k
            break
    assert want is not None and done == want


def test_autograd_matches_finite_differences():
    B, H, N = 1, 2, 6
    _, _, C, lmu, lnu, eps = _case(B, H, N, seed=4)
    g = torch.Generator().manual_seed(5)
    wu, wv = torch.randn(B, H, N, generator=g, **F64), torch.randn(B, H, N, generator=g, **F64)
    V = torch.randn(B, H, N, 3, generator=g, **F64)
    Gt = torch.randn(B, H, N, 3, generator=g, **F64)
    wo = torch.randn(B, N, H * 3, generator=g, **F64)

    def loss(Cc, mu, nu):
        lu, lv = dref.sinkhorn_solve(Cc, mu, nu, eps, K=5)
        o, Tn, _ = dref.compute_transport_output(V, Gt, lu, lv, Cc, eps)
        return (lu * wu).sum() + (lv * wv).sum() + (o * wo).sum()

    Cr, mur, nur = (t.clone().requires_grad_(True) for t in (C, lmu, lnu))
    loss(Cr, mur, nur).backward()
    h = 1e-6
    for t, gr in ((C, Cr.grad), (lmu, mur.grad), (lnu, nur.grad)):
        flat = t.view(-1)
        for idx in (0, 7, flat.numel() // 2, flat.numel() - 1):
            old = float(flat[idx])
            flat[idx] = old + h
            lp = float(loss(C, lmu, lnu))
            flat[idx] = old - h
            lm = float(loss(C, lmu, lnu))
            flat[idx] = old
            fd = (lp - lm) / (2 * h)
            assert abs(fd - float(gr.view(-1)[idx])) < 1e-6 * max(1.0, abs(fd))
