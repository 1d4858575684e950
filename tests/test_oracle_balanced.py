"""CPU pinning of the balanced-transport oracle (oracle/balanced_transport.py).

Checks against facts fixed by the mathematics, with the cost rebuilt here in
numpy from its definition (flash_sinkhorn_transport.py:254-261), not by
re-running the oracle's own formula:
* one iteration (column update first, then the row update) gives the plan
  row-normalise(Kg diag(1 / colsum Kg)), Kg = exp(-C / eps);
* Sinkhorn scaling keeps every cross ratio T_ij T_kl / (T_il T_kj) equal to
  Kg's, for any iteration count: this pins the cost, its geometry term, the
  sigmoid mixing weight and the clamp of r;
* a 2 x 2 problem converges to the closed-form entropic OT plan;
* a constant cost makes the feature centroid the masked mean of V;
* batched == per-sample, masked == unpadded, padded rows are zero, and the dual's
  coordinate centroid equals the single one (tests/test_dual_transport.py);
* autograd gradients match central finite differences.
"""

import numpy as np
import pytest
import torch

from oracle import balanced_transport as bt


def _inputs(B, H, N, d, seed, r=10.0):
    g = torch.Generator().manual_seed(seed)
    Q = torch.nn.functional.normalize(torch.randn(B, H, N, d, generator=g, dtype=torch.float64), dim=-1)
    K = torch.nn.functional.normalize(torch.randn(B, H, N, d, generator=g, dtype=torch.float64), dim=-1)
    x = torch.randn(B, N, 3, generator=g, dtype=torch.float64) * 3
    V = torch.randn(B, H, N, d, generator=g, dtype=torch.float64)
    eps = torch.tensor([0.5, 1.0, 2.0, 4.0][:H] * (H // 4 if H >= 4 else 1), dtype=torch.float64)[:H]
    if eps.numel() < H:
        eps = torch.linspace(0.5, 2.0, H, dtype=torch.float64)
    alpha = torch.randn(H, generator=g, dtype=torch.float64)
    rh = torch.full((H,), r, dtype=torch.float64)
    return Q, K, x, V, eps, alpha, rh


def _np_gibbs(Q, K, x, eps, alpha, rh, b, h):
    """exp(-C/eps) for one (b, h), built from the definition in numpy."""
    q, k, xx = Q[b, h].numpy(), K[b, h].numpy(), x[b].numpy()
    w = 1.0 / (1.0 + np.exp(-float(alpha[h])))
    r = max(abs(float(rh[h])), 0.1)
    diff = xx[:, None, :] - xx[None, :, :]
    dist = np.maximum(np.sqrt((diff ** 2).sum(-1)), 1e-8)
    C = (1 - w) * (1 - q @ k.T) + w * dist / (r + dist)
    return np.exp(-C / float(eps[h]))


def test_one_iteration_closed_form():
    B, H, N, d = 2, 3, 9, 4
    Q, K, x, V, eps, alpha, rh = _inputs(B, H, N, d, seed=1)
    (xc, hc), Tn, _, _ = bt.sinkhorn_cpu(Q, K, x, eps, alpha, rh, None, N, 1, V_h=V, return_plan=True)
    for b in range(B):
        for h in range(H):
            Kg = _np_gibbs(Q, K, x, eps, alpha, rh, b, h)
            P = Kg / Kg.sum(0, keepdims=True)
            P = P / P.sum(1, keepdims=True)
            np.testing.assert_allclose(Tn[b, h].numpy(), P, rtol=1e-12, atol=1e-15)
            np.testing.assert_allclose(xc[b, h].numpy(), P @ x[b].numpy(), rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(hc[b, h].numpy(), P @ V[b, h].numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("K_iter,r", [(3, 10.0), (20, 0.05), (7, -2.5)])
def test_cross_ratios_are_those_of_the_gibbs_kernel(K_iter, r):
    B, H, N, d = 1, 2, 7, 5
    Q, K, x, V, eps, alpha, rh = _inputs(B, H, N, d, seed=2, r=r)
    _, Tn, _, _ = bt.sinkhorn_cpu(Q, K, x, eps, alpha, rh, None, N, K_iter, return_plan=True)
    rng = np.random.default_rng(0)
    for h in range(H):
        Kg = _np_gibbs(Q, K, x, eps, alpha, rh, 0, h)
        T = Tn[0, h].numpy()
        for _ in range(20):
            i, k = rng.choice(N, 2, replace=False)
            j, l = rng.choice(N, 2, replace=False)
            want = Kg[i, j] * Kg[k, l] / (Kg[i, l] * Kg[k, j])
            got = T[i, j] * T[k, l] / (T[i, l] * T[k, j])
            assert abs(got / want - 1) < 1e-10


def test_two_by_two_converges_to_entropic_plan():
    B, H, N, d = 1, 1, 2, 3
    Q, K, x, V, eps, alpha, rh = _inputs(B, H, N, d, seed=3)
    _, Tn, _, _ = bt.sinkhorn_cpu(Q, K, x, eps, alpha, rh, None, N, 400, return_plan=True)
    Kg = _np_gibbs(Q, K, x, eps, alpha, rh, 0, 0)
    rho = Kg[0, 0] * Kg[1, 1] / (Kg[0, 1] * Kg[1, 0])
    a = np.sqrt(rho) / (1 + np.sqrt(rho))  # T_norm = [[a, 1-a], [1-a, a]] for uniform marginals
    np.testing.assert_allclose(Tn[0, 0].numpy(), [[a, 1 - a], [1 - a, a]], rtol=1e-10)


def test_constant_cost_gives_masked_mean():
    B, H, N, d = 2, 2, 8, 4
    _, _, _, V, eps, alpha, rh = _inputs(B, H, N, d, seed=4)
    Q = torch.zeros(B, H, N, d, dtype=torch.float64)
    x = torch.ones(B, N, 3, dtype=torch.float64)  # all points coincide: geometry term constant
    mask = torch.ones(B, N, dtype=torch.float64)
    mask[1, 5:] = 0
    xc, hc = bt.balanced_transport_dual(Q, Q, x, V, eps, alpha, rh, K_iter=3, mask=mask)
    for b, n in ((0, 8), (1, 5)):
        want = V[b, :, :n].mean(1, keepdim=True).expand(H, n, d)
        torch.testing.assert_close(hc[b, :, :n], want, rtol=1e-12, atol=1e-12)
        assert torch.all(hc[b, :, n:] == 0) and torch.all(xc[b, :, n:] == 0)


def _np_gpu_path(Q, K, x, V, eps, alpha, rh, K_iter, mask, b, h):
    """The reference GPU path's masked iteration (flash_sinkhorn_transport.py:57-113,
    :289-313): -1e9 on padded columns in the row update and on padded rows in the
    column update, one log marginal for every row and column, then the centroid
    pass (:117-167) restricted to valid columns."""
    Kg = _np_gibbs(Q, K, x, eps, alpha, rh, b, h)
    L = np.log(Kg)
    mb = np.where(mask[b].numpy() > 0.5, 0.0, -1e9)
    lm = -np.log(3.0)  # any constant: the normalised plan does not depend on it
    u = np.zeros(L.shape[0])
    v = np.zeros(L.shape[0])
    lse = lambda a, ax: a.max(ax) + np.log(np.exp(a - a.max(ax, keepdims=True)).sum(ax))
    for _ in range(K_iter):
        v = lm - lse(L + u[:, None] + mb[:, None], 0)
        u = lm - lse(L + v[None, :] + mb[None, :], 1)
    s = L + u[:, None] + v[None, :] + mb[None, :]
    P = np.exp(s - s.max(1, keepdims=True))
    P /= P.sum(1, keepdims=True)
    return P @ x[b].numpy(), P @ V[b, h].numpy()


def test_batched_equals_per_sample():
    B, H, N, d = 3, 2, 10, 4
    Q, K, x, V, eps, alpha, rh = _inputs(B, H, N, d, seed=5)
    xc, hc = bt.balanced_transport_dual(Q, K, x, V, eps, alpha, rh, K_iter=9)
    for b in range(B):
        xo, ho = bt.balanced_transport_dual(Q[b:b + 1], K[b:b + 1], x[b:b + 1], V[b:b + 1], eps, alpha, rh,
                                            K_iter=9)
        torch.testing.assert_close(xc[b:b + 1], xo, rtol=1e-13, atol=1e-13)
        torch.testing.assert_close(hc[b:b + 1], ho, rtol=1e-13, atol=1e-13)


def test_masked_matches_reference_gpu_path_on_valid_rows():
    B, H, N, d = 3, 2, 10, 4
    Q, K, x, V, eps, alpha, rh = _inputs(B, H, N, d, seed=5)
    mask = torch.ones(B, N, dtype=torch.float64)
    mask[1, 6:] = 0
    mask[2, [0, 4, 5, 9]] = 0  # holes, not only a padded tail
    xc, hc = bt.balanced_transport_dual(Q, K, x, V, eps, alpha, rh, K_iter=9, mask=mask)
    for b in range(B):
        ok = mask[b].numpy() > 0.5
        for h in range(H):
            xw, hw = _np_gpu_path(Q, K, x, V, eps, alpha, rh, 9, mask, b, h)
            np.testing.assert_allclose(xc[b, h].numpy()[ok], xw[ok], rtol=1e-10, atol=1e-12)
            np.testing.assert_allclose(hc[b, h].numpy()[ok], hw[ok], rtol=1e-10, atol=1e-12)
        assert torch.all(xc[b, :, ~torch.from_numpy(ok)] == 0) and torch.all(hc[b, :, ~torch.from_numpy(ok)] == 0)
    x1 = bt.balanced_transport(Q, K, x, eps, alpha, rh, K_iter=9, mask=mask)
    assert torch.equal(x1, xc)


def test_reference_cpu_form_leaks_mass_to_padded_columns():
    """Documents why the masked parity definition is the unpadded one: the CPU form
    (flash_sinkhorn_transport.py:262-270) gives each padded column about 1/n of mass."""
    B, H, N, d = 1, 1, 8, 4
    Q, K, x, V, eps, alpha, rh = _inputs(B, H, N, d, seed=8)
    mask = torch.ones(B, N, dtype=torch.float64)
    mask[0, 6:] = 0
    lm = torch.log(mask.clamp(min=1e-8))
    log_K = -(bt.balanced_cost(Q, K, x, alpha, rh) / eps.view(1, H, 1, 1)) + lm[:, None, :, None] + lm[:, None, None, :]
    lmarg = -torch.log(mask.sum(-1))
    lu = torch.zeros(B, H, N, 1, dtype=torch.float64)
    for _ in range(30):
        lv = lmarg - torch.logsumexp(log_K + lu, dim=-2, keepdim=True)
        lu = lmarg - torch.logsumexp(log_K + lv, dim=-1, keepdim=True)
    T = (lu + log_K + lv).exp()[0, 0]
    col_mass = T[:6, 6:].sum(0)  # mass the valid rows send to each padded column
    assert torch.all(col_mass > 0.5 / 6)


def test_autograd_matches_finite_differences():
    B, H, N, d = 1, 2, 6, 3
    Q, K, x, V, eps, alpha, rh = _inputs(B, H, N, d, seed=6, r=0.7)
    mask = torch.tensor([[1.0, 1, 1, 1, 1, 0]], dtype=torch.float64)
    g = torch.Generator().manual_seed(7)
    wx = torch.randn(B, H, N, 3, generator=g, dtype=torch.float64)
    wh = torch.randn(B, H, N, d, generator=g, dtype=torch.float64)

    def loss(Q, K, x, V, alpha, rh):
        xc, hc = bt.balanced_transport_dual(Q, K, x, V, eps, alpha, rh, K_iter=6, mask=mask)
        return (xc * wx).sum() + (hc * wh).sum()

    leaves = [t.clone().requires_grad_(True) for t in (Q, K, x, V, alpha, rh)]
    loss(*leaves).backward()
    step = 1e-6
    for li, idx in [(0, (0, 1, 2, 1)), (1, (0, 0, 4, 2)), (2, (0, 3, 1)), (3, (0, 1, 0, 2)), (4, (1,)), (5, (0,))]:
        p = [t.detach().clone() for t in leaves]
        m = [t.detach().clone() for t in leaves]
        p[li][idx] += step
        m[li][idx] -= step
        fd = float(loss(*p) - loss(*m)) / (2 * step)
        got = float(leaves[li].grad[idx])
        assert abs(got - fd) <= 1e-6 * max(1.0, abs(fd)), (li, idx, got, fd)
