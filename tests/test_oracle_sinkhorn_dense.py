"""Pins oracle/sinkhorn_dense_torch.py (the full-size checker) to the numpy oracle.

Both run in float64 on the CPU here; they must agree to rounding on every output
and gradient, for both IFT sign conventions, uniform and general marginals, and
with or without the x_centroid path.
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_rel
from oracle import sinkhorn as ref
from oracle import sinkhorn_dense_torch as dense


def _case(B, H, N, d, seed, eps):
    g = torch.Generator().manual_seed(seed)
    t = dict(
        Q=torch.randn(B, H, N, d, generator=g, dtype=torch.float64) / d ** 0.5,
        K=torch.randn(B, H, N, d, generator=g, dtype=torch.float64) / d ** 0.5,
        V=torch.randn(B, H, N, d, generator=g, dtype=torch.float64),
        G=torch.randn(B, H, N, d, generator=g, dtype=torch.float64),
        x_res=torch.randn(B, N, 3, generator=g, dtype=torch.float64),
        eps=torch.tensor(eps, dtype=torch.float64),
        log_mu=torch.log_softmax(torch.randn(B, H, N, generator=g, dtype=torch.float64), -1),
        log_nu=torch.log_softmax(torch.randn(B, H, N, generator=g, dtype=torch.float64), -1),
    )
    go = torch.randn(B, N, H * d, generator=g, dtype=torch.float64)
    gxc = torch.randn(B, H, N, 3, generator=g, dtype=torch.float64)
    return t, go, gxc


def _np_inputs(t, K_iter):
    B, H, N, d = t["Q"].shape
    return dict(Q=t["Q"].numpy(), K=t["K"].numpy(), V=t["V"].numpy(), G=t["G"].numpy(),
                x_res=t["x_res"].numpy(), pos_weight=np.zeros((H, 68)), pos_bins=None,
                eps=t["eps"].numpy(), w_dist=np.zeros(H), log_mu=t["log_mu"].numpy(),
                log_nu=t["log_nu"].numpy(), K_iter=K_iter, lam=1.0, r_0=10.0)


@pytest.mark.parametrize("B,H,N,d,eps,K", [(1, 2, 24, 8, [0.5, 1.0], 9), (2, 3, 17, 16, [0.25, 0.5, 2.0], 30)])
def test_dense_forward_equals_numpy_oracle(B, H, N, d, eps, K):
    t, _, _ = _case(B, H, N, d, 11 + N, eps)
    got = dense.forward(t["Q"], t["K"], t["V"], t["G"], t["eps"], t["log_mu"], t["log_nu"], K, x_res=t["x_res"])
    want = ref.forward(**_np_inputs(t, K))
    for k in ("o_flat", "x_centroid", "log_u", "log_v", "O_avg"):
        assert_close_rel(got[k].numpy(), want[k], 1e-11, k)


@pytest.mark.parametrize("with_xc", [False, True])
def test_dense_backward_cg_reference_equals_numpy_oracle(with_xc):
    B, H, N, d, K, n_cg = 2, 2, 20, 8, 25, 12
    t, go, gxc = _case(B, H, N, d, 5, [0.5, 1.0])
    gxc = gxc if with_xc else None
    fo = dense.forward(t["Q"], t["K"], t["V"], t["G"], t["eps"], t["log_mu"], t["log_nu"], K, x_res=t["x_res"])
    got = dense.backward_cg(t["Q"], t["K"], t["V"], t["G"], t["eps"], fo, go, n_cg, grad_xc=gxc, x_res=t["x_res"])
    oi = _np_inputs(t, K)
    fn = ref.forward(**oi)
    want = ref.backward_reference(oi, fn, go.numpy(), None if gxc is None else gxc.numpy(), solver="cg", n_cg=n_cg)
    for k in ("Q", "K", "V", "G", "log_mu", "log_nu"):
        assert_close_rel(got[k].numpy(), want[k], 1e-9, k)


@pytest.mark.parametrize("K_back", [1, 3, 25])
def test_dense_backward_fixed_point_equals_numpy_oracle(K_back):
    """The reference's Gauss-Seidel sweeps, sweep for sweep (a short K_back leaves the
    solve unconverged, so the sweep order and count are what is compared)."""
    B, H, N, d, K = 2, 2, 20, 8, 25
    t, go, gxc = _case(B, H, N, d, 13, [0.5, 1.0])
    fo = dense.forward(t["Q"], t["K"], t["V"], t["G"], t["eps"], t["log_mu"], t["log_nu"], K, x_res=t["x_res"])
    got = dense.backward(t["Q"], t["K"], t["V"], t["G"], t["eps"], fo, go, K_back, grad_xc=gxc, x_res=t["x_res"],
                         solver="fixed_point")
    oi = _np_inputs(t, K)
    want = ref.backward_reference(oi, ref.forward(**oi), go.numpy(), gxc.numpy(), K_back=K_back)
    for k in ("Q", "K", "V", "G", "log_mu", "log_nu"):
        assert_close_rel(got[k].numpy(), want[k], 1e-9, k)
    if K_back == 1:  # one sweep differs from the converged solve: the comparison discriminates
        conv = ref.backward_reference(oi, ref.forward(**oi), go.numpy(), gxc.numpy(), K_back=60)
        assert np.max(np.abs(got["log_nu"].numpy() - conv["log_nu"])) > 1e-6


def test_dense_backward_analytic_equals_numpy_oracle():
    """Analytic signs; CG run long enough to reach the exact solve of the numpy oracle."""
    B, H, N, d, K = 1, 2, 20, 8, 40
    t, go, gxc = _case(B, H, N, d, 7, [0.5, 2.0])
    fo = dense.forward(t["Q"], t["K"], t["V"], t["G"], t["eps"], t["log_mu"], t["log_nu"], K, x_res=t["x_res"])
    got = dense.backward_cg(t["Q"], t["K"], t["V"], t["G"], t["eps"], fo, go, 60, mode="analytic", grad_xc=gxc,
                            x_res=t["x_res"])
    oi = _np_inputs(t, K)
    want = ref.backward_analytic(oi, ref.forward(**oi), go.numpy(), gxc.numpy())
    for k in ("Q", "K", "V", "G", "log_mu", "log_nu"):
        assert_close_rel(got[k].numpy(), want[k], 1e-8, k)


def test_dense_planted_sign_error_is_caught():
    """The reference and analytic sign conventions differ measurably (the check discriminates)."""
    B, H, N, d, K = 1, 1, 16, 8, 30
    t, go, _ = _case(B, H, N, d, 9, [0.5])
    fo = dense.forward(t["Q"], t["K"], t["V"], t["G"], t["eps"], t["log_mu"], t["log_nu"], K)
    a = dense.backward_cg(t["Q"], t["K"], t["V"], t["G"], t["eps"], fo, go, 30, mode="reference")
    b = dense.backward_cg(t["Q"], t["K"], t["V"], t["G"], t["eps"], fo, go, 30, mode="analytic")
    rel = float((a["Q"] - b["Q"]).abs().max() / a["Q"].abs().max())
    assert rel > 1e-3
