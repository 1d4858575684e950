"""GPU parity of the remaining Sinkhorn-path APIs:

* ``flash_sinkhorn`` / ``FlashSinkhornFunction.apply`` (sinkhorn_kernel.py:1921-2468):
  ungated O_avg, x_centroid and potentials against the oracle forward (gate
  logits +30, sigma = 1 - 1e-13), gradients of ``ift_mode="reference"`` against
  the oracle's reference-mode IFT backward (the default unrolled gradient is
  tests/test_gpu_unrolled.py's); the additive mask_bias form; unbatched inputs.
* ``conjugate_gradient`` / ``CGInfo`` (utils/cg.py:28-97): the solution against
  torch.linalg.solve, and the iteration count / residual record against the
  oracle's restatement of the reference steps.
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_rel
from oracle import sinkhorn as ref
from test_gpu_sinkhorn_fwd import make_inputs, oracle_inputs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GRADS = ("Q", "K", "V", "x_res", "pos_weight", "w_dist", "log_mu", "log_nu")


def gate_free_oracle(inp, dtype, K_iter):
    oi = oracle_inputs(inp, dtype)
    oi["G"] = np.full_like(oi["Q"], 30.0)  # sigmoid(30) = 1 - 9e-14
    return oi, ref.forward(**oi, K_iter=K_iter)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_flash_sinkhorn_forward_backward(dtype, tol):
    from deepfold_amd import flash_sinkhorn

    B, H, N, d, K = 2, 2, 70, 32, 7
    inp = make_inputs(B, H, N, d, seed=501, eps=[0.5, 1.0], pos_geo=True)
    leaves = {k: (None if v is None else v.to(DEV)) for k, v in inp.items()}
    for k in ("Q", "K", "V"):
        leaves[k] = leaves[k].to(dtype)
    for k in GRADS:
        leaves[k] = leaves[k].detach().requires_grad_(True)
    O, xc, lu, lv = flash_sinkhorn(leaves["Q"], leaves["K"], leaves["V"], leaves["x_res"], leaves["pos_weight"],
                                   leaves["pos_bins"], leaves["eps"], leaves["w_dist"], leaves["log_mu"],
                                   leaves["log_nu"], K_iter=K, ift_mode="reference")
    assert O.shape == (B, H, N, d)
    g = torch.Generator().manual_seed(502)
    gO = torch.randn(B, H, N, d, generator=g)
    gxc = torch.randn(B, H, N, 3, generator=g)
    ((O * gO.to(DEV)).sum() + (xc * gxc.to(DEV)).sum()).backward()
    oi, fo = gate_free_oracle(inp, dtype, K)
    assert_close_rel(O.detach().cpu().numpy(), fo["O_avg"], tol, "O_avg")
    assert_close_rel(xc.detach().cpu().numpy(), fo["x_centroid"], tol, "x_centroid")
    assert_close_rel(lu.detach().cpu().numpy(), fo["log_u"], tol, "log_u")
    assert_close_rel(lv.detach().cpu().numpy(), fo["log_v"], tol, "log_v")
    # the oracle's gate is sigma = 1 - 9e-14: d o_flat = gO permuted
    go_flat = gO.permute(0, 2, 1, 3).reshape(B, N, H * d).numpy()
    want = ref.backward_reference(dict(oi, K_iter=K), fo, go_flat, gxc.numpy())
    for k in GRADS:
        assert_close_rel(leaves[k].grad.float().cpu().numpy(), want[k], max(tol, 2e-4), "d" + k)


def test_flash_sinkhorn_function_mask_bias_and_unbatched():
    from deepfold_amd import FlashSinkhornFunction, flash_sinkhorn

    B, H, N, d, K = 1, 2, 40, 32, 5
    inp = make_inputs(B, H, N, d, seed=511, eps=[0.5, 1.0])
    t = {k: (None if v is None else v.to(DEV)) for k, v in inp.items()}
    mask = torch.ones(B, N, device=DEV)
    mask[0, 31:] = 0
    mask_bias = (1 - mask) * -1e9
    a = FlashSinkhornFunction.apply(t["Q"], t["K"], t["V"], t["x_res"], t["pos_weight"], t["pos_bins"], t["eps"],
                                    t["w_dist"], t["log_mu"], t["log_nu"], K, 1.0, 10.0, None, None, 64, mask_bias)
    b = flash_sinkhorn(t["Q"], t["K"], t["V"], t["x_res"], t["pos_weight"], t["pos_bins"], t["eps"], t["w_dist"],
                       t["log_mu"], t["log_nu"], K_iter=K, mask=mask)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert torch.all(a[0][0, :, 31:] == 0)
    u = flash_sinkhorn(t["Q"][0], t["K"][0], t["V"][0], t["x_res"][0], t["pos_weight"], None, t["eps"],
                       t["w_dist"], t["log_mu"][0], t["log_nu"][0], K_iter=K)
    full = flash_sinkhorn(t["Q"], t["K"], t["V"], t["x_res"], t["pos_weight"], None, t["eps"], t["w_dist"],
                          t["log_mu"], t["log_nu"], K_iter=K)
    assert u[0].shape == (H, N, d)
    for x, y in zip(u, full):
        assert torch.equal(x, y[0])


@pytest.mark.parametrize("precond,stabilise", [(False, 0), (True, 0), (False, 3)])
def test_conjugate_gradient(precond, stabilise):
    from deepfold_amd import CGInfo, conjugate_gradient

    g = torch.Generator().manual_seed(521)
    A0 = torch.randn(64, 64, generator=g, dtype=torch.float64)
    A = A0 @ A0.T + 64 * torch.eye(64, dtype=torch.float64)
    b = torch.randn(64, generator=g, dtype=torch.float64)
    Ad, bd = A.to(DEV), b.to(DEV)
    pre = (lambda r: r / torch.diagonal(Ad)) if precond else None
    x, info = conjugate_gradient(lambda v: Ad @ v, bd, rtol=1e-10, atol=1e-12, preconditioner=pre,
                                 stabilise_every=stabilise, max_iter=200)
    assert isinstance(info, CGInfo) and info.converged
    np.testing.assert_allclose(x.cpu().numpy(), torch.linalg.solve(A, b).numpy(), rtol=1e-8)
    pre_np = (lambda r: r / np.diag(A.numpy())) if precond else None
    _, want = ref.conjugate_gradient(lambda v: A.numpy() @ v, b.numpy(), rtol=1e-10, atol=1e-12,
                                     preconditioner=pre_np, stabilise_every=stabilise, max_iter=200)
    assert info.iters == want["iters"]
    assert info.initial_residual == pytest.approx(want["initial_residual"], rel=1e-12)
    # identity: one step, warm start at the solution: zero steps needed beyond the first check
    x1, i1 = conjugate_gradient(lambda v: v, bd)
    assert i1.converged and i1.iters == 1
    torch.testing.assert_close(x1, bd)
