"""CPU pinning of the numpy oracle (oracle/sinkhorn.py) -- no GPU needed.

The oracle is only trusted as far as these checks pin it:

* golden vectors written by the reference's own FlashSinkhornAttn forward and
  backward (tests/golden/make_golden.py);
* closed forms: Q = K = 0 with no position / geometry term gives L = 0, so the
  potentials follow scalar recurrences over the n valid tokens and O_avg is the
  masked mean of V;
* invariants the reference's tests assert: batched == per-sample
  (tests/test_flash_sinkhorn_batch.py:29-107), masked == unpadded with zero
  padded potentials (tests/test_sinkhorn_batch.py:43-113), T_norm rows sum to 1
  (tests/test_primitives.py:149-150), warm-start composition K=7 then 4 == K=11
  (scripts/benchmark_correctness.py:503-531);
* optimality: the converged potentials are a stationary point of the entropic
  unbalanced-OT primal (Chizat et al. 2018), checked by finite differences of
  the primal objective, which the oracle never evaluates;
* the analytic IFT adjoint against float64 finite differences of a converged
  forward, and the reference-mode adjoint tied to it by
  z_v(ref) = lambda_v(analytic), z_u(ref) = -lambda_u(analytic);
* CG: against numpy.linalg.solve on SPD systems (tests/test_cg.py:9-28) and
  against the converged fixed point on the IFT system;
* planted mistakes (a transposed cost, the analytic signs) fail the golden
  checks, so those checks can tell.
"""

import glob
import math
import os

import numpy as np
import pytest

from conftest import max_rel_err
from oracle import sinkhorn as ref

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = sorted(glob.glob(os.path.join(HERE, "golden", "flash_sinkhorn_*.npz")))
FWD_KEYS = ("o_flat", "x_centroid", "log_u", "log_v")
GRADS = ("Q", "K", "V", "G", "x_res", "pos_weight", "w_dist", "log_mu", "log_nu")
INPUTS = ("Q", "K", "V", "G", "x_res", "pos_weight", "pos_bins", "eps", "w_dist", "log_mu", "log_nu")


def load_golden(path):
    z = dict(np.load(path))
    inp = {k: z[k] for k in INPUTS}
    scal = dict(K_iter=int(z["K_iter"]), lam=float(z["lam"]), r_0=float(z["r_0"]))
    return z, inp, scal


def grad_err(got, want, k):
    """Relative error; gradients that are pure cancellation noise in the reference
    (d pos_weight / d w_dist with those terms identically zero) are measured on the
    scale of the largest gradient instead."""
    w = np.asarray(want, dtype=np.float64)
    if float(np.max(np.abs(w))) < 1e-4:
        return float(np.max(np.abs(np.asarray(got) - w)))
    return max_rel_err(got, w)


def make_inputs(B, H, N, d, seed, eps, pos_geo=True, mask_lengths=None):
    rng = np.random.default_rng(seed)
    inp = dict(
        Q=rng.standard_normal((B, H, N, d)) / math.sqrt(d),
        K=rng.standard_normal((B, H, N, d)) / math.sqrt(d),
        V=rng.standard_normal((B, H, N, d)),
        G=rng.standard_normal((B, H, N, d)),
        x_res=rng.standard_normal((B, N, 3)) * 3.0 if pos_geo else np.zeros((B, N, 3)),
        pos_weight=rng.standard_normal((H, 68)) * 0.5 if pos_geo else np.zeros((H, 68)),
        pos_bins=rng.integers(0, 68, (B, N, N)).astype(np.int32) if pos_geo else None,
        eps=np.asarray(eps, dtype=np.float64),
        w_dist=rng.random(H) if pos_geo else np.zeros(H),
    )
    lm = rng.standard_normal((B, H, N))
    ln = rng.standard_normal((B, H, N))
    inp["log_mu"] = lm - np.log(np.exp(lm).sum(-1, keepdims=True))
    inp["log_nu"] = ln - np.log(np.exp(ln).sum(-1, keepdims=True))
    return inp


# ---------------------------------------------------------------- golden vectors


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[15:-4] for p in GOLDEN])
def test_forward_matches_reference_golden(path):
    z, inp, scal = load_golden(path)
    fo = ref.forward(**inp, **scal)
    # ragged_tile (N = 70, geometry on): torch.cdist's matmul path rounds the
    # reference's distances (~5e-5 relative on the outputs); the rest agree to 1e-6.
    tol = 1e-4 if "ragged_tile" in path else 1e-6
    for k in FWD_KEYS:
        assert max_rel_err(fo[k], z[k]) <= tol, k


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[15:-4] for p in GOLDEN])
def test_backward_reference_matches_reference_golden(path):
    z, inp, scal = load_golden(path)
    fo = ref.forward(**inp, **scal)
    g = ref.backward_reference(dict(inp, **scal), fo, z["grad_o"], z["grad_xc"])
    tol = 1e-3 if "ragged_tile" in path else 2e-5
    for k in GRADS:
        assert grad_err(g[k], z["grad_" + k], k) <= tol, k


def test_planted_transposed_cost_fails_golden(monkeypatch):
    """A transposed cost (q_j.k_i instead of q_i.k_j) must be caught by the golden check."""
    z, inp, scal = load_golden(GOLDEN[0])
    orig = ref.cost_matrix

    def transposed(*a, **kw):
        C, dist, diff = orig(*a, **kw)
        return C.T, dist, diff

    monkeypatch.setattr(ref, "cost_matrix", transposed)
    fo = ref.forward(**inp, **scal)
    assert max(max_rel_err(fo[k], z[k]) for k in ("log_u", "log_v", "o_flat")) > 1e-2


def test_planted_analytic_signs_fail_reference_golden():
    """The analytic adjoint differs from the reference's in two signs; the reference
    golden vectors must tell them apart (and so would catch either sign in the oracle)."""
    path = [p for p in GOLDEN if "converged" in p][0]
    z, inp, scal = load_golden(path)
    fo = ref.forward(**inp, **scal)
    g = ref.backward_analytic(dict(inp, **scal), fo, z["grad_o"], z["grad_xc"])
    assert max_rel_err(g["log_mu"], z["grad_log_mu"]) > 0.5
    assert max_rel_err(g["Q"], z["grad_Q"]) > 1e-2
    # ... while d log_nu (z_v) is the same in both conventions
    assert max_rel_err(g["log_nu"], z["grad_log_nu"]) < 1e-4


# ---------------------------------------------------------------- closed forms


@pytest.mark.parametrize("n,N,eps,K_iter", [(5, 8, 0.5, 7), (8, 8, 1.0, 3), (13, 20, 0.25, 11)])
def test_zero_logits_closed_form(n, N, eps, K_iter):
    """Q = K = 0 and no position / geometry term: L = 0.  Then u and v are constant
    over valid tokens, a_k = kappa (log mu - log n - b_{k-1}), b_k = kappa (log nu -
    log n - a_k) with b_0 = 0, and O_avg = n / (n + 1e-6) * mean of V over valid keys."""
    B, H, d = 1, 2, 4
    rng = np.random.default_rng(n)
    V = rng.standard_normal((B, H, N, d))
    mask = np.zeros((B, N))
    mask[0, :n] = 1.0
    lmu, lnu = -0.3, -1.7
    out = ref.forward(np.zeros((B, H, N, d)), np.zeros((B, H, N, d)), V, np.zeros((B, H, N, d)),
                      np.zeros((B, N, 3)), np.zeros((H, 68)), None, np.full(H, eps), np.zeros(H),
                      np.full((B, H, N), lmu), np.full((B, H, N), lnu), K_iter=K_iter, mask=mask)
    kappa = 1.0 / (1.0 + eps)
    a = b = 0.0
    for _ in range(K_iter):
        a = kappa * (lmu - math.log(n) - b)
        b = kappa * (lnu - math.log(n) - a)
    np.testing.assert_allclose(out["log_u"][0, :, :n], a, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(out["log_v"][0, :, :n], b, rtol=1e-13, atol=1e-13)
    assert np.all(out["log_u"][0, :, n:] == 0) and np.all(out["log_v"][0, :, n:] == 0)
    want = V[0, :, :n].sum(1) / (n + 1e-6)  # (H, d), the same for every query row
    np.testing.assert_allclose(out["O_avg"][0, :, :n], np.broadcast_to(want[:, None], (H, n, d)),
                               rtol=1e-12, atol=1e-13)
    o = out["o_flat"].reshape(B, N, H, d)
    assert np.all(o[0, n:] == 0)
    np.testing.assert_allclose(o[0, :n], 0.5 * np.broadcast_to(want[None], (n, H, d)), rtol=1e-12)


def test_cost_terms_closed_form():
    """Position term = pos_weight[h, bins]; geometry term = w d/(r0 + d) on a 3-4-5 triangle."""
    rng = np.random.default_rng(3)
    pw = rng.standard_normal(68)
    bins = rng.integers(0, 68, (6, 6))
    x = np.zeros((6, 3))
    C, _, _ = ref.cost_matrix(np.zeros((6, 4)), np.zeros((6, 4)), x, pw, bins, 0.0, 10.0)
    np.testing.assert_array_equal(C, pw[bins])
    x = np.array([[0.0, 0.0, 0.0], [3.0, 4.0, 0.0]])
    C, dist, _ = ref.cost_matrix(np.zeros((2, 4)), np.zeros((2, 4)), x, pw, None, 2.0, 10.0)
    np.testing.assert_allclose(C, [[0.0, 10.0 / 15.0], [10.0 / 15.0, 0.0]], rtol=1e-15)
    q = np.array([[1.0, 2.0, 0.0, 0.0]])
    k = np.array([[3.0, -1.0, 0.0, 0.0]])
    C, _, _ = ref.cost_matrix(q, k, np.zeros((1, 3)), pw, None, 0.0, 10.0)
    assert C[0, 0] == pytest.approx(-(3.0 - 2.0) / 2.0)


# ---------------------------------------------------------------- invariants


def test_batched_equals_per_sample():
    inp = make_inputs(3, 2, 12, 8, seed=5, eps=[0.5, 2.0])
    full = ref.forward(**inp, K_iter=6)
    for b in range(3):
        one = {k: (v if k in ("pos_weight", "eps", "w_dist") else v[b:b + 1]) for k, v in inp.items()}
        single = ref.forward(**one, K_iter=6)
        for k in FWD_KEYS:
            np.testing.assert_allclose(full[k][b:b + 1], single[k], rtol=1e-13, atol=1e-14)


def test_masked_equals_unpadded():
    B, H, N, d, n = 1, 2, 16, 8, 11
    inp = make_inputs(B, H, N, d, seed=6, eps=[0.5, 1.0])
    mask = np.zeros((B, N))
    mask[0, :n] = 1.0
    padded = ref.forward(**inp, K_iter=9, mask=mask)
    sl = dict(inp)
    for k in ("Q", "K", "V", "G", "log_mu", "log_nu"):
        sl[k] = inp[k][:, :, :n]
    sl["x_res"] = inp["x_res"][:, :n]
    sl["pos_bins"] = inp["pos_bins"][:, :n, :n]
    unpadded = ref.forward(**sl, K_iter=9)
    np.testing.assert_allclose(padded["log_u"][:, :, :n], unpadded["log_u"], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(padded["log_v"][:, :, :n], unpadded["log_v"], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(padded["o_flat"][:, :n], unpadded["o_flat"], rtol=1e-12, atol=1e-13)
    assert np.all(padded["log_u"][:, :, n:] == 0) and np.all(padded["log_v"][:, :, n:] == 0)
    assert np.all(padded["o_flat"][:, n:] == 0)


def test_plan_rows_sum_to_one():
    """T_norm rows sum to 1 up to the 1e-6 guard: O_avg of V = 1 is 1 within 1e-6."""
    inp = make_inputs(1, 3, 10, 4, seed=7, eps=[0.25, 1.0, 4.0])
    inp["V"] = np.ones_like(inp["V"])
    out = ref.forward(**inp, K_iter=5)
    assert np.max(np.abs(out["O_avg"] - 1.0)) <= 1e-6


def test_warm_start_composition():
    inp = make_inputs(2, 2, 9, 4, seed=8, eps=[0.5, 1.0])
    a = ref.forward(**inp, K_iter=7)
    b = ref.forward(**inp, K_iter=4, log_u_init=a["log_u"], log_v_init=a["log_v"])
    c = ref.forward(**inp, K_iter=11)
    for k in FWD_KEYS:
        np.testing.assert_allclose(b[k], c[k], rtol=1e-13, atol=1e-14)


def _uot_primal(T, C, eps, lam, mu, nu):
    r, c = T.sum(1), T.sum(0)
    kl = lambda p, q: float(np.sum(p * np.log(p / q) - p + q))
    return float(np.sum(T * C)) + eps * float(np.sum(T * np.log(T) - T)) + lam * kl(r, mu) + lam * kl(c, nu)


def test_converged_potentials_minimise_uot_primal():
    """exp(u + L + v) at convergence minimises <T,C> + eps sum(T log T - T) +
    lam KL~(T1|mu) + lam KL~(T^T 1|nu): every directional derivative of the primal
    (by central differences) vanishes there, and does not after 2 iterations."""
    rng = np.random.default_rng(9)
    H, N, d, eps, lam = 1, 7, 4, 0.5, 1.0
    inp = make_inputs(1, H, N, d, seed=9, eps=[eps])
    C, _, _ = ref.cost_matrix(inp["Q"][0, 0], inp["K"][0, 0], inp["x_res"][0], inp["pos_weight"][0],
                              inp["pos_bins"][0], inp["w_dist"][0], 10.0)
    mu, nu = np.exp(inp["log_mu"][0, 0]), np.exp(inp["log_nu"][0, 0])

    def slopes(K_iter):
        out = ref.forward(**inp, K_iter=K_iter, lam=lam)
        u, v = out["log_u"][0, 0], out["log_v"][0, 0]
        T = np.exp(u[:, None] - C / eps + v[None, :])
        res = []
        for _ in range(6):
            D = rng.standard_normal(T.shape)
            h = 1e-5
            fp = _uot_primal(T * np.exp(h * D), C, eps, lam, mu, nu)
            fm = _uot_primal(T * np.exp(-h * D), C, eps, lam, mu, nu)
            res.append(abs(fp - fm) / (2 * h))
        return max(res)

    assert slopes(400) < 1e-8
    assert slopes(2) > 1e-3


# ---------------------------------------------------------------- IFT backward


def _loss(inp, K_iter, go, gxc):
    out = ref.forward(**inp, K_iter=K_iter)
    return float(np.sum(out["o_flat"] * go) + np.sum(out["x_centroid"] * gxc))


def test_analytic_adjoint_matches_finite_differences():
    """d loss / d theta of a converged float64 forward (central differences) equals
    the analytic IFT gradient, for every differentiable input kind."""
    B, H, N, d, K_iter = 1, 2, 8, 4, 400
    inp = make_inputs(B, H, N, d, seed=10, eps=[0.5, 1.0])
    rng = np.random.default_rng(11)
    go = rng.standard_normal((B, N, H * d))
    gxc = rng.standard_normal((B, H, N, 3))
    fo = ref.forward(**inp, K_iter=K_iter)
    g = ref.backward_analytic(dict(inp, K_iter=K_iter), fo, go, gxc)
    h = 1e-6
    probes = [("Q", (0, 0, 3, 1)), ("Q", (0, 1, 6, 2)), ("K", (0, 0, 2, 0)), ("K", (0, 1, 7, 3)),
              ("V", (0, 1, 4, 2)), ("G", (0, 0, 5, 1)), ("x_res", (0, 3, 1)), ("x_res", (0, 6, 2)),
              ("pos_weight", (1, int(inp["pos_bins"][0, 2, 5]))), ("w_dist", (0,)), ("w_dist", (1,)),
              ("log_mu", (0, 0, 2)), ("log_mu", (0, 1, 5)), ("log_nu", (0, 0, 4)), ("log_nu", (0, 1, 1))]
    for name, idx in probes:
        p, m = dict(inp), dict(inp)
        p[name] = inp[name].copy()
        m[name] = inp[name].copy()
        p[name][idx] += h
        m[name][idx] -= h
        fd = (_loss(p, K_iter, go, gxc) - _loss(m, K_iter, go, gxc)) / (2 * h)
        scale = max(1.0, float(np.max(np.abs(g[name]))))
        # 1e-5: the forward's T / (sum T + 1e-6) guard perturbs the loss at the 1e-6
        # level and is not differentiated by the adjoint (nor by the reference's)
        assert abs(g[name][idx] - fd) <= 1e-5 * scale, (name, idx, g[name][idx], fd)


def test_reference_mode_tied_to_analytic_adjoint():
    """With g_u = 0 the reference's Gauss-Seidel z solves the same system:
    z_v(ref) = lambda_v(analytic) and z_u(ref) = -lambda_u(analytic)."""
    inp = make_inputs(1, 2, 10, 4, seed=12, eps=[0.5, 2.0])
    rng = np.random.default_rng(13)
    go = rng.standard_normal((1, 10, 8))
    fo = ref.forward(**inp, K_iter=300)
    r = ref.backward_reference(dict(inp, K_iter=300), fo, go, None, K_back=400)
    a = ref.backward_analytic(dict(inp, K_iter=300), fo, go, None)
    np.testing.assert_allclose(r["log_nu"], a["log_nu"], rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(r["log_mu"], -a["log_mu"], rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(r["V"], a["V"], rtol=1e-12)


def test_backward_batched_equals_per_sample():
    inp = make_inputs(2, 2, 9, 4, seed=14, eps=[0.5, 1.0])
    rng = np.random.default_rng(15)
    go = rng.standard_normal((2, 9, 8))
    gxc = rng.standard_normal((2, 2, 9, 3))
    fo = ref.forward(**inp, K_iter=5)
    full = ref.backward_reference(dict(inp, K_iter=5), fo, go, gxc)
    acc_pw = np.zeros_like(full["pos_weight"])
    for b in range(2):
        one = {k: (v if k in ("pos_weight", "eps", "w_dist") else v[b:b + 1]) for k, v in inp.items()}
        f1 = ref.forward(**one, K_iter=5)
        g1 = ref.backward_reference(dict(one, K_iter=5), f1, go[b:b + 1], gxc[b:b + 1])
        for k in ("Q", "K", "V", "G", "x_res", "log_mu", "log_nu"):
            np.testing.assert_allclose(full[k][b:b + 1], g1[k], rtol=1e-12, atol=1e-14)
        acc_pw += g1["pos_weight"]
    np.testing.assert_allclose(full["pos_weight"], acc_pw, rtol=1e-12, atol=1e-14)


# ---------------------------------------------------------------- conjugate gradient


def test_cg_identity():
    b = np.arange(1.0, 6.0)
    x, info = ref.conjugate_gradient(lambda v: v, b)
    np.testing.assert_allclose(x, b, rtol=1e-15)
    assert info["converged"] and info["iters"] == 1


@pytest.mark.parametrize("precond", [False, True])
def test_cg_spd_matches_solve(precond):
    rng = np.random.default_rng(16)
    A0 = rng.standard_normal((30, 30))
    A = A0 @ A0.T + 30 * np.eye(30)
    b = rng.standard_normal(30)
    pre = (lambda r: r / np.diag(A)) if precond else None
    x, info = ref.conjugate_gradient(lambda v: A @ v, b, rtol=1e-12, atol=1e-14, preconditioner=pre,
                                     max_iter=200)
    assert info["converged"]
    np.testing.assert_allclose(x, np.linalg.solve(A, b), rtol=1e-9)


def test_cg_system_matches_fixed_point():
    """CG on the symmetric form solves the reference's fixed-point system: equal z."""
    inp = make_inputs(1, 1, 12, 4, seed=17, eps=[0.5])
    rng = np.random.default_rng(18)
    go = rng.standard_normal((1, 12, 4))
    fo = ref.forward(**inp, K_iter=20)
    fp = ref.backward_reference(dict(inp, K_iter=20), fo, go, None, K_back=600, return_internals=True)
    cg = ref.backward_reference(dict(inp, K_iter=20), fo, go, None, solver="cg", n_cg=40,
                                return_internals=True)
    np.testing.assert_allclose(cg["_internals"][(0, 0)]["z_v"], fp["_internals"][(0, 0)]["z_v"],
                               rtol=1e-10, atol=1e-13)
    for k in GRADS:
        np.testing.assert_allclose(cg[k], fp[k], rtol=1e-9, atol=1e-12)


def test_backward_masked_is_per_sample_unpadded():
    B, H, N, d = 2, 2, 10, 4
    inp = make_inputs(B, H, N, d, seed=19, eps=[0.5, 1.0])
    mask = np.zeros((B, N))
    mask[0, :7] = 1
    mask[1, :10] = 1
    rng = np.random.default_rng(20)
    go = rng.standard_normal((B, N, H * d))
    fo, gr = ref.backward_masked(dict(inp, K_iter=4, mask=mask), go)
    sl = {k: (v if k in ("pos_weight", "eps", "w_dist") else v[0:1]) for k, v in inp.items()}
    for k in ("Q", "K", "V", "G", "log_mu", "log_nu"):
        sl[k] = sl[k][:, :, :7]
    sl["x_res"] = sl["x_res"][:, :7]
    sl["pos_bins"] = sl["pos_bins"][:, :7, :7]
    f0 = ref.forward(**sl, K_iter=4)
    g0 = ref.backward_reference(dict(sl, K_iter=4), f0, go[0:1, :7], None)
    np.testing.assert_allclose(gr["Q"][0:1, :, :7], g0["Q"], rtol=1e-12, atol=1e-14)
    assert np.all(gr["Q"][0, :, 7:] == 0) and np.all(gr["log_mu"][0, :, 7:] == 0)
