"""GPU parity of the dense (materialised-cost) Sinkhorn functions
(sinkhorn_solve, compute_transport_output) against the float64 CPU oracle
(oracle/sinkhorn_dense_ref.py, gradients by autograd as in the reference).

Relative error = max |gpu - oracle| / max |oracle| per tensor, bar 1e-4 (fp32).
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_rel
from oracle import sinkhorn_dense_ref as dref

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 1e-4


def _case(B, H, N, d=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, N, d, generator=g) / d ** 0.5
    K = torch.randn(B, H, N, d, generator=g) / d ** 0.5
    C = -(Q @ K.transpose(-1, -2)) / d ** 0.5 + 0.3 * torch.rand(B, H, N, N, generator=g)
    lmu = torch.log_softmax(torch.randn(B, H, N, generator=g), -1)
    lnu = torch.log_softmax(torch.randn(B, H, N, generator=g), -1)
    eps = torch.linspace(0.4, 1.5, H)
    return C, lmu, lnu, eps, g


def _mask(B, N, lengths):
    m = torch.zeros(B, N)
    for b, n in enumerate(lengths):
        m[b, :n] = 1
    return m


def _grads(fn, leaves):
    """Run fn on float64 CPU copies (oracle) and on float32 GPU copies (HIP), return both grads."""
    out = {}
    for tag, conv in (("ref", lambda t: t.double().clone()), ("gpu", lambda t: t.float().to(DEV).clone())):
        ls = {k: (None if v is None else conv(v).requires_grad_(True)) for k, v in leaves.items()}
        loss, vals = fn(ls, tag)
        loss.backward()
        out[tag] = ({k: (None if v is None else v.grad) for k, v in ls.items()}, vals)
    out["shapes"] = {k: (None if v is None else tuple(v.shape)) for k, v in leaves.items()}
    return out


def _solve(tag):
    if tag == "ref":
        return dref.sinkhorn_solve
    from deepfold_amd import sinkhorn_solve
    return sinkhorn_solve


def _transport(tag):
    if tag == "ref":
        return dref.compute_transport_output
    from deepfold_amd import compute_transport_output
    return compute_transport_output


def _cmp(out, names, tol=TOL):
    gref, vref = out["ref"]
    ggpu, vgpu = out["gpu"]
    for k, w in vref.items():
        assert_close_rel(vgpu[k].detach().cpu().double().numpy(), w.detach().numpy(), tol, f"value {k}")
    for k in names:
        # autograd leaves .grad None on a leaf the loss does not reach (log_u_init for K >= 1)
        want = np.zeros(out["shapes"][k]) if gref[k] is None else gref[k].numpy()
        got = np.zeros_like(want) if ggpu[k] is None else ggpu[k].cpu().double().numpy()
        assert_close_rel(got, want, tol, f"grad {k}")


@pytest.mark.parametrize("B,H,N,K", [(1, 2, 40, 7), (2, 3, 70, 12), (1, 1, 5, 3)])
def test_solve_forward_backward(B, H, N, K):
    C, lmu, lnu, eps, g = _case(B, H, N, seed=N + K)
    wu, wv = torch.randn(B, H, N, generator=g), torch.randn(B, H, N, generator=g)

    def fn(ls, tag):
        e = eps.double() if tag == "ref" else eps.to(DEV)
        lu, lv = _solve(tag)(ls["C"], ls["mu"], ls["nu"], e, K=K)
        cw = (lambda t: t.double()) if tag == "ref" else (lambda t: t.to(DEV))
        return (lu * cw(wu)).sum() + (lv * cw(wv)).sum(), {"log_u": lu, "log_v": lv}

    _cmp(_grads(fn, {"C": C, "mu": lmu, "nu": lnu}), ("C", "mu", "nu"))


def test_solve_masked_warm_start_unbatched():
    B, H, N, K = 3, 2, 48, 9
    C, lmu, lnu, eps, g = _case(B, H, N, seed=3)
    mask = _mask(B, N, [48, 31, 9])
    u0, v0 = 0.1 * torch.randn(B, H, N, generator=g), 0.1 * torch.randn(B, H, N, generator=g)
    wu, wv = torch.randn(B, H, N, generator=g), torch.randn(B, H, N, generator=g)

    def fn(ls, tag):
        cw = (lambda t: t.double()) if tag == "ref" else (lambda t: t.to(DEV))
        lu, lv = _solve(tag)(ls["C"], ls["mu"], ls["nu"], cw(eps), K=K, log_u_init=ls["u0"], log_v_init=ls["v0"],
                             mask=cw(mask))
        return (lu * cw(wu)).sum() + (lv * cw(wv)).sum(), {"log_u": lu, "log_v": lv}

    out = _grads(fn, {"C": C, "mu": lmu, "nu": lnu, "u0": u0, "v0": v0})
    _cmp(out, ("C", "mu", "nu", "u0", "v0"))
    lu = out["gpu"][1]["log_u"].detach().cpu()
    assert torch.all(lu[1, :, 31:] == 0) and torch.all(lu[2, :, 9:] == 0)
    # unbatched 3-D input == B = 1
    from deepfold_amd import sinkhorn_solve
    a = sinkhorn_solve(C[0].to(DEV), lmu[0].to(DEV), lnu[0].to(DEV), eps.to(DEV), K=K)
    b = sinkhorn_solve(C[:1].to(DEV), lmu[:1].to(DEV), lnu[:1].to(DEV), eps.to(DEV), K=K)
    assert torch.equal(a[0], b[0][0]) and torch.equal(a[1], b[1][0])


def test_solve_early_stop():
    from deepfold_amd import sinkhorn_solve

    B, H, N = 1, 2, 32
    C, lmu, lnu, eps, _ = _case(B, H, N, seed=7)
    thr = 1e-5
    lu_r, lv_r, done = dref.sinkhorn_solve(C.double(), lmu.double(), lnu.double(), eps.double(), K=200,
                                           threshold=thr, check_every=2, return_iters=True)
    assert done < 200
    lu, lv = sinkhorn_solve(C.to(DEV), lmu.to(DEV), lnu.to(DEV), eps.to(DEV), K=200, threshold=thr, check_every=2)
    assert_close_rel(lu.cpu().double().numpy(), lu_r.numpy(), TOL, "log_u")
    assert_close_rel(lv.cpu().double().numpy(), lv_r.numpy(), TOL, "log_v")


def _diff(a, b):
    a, b = a.detach().cpu(), b.detach().cpu()
    idx = (a != b).nonzero()[:8].tolist()
    return f"{len((a != b).nonzero())} differ; first {idx}: {[(float(a[tuple(i)]), float(b[tuple(i)])) for i in idx]}"


def test_solve_zero_iterations():
    """K = 0: the initial potentials pass through, with their gradients."""
    from deepfold_amd import sinkhorn_solve

    B, H, N = 1, 2, 32
    C, lmu, lnu, eps, g = _case(B, H, N, seed=8)
    u0 = torch.randn(B, H, N, generator=g, dtype=torch.float32).to(DEV).requires_grad_(True)
    v0 = torch.randn(B, H, N, generator=g, dtype=torch.float32).to(DEV).requires_grad_(True)
    Cg = C.float().to(DEV).requires_grad_(True)
    lu0, lv0 = sinkhorn_solve(Cg, lmu.to(DEV), lnu.to(DEV), eps.to(DEV), K=0, log_u_init=u0, log_v_init=v0)
    assert torch.equal(lu0, u0.detach()), _diff(lu0, u0)
    assert torch.equal(lv0, v0.detach()), _diff(lv0, v0)
    (2 * lu0.sum() + 3 * lv0.sum()).backward()
    assert torch.all(u0.grad == 2) and torch.all(v0.grad == 3)
    assert Cg.grad is None or torch.all(Cg.grad == 0)


@pytest.mark.parametrize("B,H,N,d,with_x,masked", [(1, 2, 40, 16, True, False), (2, 2, 70, 32, True, True),
                                                   (1, 3, 33, 64, False, False)])
def test_transport_forward_backward(B, H, N, d, with_x, masked):
    C, lmu, lnu, eps, g = _case(B, H, N, seed=11 + d)
    lu, lv = dref.sinkhorn_solve(C.double(), lmu.double(), lnu.double(), eps.double(), K=6)
    V = torch.randn(B, H, N, d, generator=g)
    G = torch.randn(B, H, N, d, generator=g)
    x = torch.randn(B, N, 3, generator=g) if with_x else None
    mask = _mask(B, N, [N, N - 23][:B]) if masked else None
    wo = torch.randn(B, N, H * d, generator=g)
    wT = torch.randn(B, H, N, N, generator=g)
    wx = torch.randn(B, H, N, 3, generator=g)

    def fn(ls, tag):
        cw = (lambda t: None if t is None else t.double()) if tag == "ref" else \
            (lambda t: None if t is None else t.float().to(DEV))
        o, Tn, xc = _transport(tag)(ls["V"], ls["G"], ls["lu"], ls["lv"], ls["C"], cw(eps), ls["x"], cw(mask))
        loss = (o * cw(wo)).sum() + (Tn * cw(wT)).sum()
        vals = {"o": o, "T_norm": Tn}
        if xc is not None:
            loss = loss + (xc * cw(wx)).sum()
            vals["x_centroid"] = xc
        return loss, vals

    names = ("V", "G", "lv", "C") + (("x",) if with_x else ())
    out = _grads(fn, {"V": V, "G": G, "lu": lu.float(), "lv": lv.float(), "C": C, "x": x})
    _cmp(out, names)
    # d log_u is a sum of terms that cancel exactly (T_norm does not depend on log_u)
    assert float(out["gpu"][0]["lu"].abs().max()) < 1e-4 * float(out["ref"][0]["C"].abs().max() + 1)


def test_solve_then_transport_masked_pipeline():
    """The reference's use: potentials from sinkhorn_solve feed compute_transport_output."""
    B, H, N, d, K = 2, 2, 56, 16, 8
    C, lmu, lnu, eps, g = _case(B, H, N, seed=21)
    mask = _mask(B, N, [56, 40])
    V = torch.randn(B, H, N, d, generator=g)
    G = torch.randn(B, H, N, d, generator=g)
    x = torch.randn(B, N, 3, generator=g)
    wo = torch.randn(B, N, H * d, generator=g)
    wx = torch.randn(B, H, N, 3, generator=g)

    def fn(ls, tag):
        cw = (lambda t: t.double()) if tag == "ref" else (lambda t: t.float().to(DEV))
        lu, lv = _solve(tag)(ls["C"], ls["mu"], ls["nu"], cw(eps), K=K, mask=cw(mask))
        o, Tn, xc = _transport(tag)(ls["V"], ls["G"], lu, lv, ls["C"], cw(eps), ls["x"], cw(mask))
        return (o * cw(wo)).sum() + (xc * cw(wx)).sum(), {"o": o, "x_centroid": xc}

    out = _grads(fn, {"C": C, "mu": lmu, "nu": lnu, "V": V, "G": G, "x": x})
    _cmp(out, ("C", "mu", "nu", "V", "G", "x"))
    o = out["gpu"][1]["o"].detach().cpu()
    assert torch.all(o[1, 40:] == 0)
