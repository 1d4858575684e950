"""GPU parity of the balanced Sinkhorn transport (balanced_sinkhorn_transport[_dual])
against the float64 CPU oracle (oracle/balanced_transport.py), gradients by
autograd through the oracle's unrolled iterations, as the reference's CPU path.

Relative error = max |gpu - oracle| / max |oracle| per tensor; bar 1e-4 (fp32).
The oracle sees the fp32-rounded inputs upcast to float64.  Cases cover the
reference fixture (tests/test_dual_transport.py: B1 H8 N64 d32, eps 0.5..4,
K = 20), ragged masks with holes, d = 16 and 64, K = 1, r below the 0.1 clamp and
negative r, the forward's stream storage (N = 768) and backward workgroups with
two resident tiles per wave (nr > 8).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_close_rel
from oracle import balanced_transport as bt

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 1e-4


def _case(B, H, N, d, seed, r=10.0, lens=None, holes=()):
    g = torch.Generator().manual_seed(seed)
    Q = F.normalize(torch.randn(B, H, N, d, generator=g), dim=-1)
    K = F.normalize(torch.randn(B, H, N, d, generator=g), dim=-1)
    x = torch.randn(B, N, 3, generator=g) * 4
    V = torch.randn(B, H, N, d, generator=g)
    eps = torch.tensor([0.5, 1.0, 2.0, 4.0])[torch.arange(H) * 4 // H]
    alpha = torch.randn(H, generator=g)
    rh = torch.full((H,), float(r))
    mask = None
    if lens is not None:
        mask = torch.zeros(B, N)
        for b, n in enumerate(lens):
            mask[b, :n] = 1
        for b, i in holes:
            mask[b, i] = 0
    wx = torch.randn(B, H, N, 3, generator=g)
    wh = torch.randn(B, H, N, d, generator=g)
    return dict(Q=Q, K=K, x=x, V=V, eps=eps, alpha=alpha, r=rh), mask, wx, wh


def _run(inp, mask, wx, wh, K_iter, dual, gpu):
    conv = (lambda t: t.float().to(DEV)) if gpu else (lambda t: t.double())
    leaves = {k: conv(v).requires_grad_(k != "eps") for k, v in inp.items() if dual or k != "V"}
    m = None if mask is None else conv(mask)
    if gpu:
        from deepfold_amd import balanced_sinkhorn_transport, balanced_sinkhorn_transport_dual
        fd, fs = balanced_sinkhorn_transport_dual, balanced_sinkhorn_transport
    else:
        fd, fs = bt.balanced_transport_dual, bt.balanced_transport
    L = leaves
    if dual:
        xc, hc = fd(L["Q"], L["K"], L["x"], L["V"], L["eps"], L["alpha"], L["r"], K_iter=K_iter, mask=m)
        loss = (xc * conv(wx)).sum() + (hc * conv(wh)).sum()
        vals = {"x_centroid": xc, "h_centroid": hc}
    else:
        xc = fs(L["Q"], L["K"], L["x"], L["eps"], L["alpha"], L["r"], K_iter=K_iter, mask=m)
        loss = (xc * conv(wx)).sum()
        vals = {"x_centroid": xc}
    loss.backward()
    grads = {k: v.grad for k, v in leaves.items() if k != "eps"}
    return vals, grads


CASES = [
    # B, H, N, d, K, dual, r, lens, holes
    (1, 8, 64, 32, 20, True, 10.0, None, ()),          # reference fixture
    (2, 4, 100, 32, 7, True, 10.0, [100, 61], [(0, 17)]),
    (1, 2, 33, 64, 5, False, 0.05, None, ()),          # r under the clamp: dr = 0
    (2, 3, 48, 16, 1, False, -2.5, [48, 30], ()),      # K = 1, negative r
    (1, 16, 256, 32, 20, True, 10.0, None, ()),        # TokenOTBlock shape (H16 d32 K20)
    (1, 2, 768, 32, 6, True, 10.0, [700], [(0, 3)]),    # forward in stream storage
    (4, 16, 600, 32, 2, True, 4.0, [600, 590, 577, 600], ()),  # nr > 8: two tiles per wave
]


@pytest.mark.parametrize("B,H,N,d,K,dual,r,lens,holes", CASES)
def test_matches_oracle(B, H, N, d, K, dual, r, lens, holes):
    inp, mask, wx, wh = _case(B, H, N, d, seed=N + K + d, r=r, lens=lens, holes=holes)
    print(f"case B{B} H{H} N{N} d{d} K{K} dual={dual}", flush=True)
    vg, gg = _run(inp, mask, wx, wh, K, dual, gpu=True)
    vr, gr = _run(inp, mask, wx, wh, K, dual, gpu=False)
    for k in vr:
        assert_close_rel(vg[k].detach().cpu().double().numpy(), vr[k].detach().numpy(), TOL, k)
    for k in gr:
        want = gr[k].numpy()
        got = gg[k].cpu().double().numpy()
        assert np.isfinite(got).all(), k
        if k == "r" and abs(r) < 0.1:
            assert np.all(got == 0) and np.all(want == 0), "r below the clamp gets no gradient"
            continue
        assert_close_rel(got, want, TOL, f"grad {k}")
    if mask is not None:
        pad = (mask < 0.5)
        for k, v in vg.items():
            assert torch.all(v.detach().cpu()[pad[:, None, :].expand(B, H, N)] == 0), k


def test_reference_fixture_accuracy_and_dual_vs_single():
    """tests/test_dual_transport.py: dual vs CPU reference (1e-3 absolute) and the
    dual's x centroid vs the single transport's (1e-4)."""
    from deepfold_amd import balanced_sinkhorn_transport, balanced_sinkhorn_transport_dual

    inp, _, _, _ = _case(1, 8, 64, 32, seed=0)
    inp["eps"] = torch.tensor([0.5] * 2 + [1.0] * 2 + [2.0] * 2 + [4.0] * 2)
    g = {k: v.to(DEV) for k, v in inp.items()}
    mask = torch.ones(1, 64, device=DEV)
    xd, hd = balanced_sinkhorn_transport_dual(g["Q"], g["K"], g["x"], g["V"], g["eps"], g["alpha"], g["r"],
                                              K_iter=20, mask=mask)
    xs = balanced_sinkhorn_transport(g["Q"], g["K"], g["x"], g["eps"], g["alpha"], g["r"], K_iter=20, mask=mask)
    c = {k: v.double() for k, v in inp.items()}
    xr, hr = bt.sinkhorn_cpu(c["Q"], c["K"], c["x"], c["eps"], c["alpha"], c["r"], mask.cpu().double(), 64, 20,
                             V_h=c["V"])
    assert float((xd.cpu().double() - xr).abs().max()) < 1e-3
    assert float((hd.cpu().double() - hr).abs().max()) < 1e-3
    assert float((xd - xs).abs().max()) < 1e-4


@pytest.mark.parametrize("N", [256, 512])
def test_forward_memory_is_linear(N):
    """tests/test_dual_transport.py::test_dual_memory: the forward allocates well
    under half of one (B,H,N,N) fp32 plan."""
    from deepfold_amd import balanced_sinkhorn_transport_dual

    B, H, d = 1, 16, 32
    inp, _, _, _ = _case(B, H, N, d, seed=N)
    g = {k: v.to(DEV) for k, v in inp.items()}
    mask = torch.ones(B, N, device=DEV)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    before = torch.cuda.max_memory_allocated()
    balanced_sinkhorn_transport_dual(g["Q"], g["K"], g["x"], g["V"], g["eps"], g["alpha"], g["r"], K_iter=20,
                                     mask=mask)
    torch.cuda.synchronize()
    used = torch.cuda.max_memory_allocated() - before
    assert used < 0.5 * B * H * N * N * 4, used


def test_rejects_bad_input():
    from deepfold_amd import balanced_sinkhorn_transport

    inp, _, _, _ = _case(1, 2, 16, 32, seed=1)
    g = {k: v.to(DEV) for k, v in inp.items()}
    with pytest.raises(RuntimeError, match="K_iter"):
        balanced_sinkhorn_transport(g["Q"], g["K"], g["x"], g["eps"], g["alpha"], g["r"], K_iter=0)
    with pytest.raises(RuntimeError, match="GPU"):
        balanced_sinkhorn_transport(g["Q"].cpu(), g["K"], g["x"], g["eps"], g["alpha"], g["r"])
