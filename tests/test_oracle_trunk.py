"""Pins oracle/trunk_steps.py (CPU): library routines, closed forms, invariants and
float64 gradchecks."""

import math

import torch
import torch.nn.functional as F

from oracle import trunk_steps as ts

D = torch.float64


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_layer_norm_matches_torch():
    g = _g(1)
    x = torch.randn(3, 7, 64, generator=g, dtype=D) * 3 + 1
    w = torch.randn(64, generator=g, dtype=D)
    b = torch.randn(64, generator=g, dtype=D)
    assert torch.allclose(ts.layer_norm(x, w, b), F.layer_norm(x, (64,), w, b, eps=1e-5), atol=1e-12)


def test_projections_match_library_forms_and_are_unit():
    g = _g(2)
    B, N, C, H = 2, 5, 64, 4
    h = torch.randn(B, N, C, generator=g, dtype=D)
    lw, lb = torch.randn(C, generator=g, dtype=D), torch.randn(C, generator=g, dtype=D)
    wq, wk, wv = (torch.randn(C, C, generator=g, dtype=D) / 8 for _ in range(3))
    q, k, v = ts.sink_projections(h, lw, lb, wq, wk, wv, H)
    hs = F.layer_norm(h, (C,), lw, lb)
    lin = lambda w: F.linear(hs, w).view(B, N, H, C // H).permute(0, 2, 1, 3)
    assert torch.allclose(q, F.normalize(lin(wq), dim=-1), atol=1e-12)
    assert torch.allclose(k, F.normalize(lin(wk), dim=-1), atol=1e-12)
    assert torch.allclose(v, lin(wv), atol=1e-12)
    assert torch.allclose(q.norm(dim=-1), torch.ones(B, H, N, dtype=D), atol=1e-12)
    # a projection that vanishes on a head stays zero (the eps branch), as F.normalize
    wz = wq.clone()
    wz[: C // H] = 0
    qz, _, _ = ts.sink_projections(h, lw, lb, wz, wk, None, H)
    assert torch.all(qz[:, 0] == 0)


def test_coordinate_update_closed_forms():
    g = _g(3)
    B, N, C, H = 2, 6, 64, 4
    h = torch.randn(B, N, C, generator=g, dtype=D)
    x = torch.randn(B, N, 3, generator=g, dtype=D)
    xc = torch.randn(B, H, N, 3, generator=g, dtype=D)
    lw, lb = torch.ones(C, dtype=D), torch.zeros(C, dtype=D)
    zero_w, zero_b = torch.zeros(1, C, dtype=D), torch.zeros(1, dtype=D)
    # gate = 1/2 with zero gate weights; lambda_h = tanh(atanh(c_h)) / H
    c = torch.tensor([0.5, -0.25, 0.75, 0.1], dtype=D)
    out = ts.gated_coordinate_update(h, x, xc, lw, lb, zero_w, zero_b, torch.atanh(c))
    want = x + 0.5 * sum(c[i] / H * (xc[:, i] - x) for i in range(H))
    assert torch.allclose(out, want, atol=1e-12)
    # a masked token does not move
    mask = torch.ones(B, N, dtype=D)
    mask[1, 2:] = 0
    out = ts.gated_coordinate_update(h, x, xc, lw, lb, torch.randn(1, C, generator=g, dtype=D), zero_b,
                                     torch.randn(H, generator=g, dtype=D), mask)
    assert torch.equal(out[1, 2:], x[1, 2:])
    # one head, lambda_raw = atanh(1/2) and gate = sigmoid(b): x moves gate/2 of the way to x_c
    b = torch.tensor([0.7], dtype=D)
    out = ts.gated_coordinate_update(h, x, xc[:, :1], lw, lb, zero_w, b, torch.atanh(torch.tensor([0.5], dtype=D)))
    s = 1 / (1 + math.exp(-0.7))
    assert torch.allclose(out, x + 0.5 * s * (xc[:, 0] - x), atol=1e-12)


def test_gradcheck():
    g = _g(4)
    B, N, C, H = 1, 3, 16, 2
    args = [torch.randn(B, N, C, generator=g, dtype=D), torch.randn(C, generator=g, dtype=D),
            torch.randn(C, generator=g, dtype=D)] + [torch.randn(C, C, generator=g, dtype=D) / 4 for _ in range(3)]
    args = [a.requires_grad_(True) for a in args]
    f = lambda *a: tuple(t for t in ts.sink_projections(*a, H))
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-6)
    cargs = [torch.randn(B, N, C, generator=g, dtype=D), torch.randn(B, N, 3, generator=g, dtype=D),
             torch.randn(B, H, N, 3, generator=g, dtype=D), torch.randn(C, generator=g, dtype=D),
             torch.randn(C, generator=g, dtype=D), torch.randn(1, C, generator=g, dtype=D),
             torch.randn(1, generator=g, dtype=D), torch.randn(H, generator=g, dtype=D)]
    cargs = [a.requires_grad_(True) for a in cargs]
    assert torch.autograd.gradcheck(lambda *a: ts.gated_coordinate_update(*a), cargs, eps=1e-6, atol=1e-6)
