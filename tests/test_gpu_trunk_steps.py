"""GPU parity of the TokenOTBlock steps either side of the balanced transport
(deepfold_amd.trunk_steps) against float64 CPU autograd through oracle/trunk_steps.py.

Relative error = max |gpu - oracle| / max |oracle| per tensor; bars 1e-4 (fp32
inputs) and 2e-2 (bf16 inputs, with the oracle fed the bf16-rounded h and weights).
Cases: TokenOTBlock's width (C = 512, H = 16), head dims 16 / 32 / 64, token counts
that are not multiples of the 64-token block, no V projection, unbatched input,
masks; the chained step (projections -> balanced transport -> output projection ->
coordinate update) against the chained oracle.
"""

import pytest
import torch

from conftest import assert_close_rel
from oracle import trunk_steps as ts

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _proj_inputs(B, N, C, seed, with_v=True):
    g = torch.Generator().manual_seed(seed)
    t = dict(h=torch.randn(B, N, C, generator=g) * 2 + 0.5, lw=1 + 0.2 * torch.randn(C, generator=g),
             lb=0.1 * torch.randn(C, generator=g), wq=torch.randn(C, C, generator=g) / C ** 0.5,
             wk=torch.randn(C, C, generator=g) / C ** 0.5)
    if with_v:
        t["wv"] = torch.randn(C, C, generator=g) / C ** 0.5
    return t


def _proj_grads_weights(B, N, C, H, seed):
    g = torch.Generator().manual_seed(seed + 1)
    return [torch.randn(B, H, N, C // H, generator=g) for _ in range(3)]


PROJ_CASES = [
    # B, N, C, H, dtype, tol, with_v
    (2, 100, 512, 16, torch.float32, 1e-4, True),   # TokenOTBlock width, ragged token block
    (1, 64, 128, 4, torch.float32, 1e-4, True),     # head dim 32, one block
    (1, 50, 256, 16, torch.float32, 1e-4, False),   # head dim 16, no V projection
    (2, 37, 256, 4, torch.float32, 1e-4, True),     # head dim 64
    (2, 100, 512, 16, torch.bfloat16, 2e-2, True),
]


@pytest.mark.parametrize("B,N,C,H,dtype,tol,with_v", PROJ_CASES)
def test_sink_projections_match_oracle(B, N, C, H, dtype, tol, with_v):
    from deepfold_amd import sink_projections

    print(f"case B{B} N{N} C{C} H{H} {dtype} v={with_v}", flush=True)
    t = _proj_inputs(B, N, C, seed=N + C + H, with_v=with_v)
    wts = _proj_grads_weights(B, N, C, H, seed=N)
    if dtype == torch.bfloat16:  # the oracle sees the rounded operands of the bf16 products
        for k in ("h", "wq", "wk", "wv"):
            if k in t:
                t[k] = t[k].to(torch.bfloat16).float()
    ref = {k: v.double().requires_grad_(True) for k, v in t.items()}
    qr, kr, vr = ts.sink_projections(ref["h"], ref["lw"], ref["lb"], ref["wq"], ref["wk"], ref.get("wv"), H)
    loss = (qr * wts[0].double()).sum() + (kr * wts[1].double()).sum()
    if with_v:
        loss = loss + (vr * wts[2].double()).sum()
    loss.backward()

    gpu = {k: (v.to(DEV).to(dtype) if k in ("h", "wq", "wk", "wv") else v.to(DEV)).detach().requires_grad_(True)
           for k, v in t.items()}
    q, k, v = sink_projections(gpu["h"], gpu["lw"], gpu["lb"], gpu["wq"], gpu["wk"], gpu.get("wv"), H)
    assert q.shape == (B, H, N, C // H) and q.dtype == torch.float32
    gl = (q * wts[0].to(DEV)).sum() + (k * wts[1].to(DEV)).sum()
    if with_v:
        gl = gl + (v * wts[2].to(DEV)).sum()
    gl.backward()
    for name, got, want in (("q_s", q, qr), ("k_s", k, kr)) + ((("v_s", v, vr),) if with_v else ()):
        assert_close_rel(got.detach().cpu().double().numpy(), want.detach().numpy(), tol, name)
    for name in ref:
        assert_close_rel(gpu[name].grad.float().cpu().double().numpy(), ref[name].grad.numpy(), tol, f"grad {name}")


def test_sink_projections_unbatched_and_views():
    """(N, C) input gives (1, H, N, d) views of one (N, C) buffer: the layout the
    transport reads in place."""
    from deepfold_amd import sink_projections

    t = _proj_inputs(1, 40, 128, seed=3)
    g = {k: v.to(DEV) for k, v in t.items()}
    q, k, v = sink_projections(g["h"][0], g["lw"], g["lb"], g["wq"], g["wk"], g["wv"], 4)
    qb, kb, vb = sink_projections(g["h"], g["lw"], g["lb"], g["wq"], g["wk"], g["wv"], 4)
    assert q.shape == (1, 4, 40, 32) and q.stride() == (40 * 128, 32, 128, 1)
    assert torch.equal(q, qb) and torch.equal(k, kb) and torch.equal(v, vb)


def _coord_inputs(B, N, C, H, seed):
    g = torch.Generator().manual_seed(seed)
    return dict(h=torch.randn(B, N, C, generator=g), x=torch.randn(B, N, 3, generator=g) * 3,
                xc=torch.randn(B, H, N, 3, generator=g) * 3, lw=1 + 0.2 * torch.randn(C, generator=g),
                lb=0.1 * torch.randn(C, generator=g), wg=torch.randn(1, C, generator=g) / C ** 0.5,
                bg=torch.randn(1, generator=g), lr=torch.randn(H, generator=g))


COORD_CASES = [
    # B, N, C, H, dtype, tol, lens
    (2, 70, 512, 16, torch.float32, 1e-4, [70, 41]),
    (1, 33, 128, 4, torch.float32, 1e-4, None),
    (2, 300, 256, 8, torch.float32, 1e-4, [300, 123]),  # more tokens than the 256 in flight
    (2, 70, 512, 16, torch.bfloat16, 2e-2, [70, 41]),
]


@pytest.mark.parametrize("B,N,C,H,dtype,tol,lens", COORD_CASES)
def test_coordinate_update_matches_oracle(B, N, C, H, dtype, tol, lens):
    from deepfold_amd import gated_coordinate_update

    print(f"case B{B} N{N} C{C} H{H} {dtype}", flush=True)
    t = _coord_inputs(B, N, C, H, seed=N + C)
    if dtype == torch.bfloat16:
        t["h"] = t["h"].to(torch.bfloat16).float()
    mask = None
    if lens is not None:
        mask = torch.zeros(B, N)
        for b, n in enumerate(lens):
            mask[b, :n] = 1
    w = torch.randn(B, N, 3, generator=torch.Generator().manual_seed(7))
    ref = {k: v.double().requires_grad_(True) for k, v in t.items()}
    out_r = ts.gated_coordinate_update(ref["h"], ref["x"], ref["xc"], ref["lw"], ref["lb"], ref["wg"], ref["bg"],
                                       ref["lr"], None if mask is None else mask.double())
    (out_r * w.double()).sum().backward()
    gpu = {k: (v.to(DEV).to(dtype) if k == "h" else v.to(DEV)).detach().requires_grad_(True) for k, v in t.items()}
    out = gated_coordinate_update(gpu["h"], gpu["x"], gpu["xc"], gpu["lw"], gpu["lb"], gpu["wg"], gpu["bg"],
                                  gpu["lr"], None if mask is None else mask.to(DEV))
    (out * w.to(DEV)).sum().backward()
    assert_close_rel(out.detach().cpu().double().numpy(), out_r.detach().numpy(), tol, "x_out")
    if mask is not None:
        pad = mask < 0.5
        assert torch.equal(out.detach().cpu()[pad], t["x"][pad])
    for name in ref:
        assert_close_rel(gpu[name].grad.float().cpu().double().numpy(), ref[name].grad.numpy(), tol, f"grad {name}")


class _Block(torch.nn.Module):
    """The parameters TokenOTBlock holds for its transport steps (trunk_block.py:65-96)."""

    def __init__(self, C, H, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.n_heads = H
        self.feature_transport = True
        self.ln_sink = torch.nn.LayerNorm(C)
        self.ln_gate = torch.nn.LayerNorm(C)
        self.w_q_sink = torch.nn.Linear(C, C, bias=False)
        self.w_k_sink = torch.nn.Linear(C, C, bias=False)
        self.w_v_sink = torch.nn.Linear(C, C, bias=False)
        self.w_o_sink = torch.nn.Linear(C, C, bias=False)
        self.w_gate = torch.nn.Linear(C, 1, bias=True)
        with torch.no_grad():
            for ln in (self.ln_sink, self.ln_gate):
                ln.weight.copy_(1 + 0.2 * torch.randn(C, generator=g))
                ln.bias.copy_(0.1 * torch.randn(C, generator=g))
            for lin in (self.w_q_sink, self.w_k_sink, self.w_v_sink, self.w_o_sink, self.w_gate):
                lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) / C ** 0.5)
            self.w_gate.bias.copy_(torch.randn(1, generator=g))
        self.alpha_h = torch.nn.Parameter(torch.randn(H, generator=g))
        self.r_h = torch.nn.Parameter(torch.full((H,), 10.0))
        self.lambda_h_raw = torch.nn.Parameter(torch.randn(H, generator=g))
        nr = H // 4
        self.register_buffer("eps", torch.tensor([0.5] * nr + [1.0] * nr + [2.0] * nr + [4.0] * nr))


def test_transport_step_matches_chained_oracle():
    from deepfold_amd import token_ot_transport_step

    B, N, C, H, K = 2, 48, 128, 4, 6
    blk = _Block(C, H, seed=11)
    g = torch.Generator().manual_seed(12)
    h = torch.randn(B, N, C, generator=g)
    x = torch.randn(B, N, 3, generator=g) * 4
    mask = torch.ones(B, N)
    mask[1, 30:] = 0
    wh = torch.randn(B, N, C, generator=g)
    wx = torch.randn(B, N, 3, generator=g)

    P = {"ln_sink_w": blk.ln_sink.weight, "ln_sink_b": blk.ln_sink.bias, "w_q": blk.w_q_sink.weight,
         "w_k": blk.w_k_sink.weight, "w_v": blk.w_v_sink.weight, "w_o": blk.w_o_sink.weight, "eps": blk.eps,
         "alpha_h": blk.alpha_h, "r_h": blk.r_h, "ln_gate_w": blk.ln_gate.weight, "ln_gate_b": blk.ln_gate.bias,
         "w_gate": blk.w_gate.weight, "b_gate": blk.w_gate.bias, "lambda_raw": blk.lambda_h_raw}
    R = {k: v.detach().double().requires_grad_(k != "eps") for k, v in P.items()}
    hr = h.double().requires_grad_(True)
    xr = x.double().requires_grad_(True)
    ho, xo = ts.transport_step(R, hr, xr, mask.double(), H, K_iter=K)
    ((ho * wh.double()).sum() + (xo * wx.double()).sum()).backward()

    blk = blk.to(DEV)
    hg = h.to(DEV).requires_grad_(True)
    xg = x.to(DEV).requires_grad_(True)
    hg2, xg2 = token_ot_transport_step(blk, hg, xg, mask.to(DEV), K_iter=K)
    ((hg2 * wh.to(DEV)).sum() + (xg2 * wx.to(DEV)).sum()).backward()
    assert_close_rel(hg2.detach().cpu().double().numpy(), ho.detach().numpy(), 1e-4, "h")
    assert_close_rel(xg2.detach().cpu().double().numpy(), xo.detach().numpy(), 1e-4, "x_res")
    assert_close_rel(hg.grad.cpu().double().numpy(), hr.grad.numpy(), 1e-4, "grad h")
    assert_close_rel(xg.grad.cpu().double().numpy(), xr.grad.numpy(), 1e-4, "grad x_res")
    mods = {"ln_sink_w": blk.ln_sink.weight, "w_q": blk.w_q_sink.weight, "w_k": blk.w_k_sink.weight,
            "w_v": blk.w_v_sink.weight, "w_o": blk.w_o_sink.weight, "alpha_h": blk.alpha_h, "r_h": blk.r_h,
            "ln_gate_w": blk.ln_gate.weight, "w_gate": blk.w_gate.weight, "lambda_raw": blk.lambda_h_raw}
    for k, p in mods.items():
        assert_close_rel(p.grad.cpu().double().numpy(), R[k].grad.numpy(), 1e-4, f"grad {k}")
