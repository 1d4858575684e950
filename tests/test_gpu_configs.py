"""GPU parity at the BASELINE configurations as stated, and at the resident
multi-tile layouts the headline workload runs in.

* B1 H4 N256 d32 fp32, uniform marginals -log 256, V / sqrt(d),
  eps 1.0, K 20, no mask, forward only (flash_sinkhorn_attn.py:144-218).
* configs[1] (the headline, the bench workload exactly as bench.py builds and
  runs it): B2 H8 N768 d32 bf16, seed 1002 -> n_b = [501, 759], eps 0.5, K 50,
  20 CG steps, then the same with the reference fixed-point solver
  (flash_sinkhorn_attn.py:246-667).  At B*H = 16 each (b,h) is served by 16
  workgroups, so a member owns 2 (n = 501) or 3 (n = 759) resident 16-row
  tiles: the forward's multi-tile sweeps and the backward's split heavy passes
  (8 / n_tiles waves per tile) are the code under test.
* fp32 and bf16 resident cases with 2, 3 and 8 tiles per member (B*H = 64 ->
  4 workgroups per (b,h)), held to 1e-4 in fp32.
* configs[2] / configs[3] at full size: flash diffusion attention B1 H16 N1024
  d24 with dense pair bias and gate; atom-window attention over 8192 atoms
  with a per-window bias; token-to-atom 8192 x 341 and atom-to-token 341 x 8192.

Padded batches are compared with each sample evaluated on its unpadded slice
(oracle.sinkhorn.backward_masked).  Normwise relative error bars: 1e-4 (fp32
inputs), 2e-2 (bf16 inputs), on outputs, potentials and every gradient.
"""

import math

import numpy as np
import pytest
import torch

from conftest import assert_close_rel, max_rel_err
from oracle import attention as aref
from oracle import sinkhorn as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
FWD_NAMES = ("o_flat", "x_centroid", "log_u", "log_v")
GRAD_NAMES = ("Q", "K", "V", "G", "log_mu", "log_nu")


def members_per_head(B, H, N):
    """Workgroups serving one (b,h): the C library's group size rule."""
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    G = max(1, cus // (8 * ((B * H + 7) // 8)))
    return min(G, (N + 15) // 16)


def tiles_per_member(n, G):
    tiles = (n + 15) // 16
    return sorted({tiles * (m + 1) // G - tiles * m // G for m in range(G)})


def run_layer(t, K_iter, *, grads=True, **kw):
    """One forward (+ backward with upstream t['dO']) through the public op, as
    bench.py's step does: no bins, w_dist None, gradients of Q, K, V, G, log mu, log nu."""
    from deepfold_amd import flash_sinkhorn_attn

    leaves = {k: t[k].detach().clone().requires_grad_(grads) for k in GRAD_NAMES}
    o, xc, lu, lv = flash_sinkhorn_attn(leaves["Q"], leaves["K"], leaves["V"], leaves["G"], t["x_res"],
                                        t["pos_weight"], None, t["eps"], None, leaves["log_mu"],
                                        leaves["log_nu"], K_iter=K_iter, mask=t.get("mask"), **kw)
    if grads:
        o.backward(t["dO"])
    torch.cuda.synchronize()
    out = {n: v.detach().float().cpu().numpy() for n, v in zip(FWD_NAMES, (o, xc, lu, lv))}
    g = {k: leaves[k].grad.float().cpu().numpy() for k in GRAD_NAMES} if grads else None
    return out, g


def oracle_fwd_inputs(cpu, K_iter):
    f64 = lambda x: x.to(torch.float64).numpy()
    return dict(Q=f64(cpu["Q"]), K=f64(cpu["K"]), V=f64(cpu["V"]), G=f64(cpu["G"]), x_res=f64(cpu["x_res"]),
                pos_weight=f64(cpu["pos_weight"]), pos_bins=None, eps=f64(cpu["eps"]), w_dist=f64(cpu["w_dist"]),
                log_mu=f64(cpu["log_mu"]), log_nu=f64(cpu["log_nu"]), K_iter=K_iter, lam=1.0, r_0=10.0,
                mask=None if cpu.get("mask") is None else cpu["mask"].numpy())


def check_layer(got, ggot, want, gwant, tol, label, lengths=None):
    for k in FWD_NAMES:
        assert_close_rel(got[k], want[k], tol, f"{label}:{k}")
    if lengths is not None:  # padded positions exactly zero
        for b, n in enumerate(lengths):
            assert np.all(got["o_flat"][b, n:] == 0) and np.all(got["log_u"][b, :, n:] == 0)
    if gwant is None:
        return
    for k in GRAD_NAMES:
        assert_close_rel(ggot[k], gwant[k], tol, f"{label}:d{k}")
        if lengths is not None:
            for b, n in enumerate(lengths):
                assert np.all(ggot[k][b, :, n:] == 0), f"{label}:d{k} nonzero on padding"


# ---------------------------------------------------------------------------
# configs[0]
def test_config0_forward():
    B, H, N, d, K = 1, 4, 256, 32, 20
    g = torch.Generator().manual_seed(1001)
    cpu = dict(Q=torch.randn(B, H, N, d, generator=g) / math.sqrt(d),
               K=torch.randn(B, H, N, d, generator=g) / math.sqrt(d),
               V=torch.randn(B, H, N, d, generator=g) / math.sqrt(d),
               G=torch.zeros(B, H, N, d), x_res=torch.zeros(B, N, 3), pos_weight=torch.zeros(H, 68),
               eps=torch.ones(H), w_dist=torch.zeros(H),
               log_mu=torch.full((B, H, N), -math.log(N)), log_nu=torch.full((B, H, N), -math.log(N)))
    t = {k: v.to(DEV) for k, v in cpu.items()}
    got, _ = run_layer(t, K, grads=False)
    want = ref.forward(**{k: v for k, v in oracle_fwd_inputs(cpu, K).items() if k != "mask"})
    check_layer(got, None, want, None, 1e-4, "config0")


# ---------------------------------------------------------------------------
# configs[1], the headline: exactly the bench workload
def _headline():
    import bench

    cfg = bench.SINKHORN["cfg2"]
    cpu, t = bench.make_workload(cfg, DEV)
    return cfg, cpu, t


@pytest.mark.parametrize("solver", ["cg", "fixed_point"])
def test_headline_config1(solver):
    cfg, cpu, t = _headline()
    assert cpu["lengths"] == [501, 759]
    G = members_per_head(cfg["B"], cfg["H"], cfg["N"])
    # the layout the bench times: 2 and 3 resident tiles per member
    assert tiles_per_member(501, G) == [2] and tiles_per_member(759, G) == [3], (G, cpu["lengths"])
    iters = cfg["n_cg"] if solver == "cg" else cfg["K_iter"]
    got, ggot = run_layer(t, cfg["K_iter"], ift_solver=solver, ift_iters=iters)
    fo, gr = ref.backward_masked(oracle_fwd_inputs(cpu, cfg["K_iter"]), cpu["dO"].numpy(), None,
                                 solver=solver, n_cg=cfg["n_cg"], K_back=cfg["K_iter"])
    check_layer(got, ggot, fo, gr, 2e-2, f"config1-{solver}", cpu["lengths"])


# ---------------------------------------------------------------------------
# resident layouts with several tiles per member
def _ragged_case(B, H, N, d, lengths, seed, dtype, eps):
    g = torch.Generator().manual_seed(seed)
    cpu = dict(Q=(torch.randn(B, H, N, d, generator=g) / math.sqrt(d)).to(dtype),
               K=(torch.randn(B, H, N, d, generator=g) / math.sqrt(d)).to(dtype),
               V=torch.randn(B, H, N, d, generator=g).to(dtype),
               G=torch.randn(B, H, N, d, generator=g).to(dtype),
               x_res=torch.zeros(B, N, 3), pos_weight=torch.zeros(H, 68),
               eps=torch.tensor(eps, dtype=torch.float32), w_dist=torch.zeros(H))
    mask = torch.zeros(B, N)
    lmu, lnu = torch.zeros(B, H, N), torch.zeros(B, H, N)
    for b, n in enumerate(lengths):
        mask[b, :n] = 1
        lmu[b, :, :n] = torch.log_softmax(torch.randn(H, n, generator=g), -1)
        lnu[b, :, :n] = torch.log_softmax(torch.randn(H, n, generator=g), -1)
    cpu.update(mask=mask, log_mu=lmu, log_nu=lnu,
               dO=(torch.randn(B, N, H * d, generator=g).to(dtype).float() * mask[:, :, None]))
    return cpu


@pytest.mark.parametrize("dtype,tol,N,lengths,expect,solver", [
    # B*H = 64 -> 4 members per head: 3, 2-3, 3 and 2 tiles per member
    (torch.float32, 1e-4, 192, [192, 161, 177, 128], {2, 3}, "cg"),
    (torch.float32, 1e-4, 192, [192, 161, 177, 128], {2, 3}, "fixed_point"),
    (torch.bfloat16, 2e-2, 192, [192, 161, 177, 128], {2, 3}, "cg"),
    # 8 tiles per member (one wave per tile in the split passes)
    (torch.bfloat16, 2e-2, 512, [512, 497, 400, 330], {6, 7, 8}, "cg"),
    # 9-10 tiles per member: the heavy passes give waves whole tiles, the forward's sweep
    # runs resident chunks of 4 + 4 + 1-2 tiles
    (torch.bfloat16, 2e-2, 640, [640, 600, 560, 530], {9, 10}, "cg"),
])
def test_resident_multi_tile(dtype, tol, N, lengths, expect, solver):
    B, H, d, K = 4, 16, 32, 12
    G = members_per_head(B, H, N)
    seen = set()
    for n in lengths:
        seen.update(tiles_per_member(n, G))
    assert expect <= seen, (G, seen)
    eps = [0.5, 1.0, 0.25, 2.0] * 4
    cpu = _ragged_case(B, H, N, d, lengths, seed=77 + N, dtype=dtype, eps=eps)
    t = {k: v.to(DEV) for k, v in cpu.items()}
    iters = 16 if solver == "cg" else K
    got, ggot = run_layer(t, K, ift_solver=solver, ift_iters=iters, storage="resident")
    fo, gr = ref.backward_masked(oracle_fwd_inputs(cpu, K), cpu["dO"].numpy(), None, solver=solver,
                                 n_cg=iters, K_back=K)
    check_layer(got, ggot, fo, gr, tol, f"resident-{dtype}-{N}-{solver}", lengths)


# ---------------------------------------------------------------------------
# configs[2] and configs[3] at full size
def _attn_run(fn, tensors, grad_out, wrt, **kw):
    leaves = {k: (None if v is None else (v.to(DEV).requires_grad_(True) if k in wrt else v.to(DEV)))
              for k, v in tensors.items()}
    out = fn(**leaves, **kw)
    out.backward(grad_out.to(DEV).to(out.dtype))
    torch.cuda.synchronize()
    return out.detach().float().cpu(), {k: leaves[k].grad.float().cpu() for k in wrt}


def _attn_check(label, out, g, o_ref, g_ref, wrt, tol=2e-2):
    err = max_rel_err(out.numpy(), o_ref.numpy())
    assert err <= tol, f"{label}: O rel err {err:.3e}"
    for k in wrt:
        err = max_rel_err(g[k].numpy(), g_ref[k].numpy())
        assert err <= tol, f"{label}: d{k} rel err {err:.3e}"


def _bf16(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def test_config2_diffusion_dense_bias_gate():
    from deepfold_amd import flash_diffusion_attn

    B, H, N, D = 1, 16, 1024, 24
    gen = torch.Generator().manual_seed(1003)
    Q, K, V = (_bf16(B, H, N, D, gen=gen, scale=D ** -0.5) for _ in range(3))
    bias = _bf16(B, H, N, N, gen=gen)
    G = _bf16(B, H, N, D, gen=gen)
    go = _bf16(B, H, N, D, gen=gen)
    inp = dict(Q=Q, K=K, V=V, pos_weight=None, pos_bins=None, pair_bias=bias, gate=G)
    wrt = ("Q", "K", "V", "pair_bias", "gate")
    out, g = _attn_run(flash_diffusion_attn, inp, go, wrt)
    o_ref, g_ref = aref.grads(aref.diffusion_attn, {k: (None if v is None else v.double()) for k, v in inp.items()},
                              go.double(), wrt)
    _attn_check("config2", out, g, o_ref, g_ref, wrt)


def test_config3_atom_window_with_bias():
    from deepfold_amd import flash_atom_attn

    B, H, M, D = 1, 4, 8192, 32
    gen = torch.Generator().manual_seed(1004)
    Q, K, V = (_bf16(B, H, M, D, gen=gen, scale=D ** -0.5) for _ in range(3))
    wb = _bf16(M // 32, H, 32, 128, gen=gen)
    go = _bf16(B, H, M, D, gen=gen)
    inp = dict(Q=Q, K=K, V=V, mask=None, window_bias=wb)
    wrt = ("Q", "K", "V", "window_bias")
    out, g = _attn_run(flash_atom_attn, inp, go, wrt)
    o_ref, g_ref = aref.grads(aref.atom_attn, {k: (None if v is None else v.double()) for k, v in inp.items()},
                              go.double(), wrt)
    _attn_check("config3-window", out, g, o_ref, g_ref, wrt)


def test_config3_token_to_atom():
    from deepfold_amd import token_to_atom_attn

    B, H, M, N, D = 1, 4, 8192, 341, 32
    gen = torch.Generator().manual_seed(1005)
    Q = _bf16(B, H, M, D, gen=gen, scale=D ** -0.5)
    K, V = _bf16(B, H, N, D, gen=gen, scale=D ** -0.5), _bf16(B, H, N, D, gen=gen, scale=D ** -0.5)
    go = _bf16(B, H, M, D, gen=gen)
    inp = dict(Q=Q, K=K, V=V, atom_mask=None, token_mask=None)
    wrt = ("Q", "K", "V")
    out, g = _attn_run(token_to_atom_attn, inp, go, wrt)
    o_ref, g_ref = aref.grads(aref.token_to_atom, {k: (None if v is None else v.double()) for k, v in inp.items()},
                              go.double(), wrt)
    _attn_check("config3-t2a", out, g, o_ref, g_ref, wrt)


def test_config3_atom_to_token():
    from deepfold_amd import atom_to_token_attn

    B, H, N, D = 1, 4, 341, 32
    counts = torch.full((B, N), 24, dtype=torch.int32)
    counts[0, -1] = 32  # 341 * 24 + 8 = 8192 atoms
    starts = (torch.cumsum(counts, 1) - counts).int()
    M = int(counts.sum())
    assert M == 8192
    gen = torch.Generator().manual_seed(1006)
    Q = _bf16(B, H, N, D, gen=gen, scale=D ** -0.5)
    K, V = _bf16(B, H, M, D, gen=gen, scale=D ** -0.5), _bf16(B, H, M, D, gen=gen, scale=D ** -0.5)
    go = _bf16(B, H, N, D, gen=gen)
    inp = dict(Q=Q, K=K, V=V, token_atom_starts=starts, token_atom_counts=counts, token_mask=None)
    wrt = ("Q", "K", "V")
    out, g = _attn_run(atom_to_token_attn, inp, go, wrt)
    ref_inp = dict(Q=Q.double(), K=K.double(), V=V.double(), starts=starts, counts=counts, token_mask=None)
    o_ref, g_ref = aref.grads(aref.atom_to_token, ref_inp, go.double(), wrt)
    _attn_check("config3-a2t", out, g, o_ref, g_ref, wrt)


# ---------------------------------------------------------------------------
# register storage (logits held in registers, 2-D member blocks) at the headline
# layout and in fp32, neutral cost (AUTO routes only biased costs there)
@pytest.mark.parametrize("solver", ["cg", "fixed_point"])
def test_headline_config1_register_storage(solver):
    cfg, cpu, t = _headline()
    iters = cfg["n_cg"] if solver == "cg" else cfg["K_iter"]
    got, ggot = run_layer(t, cfg["K_iter"], ift_solver=solver, ift_iters=iters, storage="register")
    fo, gr = ref.backward_masked(oracle_fwd_inputs(cpu, cfg["K_iter"]), cpu["dO"].numpy(), None,
                                 solver=solver, n_cg=cfg["n_cg"], K_back=cfg["K_iter"])
    check_layer(got, ggot, fo, gr, 2e-2, f"config1-register-{solver}", cpu["lengths"])


@pytest.mark.parametrize("dtype,tol,N,lengths", [
    (torch.float32, 1e-4, 192, [192, 161]),
    (torch.bfloat16, 2e-2, 512, [497, 330]),
    (torch.float32, 1e-4, 448, [448, 400]),
])
def test_register_storage_multi_head(dtype, tol, N, lengths):
    B, H, d, K = 2, 8, 32, 12
    eps = [0.5, 1.0, 0.25, 2.0] * 2
    cpu = _ragged_case(B, H, N, d, lengths, seed=91 + N, dtype=dtype, eps=eps)
    t = {k: v.to(DEV) for k, v in cpu.items()}
    got, ggot = run_layer(t, K, ift_solver="cg", ift_iters=16, storage="register")
    fo, gr = ref.backward_masked(oracle_fwd_inputs(cpu, K), cpu["dO"].numpy(), None, solver="cg", n_cg=16, K_back=K)
    check_layer(got, ggot, fo, gr, tol, f"register-{dtype}-{N}", lengths)
