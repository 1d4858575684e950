"""Write golden vectors for the reference-mode IFT backward of flash_sinkhorn_attn.

Run ONLY in the survey/build container (the reference never travels to the GPU box):

    python tests/golden/make_golden.py /root/reference/src

``FlashSinkhornAttn.backward`` (src/deepfold/model/kernels/flash_sinkhorn_attn.py:246-667)
is the one function on the path that no reference test, closed form or invariant
pins (its sign convention and mask handling are only defined by its code), so its
input/output vectors are taken from the reference itself.  The forward outputs of
the same calls are stored alongside.  On CPU tensors the reference's Triton launch
raises and its bare ``except`` runs the dense fallback forward
(flash_sinkhorn_attn.py:144-207), which is what these vectors capture.

Each case writes ``tests/golden/flash_sinkhorn_<name>.npz`` with the float32
inputs (Q, K, V, G, x_res, pos_weight, pos_bins, eps, w_dist, log_mu, log_nu,
grad_o, grad_xc, and the scalars K_iter, lam, r_0) and outputs (o_flat, x_centroid,
log_u, log_v, and grad_<name> for every differentiable input).
"""

import os
import sys

import numpy as np
import torch

CASES = [
    # name, B, H, N, d, K_iter, eps list (len H), with_pos_geo, seed
    ("small_full", 1, 4, 16, 8, 3, [0.5, 1.0, 2.0, 4.0], True, 11),
    ("batch2_full", 2, 2, 24, 16, 5, [0.5, 1.0], True, 12),
    ("cfg1_like", 1, 2, 64, 32, 20, [1.0, 1.0], False, 13),
    ("converged", 1, 2, 48, 16, 50, [0.5, 0.5], False, 14),
    ("ragged_tile", 1, 2, 70, 8, 7, [0.25, 2.0], True, 15),
]


def make_inputs(B, H, N, d, eps_list, with_pos_geo, seed):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, N, d, generator=g) / d ** 0.5
    K = torch.randn(B, H, N, d, generator=g) / d ** 0.5
    V = torch.randn(B, H, N, d, generator=g)
    G = torch.randn(B, H, N, d, generator=g)
    if with_pos_geo:
        x_res = torch.randn(B, N, 3, generator=g) * 3.0
        pos_weight = torch.randn(H, 68, generator=g) * 0.5
        pos_bins = torch.randint(0, 68, (B, N, N), generator=g, dtype=torch.int32)
        w_dist = torch.rand(H, generator=g)
    else:
        x_res = torch.zeros(B, N, 3)
        pos_weight = torch.zeros(H, 68)
        pos_bins = torch.zeros(B, N, N, dtype=torch.int32)
        w_dist = torch.zeros(H)
    eps = torch.tensor(eps_list, dtype=torch.float32)
    log_mu = torch.log_softmax(torch.randn(B, H, N, generator=g), dim=-1)
    log_nu = torch.log_softmax(torch.randn(B, H, N, generator=g), dim=-1)
    grad_o = torch.randn(B, N, H * d, generator=g)
    grad_xc = torch.randn(B, H, N, 3, generator=g) * (1.0 if with_pos_geo else 0.0)
    return dict(Q=Q, K=K, V=V, G=G, x_res=x_res, pos_weight=pos_weight, pos_bins=pos_bins,
                eps=eps, w_dist=w_dist, log_mu=log_mu, log_nu=log_nu,
                grad_o=grad_o, grad_xc=grad_xc)


def main(ref_src):
    sys.path.insert(0, ref_src)
    from deepfold.model.kernels.flash_sinkhorn_attn import FlashSinkhornAttn  # noqa: E402

    out_dir = os.path.dirname(os.path.abspath(__file__))
    for name, B, H, N, d, K_iter, eps_list, with_pg, seed in CASES:
        inp = make_inputs(B, H, N, d, eps_list, with_pg, seed)
        lam, r_0 = 1.0, 10.0
        leaves = {k: inp[k].clone().requires_grad_(True)
                  for k in ("Q", "K", "V", "G", "x_res", "pos_weight", "w_dist", "log_mu", "log_nu")}
        o_flat, xc, lu, lv = FlashSinkhornAttn.apply(
            leaves["Q"], leaves["K"], leaves["V"], leaves["G"], leaves["x_res"],
            leaves["pos_weight"], inp["pos_bins"], inp["eps"], leaves["w_dist"],
            leaves["log_mu"], leaves["log_nu"], K_iter, lam, r_0, None, None, None)
        loss = (o_flat * inp["grad_o"]).sum() + (xc * inp["grad_xc"]).sum()
        loss.backward()
        rec = {k: v.detach().numpy() for k, v in inp.items()}
        rec.update(K_iter=np.int64(K_iter), lam=np.float64(lam), r_0=np.float64(r_0),
                   o_flat=o_flat.detach().numpy(), x_centroid=xc.detach().numpy(),
                   log_u=lu.detach().numpy(), log_v=lv.detach().numpy())
        for k, t in leaves.items():
            rec["grad_" + k] = t.grad.detach().numpy()
        path = os.path.join(out_dir, f"flash_sinkhorn_{name}.npz")
        np.savez_compressed(path, **rec)
        print(f"wrote {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
