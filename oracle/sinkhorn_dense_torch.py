"""Dense torch restatement of the flash-Sinkhorn oracle, for checks at full size.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports it; only
``tests/`` use it, as a checker.

The numpy oracle (``oracle/sinkhorn.py``) runs one (b, h) at a time in float64
and needs minutes at BASELINE configs[4] (B=1, H=16, N=4096).  This module states
the same algorithm with batched torch tensors, so a GPU test can evaluate it
at that size in fp32 in under a second.  It covers the content-only cost
(C = -Q K^T / sqrt(d): no position bins, no geometry, no mask), which is what
that configuration uses; the other cost terms are checked against the numpy
oracle at small sizes.

* ``forward``     -- flash_sinkhorn_attn.py:144-218 (== oracle.sinkhorn.forward)
* ``backward``    -- flash_sinkhorn_attn.py:246-667 with the IFT system solved either
                     by the reference's Gauss-Seidel sweeps (solver="fixed_point",
                     :471-542; == oracle.sinkhorn.backward_reference) or by CG on its
                     symmetric form (solver="cg"; == backward_reference with
                     solver="cg"); ``mode="analytic"`` flips the signs as
                     oracle.sinkhorn.backward_analytic does.  ``backward_cg`` is the
                     CG form.

bench.py's CPU baseline times ``forward`` + ``backward(solver="fixed_point")``
(the reference CPU fallback's algorithm) in float32 on the host cores.

Pinned by tests/test_oracle_sinkhorn_dense.py: equal to the numpy oracle in
float64 on CPU (both modes, several shapes, general marginals).
"""

from __future__ import annotations

import math

import torch


def _logits(Q, K, eps):
    """L = -C / eps = (Q K^T) / (sqrt(d) eps), shape (B, H, N, N)."""
    d = Q.shape[-1]
    return torch.matmul(Q, K.transpose(-1, -2).contiguous()) / (math.sqrt(d) * eps[None, :, None, None])


def forward(Q, K, V, G, eps, log_mu, log_nu, K_iter, lam=1.0, x_res=None):
    """Batched dense UOT Sinkhorn forward; every tensor of the caller's dtype/device.

    Q, K, V, G (B,H,N,d); eps (H,); log_mu, log_nu (B,H,N); x_res (B,N,3) or None.
    Returns o_flat (B,N,H*d), x_centroid (B,H,N,3), log_u, log_v, O_avg, sig_G,
    log_z = LSE_j(u_i + L_ij + v_j) and col_lse = LSE_i(L_ij + u_i) (last update).
    """
    B, H, N, d = Q.shape
    kappa = (lam / (lam + eps))[None, :, None]
    L = _logits(Q, K, eps)
    lu = torch.zeros(B, H, N, dtype=Q.dtype, device=Q.device)
    lv = torch.zeros_like(lu)
    col_lse = torch.zeros_like(lu)
    for _ in range(K_iter):                                           # :178-192
        lu = kappa * (log_mu - torch.logsumexp(L + lv[:, :, None, :], dim=-1))
        col_lse = torch.logsumexp(L + lu[:, :, :, None], dim=-2)
        lv = kappa * (log_nu - col_lse)
    ls = lu[:, :, :, None] + L + lv[:, :, None, :]                    # :194-198
    T = torch.exp(ls - ls.amax(dim=-1, keepdim=True))
    T_norm = T / (T.sum(dim=-1, keepdim=True) + 1e-6)
    O_avg = torch.matmul(T_norm, V)                                   # :199
    x = torch.zeros(B, N, 3, dtype=Q.dtype, device=Q.device) if x_res is None else x_res
    xc = torch.matmul(T_norm, x[:, None].expand(B, H, N, 3).contiguous())  # :200
    sig_G = torch.sigmoid(G)
    o_flat = (sig_G * O_avg).permute(0, 2, 1, 3).reshape(B, N, H * d)
    log_z = torch.logsumexp(ls, dim=-1)
    return dict(o_flat=o_flat, x_centroid=xc, log_u=lu, log_v=lv, O_avg=O_avg, sig_G=sig_G,
                log_z=log_z, col_lse=col_lse)


def _cg(matvec, b, n_iter):
    """Batched CG from x0 = 0 (utils/cg.py:56-97), exactly n_iter steps; vectors (..., N)."""
    x = torch.zeros_like(b)
    r = b.clone()
    p = r.clone()
    rr = (r * r).sum(-1, keepdim=True)
    for _ in range(n_iter):
        Ap = matvec(p)
        pAp = (p * Ap).sum(-1, keepdim=True)
        alpha = torch.where(pAp != 0, rr / torch.where(pAp != 0, pAp, torch.ones_like(pAp)), torch.zeros_like(pAp))
        x = x + alpha * p
        r = r - alpha * Ap
        rr_new = (r * r).sum(-1, keepdim=True)
        beta = torch.where(rr != 0, rr_new / torch.where(rr != 0, rr, torch.ones_like(rr)), torch.zeros_like(rr))
        p = r + beta * p
        rr = rr_new
    return x


def backward_cg(Q, K, V, G, eps, fwd, grad_o_flat, n_cg, lam=1.0, mode="reference", grad_xc=None, x_res=None):
    """IFT backward with the system solved by n_cg CG steps (see ``backward``)."""
    return backward(Q, K, V, G, eps, fwd, grad_o_flat, n_cg, lam=lam, mode=mode, grad_xc=grad_xc, x_res=x_res,
                    solver="cg")


def backward(Q, K, V, G, eps, fwd, grad_o_flat, n_iter, lam=1.0, mode="reference", grad_xc=None, x_res=None,
             solver="cg"):
    """IFT backward of ``forward`` (flash_sinkhorn_attn.py:246-667), dense, batched.

    The linear system (I - kappa^2 S_row^T S_col) z_v = g_v is solved either by
    n_iter reference Gauss-Seidel sweeps from z = g (solver="fixed_point",
    :471-542: z_u = kappa S_col z_v, z_v = g_v + kappa S_row^T z_u) or by n_iter CG
    steps on (I - kappa^2 W^T W) y = D_c^{-1/2} g_v, W = D_r^{-1/2} T D_c^{-1/2}.
    Returns dict of gradients Q, K, V, G, log_mu, log_nu.
    """
    B, H, N, d = Q.shape
    kappa = (lam / (lam + eps))[None, :, None]
    e4 = eps[None, :, None, None]
    O_avg, sig_G, xc = fwd["O_avg"], fwd["sig_G"], fwd["x_centroid"]
    lu, lv = fwd["log_u"], fwd["log_v"]
    g = grad_o_flat.reshape(B, N, H, d).permute(0, 2, 1, 3)
    gO = sig_G * g                                                    # :278-282
    dG = sig_G * (1 - sig_G) * O_avg * g
    x = torch.zeros(B, N, 3, dtype=Q.dtype, device=Q.device) if x_res is None else x_res
    gxc = torch.zeros_like(xc) if grad_xc is None else grad_xc
    D = (gO * O_avg).sum(-1) + (gxc * xc).sum(-1)                     # :290
    L = _logits(Q, K, eps)
    s = lu[:, :, :, None] + L + lv[:, :, None, :]
    logZ = torch.logsumexp(s, dim=-1)                                 # :297-334
    T = torch.exp(s - logZ[:, :, :, None])                            # :374-379
    row_lse = torch.logsumexp(L + lv[:, :, None, :], dim=-1)          # :407-437
    col_lse = torch.logsumexp(L + lu[:, :, :, None], dim=-2)          # :439-469
    S_row = torch.exp(L + lv[:, :, None, :] - row_lse[:, :, :, None])
    S_col = torch.exp(L + lu[:, :, :, None] - col_lse[:, :, None, :])
    xb = x[:, None].expand(B, H, N, 3)
    dT = torch.matmul(gO, V.transpose(-1, -2).contiguous()) + torch.matmul(gxc, xb.transpose(-1, -2).contiguous())
    gls = T * (dT - D[:, :, :, None])                                 # :386
    g_v = gls.sum(-2)                                                 # :388
    dV = torch.matmul(T.transpose(-1, -2).contiguous(), gO)           # :389
    if solver == "fixed_point":
        S_row_t = S_row.transpose(-1, -2).contiguous()
        z_v = g_v.clone()                                             # :472-473 (g_u = 0)
        z_u = torch.zeros_like(g_v)
        for _ in range(n_iter):                                       # :475-542
            z_u = kappa * torch.matmul(S_col, z_v[..., None])[..., 0]
            z_v = g_v + kappa * torch.matmul(S_row_t, z_u[..., None])[..., 0]
    elif solver == "cg":
        # CG on the symmetric form: T_un = exp(u + L + v - max logZ) (a scalar rescaling of T)
        T_un = T * torch.exp(logZ - logZ.amax(dim=-1, keepdim=True))[:, :, :, None]
        r = T_un.sum(-1)
        c = T_un.sum(-2)
        W = T_un / r.sqrt()[:, :, :, None] / c.sqrt()[:, :, None, :]
        Wt = W.transpose(-1, -2).contiguous()
        k2 = (kappa * kappa)

        def A(y):
            t = torch.matmul(W, y[..., None])[..., 0]
            return y - k2 * torch.matmul(Wt, t[..., None])[..., 0]

        y = _cg(A, g_v / c.sqrt(), n_iter)
        z_v = c.sqrt() * y
        z_u = kappa * torch.matmul(S_col, z_v[..., None])[..., 0]
    else:
        raise ValueError(f"unknown solver {solver!r}")
    sgn = -1.0 if mode == "reference" else 1.0
    # reference: dC = -(1/eps) gls - (kappa/eps)(z_u S_row + z_v S_col)          (:594-615)
    # analytic : lambda_v = z_v, lambda_u = -z_u; dC = -(1/eps) gls + (kappa/eps)(lambda_u S_row + lambda_v S_col)
    dC = -gls / e4 - (kappa[..., None] / e4) * z_u[:, :, :, None] * S_row \
        + sgn * (kappa[..., None] / e4) * z_v[:, :, None, :] * S_col
    inv = 1.0 / math.sqrt(d)
    dQ = -inv * torch.matmul(dC, K)
    dK = -inv * torch.matmul(dC.transpose(-1, -2).contiguous(), Q)
    dlog_mu = (kappa if mode == "reference" else -kappa) * z_u          # :645
    dlog_nu = kappa * z_v                                              # :646
    return dict(Q=dQ, K=dK, V=dV, G=dG, log_mu=dlog_mu, log_nu=dlog_nu, z_v=z_v, z_u=z_u)
