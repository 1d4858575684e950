"""CPU oracle for the dense, materialised-cost Sinkhorn functions.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports it; only
``tests/`` use it, as the checker.

Restates, with differentiable torch ops (float64 on the CPU in the tests), the
two functions of vv137/deepfold-linear's src/deepfold/model/sinkhorn.py:

* ``sinkhorn_solve``           -- :17-112: K log-domain UOT iterations on a given
                                  cost C, row update then column update, masks as
                                  -1e9 biases, optional early stop on the L-inf
                                  change every ``check_every`` iterations, padded
                                  potentials zeroed;
* ``compute_transport_output`` -- :115-198: T_norm with the running-max trick and
                                  the 1e-6 guard, padded rows zeroed, O = T_norm V,
                                  sigmoid gate, permute to (B, N, H*d), EGNN centroid.

Gradients are torch autograd through these restatements -- the reference's own
method (plain autograd through the executed iterations, sinkhorn.py:1-8).

Pinned by tests/test_oracle_sinkhorn_dense_ref.py: the potentials equal the flash
oracle (oracle/sinkhorn.py, an independent restatement of the same iteration)
when C is the flash cost; the reference's own invariants from
tests/test_sinkhorn_batch.py (batched == per-sample, masked == unpadded,
padded potentials exactly 0, rows of T_norm sum to 1); early stop stops at the
first checked iteration whose change is below the threshold; and float64
central finite differences of the losses agree with the autograd gradients.
"""

from __future__ import annotations

import torch


def sinkhorn_solve(C, log_mu, log_nu, eps, lam=1.0, K=7, log_u_init=None, log_v_init=None,
                   threshold=None, check_every=2, mask=None, return_iters=False):
    """Dense UOT Sinkhorn (sinkhorn.py:17-112).  Shapes as in the reference:
    C (H,N,N) or (B,H,N,N); log_mu, log_nu (H,N) or (B,H,N); eps (H,); mask (B,N)."""
    unbatched = C.dim() == 3
    if unbatched:
        C, log_mu, log_nu = C.unsqueeze(0), log_mu.unsqueeze(0), log_nu.unsqueeze(0)
        log_u_init = None if log_u_init is None else log_u_init.unsqueeze(0)
        log_v_init = None if log_v_init is None else log_v_init.unsqueeze(0)
    kappa = lam / (lam + eps)
    log_u = log_u_init if log_u_init is not None else torch.zeros_like(log_mu)
    log_v = log_v_init if log_v_init is not None else torch.zeros_like(log_nu)
    log_K = -C / eps[None, :, None, None]
    if mask is not None:
        mf = mask.to(C.dtype)
        col_b = (1 - mf)[:, None, None, :] * (-1e9)
        row_b = (1 - mf)[:, None, :, None] * (-1e9)
    else:
        col_b = row_b = 0
    done = 0
    for i in range(K):
        u_prev, v_prev = log_u, log_v
        log_u = kappa[None, :, None] * (log_mu - torch.logsumexp(log_K + log_v[:, :, None, :] + col_b, dim=-1))
        log_v = kappa[None, :, None] * (log_nu - torch.logsumexp(log_K + log_u[:, :, :, None] + row_b, dim=-2))
        done = i + 1
        if threshold is not None and (i + 1) % check_every == 0:
            ch = max(float((log_u - u_prev).abs().max()), float((log_v - v_prev).abs().max()))
            if ch < threshold:
                break
    if mask is not None:
        m = mask.to(C.dtype)[:, None, :]
        log_u = log_u * m
        log_v = log_v * m
    if unbatched:
        log_u, log_v = log_u.squeeze(0), log_v.squeeze(0)
    if return_iters:
        return log_u, log_v, done
    return log_u, log_v


def compute_transport_output(V, G, log_u, log_v, C, eps, x_res=None, mask=None):
    """Transport output (sinkhorn.py:115-198) -> (o, T_norm, x_centroid or None)."""
    unbatched = C.dim() == 3
    if unbatched:
        C, V, G = C.unsqueeze(0), V.unsqueeze(0), G.unsqueeze(0)
        log_u, log_v = log_u.unsqueeze(0), log_v.unsqueeze(0)
        x_res = None if x_res is None else x_res.unsqueeze(0)
    log_K = -C / eps[None, :, None, None]
    ls = log_u[:, :, :, None] + log_K + log_v[:, :, None, :]
    if mask is not None:
        mf = mask.to(C.dtype)
        ls = ls + (1 - mf)[:, None, None, :] * (-1e9)
    row_max = ls.max(dim=-1, keepdim=True).values
    T = torch.exp(ls - row_max)
    T_norm = T / (T.sum(dim=-1, keepdim=True) + 1e-6)
    if mask is not None:
        T_norm = T_norm * mf[:, None, :, None]
    O_avg = torch.matmul(T_norm, V)
    o = torch.sigmoid(G) * O_avg
    B, H, N, d = o.shape
    o = o.permute(0, 2, 1, 3).reshape(B, N, H * d)
    if mask is not None:
        o = o * mf[:, :, None]
    xc = None
    if x_res is not None:
        xc = torch.matmul(T_norm, x_res[:, None].expand(B, H, N, 3))
    if unbatched:
        return o.squeeze(0), T_norm.squeeze(0), (None if xc is None else xc.squeeze(0))
    return o, T_norm, xc
