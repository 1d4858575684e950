"""CPU oracle for the balanced Sinkhorn transport (TokenOTBlock's centroid step).

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports it; only
``tests/`` (and the bench's CPU baseline leg) use it, as the checker.

Restates, with differentiable torch ops (float64 on the CPU in the tests), the CPU
form of vv137/deepfold-linear's balanced transport,
src/deepfold/model/kernels/flash_sinkhorn_transport.py:

* ``balanced_cost``   -- :254-261: C = (1 - w)(1 - Q K^T) + w d/(r + d) with
                         d = max(|x_i - x_j|, 1e-8), w = sigmoid(alpha_h),
                         r = max(|r_h|, 0.1);
* ``sinkhorn_cpu``    -- :253-282 (``_sinkhorn_cpu``): log K = -C/eps plus log of
                         the clamped mask on both sides; per-sample log marginal
                         -log(n_valid); K iterations of column update, then row
                         update (u starts at 0); T masked; T_norm = T / rowsum
                         (clamped 1e-8); x_cent = T_norm x, h_cent = T_norm V;
* ``balanced_transport`` / ``balanced_transport_dual`` -- the public functions
                         (:376-400, :519-545) on the CPU: fp32 compute dtype
                         unless the inputs are float64.  With a mask they
                         evaluate each sample on its valid tokens (padded
                         outputs zero); see below.

Masks.  The reference's two paths disagree on padded tokens.  Its CPU form keeps
the marginal 1/n on padded rows and columns and only scales their kernel by 1e-8
per side, so the column potentials of padded columns grow until those columns
take a full 1/n of mass from the valid rows: the valid rows' plan is not the one
of the unpadded sample.  Its GPU path adds -1e9 to padded columns in the row
update and to padded rows in the column update (:73-74, :102-103), which on the
valid rows equals the unpadded sample (padded rows still get a plan over the
valid columns).  The parity definition here, as for the UOT attention, is the
per-sample unpadded evaluation: valid rows as the GPU path, padded rows zero as
the CPU form.  ``sinkhorn_cpu`` keeps the CPU form's own mask handling.

Gradients are torch autograd through these restatements, which is what the
reference's CPU path does (checkpointed autograd, :397-399).  Its GPU path
(BalancedSinkhornFn, :287-373) differs in two documented details that this
oracle does not follow: a batch-mean log marginal (:294; this oracle and the
MI355X kernels use the per-sample one of the CPU path) and a geometry distance
sqrt(d^2 + 1e-8) (:52) instead of max(d, 1e-8).

Pinned by tests/test_oracle_balanced.py: for one iteration the plan is the
closed form row-normalise(K diag(1 / colsum K)) (column update first); Sinkhorn
scaling keeps every cross ratio T_ij T_kl / (T_il T_kj) equal to that of the
Gibbs kernel exp(-C/eps), whose cost is built independently in the test; a 2 x 2
problem converges to the closed-form entropic OT plan; a constant cost gives the
masked mean; batched == per-sample; the masked result equals the reference GPU
path's masked iteration (restated in numpy in the test) on valid rows; the
dual's x centroid equals the single's; autograd gradients match central finite
differences.
"""

from __future__ import annotations

import torch


def balanced_cost(Q, K, x, alpha_h, r_h):
    """(B,H,N,N) cost of flash_sinkhorn_transport.py:254-261."""
    H = Q.shape[1]
    dt = Q.dtype
    c_feat = 1.0 - Q @ K.transpose(-1, -2)
    dist = (x.unsqueeze(2) - x.unsqueeze(1)).norm(dim=-1).clamp(min=1e-8)  # (B,N,N)
    r_pos = r_h.to(dt).abs().clamp(min=0.1).view(1, H, 1, 1)
    c_geom = dist.unsqueeze(1) / (r_pos + dist.unsqueeze(1))
    w = torch.sigmoid(alpha_h.to(dt)).view(1, H, 1, 1)
    return (1 - w) * c_feat + w * c_geom


def sinkhorn_cpu(Q_s, K_s, x_f, eps, alpha_h, r_h, mask_f, N, K_iter, V_h=None, return_plan=False):
    """_sinkhorn_cpu (flash_sinkhorn_transport.py:253-282).  Q_s, K_s (B,H,N,d);
    x_f (B,N,3); eps, alpha_h, r_h (H,); mask_f (B,N) or None; V_h (B,H,N,dv) or None."""
    B, H = Q_s.shape[:2]
    dt = Q_s.dtype
    log_K = -(balanced_cost(Q_s, K_s, x_f, alpha_h, r_h) / eps.to(dt).view(1, H, 1, 1))
    if mask_f is not None:
        lm = torch.log(mask_f.clamp(min=1e-8))
        log_K = log_K + lm.unsqueeze(1).unsqueeze(-1) + lm.unsqueeze(1).unsqueeze(-2)
        log_marg = -torch.log(mask_f.sum(-1, keepdim=True).clamp(min=1)).unsqueeze(1).unsqueeze(-1)
    else:
        log_marg = -torch.log(torch.tensor(float(N), dtype=dt))
    lu = torch.zeros(B, H, N, 1, dtype=dt)
    lv = torch.zeros(B, H, 1, N, dtype=dt)
    for _ in range(K_iter):
        lv = log_marg - torch.logsumexp(log_K + lu, dim=-2, keepdim=True)  # column update first
        lu = log_marg - torch.logsumexp(log_K + lv, dim=-1, keepdim=True)  # row update last
    T = (lu + log_K + lv).exp()
    if mask_f is not None:
        T = T * mask_f.view(B, 1, N, 1) * mask_f.view(B, 1, 1, N)
    T_norm = T / T.sum(dim=-1, keepdim=True).clamp(min=1e-8)
    x_cent = T_norm @ x_f.unsqueeze(1)
    out = (x_cent, T_norm @ V_h.to(dt)) if V_h is not None else x_cent
    if return_plan:
        return out, T_norm, lu.squeeze(-1), lv.squeeze(-2)
    return out


def _per_sample(Q, K, x, V, eps, alpha_h, r_h, K_iter, mask):
    """Each sample on its valid tokens (mask > 0.5), scattered back with zeros."""
    B, H, N, _ = Q.shape
    xs, hs = [], []
    for b in range(B):
        idx = torch.nonzero(mask[b] > 0.5).flatten()
        xc = torch.zeros(1, H, N, 3, dtype=Q.dtype)
        hc = torch.zeros(1, H, N, V.shape[-1], dtype=Q.dtype) if V is not None else None
        if idx.numel() > 0:
            sub = sinkhorn_cpu(Q[b:b + 1, :, idx], K[b:b + 1, :, idx], x[b:b + 1, idx], eps, alpha_h, r_h, None,
                               idx.numel(), K_iter, None if V is None else V[b:b + 1, :, idx])
            if V is None:
                xc = xc.index_copy(2, idx, sub)
            else:
                xc = xc.index_copy(2, idx, sub[0])
                hc = hc.index_copy(2, idx, sub[1])
        xs.append(xc)
        hs.append(hc)
    xc = torch.cat(xs)
    return xc if V is None else (xc, torch.cat(hs))


def balanced_transport(Q_s, K_s, x_res, eps, alpha_h, r_h, K_iter=20, mask=None):
    """balanced_sinkhorn_transport on the CPU (flash_sinkhorn_transport.py:376-400)."""
    N = Q_s.shape[2]
    cd = Q_s.dtype if Q_s.dtype == torch.float64 else torch.float32
    if mask is not None:
        return _per_sample(Q_s.to(cd), K_s.to(cd), x_res.to(cd), None, eps, alpha_h, r_h, K_iter, mask)
    return sinkhorn_cpu(Q_s.to(cd), K_s.to(cd), x_res.to(cd), eps, alpha_h, r_h, None, N, K_iter)


def balanced_transport_dual(Q_s, K_s, x_res, V_h, eps, alpha_h, r_h, K_iter=20, mask=None):
    """balanced_sinkhorn_transport_dual on the CPU (flash_sinkhorn_transport.py:519-545)."""
    N = Q_s.shape[2]
    cd = Q_s.dtype if Q_s.dtype == torch.float64 else torch.float32
    if mask is not None:
        return _per_sample(Q_s.to(cd), K_s.to(cd), x_res.to(cd), V_h.to(cd), eps, alpha_h, r_h, K_iter, mask)
    return sinkhorn_cpu(Q_s.to(cd), K_s.to(cd), x_res.to(cd), eps, alpha_h, r_h, None, N, K_iter, V_h.to(cd))
