"""CPU oracle for the flash-Sinkhorn optimal-transport attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package (``deepfold_amd``) or
in the HIP library imports, links or calls this module.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker / the timed CPU baseline.

It restates, in numpy (float64 unless ``dtype`` says otherwise), the algorithm of
vv137/deepfold-linear's CPU fallback for ``flash_sinkhorn_attn``:

* ``forward``            -- ``FlashSinkhornAttn.forward`` dense per-sample branch,
                            src/deepfold/model/kernels/flash_sinkhorn_attn.py:144-218
                            (the same math as model/sinkhorn.py:17-198).
* ``backward_reference`` -- ``FlashSinkhornAttn.backward`` (Python-tiled IFT),
                            flash_sinkhorn_attn.py:246-667, evaluated densely per
                            (b, h) (only the summation order differs from the
                            64x64 tiling).
* ``backward_analytic``  -- the true implicit adjoint of the converged map
                            (implicit-function adjoint of the fixed point; differs from the reference
                            in the sign of the z_v*S_col term and of d log_mu).
* ``cg_system``          -- the symmetric positive-definite form
                            (I - kappa^2 W^T W) y = D_c^{-1/2} g_v of the IFT
                            linear system that the GPU solver runs CG on.

Pinning (tests/test_oracle_sinkhorn.py): golden vectors written by the reference
itself (tests/golden/), closed forms (Q=K=0 -> scalar recurrences, O = masked
mean of V), invariants (batched == per-sample, masked == unpadded, T_norm rows
sum to 1, warm-start composition K=7+4 == K=11), float64 brute-force
finite differences for the analytic adjoint, and the algebraic identities
z_v(ref) = lambda_v(analytic), z_u(ref) = -lambda_u(analytic).
"""

from __future__ import annotations

import numpy as np

NUM_BINS = 68
MASK_BIAS = -1e9  # flash_sinkhorn_attn.py:118


def logsumexp(a: np.ndarray, axis: int) -> np.ndarray:
    """Max-shifted log-sum-exp along ``axis`` (torch.logsumexp semantics)."""
    m = np.max(a, axis=axis, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    s = np.sum(np.exp(a - m), axis=axis, keepdims=True)
    return np.squeeze(m + np.log(s), axis=axis)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def cost_matrix(Q, K, x, pw_h, bins, w_h, r_0, dist_mode="exact"):
    """C_ij = -(q_i.k_j)/sqrt(d) + pw_h[bins_ij] + w_h * dist_ij / (r_0 + dist_ij).

    Reference: forward fallback flash_sinkhorn_attn.py:155-159 (``torch.cdist``),
    backward tiles flash_sinkhorn_attn.py:27-53 (``sqrt(sum dx^2).clamp(min=1e-8)``).
    ``dist_mode="exact"`` uses the difference-based Euclidean distance (0 on the
    diagonal, what ``torch.cdist`` computes up to its rounding); ``"clamp"``
    applies the backward's 1e-8 floor.  ``bins=None`` means no position term.
    Returns (C, dist, diff).
    """
    d = Q.shape[-1]
    content = -(Q @ K.T) / np.sqrt(d)
    diff = x[:, None, :] - x[None, :, :]
    dist = np.sqrt(np.sum(diff * diff, axis=-1))
    if dist_mode == "clamp":
        dist = np.maximum(dist, 1e-8)
    geo = w_h * dist / (r_0 + dist)
    C = content + geo
    if bins is not None:
        C = C + pw_h[np.asarray(bins, dtype=np.int64)]
    return C, dist, diff


def forward(Q, K, V, G, x_res, pos_weight, pos_bins, eps, w_dist, log_mu, log_nu,
            K_iter=7, lam=1.0, r_0=10.0, log_u_init=None, log_v_init=None, mask=None,
            dtype=np.float64):
    """Batched UOT flash-Sinkhorn forward (flash_sinkhorn_attn.py:98-218).

    Shapes: Q, K, V, G (B,H,N,d); x_res (B,N,3); pos_weight (H,68);
    pos_bins (B,N,N) int or None; eps, w_dist (H,); log_mu, log_nu (B,H,N);
    mask (B,N) 1=real 0=pad or None.
    Returns dict with o_flat (B,N,H*d), x_centroid (B,H,N,3), log_u, log_v (B,H,N)
    (masked), plus the internals O_avg (B,H,N,d) and sig_G.
    """
    f = lambda a: None if a is None else np.asarray(a, dtype=dtype)
    Q, K, V, G, x_res = f(Q), f(K), f(V), f(G), f(x_res)
    pos_weight, eps, w_dist, log_mu, log_nu = f(pos_weight), f(eps), f(w_dist), f(log_mu), f(log_nu)
    B, H, N, d = Q.shape
    mask = np.ones((B, N), dtype=dtype) if mask is None else f(mask)
    maskb = (1.0 - mask) * MASK_BIAS                      # :118
    kappa = lam / (lam + eps)                              # :146
    O_avg = np.zeros((B, H, N, d), dtype=dtype)
    xc = np.zeros((B, H, N, 3), dtype=dtype)
    lu_all = np.zeros((B, H, N), dtype=dtype)
    lv_all = np.zeros((B, H, N), dtype=dtype)
    for b in range(B):
        C = np.zeros((H, N, N), dtype=dtype)
        for h in range(H):                                 # :154-159
            bins = None if pos_bins is None else pos_bins[b]
            C[h], _, _ = cost_matrix(Q[b, h], K[b, h], x_res[b], pos_weight[h], bins,
                                     w_dist[h], r_0)
        logK = -C / eps[:, None, None]                     # :161
        lu = np.zeros((H, N), dtype=dtype) if log_u_init is None else f(log_u_init)[b].copy()
        lv = np.zeros((H, N), dtype=dtype) if log_v_init is None else f(log_v_init)[b].copy()
        mv = maskb[b]
        for _ in range(K_iter):                            # :178-192
            lu = kappa[:, None] * (log_mu[b] - logsumexp(logK + lv[:, None, :] + mv[None, None, :], -1))
            lv = kappa[:, None] * (log_nu[b] - logsumexp(logK + lu[:, :, None] + mv[None, :, None], -2))
        ls = lu[:, :, None] + logK + lv[:, None, :] + mv[None, None, :]   # :194-198
        T = np.exp(ls - ls.max(axis=-1, keepdims=True))
        T_norm = T / (T.sum(axis=-1, keepdims=True) + 1e-6)
        O_avg[b] = T_norm @ V[b]                           # :199
        xc[b] = T_norm @ x_res[b]                          # :200
        lu_all[b], lv_all[b] = lu, lv
    sig_G = sigmoid(G)                                     # :210-212
    o = (sig_G * O_avg).transpose(0, 2, 1, 3).reshape(B, N, H * d)
    o = o * mask[:, :, None]                               # :215-218
    return dict(o_flat=o, x_centroid=xc, log_u=lu_all * mask[:, None, :],
                log_v=lv_all * mask[:, None, :], O_avg=O_avg, sig_G=sig_G)


def _gate_and_D(O_avg, sig_G, x_centroid, grad_o_flat, grad_xc):
    """Gate backward and D (flash_sinkhorn_attn.py:278-292)."""
    B, H, N, d = O_avg.shape
    g = grad_o_flat.reshape(B, N, H, d).transpose(0, 2, 1, 3)
    gO = sig_G * g
    dG = sig_G * (1.0 - sig_G) * O_avg * g
    if grad_xc is None:
        grad_xc = np.zeros_like(x_centroid)
    D = (gO * O_avg).sum(-1) + (grad_xc * x_centroid).sum(-1)
    return gO, dG, grad_xc, D


def _plan_pieces(Qbh, Kbh, xb, pw_h, bins, w_h, r_0, eps_h, lu, lv):
    """Dense versions of the backward's per-tile quantities (:297-469)."""
    C, dist, diff = cost_matrix(Qbh, Kbh, xb, pw_h, bins, w_h, r_0, dist_mode="clamp")
    L = -C / eps_h
    logZ = logsumexp(lu[:, None] + L + lv[None, :], -1)           # :297-334
    T = np.exp(lu[:, None] + L + lv[None, :] - logZ[:, None])      # :374-379
    row_lse = logsumexp(L + lv[None, :], -1)                       # :407-437
    col_lse = logsumexp(L + lu[:, None], 0)                        # :439-469
    S_row = np.exp(L + lv[None, :] - row_lse[:, None])             # :532-537
    S_col = np.exp(L + lu[:, None] - col_lse[None, :])             # :504-509
    return dict(C=C, dist=dist, diff=diff, L=L, logZ=logZ, T=T, row_lse=row_lse,
                col_lse=col_lse, S_row=S_row, S_col=S_col)


def _cost_chain(dC, Qbh, Kbh, dist, diff, bins, w_h, r_0):
    """dC -> dQ, dK, dx_cost, dw, dpos_w (flash_sinkhorn_attn.py:617-637)."""
    d = Qbh.shape[-1]
    inv = 1.0 / np.sqrt(d)
    dQ = -inv * (dC @ Kbh)
    dK = -inv * (dC.T @ Qbh)
    coeff = w_h * r_0 / (r_0 + dist) ** 2
    wgt = dC * coeff / dist
    dx = (wgt[:, :, None] * diff).sum(1) - (wgt[:, :, None] * diff).sum(0)
    dw = float((dC * dist / (r_0 + dist)).sum())
    dpw = np.zeros(NUM_BINS, dtype=dC.dtype)
    if bins is not None:
        dpw = np.bincount(np.asarray(bins, dtype=np.int64).ravel(), weights=dC.ravel(),
                          minlength=NUM_BINS).astype(dC.dtype)
    return dQ, dK, dx, dw, dpw


def backward_reference(fwd_inputs: dict, fwd_out: dict, grad_o_flat, grad_xc=None,
                       K_back=None, solver="fixed_point", n_cg=None, dtype=np.float64,
                       return_internals=False):
    """Reference-mode IFT backward, flash_sinkhorn_attn.py:246-667, NO mask.

    ``fwd_inputs`` holds the forward's arguments (as for ``forward``); ``fwd_out``
    the forward's results (log_u, log_v, O_avg, x_centroid, sig_G).
    ``solver="fixed_point"`` runs the reference's K_back Gauss-Seidel sweeps
    (:471-542); ``solver="cg"`` solves the same linear system to convergence
    with ``n_cg`` CG steps on the symmetric form (see ``cg_system``) and is the
    limit of the fixed point as K_back -> infinity.
    Returns a dict of gradients keyed like the forward's arguments.
    """
    p = {k: (None if v is None or k in ("K_iter", "lam", "r_0", "pos_bins")
             else np.asarray(v, dtype=dtype)) for k, v in fwd_inputs.items()}
    pos_bins = fwd_inputs.get("pos_bins")
    lam = float(fwd_inputs.get("lam", 1.0))
    r_0 = float(fwd_inputs.get("r_0", 10.0))
    K_back = int(fwd_inputs.get("K_iter", 7)) if K_back is None else int(K_back)
    Q, K, V, x = p["Q"], p["K"], p["V"], p["x_res"]
    eps, w_dist, pos_weight = p["eps"], p["w_dist"], p["pos_weight"]
    lu_all = np.asarray(fwd_out["log_u"], dtype=dtype)
    lv_all = np.asarray(fwd_out["log_v"], dtype=dtype)
    O_avg = np.asarray(fwd_out["O_avg"], dtype=dtype)
    xc = np.asarray(fwd_out["x_centroid"], dtype=dtype)
    sig_G = np.asarray(fwd_out["sig_G"], dtype=dtype)
    grad_o_flat = np.asarray(grad_o_flat, dtype=dtype)
    grad_xc = None if grad_xc is None else np.asarray(grad_xc, dtype=dtype)
    B, H, N, d = Q.shape
    kappa = lam / (lam + eps)
    gO, dG, grad_xc, D = _gate_and_D(O_avg, sig_G, xc, grad_o_flat, grad_xc)
    out = dict(Q=np.zeros_like(Q), K=np.zeros_like(K), V=np.zeros_like(V), G=dG,
               x_res=np.zeros_like(x), pos_weight=np.zeros_like(pos_weight),
               w_dist=np.zeros_like(w_dist), log_mu=np.zeros((B, H, N), dtype=dtype),
               log_nu=np.zeros((B, H, N), dtype=dtype))
    internals = {}
    for b in range(B):
        bins = None if pos_bins is None else np.asarray(pos_bins[b])
        for h in range(H):
            k_h, e_h = kappa[h], eps[h]
            pc = _plan_pieces(Q[b, h], K[b, h], x[b], pos_weight[h], bins, w_dist[h], r_0,
                              e_h, lu_all[b, h], lv_all[b, h])
            T = pc["T"]
            dT = gO[b, h] @ V[b, h].T + grad_xc[b, h] @ x[b].T          # :381-384
            gls = T * (dT - D[b, h][:, None])                            # :386
            g_v = gls.sum(0)                                             # :388
            out["V"][b, h] = T.T @ gO[b, h]                              # :389
            out["x_res"][b] += T.T @ grad_xc[b, h]                       # :390
            S_row, S_col = pc["S_row"], pc["S_col"]
            if solver == "fixed_point":
                z_u = np.zeros(N, dtype=dtype)                           # :472 (g_u = 0)
                z_v = g_v.copy()                                         # :473
                for _ in range(K_back):                                  # :475-542
                    z_u = k_h * (S_col @ z_v)
                    z_v = g_v + k_h * (S_row.T @ z_u)
            elif solver == "cg":
                # unnormalised plan exp(u + L + v) up to the scalar exp(-max logZ)
                lz = pc["logZ"]
                T_un = T * np.exp(lz - lz.max())[:, None]
                z_v = cg_system(T_un, k_h, g_v, n_cg if n_cg is not None else 50)
                z_u = k_h * (S_col @ z_v)
            else:
                raise ValueError(f"unknown solver {solver!r}")
            dC = gls * (-1.0 / e_h) - (k_h / e_h) * (z_u[:, None] * S_row + z_v[None, :] * S_col)
            dQ, dK, dx, dw, dpw = _cost_chain(dC, Q[b, h], K[b, h], pc["dist"], pc["diff"],
                                              bins, w_dist[h], r_0)
            out["Q"][b, h] = dQ
            out["K"][b, h] = dK
            out["x_res"][b] += dx
            out["w_dist"][h] += dw
            out["pos_weight"][h] += dpw
            out["log_mu"][b, h] = k_h * z_u                              # :645
            out["log_nu"][b, h] = k_h * z_v                              # :646
            if return_internals:
                internals[(b, h)] = dict(z_u=z_u, z_v=z_v, g_v=g_v, **pc)
    if return_internals:
        out["_internals"] = internals
    return out


def cg_system(T, kappa, g_v, n_iter, *, tol=0.0):
    """Solve (I - kappa^2 S_row^T S_col) z_v = g_v by CG on its symmetric form.

    ``T`` is the transport plan T_ij = exp(u_i + L_ij + v_j) up to one positive
    scalar factor (a scalar leaves S_row = D_r^{-1} T and S_col = T D_c^{-1}
    unchanged; a row rescaling would change S_col).  With r = T 1, c = T^T 1 and
    W = D_r^{-1/2} T D_c^{-1/2}:  S_row^T S_col = D_c^{1/2} W^T W D_c^{-1/2}, so with
    y = D_c^{-1/2} z_v the system is (I - kappa^2 W^T W) y = D_c^{-1/2} g_v, whose
    spectrum lies in [1 - kappa^2, 1].  CG steps follow utils/cg.py:56-97 (x0 = 0).
    """
    T = np.asarray(T)
    r = T.sum(1)
    c = T.sum(0)
    W = T / np.sqrt(r)[:, None] / np.sqrt(c)[None, :]
    b = g_v / np.sqrt(c)
    A = lambda y: y - kappa * kappa * (W.T @ (W @ y))
    y, _ = conjugate_gradient(A, b, max_iter=n_iter, rtol=tol, atol=tol)
    return np.sqrt(c) * y


def conjugate_gradient(matvec, b, *, x0=None, max_iter=300, rtol=1e-6, atol=1e-6,
                       preconditioner=None, stabilise_every=0):
    """Preconditioned CG, restating utils/cg.py:28-97 on numpy vectors.

    Returns (x, info) with info = dict(converged, iters, residual, initial_residual).
    """
    b = np.asarray(b)
    if x0 is None:
        x = np.zeros_like(b)
        r = b.copy()
    else:
        x = np.array(x0, copy=True)
        r = b - matvec(x)
    z = preconditioner(r) if preconditioner is not None else r
    p = z.copy()
    rz_old = float(r @ z)
    init_res = float(np.linalg.norm(r))
    tol = max(atol, rtol * init_res)
    for it in range(int(max_iter)):
        Ap = matvec(p)
        denom = float(p @ Ap)
        if denom == 0.0:
            break
        alpha = rz_old / denom
        x = x + alpha * p
        r = r - alpha * Ap
        if stabilise_every and (it + 1) % stabilise_every == 0:
            r = b - matvec(x)
        res = float(np.linalg.norm(r))
        if res <= tol:
            return x, dict(converged=True, iters=it + 1, residual=res, initial_residual=init_res)
        z = preconditioner(r) if preconditioner is not None else r
        rz_new = float(r @ z)
        beta = rz_new / rz_old
        p = z + beta * p
        rz_old = rz_new
    res = float(np.linalg.norm(r))
    return x, dict(converged=False, iters=int(max_iter), residual=res, initial_residual=init_res)


def backward_analytic(fwd_inputs: dict, fwd_out: dict, grad_o_flat, grad_xc=None,
                      dtype=np.float64):
    """True implicit-function-theorem adjoint of the converged Sinkhorn map.

    F_u = u - kappa (log mu - LSE_j(L + v)), F_v = v - kappa (log nu - LSE_i(L + u)).
    J^T lambda = g with g_u = 0:  lambda_v = (I - kappa^2 S_row^T S_col)^{-1} g_v,
    lambda_u = -kappa S_col lambda_v;  dC = -(1/eps) gls + (kappa/eps)
    (lambda_u S_row + lambda_v S_col);  d log_mu = kappa lambda_u,
    d log_nu = kappa lambda_v.  Solved exactly (numpy.linalg.solve), no mask.
    """
    ref = backward_reference(fwd_inputs, fwd_out, grad_o_flat, grad_xc, K_back=0,
                             dtype=dtype, return_internals=True)
    internals = ref.pop("_internals")
    p = {k: (None if v is None or k in ("K_iter", "lam", "r_0", "pos_bins")
             else np.asarray(v, dtype=dtype)) for k, v in fwd_inputs.items()}
    pos_bins = fwd_inputs.get("pos_bins")
    lam = float(fwd_inputs.get("lam", 1.0))
    r_0 = float(fwd_inputs.get("r_0", 10.0))
    Q, K, x = p["Q"], p["K"], p["x_res"]
    eps, w_dist = p["eps"], p["w_dist"]
    B, H, N, d = Q.shape
    kappa = lam / (lam + eps)
    gO, dG, gxc, D = _gate_and_D(np.asarray(fwd_out["O_avg"], dtype=dtype),
                                 np.asarray(fwd_out["sig_G"], dtype=dtype),
                                 np.asarray(fwd_out["x_centroid"], dtype=dtype),
                                 np.asarray(grad_o_flat, dtype=dtype),
                                 None if grad_xc is None else np.asarray(grad_xc, dtype=dtype))
    out = dict(ref)
    out["Q"] = np.zeros_like(Q)
    out["K"] = np.zeros_like(K)
    out["pos_weight"] = np.zeros_like(p["pos_weight"])
    out["w_dist"] = np.zeros_like(w_dist)
    # x_res keeps only the transport part from ref; recompute the cost part below
    x_tr = np.zeros_like(x)
    for b in range(B):
        for h in range(H):
            x_tr[b] += internals[(b, h)]["T"].T @ gxc[b, h]
    out["x_res"] = x_tr
    for b in range(B):
        bins = None if pos_bins is None else np.asarray(pos_bins[b])
        for h in range(H):
            it = internals[(b, h)]
            k_h, e_h = kappa[h], eps[h]
            S_row, S_col, T = it["S_row"], it["S_col"], it["T"]
            dT = gO[b, h] @ p["V"][b, h].T + gxc[b, h] @ x[b].T
            gls = T * (dT - D[b, h][:, None])
            g_v = gls.sum(0)
            A = np.eye(N, dtype=dtype) - k_h * k_h * (S_row.T @ S_col)
            lam_v = np.linalg.solve(A, g_v)
            lam_u = -k_h * (S_col @ lam_v)
            dC = gls * (-1.0 / e_h) + (k_h / e_h) * (lam_u[:, None] * S_row + lam_v[None, :] * S_col)
            dQ, dK, dx, dw, dpw = _cost_chain(dC, Q[b, h], K[b, h], it["dist"], it["diff"],
                                              bins, w_dist[h], r_0)
            out["Q"][b, h] = dQ
            out["K"][b, h] = dK
            out["x_res"][b] += dx
            out["w_dist"][h] += dw
            out["pos_weight"][h] += dpw
            out["log_mu"][b, h] = k_h * lam_u
            out["log_nu"][b, h] = k_h * lam_v
    return out


def backward_masked(fwd_inputs: dict, grad_o_flat, grad_xc=None, mode="reference",
                    solver="fixed_point", n_cg=None, K_back=None, dtype=np.float64):
    """Parity target for padded batches: each sample evaluated on its unpadded slice.

    The reference backward ignores the padding mask (flash_sinkhorn_attn.py:323-327,
    374-379, 583-588), so a padded batch leaks padded tokens into the gradients.
    The consistent definition -- and the one the GPU path implements -- runs the
    forward + backward separately on each sample's first n_b = sum(mask[b]) tokens
    (valid tokens must be a prefix), and reports zeros at padded positions.
    Returns (forward dict, gradient dict), both padded to N.
    """
    p = dict(fwd_inputs)
    mask = p.pop("mask", None)
    Q = np.asarray(p["Q"])
    B, H, N, d = Q.shape
    mask = np.ones((B, N)) if mask is None else np.asarray(mask)
    fo = dict(o_flat=np.zeros((B, N, H * d), dtype=dtype), x_centroid=np.zeros((B, H, N, 3), dtype=dtype),
              log_u=np.zeros((B, H, N), dtype=dtype), log_v=np.zeros((B, H, N), dtype=dtype),
              O_avg=np.zeros((B, H, N, d), dtype=dtype), sig_G=np.zeros((B, H, N, d), dtype=dtype))
    gr = None
    g_o = None if grad_o_flat is None else np.asarray(grad_o_flat)
    for b in range(B):
        n = int(round(float(mask[b].sum())))
        assert np.all(mask[b, :n] == 1) and np.all(mask[b, n:] == 0), "valid tokens must be a prefix"
        sl = {}
        for k, v in p.items():
            if v is None or k in ("K_iter", "lam", "r_0"):
                sl[k] = v
            elif k in ("pos_weight", "eps", "w_dist"):
                sl[k] = np.asarray(v)
            elif k == "pos_bins":
                sl[k] = np.asarray(v)[b:b + 1, :n, :n]
            elif k == "x_res":
                sl[k] = np.asarray(v)[b:b + 1, :n]
            elif k in ("log_u_init", "log_v_init", "log_mu", "log_nu"):
                sl[k] = np.asarray(v)[b:b + 1, :, :n]
            else:
                sl[k] = np.asarray(v)[b:b + 1, :, :n]
        f1 = forward(**{kk: sl[kk] for kk in ("K_iter", "lam", "r_0") if kk in sl},
                     Q=sl["Q"], K=sl["K"], V=sl["V"], G=sl["G"], x_res=sl["x_res"],
                     pos_weight=sl["pos_weight"], pos_bins=sl.get("pos_bins"), eps=sl["eps"],
                     w_dist=sl["w_dist"], log_mu=sl["log_mu"], log_nu=sl["log_nu"],
                     log_u_init=sl.get("log_u_init"), log_v_init=sl.get("log_v_init"), dtype=dtype)
        fo["o_flat"][b, :n] = f1["o_flat"][0]
        fo["x_centroid"][b, :, :n] = f1["x_centroid"][0]
        fo["log_u"][b, :, :n] = f1["log_u"][0]
        fo["log_v"][b, :, :n] = f1["log_v"][0]
        fo["O_avg"][b, :, :n] = f1["O_avg"][0]
        fo["sig_G"][b, :, :n] = f1["sig_G"][0]
        if g_o is None:
            continue
        go = g_o[b:b + 1, :n]
        gx = None if grad_xc is None else np.asarray(grad_xc)[b:b + 1, :, :n]
        if mode == "reference":
            g1 = backward_reference(sl, f1, go, gx, K_back=K_back, solver=solver, n_cg=n_cg, dtype=dtype)
        else:
            g1 = backward_analytic(sl, f1, go, gx, dtype=dtype)
        if gr is None:
            gr = dict(Q=np.zeros((B, H, N, d), dtype=dtype), K=np.zeros((B, H, N, d), dtype=dtype),
                      V=np.zeros((B, H, N, d), dtype=dtype), G=np.zeros((B, H, N, d), dtype=dtype),
                      x_res=np.zeros((B, N, 3), dtype=dtype),
                      pos_weight=np.zeros_like(np.asarray(p["pos_weight"], dtype=dtype)),
                      w_dist=np.zeros_like(np.asarray(p["w_dist"], dtype=dtype)),
                      log_mu=np.zeros((B, H, N), dtype=dtype), log_nu=np.zeros((B, H, N), dtype=dtype))
        for k in ("Q", "K", "V", "G"):
            gr[k][b, :, :n] = g1[k][0]
        gr["x_res"][b, :n] = g1["x_res"][0]
        gr["log_mu"][b, :, :n] = g1["log_mu"][0]
        gr["log_nu"][b, :, :n] = g1["log_nu"][0]
        gr["pos_weight"] += g1["pos_weight"]
        gr["w_dist"] += g1["w_dist"]
    return fo, gr
