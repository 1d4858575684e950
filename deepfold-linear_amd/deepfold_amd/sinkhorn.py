"""Dense, materialised-cost Sinkhorn on MI355X: ``sinkhorn_solve`` and ``compute_transport_output``.

Drop-in for ``deepfold.model.sinkhorn`` of vv137/deepfold-linear
(src/deepfold/model/sinkhorn.py): same names, argument order, defaults, return
tuples and unbatched (3-D cost) handling.  Both run as HIP kernels through the C
ABI (``dfl_dense_sinkhorn_*``, ``dfl_dense_transport_*`` in include/dfl_amd.h);
gradients are those of the reference's plain autograd through the executed
iterations (sinkhorn.py:1-8), computed by an unrolled HIP backward.  Computation
is fp32 (inputs are cast); ``eps`` gets no gradient (a fixed per-head buffer).
There is no CPU fallback: CPU tensors raise.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def _f32(t):
    return None if t is None else t.detach().to(torch.float32).contiguous()


class _DenseSinkhorn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, C, log_mu, log_nu, eps, lam, K, log_u_init, log_v_init, threshold, check_every, mask):
        dev = _lib.require_gpu(C, log_mu, log_nu, eps, log_u_init, log_v_init, mask)
        B, H, N, _ = C.shape
        Cf, mu, nu, ep = _f32(C), _f32(log_mu), _f32(log_nu), _f32(eps).reshape(H)
        u0, v0, m = _f32(log_u_init), _f32(log_v_init), _f32(mask)
        f32 = dict(device=dev, dtype=torch.float32)
        log_u = torch.empty(B, H, N, **f32)
        log_v = torch.empty(B, H, N, **f32)
        history = torch.empty(4, K + 1, B, H, N, **f32)
        done = ctypes.c_int(0)
        lib = _lib.load()
        ws = _lib.workspace(dev, lib.dfl_dense_sinkhorn_workspace_size(B, H, N, K), kind="dense")
        p = _lib.DenseSinkhornParams(
            Cf.data_ptr(), mu.data_ptr(), nu.data_ptr(), ep.data_ptr(), _lib.ptr(u0), _lib.ptr(v0), _lib.ptr(m),
            B, H, N, int(K), float(lam), -1.0 if threshold is None else float(threshold), int(check_every),
            log_u.data_ptr(), log_v.data_ptr(), history.data_ptr(), ctypes.addressof(done))
        rc = _lib.timed_launch("dense_sinkhorn_fwd", dev, lambda: lib.dfl_dense_sinkhorn_fwd(
            ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_dense_sinkhorn_fwd")
        ctx.save_for_backward(Cf, ep, m, history)
        ctx.meta = (B, H, N, int(K), done.value, float(lam), log_u_init is not None, log_v_init is not None)
        return log_u, log_v

    @staticmethod
    def backward(ctx, grad_u, grad_v):
        Cf, ep, m, history = ctx.saved_tensors
        B, H, N, K_max, K, lam, has_u0, has_v0 = ctx.meta
        dev = Cf.device
        f32 = dict(device=dev, dtype=torch.float32)
        gu = None if grad_u is None else grad_u.detach().to(torch.float32).contiguous()
        gv = None if grad_v is None else grad_v.detach().to(torch.float32).contiguous()
        dC = torch.empty(B, H, N, N, **f32)
        dmu = torch.empty(B, H, N, **f32)
        dnu = torch.empty(B, H, N, **f32)
        du0 = torch.empty(B, H, N, **f32) if has_u0 and ctx.needs_input_grad[6] else None
        dv0 = torch.empty(B, H, N, **f32) if has_v0 and ctx.needs_input_grad[7] else None
        lib = _lib.load()
        ws = _lib.workspace(dev, lib.dfl_dense_sinkhorn_workspace_size(B, H, N, K_max), kind="dense")
        p = _lib.DenseSinkhornBwdParams(
            Cf.data_ptr(), ep.data_ptr(), _lib.ptr(m), history.data_ptr(), B, H, N, K_max, K, lam,
            _lib.ptr(gu), _lib.ptr(gv), dC.data_ptr(), dmu.data_ptr(), dnu.data_ptr(), _lib.ptr(du0), _lib.ptr(dv0))
        rc = _lib.timed_launch("dense_sinkhorn_bwd", dev, lambda: lib.dfl_dense_sinkhorn_bwd(
            ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_dense_sinkhorn_bwd")
        return dC, dmu, dnu, None, None, None, du0, dv0, None, None, None


def sinkhorn_solve(
    C: torch.Tensor,
    log_mu: torch.Tensor,
    log_nu: torch.Tensor,
    eps: torch.Tensor,
    lam: float = 1.0,
    K: int = 7,
    log_u_init: torch.Tensor | None = None,
    log_v_init: torch.Tensor | None = None,
    threshold: float | None = None,
    check_every: int = 2,
    mask: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Log-domain UOT Sinkhorn on a dense cost (sinkhorn.py:17-112).

    C (H,N,N) or (B,H,N,N); log_mu, log_nu (H,N) or (B,H,N); eps (H,); mask (B,N)
    (batched input only).  Returns log_u, log_v, zero at padded positions.  With
    ``threshold`` the iteration stops once the L-inf change is below it, checked
    every ``check_every`` iterations (each check synchronises, as in the reference).
    """
    unbatched = C.dim() == 3
    if unbatched:
        C, log_mu, log_nu = C.unsqueeze(0), log_mu.unsqueeze(0), log_nu.unsqueeze(0)
        log_u_init = None if log_u_init is None else log_u_init.unsqueeze(0)
        log_v_init = None if log_v_init is None else log_v_init.unsqueeze(0)
    lu, lv = _DenseSinkhorn.apply(C, log_mu, log_nu, eps, lam, K, log_u_init, log_v_init, threshold, check_every,
                                  mask)
    if unbatched:
        return lu.squeeze(0), lv.squeeze(0)
    return lu, lv


class _DenseTransport(torch.autograd.Function):
    @staticmethod
    def forward(ctx, V, G, log_u, log_v, C, eps, x_res, mask):
        dev = _lib.require_gpu(V, G, log_u, log_v, C, eps, x_res, mask)
        B, H, N, d = V.shape
        if d > 64:
            raise ValueError(f"compute_transport_output: head dim {d} > 64 is not supported")
        Vf, Gf, lu, lv, Cf = _f32(V), _f32(G), _f32(log_u), _f32(log_v), _f32(C)
        ep, x, m = _f32(eps).reshape(H), _f32(x_res), _f32(mask)
        f32 = dict(device=dev, dtype=torch.float32)
        o = torch.empty(B, N, H * d, **f32)
        T_norm = torch.empty(B, H, N, N, **f32)
        xc = torch.empty(B, H, N, 3, **f32) if x is not None else None
        o_avg = torch.empty(B, H, N, d, **f32)
        lib = _lib.load()
        p = _lib.DenseTransportParams(
            Vf.data_ptr(), _lib.ptr(Gf), lu.data_ptr(), lv.data_ptr(), Cf.data_ptr(), ep.data_ptr(), _lib.ptr(x),
            _lib.ptr(m), B, H, N, d, o.data_ptr(), T_norm.data_ptr(), _lib.ptr(xc), o_avg.data_ptr())
        rc = _lib.timed_launch("dense_transport_fwd", dev, lambda: lib.dfl_dense_transport_fwd(
            ctypes.byref(p), ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_dense_transport_fwd")
        ctx.save_for_backward(Vf, Gf, lu, lv, Cf, ep, x, m, T_norm, o_avg)
        ctx.meta = (B, H, N, d)
        return o, T_norm, xc

    @staticmethod
    def backward(ctx, grad_o, grad_T, grad_xc):
        Vf, Gf, lu, lv, Cf, ep, x, m, T_norm, o_avg = ctx.saved_tensors
        B, H, N, d = ctx.meta
        dev = Vf.device
        f32 = dict(device=dev, dtype=torch.float32)
        c = lambda t: None if t is None else t.detach().to(torch.float32).contiguous()
        go, gT, gx = c(grad_o), c(grad_T), (c(grad_xc) if x is not None else None)
        dV = torch.empty(B, H, N, d, **f32)
        dG = torch.empty(B, H, N, d, **f32) if Gf is not None else None
        dlu = torch.empty(B, H, N, **f32)
        dlv = torch.empty(B, H, N, **f32)
        dC = torch.empty(B, H, N, N, **f32)
        dx = torch.empty(B, N, 3, **f32) if x is not None else None
        lib = _lib.load()
        ws = _lib.workspace(dev, lib.dfl_dense_transport_workspace_size(B, H, N, d), kind="dense_transport")
        p = _lib.DenseTransportParams(
            Vf.data_ptr(), _lib.ptr(Gf), lu.data_ptr(), lv.data_ptr(), Cf.data_ptr(), ep.data_ptr(), _lib.ptr(x),
            _lib.ptr(m), B, H, N, d, None, T_norm.data_ptr(), None, o_avg.data_ptr(),
            _lib.ptr(go), _lib.ptr(gT), _lib.ptr(gx), dV.data_ptr(), _lib.ptr(dG), dlu.data_ptr(), dlv.data_ptr(),
            dC.data_ptr(), _lib.ptr(dx))
        rc = _lib.timed_launch("dense_transport_bwd", dev, lambda: lib.dfl_dense_transport_bwd(
            ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_dense_transport_bwd")
        return dV, dG, dlu, dlv, dC, None, dx, None


def compute_transport_output(
    V: torch.Tensor,
    G: torch.Tensor,
    log_u: torch.Tensor,
    log_v: torch.Tensor,
    C: torch.Tensor,
    eps: torch.Tensor,
    x_res: torch.Tensor | None = None,
    mask: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Transport-weighted average (sinkhorn.py:115-198).

    V, G (H,N,d) or (B,H,N,d); log_u, log_v (H,N) or (B,H,N); C (H,N,N) or
    (B,H,N,N); eps (H,); x_res (N,3) or (B,N,3); mask (B,N).  Returns o (N,H*d) or
    (B,N,H*d), T_norm, and x_centroid (None without x_res).
    """
    unbatched = C.dim() == 3
    if unbatched:
        C, V, G = C.unsqueeze(0), V.unsqueeze(0), G.unsqueeze(0)
        log_u, log_v = log_u.unsqueeze(0), log_v.unsqueeze(0)
        x_res = None if x_res is None else x_res.unsqueeze(0)
    o, T_norm, xc = _DenseTransport.apply(V, G, log_u, log_v, C, eps, x_res, mask)
    if unbatched:
        return o.squeeze(0), T_norm.squeeze(0), (None if xc is None else xc.squeeze(0))
    return o, T_norm, xc
