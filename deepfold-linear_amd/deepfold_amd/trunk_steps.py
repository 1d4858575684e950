"""The TokenOTBlock steps either side of the balanced transport, as fused HIP ops.

vv137/deepfold-linear runs them as eager PyTorch inside ``TokenOTBlock.forward``
(src/deepfold/model/trunk_block.py):

* before the transport (:165-175) -- ``sink_projections``:
  h_s = ln_sink(h); Q_s, K_s, V_s = w_q_sink(h_s), w_k_sink(h_s), w_v_sink(h_s) viewed
  as (B, H, N, d) heads; Q_s, K_s L2-normalised per head (F.normalize).  One kernel
  (``dfl_sink_proj_fwd``): LayerNorm, the three projections on MFMA and the head
  norms.  The results are (B, N, H*d) fp32 arrays returned as the same
  (B, H, N, d) views the reference builds with ``.view().permute()``; the balanced
  transport reads those views in place (no ``.contiguous()`` copies).
* after the transport (:189-204) -- ``gated_coordinate_update``:
  x_res + mask * sigmoid(w_gate(ln_gate(h))) * sum_h tanh(lambda_h_raw)/H (x_centroid - x_res),
  one kernel per direction (``dfl_coord_update_fwd`` / ``_bwd``).
* ``token_ot_transport_step`` chains them with the transport and the output
  projection for a module holding TokenOTBlock's parameters (:165-204).

Both directions run on the GPU through the C ABI; CPU tensors raise.  Inputs in
bf16 run the projections on bf16 MFMA with fp32 accumulation (the weights are cast
to the input dtype, as autocast does for nn.Linear); outputs are fp32.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .flash_sinkhorn_transport import balanced_sinkhorn_transport, balanced_sinkhorn_transport_dual


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.DFL_BF16
    if t.dtype == torch.float32:
        return _lib.DFL_F32
    raise TypeError(f"unsupported dtype {t.dtype} (bf16 or fp32)")


def _f32(t):
    return None if t is None else t.detach().to(torch.float32).contiguous()


def _launch(name, dev, fn, what):
    rc = _lib.timed_launch(name, dev, fn)
    _lib.check(rc, what)


class SinkProjectionFn(torch.autograd.Function):
    """h (M, C) -> q_s, k_s, v_s (M, C) fp32; q_s, k_s normalised per head of C/H."""

    @staticmethod
    def forward(ctx, h, ln_weight, ln_bias, w_q, w_k, w_v, n_heads):
        dev = _lib.require_gpu(h, ln_weight, ln_bias, w_q, w_k, w_v)
        M, C = h.shape
        H = int(n_heads)
        hc = h.detach().contiguous()
        ws = [None if w is None else w.detach().to(h.dtype).contiguous() for w in (w_q, w_k, w_v)]
        lw, lb = _f32(ln_weight), _f32(ln_bias)
        f32 = dict(device=dev, dtype=torch.float32)
        q = torch.empty(M, C, **f32)
        k = torch.empty(M, C, **f32)
        v = torch.empty(M, C, **f32) if w_v is not None else None
        qn = torch.empty(M, H, **f32)
        kn = torch.empty(M, H, **f32)
        mean = torch.empty(M, **f32)
        rstd = torch.empty(M, **f32)
        p = _lib.SinkProjParams(_dt(hc), hc.data_ptr(), lw.data_ptr(), lb.data_ptr(), ws[0].data_ptr(),
                                ws[1].data_ptr(), _lib.ptr(ws[2]), M, C, H, q.data_ptr(), k.data_ptr(), _lib.ptr(v),
                                qn.data_ptr(), kn.data_ptr(), mean.data_ptr(), rstd.data_ptr())
        lib = _lib.load()
        _launch("sink_proj_fwd", dev, lambda: lib.dfl_sink_proj_fwd(
            ctypes.byref(p), ctypes.c_void_p(_lib.stream_handle(dev))), "dfl_sink_proj_fwd")
        ctx.save_for_backward(hc, lw, lb, ws[0], ws[1], ws[2] if ws[2] is not None else hc.new_empty(0), q, k, qn,
                              kn, mean, rstd)
        ctx.has_v = w_v is not None
        ctx.H = H
        # only the dtypes of the inputs are needed to return their gradients
        ctx.dtypes = tuple(None if t is None else t.dtype for t in (h, ln_weight, ln_bias, w_q, w_k, w_v))
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        hc, lw, lb, wq, wk, wv, q, k, qn, kn, mean, rstd = ctx.saved_tensors
        if not ctx.has_v:
            wv = None
            dv = None
        dev = hc.device
        M, C = hc.shape
        f32 = dict(device=dev, dtype=torch.float32)
        dq, dk, dv = _f32(dq), _f32(dk), _f32(dv)
        dh = torch.empty(M, C, **f32)
        dlw = torch.empty(C, **f32)
        dlb = torch.empty(C, **f32)
        need = ctx.needs_input_grad
        dwq = torch.empty(C, C, **f32) if need[3] else None
        dwk = torch.empty(C, C, **f32) if need[4] else None
        dwv = torch.empty(C, C, **f32) if (wv is not None and need[5]) else None
        lib = _lib.load()
        ws = _lib.workspace(dev, lib.dfl_sink_proj_workspace_size(M, C), "trunk")
        p = _lib.SinkProjParams(_dt(hc), hc.data_ptr(), lw.data_ptr(), lb.data_ptr(), wq.data_ptr(), wk.data_ptr(),
                                _lib.ptr(wv), M, C, ctx.H, q.data_ptr(), k.data_ptr(), None, qn.data_ptr(),
                                kn.data_ptr(), mean.data_ptr(), rstd.data_ptr(), _lib.ptr(dq), _lib.ptr(dk),
                                _lib.ptr(dv), dh.data_ptr(), dlw.data_ptr(), dlb.data_ptr(), _lib.ptr(dwq),
                                _lib.ptr(dwk), _lib.ptr(dwv))
        _launch("sink_proj_bwd", dev, lambda: lib.dfl_sink_proj_bwd(
            ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(_lib.stream_handle(dev))),
            "dfl_sink_proj_bwd")
        dts = ctx.dtypes
        cast = lambda g, dt: None if g is None or dt is None else g.to(dt)
        return (cast(dh, dts[0]), cast(dlw, dts[1]), cast(dlb, dts[2]), cast(dwq, dts[3]), cast(dwk, dts[4]),
                cast(dwv, dts[5]), None)


def sink_projections(h: torch.Tensor, ln_weight: torch.Tensor, ln_bias: torch.Tensor, w_q: torch.Tensor,
                     w_k: torch.Tensor, w_v: torch.Tensor | None = None, n_heads: int = 16):
    """trunk_block.py:165-175 -> (Q_s, K_s, V_s): (B, H, N, d) views (V_s None without w_v).

    h is (B, N, C) or unbatched (N, C) (then the views are (1, H, N, d)); ln_weight,
    ln_bias are ln_sink's parameters and w_q, w_k, w_v the nn.Linear weights (C, C)."""
    if h.dim() == 2:
        h = h.unsqueeze(0)
    B, N, C = h.shape
    H = int(n_heads)
    q, k, v = SinkProjectionFn.apply(h.reshape(B * N, C), ln_weight, ln_bias, w_q, w_k, w_v, H)
    heads = lambda t: None if t is None else t.view(B, N, H, C // H).permute(0, 2, 1, 3)
    return heads(q), heads(k), heads(v)


class GatedCoordUpdateFn(torch.autograd.Function):
    """trunk_block.py:189-204: x_res (B, N, 3) -> updated coordinates (B, N, 3)."""

    @staticmethod
    def forward(ctx, h, x_res, x_centroid, ln_weight, ln_bias, w_gate, b_gate, lambda_raw, mask):
        dev = _lib.require_gpu(h, x_res, x_centroid, ln_weight, ln_bias, w_gate, b_gate, lambda_raw, mask)
        B, N, C = h.shape
        H = x_centroid.shape[1]
        hc = h.detach().contiguous()
        t = [_f32(a) for a in (x_res, x_centroid, ln_weight, ln_bias, w_gate.reshape(-1), b_gate.reshape(-1),
                               lambda_raw)]
        mk = None if mask is None else mask.detach().to(torch.float32).contiguous()
        out = torch.empty(B, N, 3, device=dev, dtype=torch.float32)
        p = _lib.CoordUpdateParams(_dt(hc), hc.data_ptr(), t[2].data_ptr(), t[3].data_ptr(), t[4].data_ptr(),
                                   t[5].data_ptr(), t[6].data_ptr(), t[1].data_ptr(), t[0].data_ptr(), _lib.ptr(mk),
                                   B, N, C, H, out.data_ptr())
        lib = _lib.load()
        _launch("coord_update_fwd", dev, lambda: lib.dfl_coord_update_fwd(
            ctypes.byref(p), ctypes.c_void_p(_lib.stream_handle(dev))), "dfl_coord_update_fwd")
        ctx.save_for_backward(hc, *t, mk if mk is not None else hc.new_empty(0))
        ctx.has_mask = mk is not None
        ctx.dtypes = tuple(t.dtype for t in (h, x_res, x_centroid, ln_weight, ln_bias, w_gate, b_gate, lambda_raw))
        ctx.shapes = (w_gate.shape, b_gate.shape)
        return out.to(x_res.dtype)

    @staticmethod
    def backward(ctx, dout):
        hc, x, xc, lw, lb, wg, bg, lr, mk = ctx.saved_tensors
        mk = mk if ctx.has_mask else None
        dev = hc.device
        B, N, C = hc.shape
        H = xc.shape[1]
        f32 = dict(device=dev, dtype=torch.float32)
        go = _f32(dout)
        dx = torch.empty(B, N, 3, **f32)
        dxc = torch.empty(B, H, N, 3, **f32)
        dh = torch.empty(B, N, C, **f32)
        dlw, dlb, dwg = (torch.empty(C, **f32) for _ in range(3))
        dbg = torch.empty(1, **f32)
        dlr = torch.empty(H, **f32)
        lib = _lib.load()
        ws = _lib.workspace(dev, lib.dfl_coord_update_workspace_size(C, H), "trunk")
        p = _lib.CoordUpdateParams(_dt(hc), hc.data_ptr(), lw.data_ptr(), lb.data_ptr(), wg.data_ptr(),
                                   bg.data_ptr(), lr.data_ptr(), xc.data_ptr(), x.data_ptr(), _lib.ptr(mk),
                                   B, N, C, H, None, go.data_ptr(), dx.data_ptr(), dxc.data_ptr(), dh.data_ptr(),
                                   dlw.data_ptr(), dlb.data_ptr(), dwg.data_ptr(), dbg.data_ptr(), dlr.data_ptr())
        _launch("coord_update_bwd", dev, lambda: lib.dfl_coord_update_bwd(
            ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(_lib.stream_handle(dev))),
            "dfl_coord_update_bwd")
        dts = ctx.dtypes
        wg_shape, bg_shape = ctx.shapes
        return (dh.to(dts[0]), dx.to(dts[1]), dxc.to(dts[2]), dlw.to(dts[3]), dlb.to(dts[4]),
                dwg.reshape(wg_shape).to(dts[5]), dbg.reshape(bg_shape).to(dts[6]), dlr.to(dts[7]), None)


def gated_coordinate_update(h: torch.Tensor, x_res: torch.Tensor, x_centroid: torch.Tensor, ln_weight: torch.Tensor,
                            ln_bias: torch.Tensor, w_gate: torch.Tensor, b_gate: torch.Tensor,
                            lambda_raw: torch.Tensor, mask: torch.Tensor | None = None) -> torch.Tensor:
    """trunk_block.py:189-204 -> updated x_res (B, N, 3).

    h (B, N, C) is the token state after the transport's feature update; ln_weight,
    ln_bias are ln_gate's, w_gate (1, C) and b_gate (1,) w_gate's (nn.Linear(C, 1)),
    lambda_raw (H,) is lambda_h_raw; x_centroid (B, H, N, 3) comes from the transport."""
    unbatched = h.dim() == 2
    if unbatched:
        h, x_res, x_centroid = h.unsqueeze(0), x_res.unsqueeze(0), x_centroid.unsqueeze(0)
        mask = None if mask is None else mask.unsqueeze(0)
    out = GatedCoordUpdateFn.apply(h, x_res, x_centroid, ln_weight, ln_bias, w_gate, b_gate, lambda_raw, mask)
    return out.squeeze(0) if unbatched else out


def token_ot_transport_step(block, h: torch.Tensor, x_res: torch.Tensor, mask: torch.Tensor | None = None,
                            K_iter: int = 20):
    """Steps 2-4 of TokenOTBlock.forward (trunk_block.py:165-204) for a module with the
    block's parameters (ln_sink, w_q_sink, w_k_sink, w_v_sink / w_o_sink when
    feature_transport, alpha_h, r_h, eps, ln_gate, w_gate, lambda_h_raw, n_heads):
    returns the updated (h, x_res).  h (B, N, C), x_res (B, N, 3), mask (B, N)."""
    B, N, C = h.shape
    if mask is None:
        mask = h.new_ones(B, N)
    ft = getattr(block, "feature_transport", True)
    Q_s, K_s, V_s = sink_projections(h, block.ln_sink.weight, block.ln_sink.bias, block.w_q_sink.weight,
                                     block.w_k_sink.weight, block.w_v_sink.weight if ft else None, block.n_heads)
    if ft:
        x_centroid, h_centroid = balanced_sinkhorn_transport_dual(Q_s, K_s, x_res, V_s, block.eps, block.alpha_h,
                                                                  block.r_h, K_iter=K_iter, mask=mask)
        h_transport = h_centroid.permute(0, 2, 1, 3).reshape(B, N, C)
        h = h + block.w_o_sink(h_transport) * mask.unsqueeze(-1)  # dtypes promote as in the reference
    else:
        x_centroid = balanced_sinkhorn_transport(Q_s, K_s, x_res, block.eps, block.alpha_h, block.r_h,
                                                 K_iter=K_iter, mask=mask)
    x_res = gated_coordinate_update(h, x_res, x_centroid, block.ln_gate.weight, block.ln_gate.bias,
                                    block.w_gate.weight, block.w_gate.bias, block.lambda_h_raw, mask)
    return h, x_res
