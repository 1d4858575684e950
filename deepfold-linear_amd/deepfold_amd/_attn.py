"""Autograd glue of the softmax-attention kernels (``dfl_attn_*`` / ``dfl_a2t_*``).

One ``torch.autograd.Function`` drives the attention engine (diffusion,
atom-window and token-to-atom attention); another the atom-to-token kernel.
Both run only on ROCm tensors and raise otherwise.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib


def _compute_dtype(t: torch.Tensor) -> torch.dtype:
    """bf16 stays bf16; everything else computes in fp32."""
    return torch.bfloat16 if t.dtype == torch.bfloat16 else torch.float32


def _unit_inner(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _opt(t, dtype=None):
    if t is None:
        return None
    t = t.detach()
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


class AttnFn(torch.autograd.Function):
    """softmax(scale Q K^T + bias, key mask) V with zeroed masked-query rows and an
    optional sigmoid gate.  Inputs: q, k, v (B,H,*,d); g gate logits or None;
    pos_weight (H,68) + pos_bins (B,Mq,Nk) for the bins bias; bias dense
    (B,H,Mq,Nk) or window (ceil(Mq/32),H,32,128); masks (B,Mq)/(B,Nk) or None."""

    @staticmethod
    def forward(ctx, q, k, v, g, pos_weight, pos_bins, bias, q_mask, k_mask, bias_mode, window):
        dev = _lib.require_gpu(q, k, v, g, pos_weight, pos_bins, bias, q_mask, k_mask)
        lib = _lib.load()
        dt = _compute_dtype(q)
        out_dtype = q.dtype
        qc = _unit_inner(q.detach().to(dt))
        gc = None if g is None else _unit_inner(g.detach().to(dt))
        if gc is not None and gc.stride() != qc.stride():
            qc, gc = qc.contiguous(), gc.contiguous()
        kc = _unit_inner(k.detach().to(dt))
        vc = _unit_inner(v.detach().to(dt))
        if kc.stride() != vc.stride():
            kc, vc = kc.contiguous(), vc.contiguous()
        B, H, Mq, d = qc.shape
        Nk = kc.shape[2]
        pw = _opt(pos_weight, torch.float32)
        bins = _opt(pos_bins, torch.int32)
        bs = _opt(bias, dt)
        qm = _opt(q_mask, torch.float32)
        km = _opt(k_mask, torch.float32)
        o = torch.empty(B, H, Mq, d, dtype=dt, device=dev)
        lse = torch.empty(B, H, Mq, dtype=torch.float32, device=dev)
        p = _lib.AttnParams(
            dtype=_lib.DFL_BF16 if dt == torch.bfloat16 else _lib.DFL_F32,
            q=qc.data_ptr(), k=kc.data_ptr(), v=vc.data_ptr(), g=_lib.ptr(gc),
            q_stride_b=qc.stride(0), q_stride_h=qc.stride(1), q_stride_n=qc.stride(2),
            k_stride_b=kc.stride(0), k_stride_h=kc.stride(1), k_stride_n=kc.stride(2),
            q_mask=_lib.ptr(qm), k_mask=_lib.ptr(km), bias_mode=bias_mode,
            pos_weight=_lib.ptr(pw), pos_bins=_lib.ptr(bins), bias=_lib.ptr(bs), window=int(window),
            B=B, H=H, Mq=Mq, Nk=Nk, d=d, scale=1.0 / math.sqrt(d), o=o.data_ptr(), lse=lse.data_ptr())
        rc = _lib.timed_launch("attn_fwd", dev, lambda: lib.dfl_attn_fwd(
            ctypes.byref(p), ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_attn_fwd")
        ctx.save_for_backward(qc, kc, vc, gc, pw, bins, bs, qm, km, o, lse)
        ctx.meta = (bias_mode, int(window), dt, out_dtype, q.dtype, k.dtype, v.dtype,
                    None if g is None else g.dtype, None if bias is None else bias.dtype)
        ctx.set_materialize_grads(False)
        return o if o.dtype == out_dtype else o.to(out_dtype)

    @staticmethod
    def backward(ctx, grad_o):
        qc, kc, vc, gc, pw, bins, bs, qm, km, o, lse = ctx.saved_tensors
        bias_mode, window, dt, _, qdt, kdt, vdt, gdt, bdt = ctx.meta
        n_in = 11
        if grad_o is None:
            return (None,) * n_in
        dev = qc.device
        lib = _lib.load()
        B, H, Mq, d = qc.shape
        Nk = kc.shape[2]
        go = grad_o.detach().to(dt).contiguous()
        dq = torch.empty(B, H, Mq, d, dtype=dt, device=dev)
        dk = torch.empty(B, H, Nk, d, dtype=dt, device=dev)
        dv = torch.empty(B, H, Nk, d, dtype=dt, device=dev)
        need = ctx.needs_input_grad
        dg = torch.empty(B, H, Mq, d, dtype=dt, device=dev) if gc is not None else None
        dbias = None
        if bs is not None and need[6]:
            dbias = torch.empty_like(bs)  # every entry is written (window: zeros outside the sequence)
        dpw = torch.empty(H, 68, dtype=torch.float32, device=dev) if (bins is not None and need[4]) else None
        ws = _lib.workspace(dev, lib.dfl_attn_workspace_size(B, H, Mq, Nk, d), kind="attn")

        # (a window bias is shared by the batch; the library sums its per-row gradients)
        p = _lib.AttnParams(
            dtype=_lib.DFL_BF16 if dt == torch.bfloat16 else _lib.DFL_F32,
            q=qc.data_ptr(), k=kc.data_ptr(), v=vc.data_ptr(), g=_lib.ptr(gc),
            q_stride_b=qc.stride(0), q_stride_h=qc.stride(1), q_stride_n=qc.stride(2),
            k_stride_b=kc.stride(0), k_stride_h=kc.stride(1), k_stride_n=kc.stride(2),
            q_mask=_lib.ptr(qm), k_mask=_lib.ptr(km), bias_mode=bias_mode,
            pos_weight=_lib.ptr(pw), pos_bins=_lib.ptr(bins), bias=_lib.ptr(bs),
            window=window, B=B, H=H, Mq=Mq, Nk=Nk, d=d, scale=1.0 / math.sqrt(d),
            o=o.data_ptr(), lse=lse.data_ptr(), grad_o=go.data_ptr(), dq=dq.data_ptr(),
            dk=dk.data_ptr(), dv=dv.data_ptr(), dg=_lib.ptr(dg), dbias=_lib.ptr(dbias),
            dpos_weight=_lib.ptr(dpw))
        rc = _lib.timed_launch("attn_bwd", dev, lambda: lib.dfl_attn_bwd(
            ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
            ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_attn_bwd")
        cast = lambda t, dtp: None if t is None else (t if t.dtype == dtp else t.to(dtp))
        return (cast(dq, qdt) if need[0] else None, cast(dk, kdt) if need[1] else None,
                cast(dv, vdt) if need[2] else None, cast(dg, gdt) if need[3] else None,
                dpw if need[4] else None, None, cast(dbias, bdt), None, None, None, None)


class A2TFn(torch.autograd.Function):
    """Token n attends to atoms [starts[n], starts[n] + counts[n])."""

    @staticmethod
    def forward(ctx, q, k, v, starts, counts, token_mask):
        dev = _lib.require_gpu(q, k, v, starts, counts, token_mask)
        lib = _lib.load()
        dt = _compute_dtype(q)
        qc = q.detach().to(dt).contiguous()
        kc = k.detach().to(dt).contiguous()
        vc = v.detach().to(dt).contiguous()
        st = starts.detach().to(torch.int32).contiguous()
        ct = counts.detach().to(torch.int32).contiguous()
        tm = _opt(token_mask, torch.float32)
        B, H, N, d = qc.shape
        M = kc.shape[2]
        o = torch.empty(B, H, N, d, dtype=dt, device=dev)
        lse = torch.empty(B, H, N, dtype=torch.float32, device=dev)
        p = _lib.A2TParams(dtype=_lib.DFL_BF16 if dt == torch.bfloat16 else _lib.DFL_F32,
                           q=qc.data_ptr(), k=kc.data_ptr(), v=vc.data_ptr(), starts=st.data_ptr(),
                           counts=ct.data_ptr(), token_mask=_lib.ptr(tm), B=B, H=H, N=N, M=M, d=d,
                           scale=1.0 / math.sqrt(d), o=o.data_ptr(), lse=lse.data_ptr())
        rc = _lib.timed_launch("a2t_fwd", dev, lambda: lib.dfl_a2t_fwd(
            ctypes.byref(p), ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_a2t_fwd")
        ctx.save_for_backward(qc, kc, vc, st, ct, tm, o, lse)
        ctx.dtypes = (dt, q.dtype, k.dtype, v.dtype)
        ctx.set_materialize_grads(False)
        return o if o.dtype == q.dtype else o.to(q.dtype)

    @staticmethod
    def backward(ctx, grad_o):
        if grad_o is None:
            return (None,) * 6
        qc, kc, vc, st, ct, tm, o, lse = ctx.saved_tensors
        dt, qdt, kdt, vdt = ctx.dtypes
        dev = qc.device
        lib = _lib.load()
        B, H, N, d = qc.shape
        M = kc.shape[2]
        go = grad_o.detach().to(dt).contiguous()
        dq = torch.empty_like(qc)
        dk = torch.empty_like(kc)
        dv = torch.empty_like(vc)
        ws = _lib.workspace(dev, lib.dfl_a2t_workspace_size(B, H, M, d), kind="a2t")
        p = _lib.A2TParams(dtype=_lib.DFL_BF16 if dt == torch.bfloat16 else _lib.DFL_F32,
                           q=qc.data_ptr(), k=kc.data_ptr(), v=vc.data_ptr(), starts=st.data_ptr(),
                           counts=ct.data_ptr(), token_mask=_lib.ptr(tm), B=B, H=H, N=N, M=M, d=d,
                           scale=1.0 / math.sqrt(d), o=o.data_ptr(), lse=lse.data_ptr(),
                           grad_o=go.data_ptr(), dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr())
        rc = _lib.timed_launch("a2t_bwd", dev, lambda: lib.dfl_a2t_bwd(
            ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
            ctypes.c_void_p(_lib.stream_handle(dev))))
        _lib.check(rc, "dfl_a2t_bwd")
        cast = lambda t, dtp: t if t.dtype == dtp else t.to(dtp)
        return cast(dq, qdt), cast(dk, kdt), cast(dv, vdt), None, None, None
