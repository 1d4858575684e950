"""The allocation-free forward (dfl_sinkhorn_fwd_noalloc) against dfl_sinkhorn_fwd.

Both entry points run the same kernels on the same inputs; the allocation-free one
keeps its exchange words, error word and bins copies in the library's static
per-GPU array instead of a caller workspace.  Two calls in a row, the second on a
smaller problem (the array keeps the first call's contents), must each give
bit-identical outputs to the regular entry point.  Problems beyond the array's
size, and stream storage, are rejected on the host before any launch.
"""

import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
OUTS = ("o_flat", "x_centroid", "log_u", "log_v", "o_avg", "log_z", "col_lse")


def _inputs(B, H, N, d, dtype, seed, lengths=None, full_cost=False):
    g = torch.Generator().manual_seed(seed)
    t = dict(q=torch.randn(B, H, N, d, generator=g) / math.sqrt(d), k=torch.randn(B, H, N, d, generator=g) / math.sqrt(d),
             v=torch.randn(B, H, N, d, generator=g), g=torch.randn(B, H, N, d, generator=g))
    t = {k: v.to(dtype) for k, v in t.items()}
    t.update(x=torch.randn(B, N, 3, generator=g) * 3.0, eps=torch.rand(H, generator=g) + 0.25,
             log_mu=torch.log_softmax(torch.randn(B, H, N, generator=g), -1),
             log_nu=torch.log_softmax(torch.randn(B, H, N, generator=g), -1))
    if full_cost:
        t.update(pw=torch.randn(H, 68, generator=g) * 0.5, wd=torch.rand(H, generator=g),
                 bins=torch.randint(0, 68, (B, N, N), generator=g, dtype=torch.int32))
    if lengths is not None:
        m = torch.zeros(B, N)
        for b, n in enumerate(lengths):
            m[b, :n] = 1
        t["mask"] = m
    return {k: v.to(DEV) for k, v in t.items()}


def _params(t, K_iter, outs, storage=0):
    from deepfold_amd import _lib

    B, H, N, d = t["q"].shape
    ptr = lambda k: t[k].data_ptr() if k in t else None
    sb, sh, sn, _ = t["q"].stride()
    return _lib.SinkhornFwdParams(
        _lib.DFL_BF16 if t["q"].dtype == torch.bfloat16 else _lib.DFL_F32,
        ptr("q"), ptr("k"), ptr("v"), ptr("g"), sb, sh, sn,
        ptr("x"), ptr("pw"), ptr("bins"), ptr("eps"), ptr("wd"), ptr("log_mu"), ptr("log_nu"),
        None, None, ptr("mask"), B, H, N, d, K_iter, 1.0, 10.0,
        *(outs[k].data_ptr() for k in OUTS), storage, None)


def _outputs(B, H, N, d):
    f = dict(device=DEV, dtype=torch.float32)
    shapes = dict(o_flat=(B, N, H * d), x_centroid=(B, H, N, 3), log_u=(B, H, N), log_v=(B, H, N),
                  o_avg=(B, H, N, d), log_z=(B, H, N), col_lse=(B, H, N))
    return {k: torch.full(s, float("nan"), **f) for k, s in shapes.items()}


def _run_both(t, K_iter):
    from deepfold_amd import _lib

    lib = _lib.load()
    B, H, N, d = t["q"].shape
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    ref = _outputs(B, H, N, d)
    nbytes = lib.dfl_sinkhorn_workspace_size(B, H, N)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    p = _params(t, K_iter, ref)
    _lib.check(lib.dfl_sinkhorn_fwd(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(), stream),
               "dfl_sinkhorn_fwd")
    got = _outputs(B, H, N, d)
    q = _params(t, K_iter, got)
    _lib.check(lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(q), stream), "dfl_sinkhorn_fwd_noalloc")
    torch.cuda.synchronize()
    _lib.raise_pending("no-alloc test")
    return ref, got


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: the headline shape with the full cost (bins copies live in the array too)
    t1 = _inputs(2, 8, 768, 32, torch.bfloat16, seed=5, lengths=[501, 759], full_cost=True)
    ref, got = _run_both(t1, 12)
    for k in OUTS:
        assert torch.equal(ref[k], got[k]), k
    # second call, smaller, on the array the first call left behind
    t2 = _inputs(1, 4, 256, 32, torch.float32, seed=6)
    ref, got = _run_both(t2, 20)
    for k in OUTS:
        assert torch.equal(ref[k], got[k]), k
    assert torch.isfinite(got["o_flat"]).all()


def test_noalloc_rejects_what_does_not_fit():
    from deepfold_amd import _lib

    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    # B*H*Np exchange words plus bins copies beyond the array: rejected before any launch
    B, H, N, d = 8, 64, 768, 32
    t = dict(q=torch.empty(B, H, N, d, device=DEV), eps=torch.ones(H, device=DEV),
             log_mu=torch.empty(B, H, N, device=DEV), pw=torch.zeros(H, 68, device=DEV),
             bins=torch.zeros(B, N, N, dtype=torch.int32, device=DEV))
    t.update(k=t["q"], v=t["q"], log_nu=t["log_mu"])
    outs = _outputs(1, 1, 1, 1)
    p = _params(t, 5, outs)
    assert lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(p), stream) != 0
    assert b"scratch" in lib.dfl_last_error()
    # stream storage needs the workspace's stream region
    t2 = _inputs(1, 2, 64, 32, torch.float32, seed=7)
    p = _params(t2, 5, _outputs(1, 2, 64, 32), storage=_lib.DFL_STORAGE_STREAM)
    assert lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(p), stream) != 0
    assert b"resident" in lib.dfl_last_error()
