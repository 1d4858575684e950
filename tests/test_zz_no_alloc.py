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
import warnings

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


def test_noalloc_error_query_reports_expired_waits():
    """dfl_noalloc_error reads the static array's error word: 0 after a good call, 2
    after a call whose waits were made to expire from the host."""
    from deepfold_amd import _lib

    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    t = _inputs(2, 4, 256, 32, torch.float32, seed=12, lengths=[256, 200])
    outs = _outputs(2, 4, 256, 32)
    p = _params(t, 30, outs)
    _lib.check(lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(p), stream), "dfl_sinkhorn_fwd_noalloc")
    assert lib.dfl_noalloc_error(stream) == 0
    try:
        lib.dfl_debug_set_spin_limit(1)
        _lib.check(lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(p), stream), "dfl_sinkhorn_fwd_noalloc")
        torch.cuda.synchronize()
        assert lib.dfl_noalloc_error(stream) == 2
    finally:
        lib.dfl_debug_set_spin_limit(0)
        lib.dfl_pending_error()  # the pinned word (if created earlier) saw it too: clear it
    _lib.check(lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(p), stream), "dfl_sinkhorn_fwd_noalloc")
    assert lib.dfl_noalloc_error(stream) == 0


def test_noalloc_graph_replays_with_new_inputs():
    """A HIP graph that captured one allocation-free call, replayed with new input
    values in the same buffers, gives the eager workspace entry point's outputs bit
    for bit on every replay: each call clears the array's exchange words with a fill
    kernel (captured with it), so a replay never accepts an earlier replay's words."""
    from deepfold_amd import _lib

    lib = _lib.load()
    B, H, N, d = 2, 8, 768, 32
    t = _inputs(B, H, N, d, torch.bfloat16, seed=20, lengths=[501, 759])
    got = _outputs(B, H, N, d)
    p = _params(t, 12, got)
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):  # eager warm-up on the capture stream
        _lib.check(lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(p), ctypes.c_void_p(side.cuda_stream)), "warm-up")
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side, capture_error_mode="thread_local"):
        rc = lib.dfl_sinkhorn_fwd_noalloc(ctypes.byref(p), ctypes.c_void_p(side.cuda_stream))
    assert rc == 0, lib.dfl_last_error()
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    ws = torch.zeros(lib.dfl_sinkhorn_workspace_size(B, H, N), dtype=torch.uint8, device=DEV)
    for seed in (21, 22, 23):
        new = _inputs(B, H, N, d, torch.bfloat16, seed=seed, lengths=[501, 759])
        for k in t:
            t[k].copy_(new[k])
        for k in got:
            got[k].fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        want = _outputs(B, H, N, d)
        q = _params(t, 12, want)
        _lib.check(lib.dfl_sinkhorn_fwd(ctypes.byref(q), ctypes.c_void_p(ws.data_ptr()), ws.numel(), stream),
                   "dfl_sinkhorn_fwd")
        torch.cuda.synchronize()
        for k in OUTS:
            assert torch.equal(want[k], got[k]), (seed, k)
    assert lib.dfl_noalloc_error(stream) == 0
    _lib.raise_pending("graph replay test")


def test_workspace_entry_points_refuse_capture():
    """The workspace forward chooses its exchange salt on the host per call, so a
    captured call would replay a stale salt: it refuses a capturing stream."""
    from deepfold_amd import _lib

    lib = _lib.load()
    B, H, N, d = 1, 2, 64, 32
    t = _inputs(B, H, N, d, torch.float32, seed=24)
    outs = _outputs(B, H, N, d)
    p = _params(t, 5, outs)
    ws = torch.zeros(lib.dfl_sinkhorn_workspace_size(B, H, N), dtype=torch.uint8, device=DEV)
    side = torch.cuda.Stream(DEV)
    graph = torch.cuda.CUDAGraph()
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="The CUDA Graph is empty")  # the refused call captured nothing
        with torch.cuda.graph(graph, stream=side, capture_error_mode="thread_local"):
            rc = lib.dfl_sinkhorn_fwd(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                      ctypes.c_void_p(side.cuda_stream))
    assert rc != 0 and b"graph" in lib.dfl_last_error()
