"""GPU tests of the library's calling contracts.

* Launch modes (dfl_set_launch_mode): the headline workload (
  exactly as bench.py builds it) run in one process with ordinary launches and then
  with cooperative launches gives bit-identical outputs and gradients (the same
  kernels, grid and reduction order), and the cooperative run matches the oracle
  at the bf16 bar.  The reference's Triton launches are independent
  (sinkhorn_kernel.py:1991-2011); the persistent kernels here wait on each other,
  which is why the mode exists.
* Failure path: with the wait limit lowered from the host
  (dfl_debug_set_spin_limit), the forward's cross-workgroup waits expire, every
  kernel exits normally, the call's error is reported by the synchronising
  workspace check (a RuntimeError from the op) and by the pinned host word
  (dfl_pending_error returns 2 once), and a call after the limit is restored
  gives the same results as before.  The reference has no counterpart: its op
  swallows every exception (flash_sinkhorn_attn.py:144, 751).
* Warm start (log_u_init / log_v_init, flash_sinkhorn_attn.py:684-685): K = 7
  cold, then 4 more iterations from (u_7, v_7), equals K = 11 cold, the
  composition scripts/benchmark_correctness.py:503-531 checks; and a
  warm-started forward matches the oracle at 1e-4 in fp32.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from conftest import assert_close_rel, max_rel_err
from oracle import sinkhorn as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
FWD_NAMES = ("o_flat", "x_centroid", "log_u", "log_v")
GRAD_NAMES = ("Q", "K", "V", "G", "log_mu", "log_nu")


def _layer(t, K_iter, grads=True, **kw):
    from deepfold_amd import flash_sinkhorn_attn

    leaves = {k: t[k].detach().clone().requires_grad_(grads) for k in GRAD_NAMES}
    o, xc, lu, lv = flash_sinkhorn_attn(leaves["Q"], leaves["K"], leaves["V"], leaves["G"], t["x_res"],
                                        t["pos_weight"], None, t["eps"], None, leaves["log_mu"],
                                        leaves["log_nu"], K_iter=K_iter, mask=t.get("mask"), **kw)
    if grads:
        o.backward(t["dO"])
    torch.cuda.synchronize()
    out = {n: v.detach().float().cpu() for n, v in zip(FWD_NAMES, (o, xc, lu, lv))}
    g = {k: leaves[k].grad.float().cpu() for k in GRAD_NAMES} if grads else None
    return out, g


def test_launch_modes_headline_bit_identical():
    import bench
    from deepfold_amd import _lib

    cfg = bench.SINKHORN["cfg2"]
    cpu, t = bench.make_workload(cfg, DEV)
    kw = dict(ift_solver="cg", ift_iters=cfg["n_cg"])
    before = _lib.get_launch_mode()
    try:
        _lib.set_launch_mode(_lib.DFL_LAUNCH_ORDINARY)
        assert _lib.get_launch_mode() == _lib.DFL_LAUNCH_ORDINARY
        o_ord, g_ord = _layer(t, cfg["K_iter"], **kw)
        _lib.set_launch_mode(_lib.DFL_LAUNCH_COOPERATIVE)
        assert _lib.get_launch_mode() == _lib.DFL_LAUNCH_COOPERATIVE
        o_coop, g_coop = _layer(t, cfg["K_iter"], **kw)
    finally:
        _lib.set_launch_mode(before)
    for k in FWD_NAMES:
        assert torch.equal(o_ord[k], o_coop[k]), k
    for k in GRAD_NAMES:
        assert torch.equal(g_ord[k], g_coop[k]), k
    f64 = lambda x: x.to(torch.float64).numpy()
    fin = dict(Q=f64(cpu["Q"]), K=f64(cpu["K"]), V=f64(cpu["V"]), G=f64(cpu["G"]), x_res=f64(cpu["x_res"]),
               pos_weight=f64(cpu["pos_weight"]), pos_bins=None, eps=f64(cpu["eps"]), w_dist=f64(cpu["w_dist"]),
               log_mu=f64(cpu["log_mu"]), log_nu=f64(cpu["log_nu"]), K_iter=cfg["K_iter"], lam=1.0, r_0=10.0,
               mask=cpu["mask"].numpy())
    fo, gr = ref.backward_masked(fin, cpu["dO"].numpy(), None, solver="cg", n_cg=cfg["n_cg"],
                                 K_back=cfg["K_iter"])
    for k in FWD_NAMES:
        assert_close_rel(o_coop[k].numpy(), fo[k], 2e-2, f"coop:{k}")
    for k in GRAD_NAMES:
        assert_close_rel(g_coop[k].numpy(), gr[k], 2e-2, f"coop:d{k}")


def test_launch_mode_rejects_unknown_value():
    from deepfold_amd import _lib

    lib = _lib.load()
    assert lib.dfl_set_launch_mode(7) != 0
    assert b"launch mode" in lib.dfl_last_error()


def _small_case(seed, B=2, H=4, N=256, d=32, lengths=(256, 190)):
    g = torch.Generator().manual_seed(seed)
    cpu = dict(Q=torch.randn(B, H, N, d, generator=g) / math.sqrt(d),
               K=torch.randn(B, H, N, d, generator=g) / math.sqrt(d),
               V=torch.randn(B, H, N, d, generator=g), G=torch.randn(B, H, N, d, generator=g),
               x_res=torch.randn(B, N, 3, generator=g), pos_weight=torch.zeros(H, 68),
               eps=torch.tensor([0.5, 1.0, 0.75, 2.0][:H]), w_dist=torch.zeros(H))
    mask = torch.zeros(B, N)
    lmu, lnu = torch.zeros(B, H, N), torch.zeros(B, H, N)
    for b, n in enumerate(lengths):
        mask[b, :n] = 1
        lmu[b, :, :n] = torch.log_softmax(torch.randn(H, n, generator=g), -1)
        lnu[b, :, :n] = torch.log_softmax(torch.randn(H, n, generator=g), -1)
    cpu.update(mask=mask, log_mu=lmu, log_nu=lnu, dO=torch.randn(B, N, H * d, generator=g) * mask[:, :, None])
    return cpu, {k: v.to(DEV) for k, v in cpu.items()}


def test_expired_wait_is_reported_and_kernels_exit():
    from deepfold_amd import _lib

    lib = _lib.load()
    cpu, t = _small_case(31)
    good, _ = _layer(t, 30, grads=False)
    assert lib.dfl_pending_error() == 0
    try:
        lib.dfl_debug_set_spin_limit(1)  # every exchange wait gives up at once
        with pytest.raises(RuntimeError, match="error code 2|wait expired"):
            _layer(t, 30, grads=False)
        torch.cuda.synchronize()  # the kernels ended: the stream drains
        assert lib.dfl_pending_error() == 2  # the pinned host word saw it too
        assert lib.dfl_pending_error() == 0  # read once, cleared
    finally:
        lib.dfl_debug_set_spin_limit(0)
    again, _ = _layer(t, 30, grads=False)
    for k in FWD_NAMES:
        assert torch.equal(good[k], again[k]), k


def test_next_op_raises_after_an_expired_wait():
    """Without the synchronising check, the failed call returns and the next op raises."""
    import os

    from deepfold_amd import _lib

    lib = _lib.load()
    cpu, t = _small_case(32)
    old = os.environ.get("DFL_AMD_CHECK")
    os.environ["DFL_AMD_CHECK"] = "0"
    try:
        lib.dfl_debug_set_spin_limit(1)
        _layer(t, 30, grads=False)  # returns; its outputs are invalid
        torch.cuda.synchronize()
        lib.dfl_debug_set_spin_limit(0)
        with pytest.raises(RuntimeError, match="error code 2"):
            _layer(t, 30, grads=False)
    finally:
        lib.dfl_debug_set_spin_limit(0)
        if old is None:
            os.environ.pop("DFL_AMD_CHECK", None)
        else:
            os.environ["DFL_AMD_CHECK"] = old
    assert lib.dfl_pending_error() == 0
    _layer(t, 30, grads=False)  # a clean call after the error was raised


def _fwd_only(t, K_iter, u0=None, v0=None):
    from deepfold_amd import flash_sinkhorn_attn

    with torch.no_grad():
        o, xc, lu, lv = flash_sinkhorn_attn(t["Q"], t["K"], t["V"], t["G"], t["x_res"], t["pos_weight"], None,
                                            t["eps"], None, t["log_mu"], t["log_nu"], K_iter=K_iter,
                                            log_u_init=u0, log_v_init=v0, mask=t.get("mask"))
    torch.cuda.synchronize()
    return dict(o_flat=o, x_centroid=xc, log_u=lu, log_v=lv)


def test_warm_start_composes():
    cpu, t = _small_case(33)
    r7 = _fwd_only(t, 7)
    r7_4 = _fwd_only(t, 4, r7["log_u"], r7["log_v"])
    r11 = _fwd_only(t, 11)
    for k in FWD_NAMES:
        err = max_rel_err(r7_4[k].cpu().numpy(), r11[k].cpu().numpy())
        # the continued run's first sweeps take the online shift and the cold run's the
        # previous LSE: the two agree to fp32 rounding, not bitwise
        assert err <= 1e-6, f"{k}: {err:.3e}"


def test_warm_started_forward_matches_oracle():
    cpu, t = _small_case(34)
    g = torch.Generator().manual_seed(35)
    B, H, N = cpu["log_mu"].shape
    u0 = torch.randn(B, H, N, generator=g) * 0.5
    v0 = torch.randn(B, H, N, generator=g) * 0.5
    got = _fwd_only(t, 9, u0.to(DEV), v0.to(DEV))
    f64 = lambda x: x.to(torch.float64).numpy()
    fin = dict(Q=f64(cpu["Q"]), K=f64(cpu["K"]), V=f64(cpu["V"]), G=f64(cpu["G"]), x_res=f64(cpu["x_res"]),
               pos_weight=f64(cpu["pos_weight"]), pos_bins=None, eps=f64(cpu["eps"]), w_dist=f64(cpu["w_dist"]),
               log_mu=f64(cpu["log_mu"]), log_nu=f64(cpu["log_nu"]), K_iter=9, lam=1.0, r_0=10.0,
               log_u_init=f64(u0), log_v_init=f64(v0), mask=cpu["mask"].numpy())
    fo, _ = ref.backward_masked(fin, cpu["dO"].numpy(), None, solver="cg", n_cg=1, K_back=1)
    for k in FWD_NAMES:
        assert_close_rel(got[k].cpu().numpy(), fo[k], 1e-4, f"warm:{k}")
