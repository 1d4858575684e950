"""Benchmark: flash-Sinkhorn forward + IFT backward per layer on one MI355X.

Default workload (the metric's configuration): B=2,
H=8, N=768 padded, d=32, bf16 inputs with fp32 accumulation, ragged valid
lengths n_b ~ U[384, 768] with a padding mask, eps=0.5, 50 Sinkhorn iterations,
20 CG iterations in the IFT solve, upstream gradient dO ~ N(0,1).  Synthetic
data, seed 1002 (= 1000 + config#).  Unspecified terms are neutral: no position
bins, no geometry term (w_dist = 0, passed as None), x_res = 0, G = 0.

One "step" = one forward (flash_sinkhorn_attn) + one backward (autograd) of the
layer, inputs resident in HBM.  Prints ONE JSON line.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
                    [--workload cfg2|cfg5|cfg3|cfg4|balanced]
    python bench.py --rocpd-summary RESULTS.db    (CPU only: kernel table of a rocprofv3 run)

Opt-in workloads: cfg5 = BASELINE configs[4] (B=1, H=16, N=4096, d=64, bf16,
Dirichlet(5) marginals, eps=0.25, K=100, 30 CG steps; stream storage mode);
cfg3 / cfg4 = the attention rows (configs[2] and [3]); balanced = the balanced
Sinkhorn transport of TokenOTBlock (balanced_sinkhorn_transport_dual fwd+bwd at
the trunk shape B=1, H=16, N=256, d=32, fp32, K=20; the timing configuration of
the reference's tests/test_dual_transport.py).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deepfold-linear_amd"))

# MI355X published peaks (dense): bf16 MFMA 2.5 PFLOP/s, HBM 8 TB/s.
PEAK_MFMA_BF16 = 2.5e15
PEAK_HBM = 8.0e12
# Measured on MI355X by `bench.py --workload peaks` (csrc/peaks.hip, two waves per
# SIMD on all 256 CUs): v_exp_f32 issue rate (15.5-17.8 T/s on two boxes: the higher),
# and the rate of the fixed-shift sweep's element (fma + exp2 + add), which does not
# overlap on gfx950 (9.54 and 9.53 T/s).
PEAK_EXP_MEASURED = 17.8e12
PEAK_SWEEP_ELEMENT_MEASURED = 9.54e12
PEAK_MFMA_F32 = 157.3e12

SINKHORN = {
    "cfg2": dict(B=2, H=8, N=768, d=32, eps=0.5, K_iter=50, n_cg=20, seed=1002, ragged=True, dirichlet=False,
                 workload="BASELINE configs[1]: flash-Sinkhorn fwd + IFT(CG) bwd"),
    "cfg5": dict(B=1, H=16, N=4096, d=64, eps=0.25, K_iter=100, n_cg=30, seed=1005, ragged=False, dirichlet=True,
                 workload="BASELINE configs[4]: large-scale flash-Sinkhorn fwd + IFT(CG) bwd (stream storage)"),
    "cfg2-full": dict(B=2, H=8, N=768, d=32, eps=0.5, K_iter=50, n_cg=20, seed=1002, ragged=True, dirichlet=False,
                      full_cost=True,
                      workload="BASELINE configs[1] with the full cost: position bins (B,N,N) in [0,68), "
                               "pos_weight ~ N(0,0.5^2), w_dist ~ U(0,1), x_res ~ N(0,3^2); fwd + IFT(CG) bwd"),
    "cfg2-unrolled": dict(B=2, H=8, N=768, d=32, eps=0.5, K_iter=50, n_cg=0, seed=1002, ragged=True,
                          dirichlet=False, unrolled=True,
                          workload="BASELINE configs[1] inputs, fwd + unrolled bwd (the reference GPU path's "
                                   "gradient through the 50 iterations)"),
}


def make_workload(cfg, device, dtype=None):
    """Synthetic inputs of one Sinkhorn configuration, built on the CPU (seeded) and copied."""
    import numpy as np
    import torch

    dtype = dtype or torch.bfloat16
    B, H, N, d = cfg["B"], cfg["H"], cfg["N"], cfg["d"]
    g = torch.Generator().manual_seed(cfg["seed"])
    lengths = torch.randint(384, N + 1, (B,), generator=g).tolist() if cfg["ragged"] else [N] * B
    Q = (torch.randn(B, H, N, d, generator=g) / math.sqrt(d)).to(dtype)
    K = (torch.randn(B, H, N, d, generator=g) / math.sqrt(d)).to(dtype)
    V = (torch.randn(B, H, N, d, generator=g) / math.sqrt(d)).to(dtype)
    G = torch.zeros(B, H, N, d, dtype=dtype)
    mask = torch.zeros(B, N)
    log_m = torch.zeros(B, H, N)
    log_n = torch.zeros(B, H, N)
    rng = np.random.default_rng(cfg["seed"])
    for b, n in enumerate(lengths):
        mask[b, :n] = 1.0
        if cfg["dirichlet"]:
            log_m[b, :, :n] = torch.from_numpy(np.log(rng.dirichlet(5.0 * np.ones(n), size=H))).float()
            log_n[b, :, :n] = torch.from_numpy(np.log(rng.dirichlet(5.0 * np.ones(n), size=H))).float()
        else:
            log_m[b, :, :n] = -math.log(n)
            log_n[b, :, :n] = -math.log(n)
    dO = torch.randn(B, N, H * d, generator=g).to(dtype).float()
    dO = dO * mask[:, :, None]
    x = torch.zeros(B, N, 3)
    pw = torch.zeros(H, 68)
    eps = torch.full((H,), cfg["eps"])
    wd = torch.zeros(H)
    bins = None
    if cfg.get("full_cost"):  # drawn after the neutral terms, so the shared inputs stay identical
        bins = torch.randint(0, 68, (B, N, N), generator=g, dtype=torch.int32)
        pw = torch.randn(H, 68, generator=g) * 0.5
        wd = torch.rand(H, generator=g)
        x = torch.randn(B, N, 3, generator=g) * 3.0
    cpu = dict(Q=Q, K=K, V=V, G=G, x_res=x, pos_weight=pw, pos_bins=bins, eps=eps, w_dist=wd, log_mu=log_m,
               log_nu=log_n, mask=None if not cfg["ragged"] else mask, dO=dO, lengths=lengths)
    dev = {k: (v.to(device) if v is not None and hasattr(v, "to") else v) for k, v in cpu.items()}
    return cpu, dev


# where the forward keeps the cost (flash_sinkhorn_attn's storage=; --storage)
STORAGE = "auto"


def step(cfg, t, want=False):
    """One layer: forward + backward with upstream dO.  want=True also makes log mu /
    log nu leaves and returns every output and gradient (the same kernels run)."""
    from deepfold_amd import flash_sinkhorn_attn

    q, k, v, g = (t[n].detach().requires_grad_(True) for n in ("Q", "K", "V", "G"))
    lmu, lnu = t["log_mu"], t["log_nu"]
    if want:
        lmu, lnu = lmu.detach().requires_grad_(True), lnu.detach().requires_grad_(True)
    if cfg.get("full_cost"):  # position weights, geometry weights and coordinates receive gradients too
        pw, wd, x = (t[n].detach().requires_grad_(True) for n in ("pos_weight", "w_dist", "x_res"))
        o, xc, lu, lv = flash_sinkhorn_attn(q, k, v, g, x, pw, t["pos_bins"], t["eps"], wd,
                                            lmu, lnu, K_iter=cfg["K_iter"], mask=t["mask"],
                                            ift_solver="cg", ift_iters=cfg["n_cg"], storage=STORAGE)
    elif cfg.get("unrolled"):
        # neutral terms: no bins and no geometry weight (w_dist = None is the reference's
        # w_dist = 0 without reading x), so the kernels built without the bias terms run
        o, xc, lu, lv = flash_sinkhorn_attn(q, k, v, g, t["x_res"], t["pos_weight"], None, t["eps"], None,
                                            lmu, lnu, K_iter=cfg["K_iter"], mask=t["mask"],
                                            ift_mode="unrolled", storage=STORAGE)
    else:
        o, xc, lu, lv = flash_sinkhorn_attn(q, k, v, g, t["x_res"], t["pos_weight"], None, t["eps"], None,
                                            lmu, lnu, K_iter=cfg["K_iter"], mask=t["mask"],
                                            ift_solver="cg", ift_iters=cfg["n_cg"], storage=STORAGE)
    o.backward(t["dO"])
    if not want:
        return q.grad
    res = dict(o_flat=o, x_centroid=xc, log_u=lu, log_v=lv, Q=q.grad, K=k.grad, V=v.grad, G=g.grad,
               log_mu=lmu.grad, log_nu=lnu.grad)
    return {n: x.detach().float().cpu().numpy() for n, x in res.items()}


def verify_head(cfg, cpu, res, tol=2e-2):
    """Parity of one (b, h) head of a bench step against the CPU oracle, run after and
    outside the timed region on the same inputs: the longest sample's head 0 on its
    valid tokens.  IFT workloads: oracle forward + reference-mode backward with the
    bench's CG step count (oracle/sinkhorn.py, flash_sinkhorn_attn.py:144-218,
    246-667); unrolled: float64 autograd through the dense iteration
    (oracle/sinkhorn_dense_ref.py, the gradient of sinkhorn_kernel.py:2085-2382).
    Normwise relative errors of the outputs, potentials and per-head gradients."""
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    from oracle import sinkhorn as ref

    B, H, d, K = cfg["B"], cfg["H"], cfg["d"], cfg["K_iter"]
    b = max(range(B), key=lambda i: cpu["lengths"][i])
    h, n = 0, cpu["lengths"][b]
    inp = _head_inputs(cfg, cpu, b, h, K)
    inp = {k: (np.asarray(v, dtype=np.float64) if isinstance(v, np.ndarray) and k != "pos_bins" else v)
           for k, v in inp.items()}
    go = cpu["dO"].reshape(B, -1, H, d)[b:b + 1, :n, h, :].double().numpy()
    fo = ref.forward(**inp)
    if cfg.get("unrolled"):
        from oracle import sinkhorn_dense_ref as dref

        f64 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).double()
        q, k, v, g = (f64(inp[n_]).requires_grad_(True) for n_ in ("Q", "K", "V", "G"))
        lmu, lnu = f64(inp["log_mu"]).requires_grad_(True), f64(inp["log_nu"]).requires_grad_(True)
        C = -(q @ k.transpose(-1, -2)) / math.sqrt(d)
        lu, lv = dref.sinkhorn_solve(C, lmu, lnu, f64(inp["eps"]), K=K)
        o, _, _ = dref.compute_transport_output(v, g, lu, lv, C, f64(inp["eps"]))
        (o * f64(go)).sum().backward()
        gr = {n_: x.grad.numpy() for n_, x in (("Q", q), ("K", k), ("V", v), ("G", g), ("log_mu", lmu),
                                                  ("log_nu", lnu))}
    else:
        gr = ref.backward_reference(inp, fo, go, None, solver="cg", n_cg=cfg["n_cg"])

    def rel(got, want):
        got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
        return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))

    errs = {
        "o_flat": rel(res["o_flat"][b, :n, h * d:(h + 1) * d], fo["o_flat"][0]),
        "x_centroid": rel(res["x_centroid"][b, h, :n], fo["x_centroid"][0, 0]),
        "log_u": rel(res["log_u"][b, h, :n], fo["log_u"][0, 0]),
        "log_v": rel(res["log_v"][b, h, :n], fo["log_v"][0, 0]),
    }
    for k_ in ("Q", "K", "V", "G", "log_mu", "log_nu"):
        errs["d" + k_] = rel(res[k_][b, h, :n], gr[k_][0, 0])
    return {"head": [b, h], "n_valid": n, "oracle": "oracle/sinkhorn.py" if not cfg.get("unrolled")
            else "oracle/sinkhorn_dense_ref.py (float64 autograd)", "tol": tol,
            "max_rel_err": {k_: float(f"{v_:.3e}") for k_, v_ in errs.items()},
            "pass": bool(all(v_ <= tol for v_ in errs.values()))}


def algorithmic_counts(cfg, lengths):
    """Per-layer algorithmic work: E = sum_b H n_b^2 valid
    plan elements; forward 2K LSE sweeps at 2d flops + one output sweep at 4d;
    backward n_CG matvec sweeps at 2d + g_v sweep 6d + gradient sweep 8d; one
    exp per element per sweep."""
    H, d, K, ncg = cfg["H"], cfg["d"], cfg["K_iter"], cfg["n_cg"]
    E = sum(H * n * n for n in lengths)
    f_fwd = E * d * (4 * K + 4)
    x_fwd = E * (2 * K + 1)
    if cfg.get("unrolled"):
        # 2K + 2 sweeps of cost recompute (2d) and one gradient product (2d), plus the
        # centroid sweeps' gO.V (2d each) and P^T gO (2d); two exponentials a sweep
        f_bwd = E * d * (8 * K + 16)
        x_bwd = E * (4 * K + 3)
    else:
        f_bwd = E * d * (14 + 2 * ncg)
        x_bwd = E * (ncg + 2)
    return E, f_fwd, f_bwd, x_fwd, x_bwd


def profiled_traffic(kernel, profile="sinkhorn_cfg2_bench.md", key="hbm_bytes_per_launch"):
    """HBM bytes per launch of ``kernel`` (or per step, key "hbm_bytes") from a committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated against a copy kernel), or None."""
    import re

    path = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(path):
        return None
    m = re.search(rf"^\s*{kernel} {key} = (\d+)", open(path).read(), flags=re.M)
    return int(m.group(1)) if m else None


def _head_inputs(cfg, cpu, b, h, K_iter):
    n = cpu["lengths"][b]
    sl = lambda a: a[b:b + 1, h:h + 1, :n].float().numpy()
    return dict(Q=sl(cpu["Q"]), K=sl(cpu["K"]), V=sl(cpu["V"]), G=sl(cpu["G"]),
                x_res=cpu["x_res"][b:b + 1, :n].numpy(), pos_weight=cpu["pos_weight"][h:h + 1].numpy(),
                pos_bins=None if cpu.get("pos_bins") is None else cpu["pos_bins"][b:b + 1, :n, :n].numpy(),
                eps=cpu["eps"][h:h + 1].numpy(), w_dist=cpu["w_dist"][h:h + 1].numpy(),
                log_mu=cpu["log_mu"][b:b + 1, h:h + 1, :n].numpy(),
                log_nu=cpu["log_nu"][b:b + 1, h:h + 1, :n].numpy(),
                K_iter=K_iter, lam=1.0, r_0=10.0)


def host_cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_torch(cfg, cpu, reps=3):
    """The reference CPU fallback's algorithm restated densely in torch (float32, all
    host cores): per sample on its valid tokens, all heads at once, the dense forward
    (K log-domain iterations, flash_sinkhorn_attn.py:144-218) and the reference-mode
    IFT backward with K_back = K_iter Gauss-Seidel sweeps (:246-667), i.e.
    oracle/sinkhorn_dense_torch.forward + backward(solver="fixed_point").  One warm-up
    layer, then the median of `reps` layers."""
    import statistics

    import torch

    sys.path.insert(0, ROOT)
    from oracle import sinkhorn_dense_torch as dense

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B, H, d, K = cfg["B"], cfg["H"], cfg["d"], cfg["K_iter"]
    lengths = cpu["lengths"]
    f32 = lambda x: x.float()

    def layer():
        t0 = time.perf_counter()
        for b, n in enumerate(lengths):
            sl = lambda a: f32(a[b:b + 1, :, :n]).contiguous()
            q, k, v, g = sl(cpu["Q"]), sl(cpu["K"]), sl(cpu["V"]), sl(cpu["G"])
            lmu, lnu = f32(cpu["log_mu"][b:b + 1, :, :n]), f32(cpu["log_nu"][b:b + 1, :, :n])
            eps = f32(cpu["eps"])
            fo = dense.forward(q, k, v, g, eps, lmu, lnu, K)
            go = f32(cpu["dO"][b:b + 1, :n]).contiguous()
            dense.backward(q, k, v, g, eps, fo, go, K, solver="fixed_point")
        return time.perf_counter() - t0

    with torch.no_grad():
        layer()
        times = [layer() for _ in range(reps)]
    med = statistics.median(times)
    return dict(value=round(med * 1e3, 1), unit="ms/layer", cores=cores, kind="port",
                sample=(f"CPU restatement of the reference fallback (oracle/sinkhorn_dense_torch.py): dense forward "
                        f"K={K} + reference fixed-point IFT backward ({K} sweeps), float32 torch on {cores} threads "
                        f"({host_cpu_model()}), the whole layer (n_b={lengths}, {H} heads), 1 warm-up + median of "
                        f"{reps} ({', '.join(f'{x * 1e3:.0f}' for x in times)} ms)"))


def cpu_baseline(cfg, cpu, budget_s=12.0):
    """The numpy oracle (float32, one thread) on a bounded sample of the layer:
    dense forward + the reference's fixed-point IFT backward (K_back = K_iter
    sweeps, flash_sinkhorn_attn.py:471-542) of whole (b, h) heads.

    cfg2: full heads (K = 50), cycling over the heads until ~budget_s of CPU time
    is spent, scaled to one layer by valid plan elements.
    cfg5: one head at K = 4 and K = 12; the per-iteration slope and the intercept
    are extrapolated to K = 100 and scaled to the 16 heads (labelled as such)."""
    import numpy as np

    try:
        from threadpoolctl import threadpool_limits
    except Exception:  # pragma: no cover
        threadpool_limits = None
    sys.path.insert(0, ROOT)
    from oracle import sinkhorn as ref

    B, H, d, K = cfg["B"], cfg["H"], cfg["d"], cfg["K_iter"]
    lengths = cpu["lengths"]
    ctx = threadpool_limits(limits=1) if threadpool_limits else None

    def one_head(b, h, k_iter):
        inp = _head_inputs(cfg, cpu, b, h, k_iter)
        n = lengths[b]
        go = cpu["dO"].reshape(B, -1, H, d)[b:b + 1, :n, h, :].numpy()
        t0 = time.perf_counter()
        fo = ref.forward(**inp, dtype=np.float32)
        ref.backward_reference(inp, fo, go, None, K_back=k_iter, dtype=np.float32)
        return time.perf_counter() - t0

    try:
        if not cfg["dirichlet"]:
            spent, heads = 0.0, []
            for b, h in [(b, h) for h in range(H) for b in range(B)] * 64:  # alternate samples
                spent += one_head(b, h, K)
                heads.append((b, h))
                if spent > budget_s:
                    break
            e_all = sum(H * n * n for n in lengths)
            e_smp = sum(lengths[b] ** 2 for b, _ in heads)
            value = spent * e_all / e_smp
            sample = (f"numpy oracle (float32, 1 thread): dense forward K={K} + reference fixed-point IFT backward "
                      f"({K} sweeps), {len(heads)} (b,h) head solves cycling over the layer's {B * H} heads "
                      f"({spent:.1f} s), scaled to one layer by valid plan elements")
        else:
            k1, k2 = 4, 12
            t1, t2 = one_head(0, 0, k1), one_head(0, 0, k2)
            slope = (t2 - t1) / (k2 - k1)
            per_head = t1 + slope * (K - k1)
            value = per_head * B * H
            sample = (f"numpy oracle (float32, 1 thread), one ({lengths[0]}-token) head: forward + reference "
                      f"fixed-point IFT backward at K=K_back={k1} ({t1:.1f} s) and {k2} ({t2:.1f} s), "
                      f"linearly extrapolated to K=K_back={K} and scaled to {B * H} heads")
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    return dict(value=round(value * 1e3, 1), unit="ms/layer", cores=1, kind="port", sample=sample)


def unrolled_cpu_baseline(cfg, cpu, budget_s=12.0):
    """Autograd through the dense iteration (the oracle's restatement of
    sinkhorn.py:17-198, the CPU form of the unrolled gradient), float32 torch on
    all host threads, one (b, h) head at a time on its valid tokens, cycling over
    the layer's heads for about budget_s and scaled to the layer by valid elements."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import sinkhorn_dense_ref as dref

    B, H, d, K = cfg["B"], cfg["H"], cfg["d"], cfg["K_iter"]
    lengths = cpu["lengths"]
    spent, heads = 0.0, []
    for b, h in [(b, h) for h in range(H) for b in range(B)]:
        n = lengths[b]
        sl = lambda t: t[b:b + 1, h:h + 1, :n].float().clone().requires_grad_(True)
        q, k, v = sl(cpu["Q"]), sl(cpu["K"]), sl(cpu["V"])
        g = cpu["G"][b:b + 1, h:h + 1, :n].float()
        go = cpu["dO"].reshape(B, -1, H, d)[b:b + 1, :n, h, :]
        t0 = time.perf_counter()
        C = -(q @ k.transpose(-1, -2)) / math.sqrt(d)
        lu, lv = dref.sinkhorn_solve(C, cpu["log_mu"][b:b + 1, h:h + 1, :n], cpu["log_nu"][b:b + 1, h:h + 1, :n],
                                     cpu["eps"][h:h + 1], K=K)
        o, _, _ = dref.compute_transport_output(v, g, lu, lv, C, cpu["eps"][h:h + 1])
        (o * go).sum().backward()
        spent += time.perf_counter() - t0
        heads.append((b, h))
        if spent > budget_s:
            break
    e_all = sum(H * n * n for n in lengths)
    e_smp = sum(lengths[b] ** 2 for b, _ in heads)
    th = torch.get_num_threads()
    return dict(value=round(spent * e_all / e_smp * 1e3, 1), unit="ms/layer", cores=th, kind="port",
                sample=f"autograd through the dense oracle iteration (float32 torch, {th} threads), K={K}, "
                       f"{len(heads)} (b,h) heads ({spent:.1f} s), scaled to the layer by valid plan elements")


def bench_sinkhorn(args, name):
    import torch
    from deepfold_amd import _lib

    cfg = SINKHORN[name]
    dev = torch.device("cuda:0")
    cpu, t = make_workload(cfg, dev)
    # warmup: every launch bracketed by events, for the per-kernel breakdown and to
    # find the dominant kernel
    _lib.launch_timings, _lib.launch_timed = [], None
    for _ in range(max(args.warmup, 1)):
        step(cfg, t)
    torch.cuda.synchronize()
    per = {}
    for kname, s, e in _lib.launch_timings:
        per.setdefault(kname, []).append(s.elapsed_time(e))
    # median: the first warmup launch carries one-time costs (code object load)
    avg = {k: float(sorted(v)[len(v) // 2]) for k, v in per.items()}
    dom = max(avg, key=avg.get)

    # timed region: exactly `steps` steps; events (on the launch stream) bracket only the
    # dominant kernel's launches, whose average gives the roofline (an event pair around
    # every launch costs a few microseconds of stream time per launch)
    _lib.launch_timings, _lib.launch_timed = [], {dom}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(cfg, t)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    timings = _lib.launch_timings
    _lib.launch_timings, _lib.launch_timed = None, None
    import deepfold_amd

    deepfold_amd.check_errors(dev)  # raises if any timed kernel gave up on a cross-workgroup wait
    dom_ms = [s.elapsed_time(e) for kname, s, e in timings if kname == dom]
    avg[dom] = sum(dom_ms) / len(dom_ms)
    ms_per_step = wall * 1e3 / args.steps

    E, f_fwd, f_bwd, x_fwd, x_bwd = algorithmic_counts(cfg, cpu["lengths"])
    f_dom = f_fwd if dom == "sinkhorn_fwd" else f_bwd
    x_dom = x_fwd if dom == "sinkhorn_fwd" else x_bwd
    achieved = f_dom / (avg[dom] * 1e-3)
    traffic = profiled_traffic(dom, {"cfg2": "sinkhorn_cfg2_bench.md", "cfg2-unrolled": "unrolled_cfg2_bench.md"}
                               .get(name, f"sinkhorn_{name}_bench.md"))
    peak = PEAK_MFMA_BF16  # bf16 inputs: both backwards run their products on the bf16 MFMA
    t_roof = max((f_fwd + f_bwd) / PEAK_MFMA_BF16, (x_fwd + x_bwd) / PEAK_SWEEP_ELEMENT_MEASURED)
    metric = ("flash-Sinkhorn fwd+IFT-bwd ms/layer @B2,H8,N768,d32 bf16; % of MFMA/HBM roof" if name == "cfg2"
              else f"flash-Sinkhorn fwd+{'unrolled' if cfg.get('unrolled') else 'IFT'}-bwd ms/layer "
                   f"@B{cfg['B']},H{cfg['H']},N{cfg['N']},d{cfg['d']} bf16")
    out = {
        "metric": metric,
        "value": round(ms_per_step, 4),
        "unit": "ms/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": (f"synthetic (seed {cfg['seed']}): Q,K,V ~ N(0,1)/sqrt(d), "
                 + ("ragged n_b ~ U[384,768], " if cfg["ragged"] else "Dirichlet(5) marginals, ")
                 + "dO ~ N(0,1)"),
        "config": {"workload": cfg["workload"], "B": cfg["B"], "H": cfg["H"], "N": cfg["N"], "d": cfg["d"],
                   "n_b": cpu["lengths"], "eps": cfg["eps"], "K_iter": cfg["K_iter"], "n_cg": cfg["n_cg"],
                   "valid_plan_elements": E},
        "kernel_ms": {k: round(v, 4) for k, v in avg.items()},
        "kernel_ms_from": f"{dom}: mean over the timed steps; the others: median over the warmup steps",
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved / 1e12, 3),
                     "peak": peak / 1e12, "unit": "TFLOP/s", "frac": round(achieved / peak, 5),
                     "traffic": traffic},
        "roofline_exp": {"kernel": dom, "achieved": x_dom / (avg[dom] * 1e-3), "peak": PEAK_EXP_MEASURED,
                         "unit": "exp/s", "frac": x_dom / (avg[dom] * 1e-3) / PEAK_EXP_MEASURED,
                         "element_peak": PEAK_SWEEP_ELEMENT_MEASURED,
                         "element_frac": x_dom / (avg[dom] * 1e-3) / PEAK_SWEEP_ELEMENT_MEASURED,
                         "layer_t_roof_ms": t_roof * 1e3, "layer_frac": t_roof * 1e3 / ms_per_step},
    }
    out["kernel_errors"] = 0  # check_errors passed after the timed steps
    if cfg["N"] <= 1024:
        # after and outside the timed region: the same step, checked against the oracle
        res = step(cfg, t, want=True)
        deepfold_amd.check_errors(dev)
        out["parity_check"] = verify_head(cfg, cpu, res)
    else:
        out["parity_check"] = {"skipped": "the float64 oracle needs minutes per N=4096 head; this workload's parity "
                                          "is tested in tests/test_gpu_sinkhorn_stream.py"}
    if not args.no_cpu_baseline:
        if cfg.get("unrolled"):
            out["cpu_baseline"] = unrolled_cpu_baseline(cfg, cpu)
        elif name == "cfg2":
            out["cpu_baseline"] = cpu_baseline_torch(cfg, cpu)
        else:
            out["cpu_baseline"] = cpu_baseline(cfg, cpu)
    print(json.dumps(out), flush=True)


def rocpd_summary(db_path):
    """Markdown table (calls, total/avg/min/max us, share) of every kernel in a
    rocprofv3 results database; used for the committed profiles/ summaries."""
    import sqlite3

    con = sqlite3.connect(db_path)
    short = lambda name: name if len(name) <= 90 else name[:87] + "..."
    rows = con.execute("select name, count(*), sum(duration), avg(duration), min(duration), max(duration) "
                       "from kernels group by name order by sum(duration) desc").fetchall()
    if rows:
        total = sum(r[2] for r in rows) or 1
        print("| kernel | calls | total us | avg us | min us | max us | % |")
        print("|---|---|---|---|---|---|---|")
        for name, n, tot, avg, mn, mx in rows:
            print(f"| `{short(name)}` | {n} | {tot / 1e3:.1f} | {avg / 1e3:.2f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} | "
                  f"{100.0 * tot / total:.1f} |")
    pmc = con.execute("select name, counter_name, count(*), avg(counter_value), min(counter_value), "
                      "max(counter_value) from pmc_events group by name, counter_name "
                      "order by name, counter_name").fetchall()
    if pmc:
        print("| kernel | counter | dispatches | avg per dispatch | min | max |")
        print("|---|---|---|---|---|---|")
        for name, counter, n, avg, mn, mx in pmc:
            print(f"| `{short(name)}` | {counter} | {n} | {avg:.1f} | {mn:.1f} | {mx:.1f} |")


def attention_workload(which, dev):
    """BASELINE configs[2] (diffusion attention, dense pair bias + gate) and
    configs[3] (atom-window attention with window bias; token-to-atom cross
    attention), synthetic data, seed 1000 + config#.  Returns (step_fn, info)."""
    import torch
    from deepfold_amd import flash_atom_attn, flash_diffusion_attn, token_to_atom_attn

    bf = torch.bfloat16
    if which == "cfg3":
        B, H, N, D = 1, 16, 1024, 24
        g = torch.Generator().manual_seed(1003)
        Q, K, V = ((torch.randn(B, H, N, D, generator=g) / math.sqrt(D)).to(bf).to(dev) for _ in range(3))
        G = torch.randn(B, H, N, D, generator=g).to(bf).to(dev)
        bias = torch.randn(B, H, N, N, generator=g).to(bf).to(dev)
        dO = torch.randn(B, H, N, D, generator=g).to(bf).to(dev)

        def step():
            q, k, v, gg, bb = (t.detach().requires_grad_(True) for t in (Q, K, V, G, bias))
            flash_diffusion_attn(q, k, v, None, None, pair_bias=bb, gate=gg).backward(dO)

        e = 2  # bf16 bytes
        bytes_alg = 3 * H * N * N * e + 10 * B * H * N * D * e  # bias read fwd+bwd, dbias write; Q,K,V,G,O,dO,dQ,dK,dV,dG
        flops = 14 * B * H * N * N * D
        info = dict(workload="BASELINE configs[2]: flash diffusion attention fwd+bwd, dense pair bias + gate",
                    B=B, H=H, N=N, d=D)
        return step, info, bytes_alg, flops
    if which == "cfg4":
        H, D, M, NT = 4, 32, 8192, 341
        W = M // 32
        g = torch.Generator().manual_seed(1004)
        Qa, Ka, Va = ((torch.randn(1, H, M, D, generator=g) / math.sqrt(D)).to(bf).to(dev) for _ in range(3))
        wb = torch.randn(W, H, 32, 128, generator=g).to(bf).to(dev)
        Kt, Vt = ((torch.randn(1, H, NT, D, generator=g) / math.sqrt(D)).to(bf).to(dev) for _ in range(2))
        dOa = torch.randn(1, H, M, D, generator=g).to(bf).to(dev)
        dOc = torch.randn(1, H, M, D, generator=g).to(bf).to(dev)

        def step():
            q, k, v, bb = (t.detach().requires_grad_(True) for t in (Qa, Ka, Va, wb))
            flash_atom_attn(q, k, v, window_bias=bb).backward(dOa)
            q2, k2, v2 = (t.detach().requires_grad_(True) for t in (Qa, Kt, Vt))
            token_to_atom_attn(q2, k2, v2).backward(dOc)

        e = 2
        bytes_alg = (3 * W * H * 32 * 128 * e + 8 * H * M * D * e) + (6 * H * M * D * e + 4 * H * NT * D * e)
        flops = 14 * H * M * 128 * D + 14 * H * M * NT * D
        info = dict(workload="BASELINE configs[3]: atom-window attention (window bias) + token-to-atom attention, "
                             "fwd+bwd", M=M, H=H, d=D, tokens=NT)
        return step, info, bytes_alg, flops
    raise SystemExit(f"unknown workload {which}")


def bench_attention(args, which):
    import torch
    from deepfold_amd import _lib

    dev = torch.device("cuda:0")
    step, info, bytes_alg, flops = attention_workload(which, dev)
    # warmup (eager): every launch bracketed by events, for the per-kernel breakdown
    # (per step: the median over the warmup steps; the first step loads code objects)
    steps_ms = []
    for _ in range(max(args.warmup, 1)):
        _lib.launch_timings = []
        step()
        torch.cuda.synchronize()
        one = {}
        for name, s_, e_ in _lib.launch_timings:
            one[name] = one.get(name, 0.0) + s_.elapsed_time(e_)
        steps_ms.append(one)
    _lib.launch_timings = None
    kernel_ms = {k: sorted(d.get(k, 0.0) for d in steps_ms)[len(steps_ms) // 2] for k in steps_ms[-1]}
    # eager step (Python autograd glue on every call: host-bound at these sizes)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    if args.eager:  # profiling runs: the eager calls are the timed region
        ms = eager_ms
    else:
        # timed region: the same step captured once in a HIP graph (the attention entry
        # points allocate nothing inside a call and record no memset), replayed `steps` times
        cur = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            step()
        cur.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        # captured on the warm-up stream, whose cached workspace then exists: no
        # allocation or zero fill is recorded into the graph
        with torch.cuda.graph(graph, stream=side):
            step()
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
    _lib.raise_pending("attention bench")
    dev_ms = ms  # the roofline over the timed step: its kernels and the gaps between them
    out = {
        "metric": f"{which} attention fwd+bwd ms/step", "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seed 1000 + config#)",
        "config": info,
        "timed": "eager Python calls" if args.eager else "HIP graph replays of the captured fwd+bwd step",
        "eager_ms_per_step": round(eager_ms, 4),
        "kernel_ms_per_step": {k: round(v, 4) for k, v in kernel_ms.items()},
        "roofline": {"bound": "hbm", "achieved": round(bytes_alg / (dev_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": round(bytes_alg / (dev_ms * 1e-3) / PEAK_HBM, 4),
                     "traffic": profiled_traffic("attention_step", f"attention_{which}_bench.md", "hbm_bytes"),
                     "traffic_per": "step (sum over the step's kernels)", "algorithmic_bytes": bytes_alg},
        "mfma": {"achieved_tflops": round(flops / (dev_ms * 1e-3) / 1e12, 2), "peak_tflops": PEAK_MFMA_BF16 / 1e12},
    }
    print(json.dumps(out), flush=True)


def balanced_workload(dev):
    """TokenOTBlock's balanced transport (trunk_block.py:164-186): Q_s, K_s
    L2-normalised, V_s, x_res, the trunk's eps buffer (0.5/1/2/4 per quarter of
    the heads), alpha_h = -1 and r_h = 10 (their initial values), no padding,
    K_ITER = 20; seed 1006."""
    import torch
    import torch.nn.functional as F

    B, H, N, d, K = 1, 16, 256, 32, 20
    g = torch.Generator().manual_seed(1006)
    cpu = dict(Q=F.normalize(torch.randn(B, H, N, d, generator=g), dim=-1),
               K=F.normalize(torch.randn(B, H, N, d, generator=g), dim=-1),
               V=torch.randn(B, H, N, d, generator=g), x=torch.randn(B, N, 3, generator=g) * 3.0,
               eps=torch.tensor([0.5] * 4 + [1.0] * 4 + [2.0] * 4 + [4.0] * 4),
               alpha=torch.full((H,), -1.0), r=torch.full((H,), 10.0), mask=torch.ones(B, N),
               gx=torch.randn(B, H, N, 3, generator=g), gh=torch.randn(B, H, N, d, generator=g))
    t = {k: v.to(dev) for k, v in cpu.items()}
    cfg = dict(B=B, H=H, N=N, d=d, K_iter=K)
    return cfg, cpu, t


def balanced_counts(cfg):
    """Algorithmic work of one fwd+bwd (no padding: E = H N^2 per sample).
    Forward: 2K LSE sweeps (QK^T, 2d flops / element) + output sweep (QK^T and
    P V, 4d).  Backward: 2K+1 sweeps of cost recompute (2d) and one gradient
    product (2d), plus the centroid sweeps' dhc.V (2d each) and P^T dhc (2d).
    Exponentials: forward 2K+1, backward 4K+1 per element."""
    E = cfg["B"] * cfg["H"] * cfg["N"] ** 2
    d, K = cfg["d"], cfg["K_iter"]
    f_fwd = E * d * (4 * K + 4)
    f_bwd = E * d * (8 * K + 10)
    return E, f_fwd, f_bwd, E * (2 * K + 1), E * (4 * K + 1)


def balanced_cpu_baseline(cpu, cfg, reps=3):
    """The oracle's restatement of the reference CPU path (_sinkhorn_cpu under
    autograd, flash_sinkhorn_transport.py:253-282, 397-399) in float32 torch on
    all host threads: forward + backward of the same workload, median of `reps`."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import balanced_transport as bt

    threads = torch.get_num_threads()
    times = []
    for _ in range(reps + 1):
        leaves = {k: cpu[k].clone().requires_grad_(True) for k in ("Q", "K", "x", "V", "alpha", "r")}
        t0 = time.perf_counter()
        xc, hc = bt.sinkhorn_cpu(leaves["Q"], leaves["K"], leaves["x"], cpu["eps"], leaves["alpha"], leaves["r"],
                                 cpu["mask"], cfg["N"], cfg["K_iter"], V_h=leaves["V"])
        ((xc * cpu["gx"]).sum() + (hc * cpu["gh"]).sum()).backward()
        times.append(time.perf_counter() - t0)
    times = sorted(times[1:])
    return dict(value=round(times[len(times) // 2] * 1e3, 2), unit="ms/step", cores=threads, kind="port",
                sample=f"oracle restatement of _sinkhorn_cpu (float32 torch autograd, {threads} threads), full "
                       f"workload, median of {reps} after one warm-up")


def bench_balanced(args):
    import torch
    from deepfold_amd import _lib, balanced_sinkhorn_transport_dual

    dev = torch.device("cuda:0")
    cfg, cpu, t = balanced_workload(dev)

    def step():
        q, k, x, v, a, r = (t[n].detach().requires_grad_(True) for n in ("Q", "K", "x", "V", "alpha", "r"))
        xc, hc = balanced_sinkhorn_transport_dual(q, k, x, v, t["eps"], a, r, K_iter=cfg["K_iter"], mask=t["mask"])
        torch.autograd.backward((xc, hc), (t["gx"], t["gh"]))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _lib.launch_timings = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = {}
    for name, s_, e_ in _lib.launch_timings:
        per.setdefault(name, []).append(s_.elapsed_time(e_))
    _lib.launch_timings = None
    avg = {k: sum(v) / len(v) for k, v in per.items()}
    ms = wall * 1e3 / args.steps
    E, f_fwd, f_bwd, x_fwd, x_bwd = balanced_counts(cfg)
    dom = max(avg, key=avg.get)
    f_dom = f_fwd if dom == "balanced_fwd" else f_bwd
    x_dom = x_fwd if dom == "balanced_fwd" else x_bwd
    achieved = f_dom / (avg[dom] * 1e-3)
    t_roof = max((f_fwd + f_bwd) / PEAK_MFMA_F32, (x_fwd + x_bwd) / PEAK_SWEEP_ELEMENT_MEASURED)
    out = {
        "metric": "balanced Sinkhorn transport (dual) fwd+bwd ms/step @B1,H16,N256,d32 fp32 K20",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seed 1006): Q,K L2-normalised N(0,1), V, x*3, upstream grads N(0,1)",
        "config": {"workload": "TokenOTBlock balanced transport, balanced_sinkhorn_transport_dual fwd+bwd",
                   "B": cfg["B"], "H": cfg["H"], "N": cfg["N"], "d": cfg["d"], "K_iter": cfg["K_iter"],
                   "valid_plan_elements": E},
        "kernel_ms": {k: round(v, 4) for k, v in avg.items()},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved / 1e12, 3),
                     "peak": PEAK_MFMA_F32 / 1e12, "unit": "TFLOP/s", "frac": round(achieved / PEAK_MFMA_F32, 5),
                     "traffic": profiled_traffic(dom, "balanced_tokenot_bench.md")},
        "roofline_exp": {"kernel": dom, "achieved": x_dom / (avg[dom] * 1e-3), "peak": PEAK_EXP_MEASURED,
                         "unit": "exp/s", "frac": x_dom / (avg[dom] * 1e-3) / PEAK_EXP_MEASURED,
                         "step_t_roof_ms": t_roof * 1e3, "step_frac": t_roof * 1e3 / ms},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = balanced_cpu_baseline(cpu, cfg)
    print(json.dumps(out), flush=True)


def tokenot_block(C, H, seed, dev):
    """The parameters TokenOTBlock holds for its transport steps (trunk_block.py:65-96):
    LayerNorms near identity, Linear weights N(0, 1/C), alpha_h = -1, r_h = 10,
    lambda_h_raw = 0.5, the trunk's eps buffer."""
    import torch

    g = torch.Generator().manual_seed(seed)
    blk = torch.nn.Module()
    blk.n_heads, blk.feature_transport = H, True
    blk.ln_sink, blk.ln_gate = torch.nn.LayerNorm(C), torch.nn.LayerNorm(C)
    for n in ("w_q_sink", "w_k_sink", "w_v_sink", "w_o_sink"):
        setattr(blk, n, torch.nn.Linear(C, C, bias=False))
    blk.w_gate = torch.nn.Linear(C, 1, bias=True)
    with torch.no_grad():
        for ln in (blk.ln_sink, blk.ln_gate):
            ln.weight.copy_(1 + 0.1 * torch.randn(C, generator=g))
            ln.bias.copy_(0.1 * torch.randn(C, generator=g))
        for lin in (blk.w_q_sink, blk.w_k_sink, blk.w_v_sink, blk.w_o_sink, blk.w_gate):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) / C ** 0.5)
        blk.w_gate.bias.zero_()
    blk.alpha_h = torch.nn.Parameter(torch.full((H,), -1.0))
    blk.r_h = torch.nn.Parameter(torch.full((H,), 10.0))
    blk.lambda_h_raw = torch.nn.Parameter(torch.full((H,), 0.5))
    nr = H // 4
    blk.register_buffer("eps", torch.tensor([0.5] * nr + [1.0] * nr + [2.0] * nr + [4.0] * nr))
    return blk.to(dev)


def bench_tokenot_step(args):
    """TokenOTBlock steps 2-4 (trunk_block.py:165-204), fwd + bwd: sink projections ->
    balanced dual transport -> w_o_sink -> gated coordinate update (token_ot_transport_step),
    at the balanced workload's shape (B1 N256, d_model 512, H16, K = 20, fp32)."""
    import torch
    import torch.nn.functional as F
    from deepfold_amd import _lib, gated_coordinate_update, sink_projections, token_ot_transport_step

    dev = torch.device("cuda:0")
    B, N, C, H, K = 1, 256, 512, 16, 20
    blk = tokenot_block(C, H, 1007, dev)
    g = torch.Generator().manual_seed(1007)
    h0 = torch.randn(B, N, C, generator=g).to(dev)
    x0 = (torch.randn(B, N, 3, generator=g) * 3).to(dev)
    gh = torch.randn(B, N, C, generator=g).to(dev)
    gx = torch.randn(B, N, 3, generator=g).to(dev)
    xc_fixed = (torch.randn(B, H, N, 3, generator=g) * 3).to(dev)
    mask = torch.ones(B, N, device=dev)

    def step():
        h = h0.detach().requires_grad_(True)
        x = x0.detach().requires_grad_(True)
        ho, xo = token_ot_transport_step(blk, h, x, mask, K_iter=K)
        torch.autograd.backward((ho, xo), (gh, gx))

    def steps_hip():  # the two steps alone, around a fixed centroid
        h = h0.detach().requires_grad_(True)
        q, k, v = sink_projections(h, blk.ln_sink.weight, blk.ln_sink.bias, blk.w_q_sink.weight,
                                   blk.w_k_sink.weight, blk.w_v_sink.weight, H)
        xo = gated_coordinate_update(h, x0, xc_fixed, blk.ln_gate.weight, blk.ln_gate.bias, blk.w_gate.weight,
                                     blk.w_gate.bias, blk.lambda_h_raw, mask)
        torch.autograd.backward((q, k, v, xo), (q.detach(), k.detach(), v.detach(), gx))

    def steps_eager():  # the reference's eager form of the same two steps (trunk_block.py:165-175, 189-204)
        h = h0.detach().requires_grad_(True)
        hs = blk.ln_sink(h)
        heads = lambda u: u.view(B, N, H, C // H).permute(0, 2, 1, 3)
        q = F.normalize(heads(blk.w_q_sink(hs)), dim=-1)
        k = F.normalize(heads(blk.w_k_sink(hs)), dim=-1)
        v = heads(blk.w_v_sink(hs))
        vec = xc_fixed - x0.unsqueeze(1)
        gate = torch.sigmoid(blk.w_gate(blk.ln_gate(h)))
        lam = torch.tanh(blk.lambda_h_raw).view(1, H, 1, 1) / H
        xo = x0 + gate * (lam * vec).sum(dim=1) * mask.unsqueeze(-1)
        torch.autograd.backward((q, k, v, xo), (q.detach(), k.detach(), v.detach(), gx))

    def timed(fn, n):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    steps_hip_ms = timed(steps_hip, args.steps)
    steps_eager_ms = timed(steps_eager, args.steps)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _lib.launch_timings = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = {}
    for name, s_, e_ in _lib.launch_timings:
        per.setdefault(name, []).append(s_.elapsed_time(e_))
    _lib.launch_timings = None
    avg = {k: sum(v) / len(v) for k, v in per.items()}
    ms = wall * 1e3 / args.steps
    # projections: 2 M C^2 flops per projection forward (3 of them); backward twice that
    M = B * N
    f_proj = 3 * 2 * M * C * C
    pf = f_proj / (avg["sink_proj_fwd"] * 1e-3)
    pb = 2 * f_proj / (avg["sink_proj_bwd"] * 1e-3)
    bcfg = dict(B=B, H=H, N=N, d=C // H, K_iter=K)
    E, f_fwd, f_bwd, _, _ = balanced_counts(bcfg)
    dom = max(avg, key=avg.get)
    f_dom = {"balanced_fwd": f_fwd, "balanced_bwd": f_bwd, "sink_proj_fwd": f_proj,
             "sink_proj_bwd": 2 * f_proj}.get(dom)
    achieved = f_dom / (avg[dom] * 1e-3) if f_dom else None
    out = {
        "metric": "TokenOTBlock transport steps (projections, balanced transport, coordinate update) fwd+bwd "
                  "ms/step @B1,N256,C512,H16 fp32 K20",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seed 1007): h ~ N(0,1), x_res ~ N(0,3^2), parameters near init, "
                                "upstream grads N(0,1)",
        "config": {"workload": "TokenOTBlock steps 2-4, token_ot_transport_step fwd+bwd", "B": B, "N": N, "C": C,
                   "H": H, "K_iter": K},
        "kernel_ms": {k: round(v, 4) for k, v in avg.items()},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": None if achieved is None else round(achieved / 1e12, 3),
                     "peak": PEAK_MFMA_F32 / 1e12, "unit": "TFLOP/s",
                     "frac": None if achieved is None else round(achieved / PEAK_MFMA_F32, 5),
                     "traffic": profiled_traffic(dom, "balanced_tokenot_bench.md")},
        "roofline_projections": {"fwd_tflops": round(pf / 1e12, 3), "bwd_tflops": round(pb / 1e12, 3),
                                 "peak": PEAK_MFMA_F32 / 1e12, "unit": "TFLOP/s (fp32 MFMA)"},
        "steps_only_ms": {"hip": round(steps_hip_ms, 4), "torch_eager": round(steps_eager_ms, 4),
                          "what": "projections + coordinate update fwd+bwd around a fixed centroid; torch_eager is "
                                  "the reference's eager formulation on the same GPU"},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = tokenot_cpu_baseline(blk, h0, x0, mask, gh, gx, K)
    print(json.dumps(out), flush=True)


def tokenot_cpu_baseline(blk, h0, x0, mask, gh, gx, K):
    """oracle/trunk_steps.transport_step (float32 torch autograd on the host threads),
    one full step, median of 3."""
    import torch
    sys.path.insert(0, ROOT)
    from oracle import trunk_steps as ts

    P = {"ln_sink_w": blk.ln_sink.weight, "ln_sink_b": blk.ln_sink.bias, "w_q": blk.w_q_sink.weight,
         "w_k": blk.w_k_sink.weight, "w_v": blk.w_v_sink.weight, "w_o": blk.w_o_sink.weight, "eps": blk.eps,
         "alpha_h": blk.alpha_h, "r_h": blk.r_h, "ln_gate_w": blk.ln_gate.weight, "ln_gate_b": blk.ln_gate.bias,
         "w_gate": blk.w_gate.weight, "b_gate": blk.w_gate.bias, "lambda_raw": blk.lambda_h_raw}
    R = {k: v.detach().float().cpu().requires_grad_(k != "eps") for k, v in P.items()}
    times = []
    for _ in range(3):
        h = h0.detach().cpu().requires_grad_(True)
        x = x0.detach().cpu().requires_grad_(True)
        t0 = time.perf_counter()
        ho, xo = ts.transport_step(R, h, x, mask.cpu(), blk.n_heads, K_iter=K)
        torch.autograd.backward((ho, xo), (gh.cpu(), gx.cpu()))
        times.append((time.perf_counter() - t0) * 1e3)
    times.sort()
    return {"value": round(times[1], 2), "unit": "ms/step", "cores": torch.get_num_threads(), "kind": "port",
            "sample": "the oracle's restatement of trunk_block.py:165-204 (with _sinkhorn_cpu) under torch "
                      "autograd, float32, one full step, median of 3"}


def bench_peaks():
    """Measured issue rates of the instructions the Sinkhorn sweeps are made of, and
    the exchange round of a 16-member group (csrc/peaks.hip), one JSON line each.
    Every probe runs one 512-thread workgroup per CU (two waves per SIMD, as the
    Sinkhorn kernels do) on all 256 CUs; rates come from HIP events around the launch,
    `clk_per_wave_op` from clock64() (per SIMD, both waves' instructions counted)."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "deepfold-linear_amd", "deepfold_amd", "libdfl_peaks.so"))
    run = lib.dfl_peak_run
    run.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_float),
                    ctypes.POINTER(ctypes.c_longlong)]
    run.restype = ctypes.c_int
    blocks, lanes = 256, 512

    def probe(mode, iters):
        ms, clk = ctypes.c_float(), ctypes.c_longlong()
        for _ in range(2):  # the first launch loads the code object
            rc = run(mode, blocks, iters, ctypes.byref(ms), ctypes.byref(clk))
            if rc:
                raise SystemExit(f"peaks: probe {mode} failed with code {rc}")
        return ms.value * 1e-3, clk.value

    rows = [(0, 100000, "v_exp_f32 (exp2) issue rate", "exp/s", 24, 1.0),
            (1, 100000, "v_fma_f32 issue rate", "FLOP/s", 24, 2.0),
            (3, 50000, "fixed-shift sweep element: s += exp2(x * a + w) (fma + exp + add)", "elements/s", 24, 1.0)]
    for mode, iters, what, unit, per, scale in rows:
        t, clk = probe(mode, iters)
        n = blocks * lanes * iters * per
        print(json.dumps({"probe": what, "value": n * scale / t, "unit": unit, "ms": t * 1e3,
                          "clk_per_wave_op": clk / (iters * per * 2)}), flush=True)
    t, clk = probe(2, 200000)
    flops = blocks * 8 * 200000 * 6 * 16 * 16 * 32 * 2
    print(json.dumps({"probe": "v_mfma_f32_16x16x32_bf16, 6 independent accumulators per wave", "value": flops / t,
                      "unit": "FLOP/s", "ms": t * 1e3, "frac_of_published": flops / t / PEAK_MFMA_BF16,
                      "clk_per_wave_op": clk / (200000 * 6 * 2)}), flush=True)
    rounds = 2000
    t, clk = probe(4, rounds)
    print(json.dumps({"probe": "exchange round: 16 workgroups on one XCD each publish 48 tagged words and poll "
                               "the group's 768 (16 groups)", "value": t * 1e6 / rounds, "unit": "us/round",
                      "clk_per_round": clk / rounds}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="cfg3 / cfg4: time the eager Python calls instead of HIP graph replays")
    ap.add_argument("--storage", default="auto", choices=["auto", "register", "resident", "stream"],
                    help="where the Sinkhorn forward keeps the cost (flash_sinkhorn_attn storage=)")
    ap.add_argument("--workload", default="cfg2",
                    choices=["cfg2", "cfg5", "cfg2-full", "cfg2-unrolled", "cfg3", "cfg4", "balanced", "tokenot-step",
                             "peaks"],
                    help="cfg2 (default): the headline flash-Sinkhorn layer; cfg5: the N=4096 layer; "
                         "cfg3 / cfg4: attention rows; peaks: the issue-rate and exchange probes "
                         "(libdfl_peaks.so) behind the roofline figures")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB -> 256 MiB elementwise copy (torch.neg), used to "
                         "calibrate the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--rocpd-summary", metavar="DB", help="print the kernel table of a rocprofv3 results "
                    "database (no GPU needed) and exit")
    args = ap.parse_args()
    global STORAGE
    STORAGE = args.storage
    if args.rocpd_summary:
        rocpd_summary(args.rocpd_summary)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the flash-Sinkhorn "
              "path shards by (b, h) with no communication between GPUs", file=sys.stderr)
        sys.exit(2)

    import torch
    import deepfold_amd  # noqa: F401

    os.environ["DFL_AMD_CHECK"] = "0"
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        n = 64 << 20  # float32 elements: 256 MiB read + 256 MiB written per launch
        a = torch.ones(n, device=dev)
        b = torch.empty_like(a)
        for _ in range(5):
            torch.neg(a, out=b)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy": {"kernel": "torch.neg", "launches": 5, "read_bytes": 4 * n,
                                             "write_bytes": 4 * n}}), flush=True)
        return
    if args.workload == "peaks":
        bench_peaks()
    elif args.workload in SINKHORN:
        bench_sinkhorn(args, args.workload)
    elif args.workload == "balanced":
        bench_balanced(args)
    elif args.workload == "tokenot-step":
        bench_tokenot_step(args)
    else:
        bench_attention(args, args.workload)


if __name__ == "__main__":
    main()
