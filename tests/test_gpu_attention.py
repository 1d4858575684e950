"""GPU parity of the attention kernels (flash diffusion, atom-window, token<->atom)
against the float64 oracle (oracle/attention.py) on identical, dtype-rounded inputs.

Bars: normwise relative error (max |gpu - oracle| / max |oracle|) <= 1e-4 for fp32
inputs and <= 2e-2 for bf16 inputs, on outputs and every gradient.  Padded query
rows must be exactly zero.  Cases follow the reference's tests
(tests/test_flash_diffusion_attn.py, test_flash_atom_attn.py, test_cross_attn_kernel.py):
several shapes incl. non-power-of-two N and D=64, padding, unbatched inputs, and
gradient checks; plus the dense pair-bias / gate and window-bias extensions.
"""

import pytest
import torch

from conftest import max_rel_err
from oracle import attention as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def tol(dtype):
    return 2e-2 if dtype == torch.bfloat16 else 1e-4


def rnd(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def padded_mask(B, N, seed, max_pad):
    g = torch.Generator().manual_seed(seed)
    mask = torch.ones(B, N)
    for b in range(B):
        pad = int(torch.randint(0, max_pad + 1, (1,), generator=g))
        if pad:
            mask[b, N - pad:] = 0
    return mask


def run_gpu(fn, tensors: dict, grad_out, wrt, **kw):
    leaves = {}
    for k, v in tensors.items():
        if v is None:
            leaves[k] = None
            continue
        t = v.to(DEV)
        if k in wrt:
            t = t.detach().requires_grad_(True)
        leaves[k] = t
    out = fn(**leaves, **kw)
    if grad_out is not None:
        out.backward(grad_out.to(DEV).to(out.dtype))
    grads = {k: leaves[k].grad.float().cpu() for k in wrt}
    return out.detach().float().cpu(), grads


def check(name, got, want, t):
    err = max_rel_err(got.numpy(), want.numpy())
    assert err <= t, f"{name}: rel err {err:.3e} > {t:.1e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,H,N,D", [(1, 4, 64, 32), (2, 16, 128, 32), (1, 16, 384, 32), (2, 8, 97, 64), (1, 2, 50, 24)])
def test_diffusion_forward_backward(B, H, N, D, dtype):
    from deepfold_amd import flash_diffusion_attn

    Q, K, V = (rnd(B, H, N, D, seed=s, dtype=dtype) for s in (1, 2, 3))
    pw = rnd(H, 68, seed=4)
    bins = torch.randint(0, 68, (B, N, N), generator=torch.Generator().manual_seed(5), dtype=torch.int32)
    mask = padded_mask(B, N, seed=6, max_pad=N // 4)
    go = rnd(B, H, N, D, seed=7, dtype=dtype)
    inp = dict(Q=Q, K=K, V=V, pos_weight=pw, pos_bins=bins, mask=mask)
    out, g = run_gpu(flash_diffusion_attn, inp, go, ("Q", "K", "V", "pos_weight"))
    o_ref, g_ref = ref.grads(ref.diffusion_attn, {k: (v.double() if v.is_floating_point() else v)
                                                  for k, v in inp.items()}, go.double(),
                             ("Q", "K", "V", "pos_weight"))
    t = tol(dtype)
    check("O", out, o_ref, t)
    for b in range(B):
        n = int(mask[b].sum())
        assert torch.all(out[b, :, n:] == 0)
    for k in ("Q", "K", "V", "pos_weight"):
        check("d" + k, g[k], g_ref[k], t)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,D", [(160, 24), (150, 20), (96, 64)])
def test_diffusion_pair_bias_and_gate(N, D, dtype):
    """cfg3-shaped extension (smaller N): dense pair bias + sigmoid gate.  N = 150 is not
    a multiple of 8, so the kernels take their element-load staging (and D = 20 is not a
    whole number of 16-byte bf16 blocks); D = 64 runs the 64-wide head instantiations."""
    from deepfold_amd import flash_diffusion_attn

    B, H = 1, 4
    Q, K, V, G = (rnd(B, H, N, D, seed=s, dtype=dtype) for s in (11, 12, 13, 14))
    bias = rnd(B, H, N, N, seed=15, dtype=dtype)
    go = rnd(B, H, N, D, seed=16, dtype=dtype)
    inp = dict(Q=Q, K=K, V=V, pos_weight=None, pos_bins=None, pair_bias=bias, gate=G)
    out, g = run_gpu(flash_diffusion_attn, inp, go, ("Q", "K", "V", "pair_bias", "gate"))
    o_ref, g_ref = ref.grads(ref.diffusion_attn, {k: (None if v is None else v.double()) for k, v in inp.items()},
                             go.double(), ("Q", "K", "V", "pair_bias", "gate"))
    t = tol(dtype)
    check("O", out, o_ref, t)
    for k in ("Q", "K", "V", "pair_bias", "gate"):
        check("d" + k, g[k], g_ref[k], t)


def test_diffusion_unbatched_and_no_mask():
    from deepfold_amd import flash_diffusion_attn

    H, N, D = 8, 64, 32
    Q, K, V = (rnd(H, N, D, seed=s, dtype=torch.bfloat16) for s in (21, 22, 23))
    pw = rnd(H, 68, seed=24)
    bins = torch.randint(0, 68, (N, N), generator=torch.Generator().manual_seed(25), dtype=torch.int32)
    out = flash_diffusion_attn(Q.to(DEV), K.to(DEV), V.to(DEV), pw.to(DEV), bins.to(DEV))
    assert out.shape == (H, N, D) and out.dtype == torch.bfloat16
    want = ref.diffusion_attn(Q[None].double(), K[None].double(), V[None].double(), pw.double(), bins[None])[0]
    check("O", out.float().cpu(), want, 2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,H,M,D,with_mask,with_bias", [
    (1, 4, 256, 32, False, False), (2, 4, 100, 32, True, False), (1, 2, 75, 64, True, True),
    (1, 4, 512, 32, True, True), (3, 2, 150, 32, True, True)])
def test_atom_window_attention(B, H, M, D, with_mask, with_bias, dtype):
    from deepfold_amd import flash_atom_attn

    Q, K, V = (rnd(B, H, M, D, seed=s, dtype=dtype) for s in (31, 32, 33))
    mask = padded_mask(B, M, seed=34, max_pad=M // 4) if with_mask else None
    W = (M + 31) // 32
    wb = rnd(W, H, 32, 128, seed=35, dtype=dtype) if with_bias else None
    go = rnd(B, H, M, D, seed=36, dtype=dtype)
    inp = dict(Q=Q, K=K, V=V, mask=mask, window_bias=wb)
    wrt = ("Q", "K", "V") + (("window_bias",) if with_bias else ())
    out, g = run_gpu(flash_atom_attn, inp, go, wrt)
    o_ref, g_ref = ref.grads(ref.atom_attn, {k: (None if v is None else v.double()) for k, v in inp.items()},
                             go.double(), wrt)
    t = tol(dtype)
    check("O", out, o_ref, t)
    for k in wrt:
        check("d" + k, g[k], g_ref[k], t)
    if with_mask:
        for b in range(B):
            n = int(mask[b].sum())
            assert torch.all(out[b, :, n:] == 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,H,M,N,D", [(1, 4, 1000, 50, 32), (2, 2, 300, 77, 64), (1, 4, 2048, 341, 32)])
def test_token_to_atom(B, H, M, N, D, dtype):
    from deepfold_amd import token_to_atom_attn

    Q = rnd(B, H, M, D, seed=41, dtype=dtype)
    K, V = rnd(B, H, N, D, seed=42, dtype=dtype), rnd(B, H, N, D, seed=43, dtype=dtype)
    amask = padded_mask(B, M, seed=44, max_pad=M // 8)
    tmask = padded_mask(B, N, seed=45, max_pad=N // 4)
    go = rnd(B, H, M, D, seed=46, dtype=dtype)
    inp = dict(Q=Q, K=K, V=V, atom_mask=amask, token_mask=tmask)
    out, g = run_gpu(token_to_atom_attn, inp, go, ("Q", "K", "V"))
    o_ref, g_ref = ref.grads(ref.token_to_atom, {k: v.double() for k, v in inp.items()}, go.double(), ("Q", "K", "V"))
    t = tol(dtype)
    check("O", out, o_ref, t)
    for k in ("Q", "K", "V"):
        check("d" + k, g[k], g_ref[k], t)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_atom_to_token(dtype):
    from deepfold_amd import atom_to_token_attn

    B, H, N, D = 2, 4, 40, 32
    gen = torch.Generator().manual_seed(51)
    counts = torch.randint(0, 30, (B, N), generator=gen)
    counts[0, 3] = 0
    counts[1, 7] = 150  # more atoms than one 64-lane chunk
    starts = torch.cumsum(counts, 1) - counts
    M = int(counts.sum(1).max()) + 5
    Q = rnd(B, H, N, D, seed=52, dtype=dtype)
    K, V = rnd(B, H, M, D, seed=53, dtype=dtype), rnd(B, H, M, D, seed=54, dtype=dtype)
    tmask = torch.ones(B, N)
    tmask[1, 10] = 0
    go = rnd(B, H, N, D, seed=55, dtype=dtype)
    inp = dict(Q=Q, K=K, V=V, token_atom_starts=starts.int(), token_atom_counts=counts.int(), token_mask=tmask)
    out, g = run_gpu(atom_to_token_attn, inp, go, ("Q", "K", "V"))
    ref_inp = dict(Q=Q.double(), K=K.double(), V=V.double(), starts=starts, counts=counts, token_mask=tmask)
    o_ref, g_ref = ref.grads(ref.atom_to_token, ref_inp, go.double(), ("Q", "K", "V"))
    t = tol(dtype)
    check("O", out, o_ref, t)
    for k in ("Q", "K", "V"):
        check("d" + k, g[k], g_ref[k], t)
    assert torch.all(out[0, :, 3] == 0) and torch.all(out[1, :, 10] == 0)


@pytest.mark.parametrize("which", ["dense_bias_gate", "window_and_token_to_atom"])
def test_attention_step_graph_replay(which):
    """The attention forward + backward, captured once in a HIP graph (the attention
    entry points allocate nothing inside a call and record no memset), replayed with
    new input values in the same buffers: outputs and every gradient equal the eager
    step's bit for bit on each replay, with eager work between the replays."""
    from deepfold_amd import flash_atom_attn, flash_diffusion_attn, token_to_atom_attn

    bf = torch.bfloat16
    if which == "dense_bias_gate":
        B, H, N, D = 1, 4, 256, 24
        shapes = dict(q=(B, H, N, D), k=(B, H, N, D), v=(B, H, N, D), g=(B, H, N, D), bias=(B, H, N, N),
                      go=(B, H, N, D))

        def step(t):
            q, k, v, g, bb = (t[n].detach().requires_grad_(True) for n in ("q", "k", "v", "g", "bias"))
            o = flash_diffusion_attn(q, k, v, None, None, pair_bias=bb, gate=g)
            o.backward(t["go"])
            return [o.detach(), q.grad, k.grad, v.grad, g.grad, bb.grad]
    else:
        H, D, M, NT = 2, 32, 512, 21
        shapes = dict(q=(1, H, M, D), k=(1, H, M, D), v=(1, H, M, D), wb=(M // 32, H, 32, 128),
                      kt=(1, H, NT, D), vt=(1, H, NT, D), go=(1, H, M, D), go2=(1, H, M, D))

        def step(t):
            q, k, v, bb = (t[n].detach().requires_grad_(True) for n in ("q", "k", "v", "wb"))
            o = flash_atom_attn(q, k, v, window_bias=bb)
            o.backward(t["go"])
            q2, k2, v2 = (t[n].detach().requires_grad_(True) for n in ("q", "kt", "vt"))
            o2 = token_to_atom_attn(q2, k2, v2)
            o2.backward(t["go2"])
            return [o.detach(), q.grad, k.grad, v.grad, bb.grad, o2.detach(), q2.grad, k2.grad, v2.grad]

    def fill(t, seed):
        for i, (n, s) in enumerate(shapes.items()):
            t[n].copy_(rnd(*s, seed=seed + i, dtype=bf, scale=0.5))

    static = {n: torch.empty(s, dtype=bf, device=DEV) for n, s in shapes.items()}
    fill(static, 100)
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):  # eager warm-up on a side stream before the capture
        for _ in range(2):
            step(static)
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    # captured on the warm-up stream: the workspace cached for it exists, so the graph
    # records no zero fill, and the replays also check that no call relies on a cleared
    # workspace
    with torch.cuda.graph(graph, stream=side):
        outs = step(static)
    for seed in (200, 300, 400):
        fill(static, seed)
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        want = step(static)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), (which, seed, i)
