"""CPU pinning of the attention oracle (oracle/attention.py) -- no GPU needed.

The restatements are checked against closed forms and against independently
built dense equivalents, not against copies of themselves:
* Q = 0 gives uniform weights, so the output is the mean of V over valid keys;
* a dominant key (or a dominant position bin) gives a one-hot row;
* the windowed attention equals dense attention under a band mask built here,
  with the window bias scattered into a dense bias;
* token-to-atom equals diffusion attention without a position term when the
  atom and token sets coincide;
* atom-to-token equals a per-token softmax written as a plain loop;
* batched == per-sample; padded query rows are zero;
* autograd gradients of the dense forms match central finite differences.
"""

import math

import pytest
import torch

from oracle import attention as ref


@pytest.fixture(autouse=True, scope="module")
def _float64_default():
    """float64 for this module's tensors only; the dtype is restored for the other modules."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def rnd(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64) * scale


def test_zero_queries_give_masked_mean():
    B, H, N, D = 2, 3, 11, 8
    V = rnd(B, H, N, D, seed=1)
    mask = torch.ones(B, N)
    mask[0, 7:] = 0
    mask[1, 9:] = 0
    Q = torch.zeros(B, H, N, D)
    K = rnd(B, H, N, D, seed=2)
    out = ref.diffusion_attn(Q, K, V, None, None, mask)
    for b in range(B):
        n = int(mask[b].sum())
        want = V[b, :, :n].mean(1)
        torch.testing.assert_close(out[b, :, :n], want[:, None].expand(H, n, D), rtol=1e-12, atol=1e-12)
        assert torch.all(out[b, :, n:] == 0)
    t2a = ref.token_to_atom(Q, K, V, atom_mask=mask, token_mask=mask)
    torch.testing.assert_close(t2a, out, rtol=1e-12, atol=1e-12)


def test_dominant_key_and_bin_give_one_hot():
    B, H, N, D = 1, 2, 9, 4
    V = rnd(B, H, N, D, seed=3)
    Q = torch.zeros(B, H, N, D)
    Q[..., 0] = 1.0
    K = torch.zeros(B, H, N, D)
    K[:, :, 5, 0] = 200.0  # key 5 dominates every row
    out = ref.diffusion_attn(Q, K, V, None, None)
    torch.testing.assert_close(out, V[:, :, 5:6].expand(B, H, N, D), rtol=0, atol=1e-12)
    # position term: bin 7 carries +80, each row i has bin 7 only at key (2i mod N)
    pw = torch.zeros(H, 68)
    pw[:, 7] = 80.0
    bins = torch.zeros(B, N, N, dtype=torch.int32)
    for i in range(N):
        bins[0, i, (2 * i) % N] = 7
    out = ref.diffusion_attn(torch.zeros(B, H, N, D), torch.zeros(B, H, N, D), V, pw, bins)
    want = torch.stack([V[:, :, (2 * i) % N] for i in range(N)], dim=2)
    torch.testing.assert_close(out, want, rtol=0, atol=1e-12)


def test_gate_and_pair_bias():
    B, H, N, D = 1, 2, 7, 4
    Q, K, V, G = (rnd(B, H, N, D, seed=s) for s in (4, 5, 6, 7))
    bias = rnd(B, H, N, N, seed=8)
    plain = torch.softmax(Q @ K.transpose(-1, -2) / 2.0 + bias, -1) @ V
    out = ref.diffusion_attn(Q, K, V, None, None, pair_bias=bias, gate=G)
    torch.testing.assert_close(out, torch.sigmoid(G) * plain, rtol=1e-12, atol=1e-12)


def band_mask(M):
    i = torch.arange(M)[:, None]
    j = torch.arange(M)[None, :]
    w0 = (i // 32) * 32
    return (j >= w0 - 48) & (j < w0 + 80)


@pytest.mark.parametrize("M,with_mask,with_bias", [(100, False, False), (160, True, False), (75, True, True)])
def test_window_attention_is_banded_dense_attention(M, with_mask, with_bias):
    B, H, D = 2, 2, 8
    Q, K, V = (rnd(B, H, M, D, seed=s) for s in (9, 10, 11))
    mask = torch.ones(B, M)
    if with_mask:
        mask[0, M - 13:] = 0
    W = (M + 31) // 32
    wb = rnd(W, H, 32, 128, seed=12) if with_bias else None
    out = ref.atom_attn(Q, K, V, mask if with_mask else None, window_bias=wb)
    scores = Q @ K.transpose(-1, -2) / math.sqrt(D)
    if with_bias:
        dense = torch.zeros(H, M, M)
        for i in range(M):
            w = i // 32
            for j in range(M):
                c = j - (32 * w - 48)
                if 0 <= c < 128:
                    dense[:, i, j] = wb[w, :, i - 32 * w, c]
        scores = scores + dense[None]
    scores = scores.masked_fill(~band_mask(M)[None, None], -1e30)
    if with_mask:
        scores = scores + (1 - mask[:, None, None, :]) * -1e9
    want = torch.softmax(scores, -1) @ V
    if with_mask:
        want = want * mask[:, None, :, None]
    torch.testing.assert_close(out, want, rtol=1e-12, atol=1e-12)


def test_atom_to_token_matches_per_token_loop():
    B, H, N, D = 2, 2, 6, 4
    counts = torch.tensor([[3, 0, 5, 1, 2, 4], [2, 2, 2, 2, 2, 2]])
    starts = torch.cumsum(counts, 1) - counts
    M = int(counts.sum(1).max())
    Q = rnd(B, H, N, D, seed=13)
    K, V = rnd(B, H, M, D, seed=14), rnd(B, H, M, D, seed=15)
    tmask = torch.ones(B, N)
    tmask[1, 4] = 0
    out = ref.atom_to_token(Q, K, V, starts, counts, tmask)
    for b in range(B):
        for n in range(N):
            s, c = int(starts[b, n]), int(counts[b, n])
            if c == 0 or tmask[b, n] == 0:
                assert torch.all(out[b, :, n] == 0)
                continue
            for h in range(H):
                sc = torch.tensor([float(Q[b, h, n] @ K[b, h, s + a]) / 2.0 for a in range(c)])
                w = torch.exp(sc - sc.max())
                w = w / w.sum()
                want = sum(w[a] * V[b, h, s + a] for a in range(c))
                torch.testing.assert_close(out[b, h, n], want, rtol=1e-12, atol=1e-12)


def test_batched_equals_per_sample():
    B, H, N, D = 3, 2, 10, 4
    Q, K, V = (rnd(B, H, N, D, seed=s) for s in (16, 17, 18))
    pw = rnd(H, 68, seed=19)
    bins = torch.randint(0, 68, (B, N, N), generator=torch.Generator().manual_seed(20), dtype=torch.int32)
    mask = torch.ones(B, N)
    mask[1, 6:] = 0
    full = ref.diffusion_attn(Q, K, V, pw, bins, mask)
    for b in range(B):
        one = ref.diffusion_attn(Q[b:b + 1], K[b:b + 1], V[b:b + 1], pw, bins[b:b + 1], mask[b:b + 1])
        torch.testing.assert_close(full[b:b + 1], one, rtol=1e-13, atol=1e-14)


def test_autograd_matches_finite_differences():
    B, H, N, D = 1, 2, 6, 4
    inp = dict(Q=rnd(B, H, N, D, seed=21), K=rnd(B, H, N, D, seed=22), V=rnd(B, H, N, D, seed=23),
               pos_weight=rnd(H, 68, seed=24),
               pos_bins=torch.randint(0, 68, (B, N, N), generator=torch.Generator().manual_seed(25)),
               mask=torch.tensor([[1.0, 1, 1, 1, 1, 0]]), pair_bias=rnd(B, H, N, N, seed=26),
               gate=rnd(B, H, N, D, seed=27))
    go = rnd(B, H, N, D, seed=28)
    fn = ref.diffusion_attn
    _, g = ref.grads(fn, inp, go, ("Q", "K", "V", "pos_weight", "pair_bias", "gate"))
    h = 1e-6
    for name, idx in [("Q", (0, 1, 2, 3)), ("K", (0, 0, 4, 1)), ("V", (0, 1, 3, 0)), ("pair_bias", (0, 1, 2, 4)),
                      ("gate", (0, 0, 1, 2)), ("pos_weight", (1, int(inp["pos_bins"][0, 2, 3])))]:
        p, m = dict(inp), dict(inp)
        p[name] = inp[name].clone()
        m[name] = inp[name].clone()
        p[name][idx] += h
        m[name][idx] -= h
        fd = float(((fn(**p) - fn(**m)) * go).sum()) / (2 * h)
        assert abs(float(g[name][idx]) - fd) <= 1e-7 * max(1.0, abs(fd)), (name, float(g[name][idx]), fd)
