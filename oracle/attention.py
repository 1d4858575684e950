"""CPU oracle for the attention kernels next to the Sinkhorn path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package (``deepfold_amd``) or
the HIP library imports, links or calls this module; only ``tests/`` use it, as
the checker.  Floating-point attention, so the restatements are dense PyTorch
(CPU, float64 by default) and gradients come from torch.autograd on these
dense forms -- the way the reference's own tests check its kernels.

Restated reference functions (vv137/deepfold-linear, src/deepfold/model/kernels/):

* ``diffusion_attn``   -- ``flash_diff_attn_ref``, flash_diffusion_attn.py:440-473:
  softmax(Q K^T / sqrt(D) + pos_weight[h, bins] + (1 - mask_key) * -1e9) V,
  rows of padded queries zeroed.  Extensions (keyword-only, default off): a
  dense additive ``pair_bias`` (B,H,N,N) and a sigmoid ``gate`` (B,H,N,D) applied
  to the output (diffusion_v2.py:171-173 applies the gate in the caller).
* ``atom_attn``        -- ``flash_atom_attn_ref``, flash_atom_attn.py:215-254:
  windows of 32 queries attending to keys [32w - 48, 32w + 80) clipped to [0, M).
  Extension: ``window_bias`` (W,H,32,128) added to the scores of window w, query
  row r = i - 32w, key column c = j - (32w - 48).
* ``token_to_atom``    -- ``token_to_atom_ref``, cross_attn_kernel.py:460-488:
  dense cross attention, token (key) mask as -1e9, atom (query) rows zeroed.
* ``atom_to_token``    -- ``atom_to_token_ref``, cross_attn_kernel.py:424-457:
  token n attends to atoms [starts[n], starts[n] + counts[n]); masked or empty
  tokens give zero rows.

Pinning (tests/test_oracle_attention.py): closed forms (Q = 0 -> uniform
weights -> masked mean of V; a dominant key -> one-hot), the window attention
against dense attention with an independently built band mask, batched ==
per-sample, token-to-atom == diffusion attention without bias on equal sizes,
atom-to-token against per-token loops, and torch.autograd gradients against
central finite differences.
"""

from __future__ import annotations

import torch

W_QUERY = 32
W_KEY = 128
HALF_EXTRA = (W_KEY - W_QUERY) // 2  # 48
MASK_BIAS = -1e9


def _t(x, dtype):
    return None if x is None else torch.as_tensor(x).to(dtype)


def _softmax_attention(scores, V, key_mask=None, query_mask=None):
    """softmax over the last axis with -1e9 key masking, then query-row zeroing."""
    if key_mask is not None:
        scores = scores + (1.0 - key_mask[:, None, None, :]) * MASK_BIAS
    attn = torch.softmax(scores, dim=-1)
    if query_mask is not None:
        attn = attn * query_mask[:, None, :, None]
    attn = attn.nan_to_num(0.0)
    return attn @ V


def diffusion_attn(Q, K, V, pos_weight, pos_bins, mask=None, *, pair_bias=None, gate=None,
                   dtype=torch.float64):
    """flash_diff_attn_ref (flash_diffusion_attn.py:440-473) + optional pair_bias / gate."""
    Q, K, V = _t(Q, dtype), _t(K, dtype), _t(V, dtype)
    B, H, N, D = Q.shape
    scores = (Q @ K.transpose(-1, -2)) * D ** -0.5
    if pos_bins is not None:
        pw = _t(pos_weight, dtype)
        bins = torch.as_tensor(pos_bins).long()
        scores = scores + pw[:, bins].permute(1, 0, 2, 3)
    if pair_bias is not None:
        scores = scores + _t(pair_bias, dtype)
    m = None if mask is None else _t(mask, dtype)
    out = _softmax_attention(scores, V, m, m)
    if gate is not None:
        out = torch.sigmoid(_t(gate, dtype)) * out
    return out


def atom_attn(Q, K, V, mask=None, *, window_bias=None, dtype=torch.float64):
    """flash_atom_attn_ref (flash_atom_attn.py:215-254) + optional per-window bias."""
    Q, K, V = _t(Q, dtype), _t(K, dtype), _t(V, dtype)
    B, H, M, D = Q.shape
    m = None if mask is None else _t(mask, dtype)
    wb = None if window_bias is None else _t(window_bias, dtype)
    out = torch.zeros_like(Q)
    for w0 in range(0, M, W_QUERY):
        q1 = min(w0 + W_QUERY, M)
        k0 = max(0, w0 - HALF_EXTRA)
        k1 = min(M, w0 + W_QUERY + HALF_EXTRA)
        scores = (Q[:, :, w0:q1] @ K[:, :, k0:k1].transpose(-1, -2)) * D ** -0.5
        if wb is not None:
            c0 = k0 - (w0 - HALF_EXTRA)
            scores = scores + wb[w0 // W_QUERY][None, :, : q1 - w0, c0:c0 + (k1 - k0)]
        km = None if m is None else m[:, k0:k1]
        qm = None if m is None else m[:, w0:q1]
        out[:, :, w0:q1] = _softmax_attention(scores, V[:, :, k0:k1], km, qm)
    return out


def token_to_atom(Q, K, V, atom_mask=None, token_mask=None, dtype=torch.float64):
    """token_to_atom_ref (cross_attn_kernel.py:460-488)."""
    Q, K, V = _t(Q, dtype), _t(K, dtype), _t(V, dtype)
    D = Q.shape[-1]
    scores = (Q @ K.transpose(-1, -2)) * D ** -0.5
    return _softmax_attention(scores, V, None if token_mask is None else _t(token_mask, dtype),
                              None if atom_mask is None else _t(atom_mask, dtype))


def atom_to_token(Q, K, V, starts, counts, token_mask=None, dtype=torch.float64):
    """atom_to_token_ref (cross_attn_kernel.py:424-457), vectorised over tokens with
    a per-(token, atom) membership mask instead of the reference's Python loop."""
    Q, K, V = _t(Q, dtype), _t(K, dtype), _t(V, dtype)
    B, H, N, D = Q.shape
    M = K.shape[2]
    starts = torch.as_tensor(starts).long()
    counts = torch.as_tensor(counts).long()
    j = torch.arange(M)
    member = (j[None, None, :] >= starts[:, :, None]) & (j[None, None, :] < (starts + counts)[:, :, None])
    if token_mask is not None:
        member = member & (torch.as_tensor(token_mask)[:, :, None] != 0)
    scores = (Q @ K.transpose(-1, -2)) * D ** -0.5                  # (B,H,N,M)
    scores = scores.masked_fill(~member[:, None], -1e30)             # exp underflows to exactly 0
    attn = torch.softmax(scores, dim=-1)
    attn = attn * member.any(-1)[:, None, :, None].to(attn.dtype)    # empty / masked tokens -> 0
    return attn @ V


def grads(fn, inputs: dict, grad_out, wrt):
    """torch.autograd gradients of <fn(**inputs), grad_out> for the names in ``wrt``."""
    leaves = {k: (v.detach().clone().requires_grad_(True) if k in wrt else v) for k, v in inputs.items()}
    out = fn(**leaves)
    (out * grad_out.to(out.dtype)).sum().backward()
    return out.detach(), {k: leaves[k].grad for k in wrt}
