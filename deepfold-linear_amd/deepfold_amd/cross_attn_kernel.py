"""Atom <-> token cross attention on MI355X.

Drop-in for ``deepfold.model.kernels.cross_attn_kernel`` of vv137/deepfold-linear
(src/deepfold/model/kernels/cross_attn_kernel.py): ``token_to_atom_attn``,
``atom_to_token_attn``, their ``*Fn.apply`` and ``*_ref`` functions.

* token_to_atom: atoms (queries, B,H,M,D) attend densely to tokens (keys,
  B,H,N,D); token mask on keys, atom mask zeroes query rows (``dfl_attn_*``).
* atom_to_token: token n attends to its atoms [starts[n], starts[n] + counts[n])
  (``dfl_a2t_*``); no host synchronisation (the reference reads
  counts.max().item(), cross_attn_kernel.py:501).
"""

from __future__ import annotations

import torch

from . import _lib
from ._attn import A2TFn, AttnFn


def atom_to_token_ref(Q, K, V, token_atom_starts, token_atom_counts, token_mask=None):
    """PyTorch reference (cross_attn_kernel.py:424-457), for tests; not used by the op."""
    B, H, N, D = Q.shape
    O = torch.zeros_like(Q)
    for b in range(B):
        for n in range(N):
            if token_mask is not None and token_mask[b, n] == 0:
                continue
            s, c = int(token_atom_starts[b, n]), int(token_atom_counts[b, n])
            if c == 0:
                continue
            scores = (Q[b, :, n, None, :] * K[b, :, s:s + c, :]).sum(-1) * D ** -0.5
            O[b, :, n, :] = (torch.softmax(scores, dim=-1).unsqueeze(-1) * V[b, :, s:s + c, :]).sum(1)
    return O


def token_to_atom_ref(Q, K, V, atom_mask=None, token_mask=None):
    """PyTorch reference (cross_attn_kernel.py:460-488), for tests; not used by the op."""
    D = Q.shape[-1]
    scores = torch.matmul(Q, K.transpose(-1, -2).contiguous()) * D ** -0.5
    if token_mask is not None:
        scores = scores + (1 - token_mask[:, None, None, :]) * (-1e9)
    attn = torch.softmax(scores, dim=-1)
    if atom_mask is not None:
        attn = attn * atom_mask[:, None, :, None]
    return torch.matmul(attn.nan_to_num(0.0), V)


class AtomToTokenAttnFn:
    """``apply(Q, K, V, token_atom_starts, token_atom_counts, token_mask)`` (cross_attn_kernel.py:496-552).

    Same entry point as the reference's autograd.Function; the gradients come
    from the HIP backward behind it."""

    @staticmethod
    def apply(Q, K, V, token_atom_starts, token_atom_counts, token_mask):
        return A2TFn.apply(Q, K, V, token_atom_starts, token_atom_counts, token_mask)


class TokenToAtomAttnFn:
    """``apply(Q, K, V, atom_mask, token_mask)`` (cross_attn_kernel.py:555-621).

    Same entry point as the reference's autograd.Function; the gradients come
    from the HIP backward behind it."""

    @staticmethod
    def apply(Q, K, V, atom_mask, token_mask):
        return AttnFn.apply(Q, K, V, None, None, None, None, atom_mask, token_mask, _lib.DFL_ATTN_BIAS_NONE, 0)


def atom_to_token_attn(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    token_atom_starts: torch.Tensor,
    token_atom_counts: torch.Tensor,
    token_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """Sparse cross-attention, tokens query their own atoms (cross_attn_kernel.py:629-661).

    Q (B,H,N,D) token queries; K, V (B,H,M,D) atom keys / values; starts, counts
    (B,N) int; token_mask (B,N) or None.  Returns (B,H,N,D)."""
    return A2TFn.apply(Q, K, V, token_atom_starts, token_atom_counts, token_mask)


def token_to_atom_attn(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    atom_mask: torch.Tensor | None = None,
    token_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dense cross-attention, atoms query all tokens (cross_attn_kernel.py:664-696).

    Q (B,H,M,D) atom queries; K, V (B,H,N,D); atom_mask (B,M), token_mask (B,N)."""
    return AttnFn.apply(Q, K, V, None, None, None, None, atom_mask, token_mask, _lib.DFL_ATTN_BIAS_NONE, 0)
