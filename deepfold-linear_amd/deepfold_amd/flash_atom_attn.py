"""Windowed atom attention on MI355X.

Drop-in for ``deepfold.model.kernels.flash_atom_attn`` of vv137/deepfold-linear
(src/deepfold/model/kernels/flash_atom_attn.py): ``flash_atom_attn``,
``FlashAtomAttnFn.apply`` and ``flash_atom_attn_ref``.  Window w holds queries
[32w, 32w + 32) and keys [32w - 48, 32w + 80) clipped to [0, M).  HIP kernels
(``dfl_attn_*`` with window = 1); dK / dV over overlapping windows are gathered
per key tile, without atomics.

Keyword-only extension: ``window_bias`` (ceil(M/32), H, 32, 128) added to the
scores of window w at query row i - 32w and key column j - (32w - 48).
"""

from __future__ import annotations

import torch

from . import _lib
from ._attn import AttnFn

W_QUERY = 32
W_KEY = 128


def flash_atom_attn_ref(Q, K, V, mask=None, w_query=W_QUERY, w_key=W_KEY):
    """Dense PyTorch reference of the op (flash_atom_attn.py:215-254), for tests.

    Not used by ``flash_atom_attn``."""
    B, H, M, D = Q.shape
    scale = D ** -0.5
    half = (w_key - w_query) // 2
    O = torch.zeros_like(Q)
    for w in range(0, M, w_query):
        q1 = min(w + w_query, M)
        k0, k1 = max(0, w - half), min(M, w + w_query + half)
        scores = torch.matmul(Q[:, :, w:q1], K[:, :, k0:k1].transpose(-1, -2).contiguous()) * scale
        if mask is not None:
            scores = scores + (1 - mask[:, None, None, k0:k1]) * (-1e9)
        attn = torch.softmax(scores, dim=-1)
        if mask is not None:
            attn = attn * mask[:, None, w:q1, None]
        O[:, :, w:q1] = torch.matmul(attn.nan_to_num(0.0), V[:, :, k0:k1])
    return O


class FlashAtomAttnFn:
    """``apply(Q, K, V, mask)`` -> O (flash_atom_attn.py:262-315).

    Same entry point as the reference's autograd.Function; the gradients come
    from the HIP backward behind it."""

    @staticmethod
    def apply(Q, K, V, mask):
        return AttnFn.apply(Q, K, V, None, None, None, None, mask, mask, _lib.DFL_ATTN_BIAS_NONE, 1)


def flash_atom_attn(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    mask: torch.Tensor | None = None,
    *,
    window_bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """Windowed atom attention, 32 queries x 128 keys (flash_atom_attn.py:318-354).

    Q, K, V: (B,H,M,D) or (H,M,D); mask (B,M) or (M,), 1 = valid.
    """
    unbatched = Q.dim() == 3
    if unbatched:
        Q, K, V = Q.unsqueeze(0), K.unsqueeze(0), V.unsqueeze(0)
        if mask is not None:
            mask = mask.unsqueeze(0)
    if window_bias is not None:
        O = AttnFn.apply(Q, K, V, None, None, None, window_bias, mask, mask, _lib.DFL_ATTN_BIAS_WINDOW, 1)
    else:
        O = AttnFn.apply(Q, K, V, None, None, None, None, mask, mask, _lib.DFL_ATTN_BIAS_NONE, 1)
    return O.squeeze(0) if unbatched else O
