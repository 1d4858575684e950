"""Flash diffusion attention with the 68-bin position bias on MI355X.

Drop-in for ``deepfold.model.kernels.flash_diffusion_attn`` of vv137/deepfold-linear
(src/deepfold/model/kernels/flash_diffusion_attn.py): ``flash_diffusion_attn``,
``FlashDiffusionAttnFn.apply`` and ``flash_diff_attn_ref`` keep their names,
arguments, defaults and unbatched handling.  The op runs as HIP kernels
(``dfl_attn_fwd`` / ``dfl_attn_bwd``); there is no Triton and no CPU path.

Keyword-only extensions (default off): ``pair_bias`` -- a dense additive bias
(B,H,N,N) with gradient -- and ``gate`` -- sigmoid gate logits (B,H,N,D),
O = sigmoid(gate) * attention (the reference applies this gate in its caller,
diffusion_v2.py:171-173).  Keys with mask 0 are excluded; rows of padded
queries are zero.
"""

from __future__ import annotations

import torch

from . import _lib
from ._attn import AttnFn

NUM_BINS = 68


def flash_diff_attn_ref(Q, K, V, pos_weight, pos_bins, mask=None):
    """Dense PyTorch reference of the op (flash_diffusion_attn.py:440-473), for tests.

    Not used by ``flash_diffusion_attn``; runs wherever its inputs live."""
    B, H, N, D = Q.shape
    scores = torch.matmul(Q, K.transpose(-1, -2).contiguous()) * D ** -0.5
    scores = scores + pos_weight[:, pos_bins.long()].permute(1, 0, 2, 3)
    if mask is not None:
        scores = scores + (1 - mask[:, None, None, :]) * (-1e9)
    attn = torch.softmax(scores, dim=-1)
    if mask is not None:
        attn = attn * mask[:, None, :, None]
    attn = attn.nan_to_num(0.0)
    return torch.matmul(attn, V)


class FlashDiffusionAttnFn:
    """``apply(Q, K, V, pos_weight, pos_bins, mask)`` -> O (flash_diffusion_attn.py:485-576).

    Same entry point as the reference's autograd.Function; the gradients come
    from the HIP backward behind it."""

    @staticmethod
    def apply(Q, K, V, pos_weight, pos_bins, mask):
        return AttnFn.apply(Q, K, V, None, pos_weight, pos_bins, None, mask, mask, _lib.DFL_ATTN_BIAS_BINS, 0)


def flash_diffusion_attn(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    pos_weight: torch.Tensor,
    pos_bins: torch.Tensor,
    mask: torch.Tensor | None = None,
    *,
    pair_bias: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
) -> torch.Tensor:
    """Flash diffusion attention with 68-bin position bias (flash_diffusion_attn.py:579-622).

    Q, K, V: (B,H,N,D) or (H,N,D); pos_weight (H,68); pos_bins (B,N,N) or (N,N)
    int (may be None when ``pair_bias`` is given); mask (B,N) or (N,), 1 = valid.
    Returns O with the shape and dtype of Q.
    """
    unbatched = Q.dim() == 3
    if unbatched:
        Q, K, V = Q.unsqueeze(0), K.unsqueeze(0), V.unsqueeze(0)
        if pos_bins is not None:
            pos_bins = pos_bins.unsqueeze(0)
        if mask is not None:
            mask = mask.unsqueeze(0)
        if pair_bias is not None and pair_bias.dim() == 3:
            pair_bias = pair_bias.unsqueeze(0)
        if gate is not None:
            gate = gate.unsqueeze(0)
    if pos_bins is not None and pair_bias is not None:
        raise ValueError("flash_diffusion_attn: give either pos_bins or pair_bias, not both")
    if pair_bias is not None:
        O = AttnFn.apply(Q, K, V, gate, None, None, pair_bias, mask, mask, _lib.DFL_ATTN_BIAS_DENSE, 0)
    elif pos_bins is not None:
        O = AttnFn.apply(Q, K, V, gate, pos_weight, pos_bins, None, mask, mask, _lib.DFL_ATTN_BIAS_BINS, 0)
    else:
        O = AttnFn.apply(Q, K, V, gate, None, None, None, mask, mask, _lib.DFL_ATTN_BIAS_NONE, 0)
    return O.squeeze(0) if unbatched else O
