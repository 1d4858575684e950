"""deepfold_amd: MI355X (gfx950) kernels for DeepFold-Linear's flash-Sinkhorn
optimal-transport attention and its neighbouring attention ops.

Module names mirror vv137/deepfold-linear's ``deepfold.model.kernels`` /
``deepfold.utils`` modules so that call sites switch by changing the import root.
"""

from . import _lib  # noqa: F401
from .cg import CGInfo, conjugate_gradient  # noqa: F401
from .cross_attn_kernel import atom_to_token_attn, token_to_atom_attn  # noqa: F401
from .flash_atom_attn import flash_atom_attn  # noqa: F401
from .flash_diffusion_attn import flash_diffusion_attn  # noqa: F401
from .flash_sinkhorn_attn import FlashSinkhornAttn, flash_sinkhorn_attn  # noqa: F401
from .flash_sinkhorn_transport import (  # noqa: F401
    BalancedSinkhornDualFn, BalancedSinkhornFn, balanced_sinkhorn_transport, balanced_sinkhorn_transport_dual)
from .sinkhorn import compute_transport_output, sinkhorn_solve  # noqa: F401
from .sinkhorn_kernel import FlashSinkhornFunction, flash_sinkhorn  # noqa: F401
from .trunk_steps import (  # noqa: F401
    GatedCoordUpdateFn, SinkProjectionFn, gated_coordinate_update, sink_projections, token_ot_transport_step)

__version__ = "0.1.0"


def check_errors(device=None) -> None:
    """Synchronise ``device`` and raise if any kernel launched so far reported an
    expired cross-workgroup wait (its outputs are then invalid).  Every op also
    checks, without synchronising, before its own launch."""
    import torch

    torch.cuda.synchronize(device)
    _lib.raise_pending("deepfold_amd.check_errors")
