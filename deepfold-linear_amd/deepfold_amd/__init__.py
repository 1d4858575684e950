"""deepfold_amd: MI355X (gfx950) kernels for DeepFold-Linear's flash-Sinkhorn
optimal-transport attention and its neighbouring attention ops.

Module names mirror vv137/deepfold-linear's ``deepfold.model.kernels`` /
``deepfold.utils`` modules so that call sites switch by changing the import root.
"""

from . import _lib  # noqa: F401
from .flash_sinkhorn_attn import FlashSinkhornAttn, flash_sinkhorn_attn  # noqa: F401

__version__ = "0.1.0"
