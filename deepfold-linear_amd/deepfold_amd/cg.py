"""Conjugate gradient for SPD systems -- API of vv137/deepfold-linear's
``deepfold.utils.cg.conjugate_gradient`` / ``CGInfo`` (src/deepfold/utils/cg.py:18-97).

The IFT backward of the flash-Sinkhorn op does not call this routine.  It runs
its own CG inside the HIP kernel, with the matvecs, inner products and updates
fused and no host synchronisation.  This module is the generic solver for
callers that bring their own matvec: the same steps, tolerances, warm start,
preconditioner, periodic residual refresh and result record as the reference.
All vectors stay on the GPU; the one host read per iteration is the residual
norm the stopping test needs (as in the reference).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

from . import _lib


@dataclass(frozen=True)
class CGInfo:
    """Convergence info from a CG solve (cg.py:18-25)."""

    converged: bool
    iters: int
    residual: float
    initial_residual: float


def conjugate_gradient(
    matvec: Callable[[torch.Tensor], torch.Tensor],
    b: torch.Tensor,
    *,
    x0: torch.Tensor | None = None,
    max_iter: int = 300,
    rtol: float = 1e-6,
    atol: float = 1e-6,
    preconditioner: Callable[[torch.Tensor], torch.Tensor] | None = None,
    stabilise_every: int = 0,
) -> tuple[torch.Tensor, CGInfo]:
    """Solve A x = b with matvec(v) = A v for SPD A (cg.py:28-97).

    Stops when ||r|| <= max(atol, rtol ||r_0||); ``stabilise_every`` > 0 replaces
    the recursive residual by b - A x every that many iterations.
    """
    _lib.require_gpu(b, x0)
    if x0 is None:
        x = torch.zeros_like(b)
        r = b.clone()
    else:
        x = x0.clone()
        r = b - matvec(x)
    z = preconditioner(r) if preconditioner is not None else r
    p = z.clone()
    rz_old = torch.dot(r, z)
    init_res = float(torch.linalg.norm(r))
    tol = max(atol, rtol * init_res)
    for it in range(int(max_iter)):
        Ap = matvec(p)
        denom = torch.dot(p, Ap)
        if float(denom.abs()) == 0.0:
            break
        alpha = rz_old / denom
        x = x + alpha * p
        r = r - alpha * Ap
        if stabilise_every and (it + 1) % stabilise_every == 0:
            r = b - matvec(x)
        res = float(torch.linalg.norm(r))
        if res <= tol:
            return x, CGInfo(converged=True, iters=it + 1, residual=res, initial_residual=init_res)
        z = preconditioner(r) if preconditioner is not None else r
        rz_new = torch.dot(r, z)
        p = z + (rz_new / rz_old) * p
        rz_old = rz_new
    res = float(torch.linalg.norm(r))
    return x, CGInfo(converged=False, iters=int(max_iter), residual=res, initial_residual=init_res)
