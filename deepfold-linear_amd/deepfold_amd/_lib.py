"""ctypes binding of libdfl_amd.so (the C ABI declared in include/dfl_amd.h).

The library is built in-tree by ``deepfold-linear_amd/build_lib.py`` (``__graft_entry__.build()``).
There is no CPU or PyTorch fallback: every public op of this package raises if the
library is missing or the tensors are not on a ROCm device.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdfl_amd.so")

DFL_BF16 = 0
DFL_F32 = 1
DFL_IFT_FIXED_POINT = 0
DFL_IFT_CG = 1
DFL_IFT_REFERENCE = 0
DFL_IFT_ANALYTIC = 1
DFL_STORAGE_AUTO = 0
DFL_STORAGE_RESIDENT = 1
DFL_STORAGE_STREAM = 2
DFL_STORAGE_REGISTER = 3
DFL_LAUNCH_AUTO = 0
DFL_LAUNCH_ORDINARY = 1
DFL_LAUNCH_COOPERATIVE = 2

_lock = threading.Lock()
_lib = None

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_longlong
F32 = ctypes.c_float


class SinkhornFwdParams(ctypes.Structure):
    """Mirror of ``dfl_sinkhorn_fwd_params``."""

    _fields_ = [
        ("dtype", I32),
        ("q", P), ("k", P), ("v", P), ("g", P),
        ("stride_b", I64), ("stride_h", I64), ("stride_n", I64),
        ("x_res", P), ("pos_weight", P), ("pos_bins", P),
        ("eps", P), ("w_dist", P), ("log_mu", P), ("log_nu", P),
        ("log_u_init", P), ("log_v_init", P), ("mask", P),
        ("B", I32), ("H", I32), ("N", I32), ("d", I32),
        ("K_iter", I32), ("lam", F32), ("r_0", F32),
        ("o_flat", P), ("x_centroid", P), ("log_u", P), ("log_v", P),
        ("o_avg", P), ("log_z", P), ("col_lse", P),
        ("storage", I32), ("hist", P),
    ]


class SinkhornUnrolledBwdParams(ctypes.Structure):
    """Mirror of ``dfl_sinkhorn_unrolled_bwd_params``."""

    _fields_ = [
        ("dtype", I32),
        ("q", P), ("k", P), ("v", P), ("g", P),
        ("stride_b", I64), ("stride_h", I64), ("stride_n", I64),
        ("x_res", P), ("pos_weight", P), ("pos_bins", P),
        ("eps", P), ("w_dist", P), ("log_mu", P), ("log_nu", P), ("log_v_init", P), ("mask", P),
        ("B", I32), ("H", I32), ("N", I32), ("d", I32), ("K_iter", I32), ("lam", F32), ("r_0", F32),
        ("o_avg", P), ("x_centroid", P), ("log_u", P), ("log_z", P), ("hist", P),
        ("grad_o", P), ("grad_xc", P),
        ("dq", P), ("dk", P), ("dv", P), ("dg", P), ("dlog_mu", P), ("dlog_nu", P), ("dlog_v_init", P),
        ("dx_res", P), ("dpos_weight", P), ("dw_dist", P),
    ]


class SinkhornBwdParams(ctypes.Structure):
    """Mirror of ``dfl_sinkhorn_bwd_params``."""

    _fields_ = [
        ("dtype", I32),
        ("q", P), ("k", P), ("v", P), ("g", P),
        ("stride_b", I64), ("stride_h", I64), ("stride_n", I64),
        ("x_res", P), ("pos_weight", P), ("pos_bins", P),
        ("eps", P), ("w_dist", P), ("mask", P),
        ("log_u", P), ("log_v", P), ("log_z", P), ("col_lse", P),
        ("o_avg", P), ("x_centroid", P), ("grad_o", P), ("grad_xc", P),
        ("B", I32), ("H", I32), ("N", I32), ("d", I32),
        ("lam", F32), ("r_0", F32),
        ("solver", I32), ("iters", I32), ("mode", I32), ("cg_rtol", F32),
        ("dq", P), ("dk", P), ("dv", P), ("dg", P),
        ("dlog_mu", P), ("dlog_nu", P), ("dx_res", P), ("dpos_weight", P), ("dw_dist", P),
        ("storage", I32),
    ]


class AttnParams(ctypes.Structure):
    """Mirror of ``dfl_attn_params``."""

    _fields_ = [
        ("dtype", I32),
        ("q", P), ("k", P), ("v", P), ("g", P),
        ("q_stride_b", I64), ("q_stride_h", I64), ("q_stride_n", I64),
        ("k_stride_b", I64), ("k_stride_h", I64), ("k_stride_n", I64),
        ("q_mask", P), ("k_mask", P),
        ("bias_mode", I32), ("pos_weight", P), ("pos_bins", P), ("bias", P),
        ("window", I32),
        ("B", I32), ("H", I32), ("Mq", I32), ("Nk", I32), ("d", I32),
        ("scale", F32),
        ("o", P), ("lse", P),
        ("grad_o", P), ("dq", P), ("dk", P), ("dv", P), ("dg", P), ("dbias", P), ("dpos_weight", P),
    ]


class A2TParams(ctypes.Structure):
    """Mirror of ``dfl_a2t_params``."""

    _fields_ = [
        ("dtype", I32),
        ("q", P), ("k", P), ("v", P),
        ("starts", P), ("counts", P), ("token_mask", P),
        ("B", I32), ("H", I32), ("N", I32), ("M", I32), ("d", I32),
        ("scale", F32),
        ("o", P), ("lse", P),
        ("grad_o", P), ("dq", P), ("dk", P), ("dv", P),
    ]


class DenseSinkhornParams(ctypes.Structure):
    """Mirror of ``dfl_dense_sinkhorn_params``."""

    _fields_ = [
        ("C", P), ("log_mu", P), ("log_nu", P), ("eps", P),
        ("log_u_init", P), ("log_v_init", P), ("mask", P),
        ("B", I32), ("H", I32), ("N", I32), ("K", I32),
        ("lam", F32), ("threshold", F32), ("check_every", I32),
        ("log_u", P), ("log_v", P), ("history", P), ("iters_done", P),
    ]


class DenseSinkhornBwdParams(ctypes.Structure):
    """Mirror of ``dfl_dense_sinkhorn_bwd_params``."""

    _fields_ = [
        ("C", P), ("eps", P), ("mask", P), ("history", P),
        ("B", I32), ("H", I32), ("N", I32), ("K_max", I32), ("K", I32), ("lam", F32),
        ("grad_log_u", P), ("grad_log_v", P),
        ("dC", P), ("dlog_mu", P), ("dlog_nu", P), ("dlog_u_init", P), ("dlog_v_init", P),
    ]


class DenseTransportParams(ctypes.Structure):
    """Mirror of ``dfl_dense_transport_params``."""

    _fields_ = [
        ("V", P), ("G", P), ("log_u", P), ("log_v", P), ("C", P), ("eps", P), ("x_res", P), ("mask", P),
        ("B", I32), ("H", I32), ("N", I32), ("d", I32),
        ("o", P), ("T_norm", P), ("x_centroid", P), ("o_avg", P),
        ("grad_o", P), ("grad_T", P), ("grad_xc", P),
        ("dV", P), ("dG", P), ("dlog_u", P), ("dlog_v", P), ("dC", P), ("dx_res", P),
    ]


class BalancedFwdParams(ctypes.Structure):
    """Mirror of ``dfl_balanced_fwd_params``."""

    _fields_ = [
        ("dtype", I32),
        ("q", P), ("k", P), ("v", P),
        ("stride_b", I64), ("stride_h", I64), ("stride_n", I64),
        ("x_res", P), ("eps", P), ("alpha_h", P), ("r_h", P), ("mask", P),
        ("B", I32), ("H", I32), ("N", I32), ("d", I32), ("K_iter", I32),
        ("x_centroid", P), ("h_centroid", P), ("log_u", P), ("log_v", P), ("log_z", P), ("hist", P),
        ("storage", I32),
    ]


class BalancedBwdParams(ctypes.Structure):
    """Mirror of ``dfl_balanced_bwd_params``."""

    _fields_ = [
        ("dtype", I32),
        ("q", P), ("k", P), ("v", P),
        ("stride_b", I64), ("stride_h", I64), ("stride_n", I64),
        ("x_res", P), ("eps", P), ("alpha_h", P), ("r_h", P), ("mask", P),
        ("B", I32), ("H", I32), ("N", I32), ("d", I32), ("K_iter", I32),
        ("x_centroid", P), ("h_centroid", P), ("hist", P), ("grad_xc", P), ("grad_hc", P),
        ("dq", P), ("dk", P), ("dv", P), ("dx_res", P), ("dalpha_h", P), ("dr_h", P),
    ]


class SinkProjParams(ctypes.Structure):
    """Mirror of ``dfl_sink_proj_params``."""

    _fields_ = [
        ("dtype", I32),
        ("h", P), ("ln_weight", P), ("ln_bias", P), ("w_q", P), ("w_k", P), ("w_v", P),
        ("M", I32), ("C", I32), ("H", I32),
        ("q_s", P), ("k_s", P), ("v_s", P), ("q_norm", P), ("k_norm", P), ("ln_mean", P), ("ln_rstd", P),
        ("dq_s", P), ("dk_s", P), ("dv_s", P),
        ("dh", P), ("dln_weight", P), ("dln_bias", P), ("dw_q", P), ("dw_k", P), ("dw_v", P),
    ]


class CoordUpdateParams(ctypes.Structure):
    """Mirror of ``dfl_coord_update_params``."""

    _fields_ = [
        ("dtype", I32),
        ("h", P), ("ln_weight", P), ("ln_bias", P), ("w_gate", P), ("b_gate", P), ("lambda_raw", P),
        ("x_centroid", P), ("x_res", P), ("mask", P),
        ("B", I32), ("N", I32), ("C", I32), ("H", I32),
        ("x_out", P),
        ("dx_out", P), ("dx_res", P), ("dx_centroid", P), ("dh", P), ("dln_weight", P), ("dln_bias", P),
        ("dw_gate", P), ("db_gate", P), ("dlambda_raw", P),
    ]


DFL_ATTN_BIAS_NONE = 0
DFL_ATTN_BIAS_BINS = 1
DFL_ATTN_BIAS_DENSE = 2
DFL_ATTN_BIAS_WINDOW = 3

# (name, restype, argtypes) of every exported symbol; tests check that the .so
# exports exactly what include/dfl_amd.h declares.
SIGNATURES = [
    ("dfl_last_error", ctypes.c_char_p, []),
    ("dfl_version", ctypes.c_char_p, []),
    ("dfl_workspace_error", I32, [P, P]),
    ("dfl_pending_error", I32, []),
    ("dfl_set_launch_mode", I32, [I32]),
    ("dfl_get_launch_mode", I32, []),
    ("dfl_debug_set_spin_limit", I32, [ctypes.c_uint]),
    ("dfl_sinkhorn_workspace_size", ctypes.c_size_t, [I32, I32, I32]),
    ("dfl_sinkhorn_bias_workspace_size", ctypes.c_size_t, [I32, I32, I32]),
    ("dfl_sinkhorn_fwd", I32, [ctypes.POINTER(SinkhornFwdParams), P, ctypes.c_size_t, P]),
    ("dfl_sinkhorn_fwd_noalloc", I32, [ctypes.POINTER(SinkhornFwdParams), P]),
    ("dfl_noalloc_error", I32, [P]),
    ("dfl_sinkhorn_bwd", I32, [ctypes.POINTER(SinkhornBwdParams), P, ctypes.c_size_t, P]),
    ("dfl_sinkhorn_unrolled_workspace_size", ctypes.c_size_t, [I32, I32, I32, I32]),
    ("dfl_sinkhorn_unrolled_bwd", I32, [ctypes.POINTER(SinkhornUnrolledBwdParams), P, ctypes.c_size_t, P]),
    ("dfl_attn_workspace_size", ctypes.c_size_t, [I32, I32, I32, I32, I32]),
    ("dfl_attn_fwd", I32, [ctypes.POINTER(AttnParams), P]),
    ("dfl_attn_bwd", I32, [ctypes.POINTER(AttnParams), P, ctypes.c_size_t, P]),
    ("dfl_a2t_workspace_size", ctypes.c_size_t, [I32, I32, I32, I32]),
    ("dfl_a2t_fwd", I32, [ctypes.POINTER(A2TParams), P]),
    ("dfl_a2t_bwd", I32, [ctypes.POINTER(A2TParams), P, ctypes.c_size_t, P]),
    ("dfl_dense_sinkhorn_workspace_size", ctypes.c_size_t, [I32, I32, I32, I32]),
    ("dfl_dense_sinkhorn_fwd", I32, [ctypes.POINTER(DenseSinkhornParams), P, ctypes.c_size_t, P]),
    ("dfl_dense_sinkhorn_bwd", I32, [ctypes.POINTER(DenseSinkhornBwdParams), P, ctypes.c_size_t, P]),
    ("dfl_dense_transport_workspace_size", ctypes.c_size_t, [I32, I32, I32, I32]),
    ("dfl_dense_transport_fwd", I32, [ctypes.POINTER(DenseTransportParams), P]),
    ("dfl_dense_transport_bwd", I32, [ctypes.POINTER(DenseTransportParams), P, ctypes.c_size_t, P]),
    ("dfl_balanced_workspace_size", ctypes.c_size_t, [I32, I32, I32, I32, I32]),
    ("dfl_balanced_fwd", I32, [ctypes.POINTER(BalancedFwdParams), P, ctypes.c_size_t, P]),
    ("dfl_balanced_bwd", I32, [ctypes.POINTER(BalancedBwdParams), P, ctypes.c_size_t, P]),
    ("dfl_sink_proj_workspace_size", ctypes.c_size_t, [I32, I32]),
    ("dfl_sink_proj_fwd", I32, [ctypes.POINTER(SinkProjParams), P]),
    ("dfl_sink_proj_bwd", I32, [ctypes.POINTER(SinkProjParams), P, ctypes.c_size_t, P]),
    ("dfl_coord_update_workspace_size", ctypes.c_size_t, [I32, I32]),
    ("dfl_coord_update_fwd", I32, [ctypes.POINTER(CoordUpdateParams), P]),
    ("dfl_coord_update_bwd", I32, [ctypes.POINTER(CoordUpdateParams), P, ctypes.c_size_t, P]),
]


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes handle; raise if the library is absent."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(
                    f"deepfold_amd: HIP library not built ({path} missing). "
                    "Run `python -c 'import __graft_entry__ as g; g.build()'` from the repo root.")
            lib = ctypes.CDLL(path)
            for name, res, args in SIGNATURES:
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
        return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().dfl_last_error().decode(errors="replace")
        raise RuntimeError(f"deepfold_amd {what} failed (code {rc}): {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("deepfold_amd ops run only on ROCm GPU tensors (no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("deepfold_amd: all tensors must be on the same device")
    if dev is None:
        raise RuntimeError("deepfold_amd: no tensor inputs")
    return dev


_ws_cache: dict = {}


def workspace(device: torch.device, nbytes: int, kind: str = "sinkhorn") -> torch.Tensor:
    """Zero-filled device workspace, cached per (device, stream, kind) and grown on demand.

    Each kind of op gets its own buffer: the Sinkhorn kernels keep tagged exchange
    words and an error word in theirs, which other ops must never overwrite."""
    key = (device.index, stream_handle(device), kind)
    ws = _ws_cache.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _ws_cache[key] = ws
    return ws


# Optional per-launch timing: when a list is installed here, every C-ABI launch
# appends (name, start_event, end_event) recorded on the launch stream.
launch_timings: list | None = None
# With launch_timings on: the launch names to bracket with events (None: every launch).
# An event pair costs a few microseconds of stream time per launch.
launch_timed: set | None = None


def raise_pending(what: str = "deepfold_amd") -> None:
    """Raise if a kernel launched earlier reported an expired cross-workgroup wait.

    Reads a pinned host word that such a kernel writes (no synchronisation): it
    sees what kernels completed so far reported.  Every C-ABI launch below calls
    it first, so a failed launch raises at the next call at the latest; call
    ``torch.cuda.synchronize()`` before it to check a finished batch of work."""
    code = load().dfl_pending_error()
    if code != 0:
        msg = load().dfl_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg}")


def timed_launch(name: str, device: torch.device, fn):
    """Run ``fn()`` (one C-ABI call), bracketing it with events if timing is on.
    Raises first if an earlier launch reported an expired wait."""
    raise_pending(name)
    if launch_timings is None or (launch_timed is not None and name not in launch_timed):
        return fn()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream(device)
    s.record(stream)
    rc = fn()
    e.record(stream)
    launch_timings.append((name, s, e))
    return rc


def set_launch_mode(mode: int) -> None:
    """Process-wide launch mode of the persistent kernels (``DFL_LAUNCH_*``)."""
    check(load().dfl_set_launch_mode(int(mode)), "dfl_set_launch_mode")


def get_launch_mode() -> int:
    return int(load().dfl_get_launch_mode())


def debug_checks() -> bool:
    return os.environ.get("DFL_AMD_CHECK", "0") not in ("", "0")


def check_workspace(ws: torch.Tensor, what: str) -> None:
    """Synchronising check of the kernel-side error word (used when DFL_AMD_CHECK=1)."""
    code = load().dfl_workspace_error(ctypes.c_void_p(ws.data_ptr()),
                                      ctypes.c_void_p(stream_handle(ws.device)))
    if code != 0:
        raise RuntimeError(f"deepfold_amd {what}: kernel reported error code {code} "
                           "(a cross-workgroup wait expired)")
