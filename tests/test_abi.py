"""CPU checks of the C ABI and the host side (no GPU, no kernel launches).

* libdfl_amd.so loads and exports every function include/dfl_amd.h declares, and
  the ctypes binding lists exactly those functions;
* the ctypes mirrors of the parameter structs have the C layout (offsets and
  sizes printed by a probe compiled with gcc against the header);
* the public op refuses CPU tensors (there is no CPU fallback);
* bench.py refuses more than one GPU.
"""

import ctypes
import os
import re
import subprocess
import sys
import tempfile

import pytest

from conftest import PKG_ROOT, ROOT

HEADER = os.path.join(ROOT, "include", "dfl_amd.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dfl_\w+)\s*\(", text)))


def header_structs():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for body, name in re.findall(r"typedef struct \w+ \{(.*?)\} (\w+);", text, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            head, names = re.match(r"(.*?[\s*])(\w+(?:\s*,\s*\w+)*)$", decl).groups()
            fields += [n.strip() for n in names.split(",")]
        out[name] = fields
    return out


@pytest.fixture(scope="module")
def lib_path():
    from deepfold_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):  # build it (hipcc cross-compiles without a GPU)
        sys.path.insert(0, PKG_ROOT)
        import build_lib

        build_lib.build(verbose=False)
    return _lib.LIB_PATH


def test_library_exports_every_header_function(lib_path):
    lib = ctypes.CDLL(lib_path)
    names = header_functions()
    assert "dfl_sinkhorn_fwd" in names and "dfl_sinkhorn_bwd" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    nm = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True)
    exported = set(re.findall(r"\bT (dfl_\w+)$", nm.stdout, flags=re.M))
    assert exported == set(names), f"extra exports: {exported - set(names)}"


def test_binding_matches_header(lib_path):
    from deepfold_amd import _lib

    assert sorted(n for n, _, _ in _lib.SIGNATURES) == header_functions()
    lib = _lib.load(lib_path)
    assert lib.dfl_version().decode().startswith("deepfold_amd")


def test_struct_layout_matches_c(lib_path):
    from deepfold_amd import _lib

    structs = header_structs()
    mirrors = {"dfl_sinkhorn_fwd_params": _lib.SinkhornFwdParams,
               "dfl_sinkhorn_unrolled_bwd_params": _lib.SinkhornUnrolledBwdParams,
               "dfl_sinkhorn_bwd_params": _lib.SinkhornBwdParams,
               "dfl_attn_params": _lib.AttnParams,
               "dfl_a2t_params": _lib.A2TParams,
               "dfl_dense_sinkhorn_params": _lib.DenseSinkhornParams,
               "dfl_dense_sinkhorn_bwd_params": _lib.DenseSinkhornBwdParams,
               "dfl_dense_transport_params": _lib.DenseTransportParams,
               "dfl_balanced_fwd_params": _lib.BalancedFwdParams,
               "dfl_balanced_bwd_params": _lib.BalancedBwdParams,
               "dfl_sink_proj_params": _lib.SinkProjParams,
               "dfl_coord_update_params": _lib.CoordUpdateParams}
    assert set(mirrors) == set(structs)
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for sname, fields in structs.items():
        lines.append(f'  printf("{sname} size %zu\\n", sizeof({sname}));')
        for f in fields:
            lines.append(f'  printf("{sname} {f} %zu\\n", offsetof({sname}, {f}));')
    lines += ["  return 0;", "}"]
    with tempfile.TemporaryDirectory() as td:
        src, exe = os.path.join(td, "probe.c"), os.path.join(td, "probe")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c99", "-o", exe, src], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    c_layout = {}
    for line in out.splitlines():
        s, f, v = line.split()
        c_layout[(s, f)] = int(v)
    for sname, cls in mirrors.items():
        py_fields = [f for f, _ in cls._fields_]
        assert py_fields == structs[sname], sname
        assert ctypes.sizeof(cls) == c_layout[(sname, "size")], sname
        for f in py_fields:
            assert getattr(cls, f).offset == c_layout[(sname, f)], (sname, f)


def test_integration_snippet_matches_binding():
    """The ctypes struct INTEGRATION.md shows a maintainer lists every field of
    dfl_sinkhorn_fwd_params, in order and with the right C types: a struct that
    stops short hands the library whatever memory follows it."""
    from deepfold_amd import _lib

    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text[text.index("class FwdParams(ctypes.Structure)"):]
    block = block[:block.index("lib.dfl_sinkhorn_workspace_size")]
    fields = re.findall(r'\("(\w+)",\s*(\w)\)', block)
    types = {"P": ctypes.c_void_p, "I": ctypes.c_int, "L": ctypes.c_longlong, "F": ctypes.c_float}
    assert [n for n, _ in fields] == [n for n, _ in _lib.SinkhornFwdParams._fields_]
    assert [n for n, _ in fields] == header_structs()["dfl_sinkhorn_fwd_params"]
    for (n, t), (_, want) in zip(fields, _lib.SinkhornFwdParams._fields_):
        assert types[t] is want, n


def test_pending_error_is_clear_without_launches(lib_path):
    """The error mailbox reads 0 before any kernel ran (and reading it needs no GPU)."""
    from deepfold_amd import _lib

    assert _lib.load(lib_path).dfl_pending_error() == 0
    _lib.raise_pending("test")


def test_attn_workspace_holds_batched_window_bias_gradient(lib_path):
    """The window bias is shared by the batch, so with B > 1 its gradient is a sum of
    per-row gradients, formed in the workspace: the size grows by B row slab sets of
    ceil(M/32) * H * 32 * 128 four-byte entries for square shapes with B > 1 (where a
    window is possible) and by nothing otherwise; a window-bias gradient call with a
    workspace one byte short is refused before any GPU work (argument checks come
    first, the pointers are never dereferenced)."""
    from deepfold_amd import _lib

    lib = _lib.load(lib_path)
    H, M, d = 2, 150, 32
    slab = -(-M // 32) * H * 32 * 128 * 4
    ws1 = lib.dfl_attn_workspace_size(1, H, M, M, d)
    ws3 = lib.dfl_attn_workspace_size(3, H, M, M, d)
    assert ws3 - 3 * ws1 >= 3 * slab - 256 * 4 and ws3 - 3 * ws1 <= 3 * slab + 256 * 4
    assert lib.dfl_attn_workspace_size(3, H, M, M + 8, d) < lib.dfl_attn_workspace_size(3, H, M, M, d)
    fake = 4096
    p = _lib.AttnParams(dtype=_lib.DFL_BF16, q=fake, k=fake, v=fake, q_stride_b=H * M * d, q_stride_h=M * d,
                        q_stride_n=d, k_stride_b=H * M * d, k_stride_h=M * d, k_stride_n=d,
                        bias_mode=_lib.DFL_ATTN_BIAS_WINDOW, bias=fake, window=1, B=3, H=H, Mq=M, Nk=M, d=d,
                        scale=1.0, o=fake, lse=fake, grad_o=fake, dq=fake, dk=fake, dv=fake, dbias=fake)
    rc = lib.dfl_attn_bwd(ctypes.byref(p), ctypes.c_void_p(fake), ws3 - 1, None)
    assert rc != 0
    assert "workspace too small" in lib.dfl_last_error().decode()


def test_ops_refuse_cpu_tensors():
    import torch
    from deepfold_amd import (atom_to_token_attn, balanced_sinkhorn_transport, balanced_sinkhorn_transport_dual,
                              compute_transport_output, conjugate_gradient, flash_atom_attn, flash_diffusion_attn,
                              flash_sinkhorn, flash_sinkhorn_attn, gated_coordinate_update, sink_projections,
                              sinkhorn_solve, token_to_atom_attn)

    B, H, N, d = 1, 2, 8, 4
    q = torch.randn(B, H, N, d)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_sinkhorn_attn(q, q, q, q, torch.zeros(B, N, 3), torch.zeros(H, 68), None, torch.ones(H),
                            torch.zeros(H), torch.zeros(B, H, N), torch.zeros(B, H, N))
    bins = torch.zeros(B, N, N, dtype=torch.int32)
    for call in (lambda: flash_diffusion_attn(q, q, q, torch.zeros(H, 68), bins),
                 lambda: flash_atom_attn(q, q, q),
                 lambda: token_to_atom_attn(q, q, q),
                 lambda: atom_to_token_attn(q, q, q, torch.zeros(B, N, dtype=torch.int32),
                                            torch.ones(B, N, dtype=torch.int32)),
                 lambda: flash_sinkhorn(q, q, q, torch.zeros(B, N, 3), torch.zeros(H, 68), None, torch.ones(H),
                                        torch.zeros(H), torch.zeros(B, H, N), torch.zeros(B, H, N)),
                 lambda: conjugate_gradient(lambda v: v, torch.ones(4)),
                 lambda: sinkhorn_solve(torch.zeros(B, H, N, N), torch.zeros(B, H, N), torch.zeros(B, H, N),
                                        torch.ones(H)),
                 lambda: compute_transport_output(q, q, torch.zeros(B, H, N), torch.zeros(B, H, N),
                                                  torch.zeros(B, H, N, N), torch.ones(H)),
                 lambda: balanced_sinkhorn_transport(q, q, torch.zeros(B, N, 3), torch.ones(H), torch.zeros(H),
                                                     torch.ones(H)),
                 lambda: balanced_sinkhorn_transport_dual(q, q, torch.zeros(B, N, 3), q, torch.ones(H),
                                                          torch.zeros(H), torch.ones(H)),
                 lambda: sink_projections(torch.randn(B, N, 64), torch.ones(64), torch.zeros(64),
                                          torch.randn(64, 64), torch.randn(64, 64), None, 2),
                 lambda: gated_coordinate_update(torch.randn(B, N, 64), torch.zeros(B, N, 3),
                                                 torch.zeros(B, H, N, 3), torch.ones(64), torch.zeros(64),
                                                 torch.zeros(1, 64), torch.zeros(1), torch.zeros(H))):
        with pytest.raises(RuntimeError, match="GPU"):
            call()


def test_missing_library_fails_loudly(tmp_path):
    from deepfold_amd import _lib

    saved = _lib._lib
    _lib._lib = None
    try:
        with pytest.raises(RuntimeError, match="not built"):
            _lib.load(str(tmp_path / "absent.so"))
    finally:
        _lib._lib = saved


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_launch_mode_setter_round_trips(lib_path):
    """dfl_set_launch_mode / dfl_get_launch_mode are host state only (no GPU call)."""
    from deepfold_amd import _lib

    lib = _lib.load(lib_path)
    before = lib.dfl_get_launch_mode()
    try:
        for mode in (_lib.DFL_LAUNCH_COOPERATIVE, _lib.DFL_LAUNCH_ORDINARY, _lib.DFL_LAUNCH_AUTO):
            assert lib.dfl_set_launch_mode(mode) == 0
            assert lib.dfl_get_launch_mode() == mode
        assert lib.dfl_set_launch_mode(3) != 0
        assert b"launch mode" in lib.dfl_last_error()
        assert lib.dfl_get_launch_mode() == _lib.DFL_LAUNCH_AUTO
    finally:
        lib.dfl_set_launch_mode(before)
    assert lib.dfl_debug_set_spin_limit(0) == 0
