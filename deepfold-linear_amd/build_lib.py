"""Build libdfl_amd.so (and the probe library libdfl_peaks.so) in-tree with hipcc for gfx950.

Every source compiles to its own object in parallel, then one link step.

Usage: python deepfold-linear_amd/build_lib.py  (also called by __graft_entry__.build()).
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "deepfold_amd", "libdfl_amd.so")
OBJ_DIR = os.path.join(HERE, "_build")
SOURCES = ["capi.hip", "sinkhorn_fwd.hip", "sinkhorn_fwd_stream.hip", "sinkhorn_fwd_reg.hip", "sinkhorn_fwd_blk.hip", "sinkhorn_bwd.hip",
           "sinkhorn_bwd_stream.hip", "attention.hip", "dense.hip", "balanced_bwd.hip",
           "unrolled_bwd.hip", "trunk_steps.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# issue-rate / exchange probes (bench.py --workload peaks only): a library of its own
PROBE_SOURCE = "peaks.hip"
PROBE_OUT = os.path.join(HERE, "deepfold_amd", "libdfl_peaks.so")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # keep hipcc from forming packed-fp32 ops by itself
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _clean(text: str) -> str:
    return "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    jobs = []
    for src in SOURCES:
        obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *FLAGS, "-c", "-o", obj, os.path.join(CSRC, src)]
        if verbose:
            print("[build]", " ".join(cmd), flush=True)
        jobs.append((src, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    probe_obj = os.path.join(OBJ_DIR, "peaks.o")
    probe_cmd = [HIPCC, *FLAGS, "-c", "-o", probe_obj, os.path.join(CSRC, PROBE_SOURCE)]
    if verbose:
        print("[build]", " ".join(probe_cmd), flush=True)
    probe = subprocess.Popen(probe_cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    errors = []
    for src, _, proc in jobs + [(PROBE_SOURCE, probe_obj, probe)]:
        out, _ = proc.communicate()
        out = _clean(out)
        if proc.returncode != 0:
            errors.append(f"{src}: hipcc failed ({proc.returncode}):\n{out}")
        elif out.strip() and verbose:
            print(out, flush=True)
    if errors:
        raise RuntimeError("\n".join(errors))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *[obj for _, obj, _ in jobs]]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed ({proc.returncode}):\n{_clean(proc.stdout + proc.stderr)}")
    os.replace(tmp, OUT)
    tmp = PROBE_OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, probe_obj]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"probe link failed ({proc.returncode}):\n{_clean(proc.stdout + proc.stderr)}")
    os.replace(tmp, PROBE_OUT)
    return OUT


if __name__ == "__main__":
    print(build())
    sys.exit(0)
