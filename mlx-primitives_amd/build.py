"""Build libmpx_attn.so (the gfx950 HIP kernels + C ABI) in-tree.

Usage: python mlx-primitives_amd/build.py [--verbose]

The library lands in mlx-primitives_amd/mlx_primitives/_lib/libmpx_attn.so,
where the Python layer loads it with ctypes. Host-only compilation: no GPU is
needed to build.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB_DIR = os.path.join(HERE, "mlx_primitives", "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libmpx_attn.so")

SOURCES = ["abi.hip", "fa_fwd.hip", "fa_fwd_drop.hip", "fa_bwd.hip", "fa_bwd32.hip",
           "paged_decode.hip", "kv_cache.hip", "rope.hip"]
# Per-source device-compiler options. MFMA accumulators in arch VGPRs
# (-amdgpu-mfma-vgpr-form): the default heuristic moves them through AGPRs with
# a copy per element per tile, and spills VGPRs into AGPRs where both are
# full; the head-dim-256 forward runs 16% faster without that, the float32
# head-dim-256 backward 16% faster and without its scratch spills. The forward
# kernels (except dropout, fa_fwd_drop.hip) and the decode kernels are
# scheduled for maximum ILP: +1-2% on the dense, windowed and float32 forward
# and on paged decode; the backward and the dropout forward run slower with it.
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
_MAX_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
EXTRA_FLAGS = {"fa_fwd.hip": _MAX_ILP + _VGPR_MFMA,
               "fa_fwd_drop.hip": _VGPR_MFMA,
               "fa_bwd.hip": _VGPR_MFMA,
               "fa_bwd32.hip": _VGPR_MFMA,
               "paged_decode.hip": _VGPR_MFMA + _MAX_ILP}
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmpx_attn.so)")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-I" + INCLUDE,
        "-I" + CSRC,
        # Packed fp32 VALU ops are kept out of the device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in proc.stderr.splitlines() if noise not in ln)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> str:
    """Compile every source to an object (in parallel), then link the library."""
    os.makedirs(LIB_DIR, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="mpx_build.") as tmpdir:
        jobs = []
        for src in SOURCES:
            obj = os.path.join(tmpdir, src.replace(".hip", ".o"))
            cmd = ([hipcc()] + compile_flags() + EXTRA_FLAGS.get(src, [])
                   + ["-c", os.path.join(CSRC, src), "-o", obj])
            jobs.append((cmd, obj))
        workers = min(len(jobs), max(1, (os.cpu_count() or 1)), 8)
        with ThreadPoolExecutor(max_workers=workers) as ex:
            for f in [ex.submit(_run, cmd, verbose) for cmd, _ in jobs]:
                f.result()
        fd, tmp = tempfile.mkstemp(prefix="libmpx_attn.", suffix=".so.tmp", dir=LIB_DIR)
        os.close(fd)
        try:
            _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC"]
                 + [obj for _, obj in jobs] + ["-o", tmp], verbose)
        except Exception:
            os.unlink(tmp)
            raise
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(verbose=args.verbose))
