"""Build recipe for libfarope.so (hand-written gfx950 HIP kernels + C ABI).

Compiles every translation unit under csrc/ with hipcc for gfx950 (in
parallel), then links one shared library next to this file, where
``_lib.py`` loads it.  Runs on a machine without a GPU: hipcc
cross-compiles.  ``python -m triton_fused_rope_flash_attn_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "libfarope.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["api.hip", "fwd.hip", "fwd_plane.hip", "bwd.hip", "bwd_fused.hip", "bwd_keys.hip", "bwd_ds.hip", "tail.hip"]
# Per-file code generation options.  fwd_plane.hip keeps its MFMA results in
# VGPRs (they feed the softmax VALU directly) and its resident operand
# fragments in AGPRs.
EXTRA_FLAGS = {"fwd_plane.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libfarope.so")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=fast",
        # The kernels never depend on NaN semantics (masked logits are -inf):
        # with IEEE mode off, fmax needs no operand canonicalization.
        "-fno-honor-nans",
        "-mno-amdgpu-ieee",
        "-mcode-object-version=5",
        # Packed-fp32 VALU forms are kept out of the generated code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        "-Wno-unused-result",
    ]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in res.stdout.splitlines() if "packed-fp32-ops" not in ln
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile and link libfarope.so; returns its path."""
    hipcc = _hipcc()
    flags = compile_flags()
    tmp = tempfile.mkdtemp(prefix="farope_build_")
    try:
        objs = []
        cmds = []
        for src in SOURCES:
            obj = os.path.join(tmp, src.replace(".hip", ".o"))
            objs.append(obj)
            cmds.append([hipcc, *flags, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
        jobs = jobs or min(len(cmds), os.cpu_count() or 1, 16)
        with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
                if verbose:
                    print(" ".join(cmd), flush=True)
                fut.result()
        out_tmp = LIB_PATH + ".tmp"
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", out_tmp])
        os.replace(out_tmp, LIB_PATH)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    if verbose:
        print(f"built {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
