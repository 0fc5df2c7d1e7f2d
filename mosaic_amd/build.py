"""Build libmosaic_bsa.so (gfx950) in-tree with hipcc.

    python -m mosaic_amd.build            # compile all sources in mosaic_amd/csrc
    python -m mosaic_amd.build --jobs 4

Each .hip source is compiled to an object in mosaic_amd/_build and linked into
mosaic_amd/libmosaic_bsa.so.  The library exports only the C ABI of include/mosaic_bsa.h.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libmosaic_bsa.so")
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-fvisibility=hidden",
    # compile without packed-fp32 VALU instructions (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wno-unused-command-line-argument",
]

# Per-source flags.  cmp.hip and bwd.hip: keep MFMA accumulators in VGPRs; by default the
# compiler puts them in AGPRs there and copies the softmax operands back and forth every tile
# (48 v_accvgpr_read per tile in cmp; 352 accumulator moves in the grad-k/v kernel).  The attention kernel keeps its default (the flag costs it
# occupancy in its two-wave instantiations).
FILE_FLAGS = {
    "cmp.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "proj.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "ffn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # the k-NN kernel's scores are never NaN: its maxima over lane exchanges then need no
    # canonicalising instruction per operand (kernels run with the IEEE mode bit clear)
    "interp.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
}


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), *extra, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int = 4, extra: list[str] | None = None, verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    extra = list(extra or [])
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), srcs))
    tmp = LIB_PATH + ".tmp"
    # --no-undefined: a kernel whose host-side stub was not emitted must fail the build here,
    # not at load time
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print("built", LIB_PATH)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--extra", nargs="*", default=[])
    args = ap.parse_args()
    build(args.jobs, args.extra, verbose=True)


if __name__ == "__main__":
    main()
