"""Builds libfmx.so (HIP kernels for gfx950 + the C-ABI) in-tree.

Usage: python -m flashmlx_amd.build   (or flashmlx_amd.build.build())
Objects go to flashmlx_amd/_build/, the library to flashmlx_amd/libfmx.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
LIB = HERE / "libfmx.so"
OBJDIR = HERE / "_build"

SOURCES = [
    "csrc/fmx_route.hip",
    "csrc/fmx_qgemm.hip",
    "csrc/fmx_pack.hip",
    "csrc/fmx_decode.hip",
    "csrc/fmx_prefill.hip",
    "csrc/fmx_elem.hip",
    "csrc/fmx_api.cpp",
    "csrc/fmx_synth.hip",
    "csrc/fmx_model.hip",
    "csrc/fmx_model.cpp",
    "csrc/fmx_loader.cpp",
    "csrc/fmx_sched.cpp",
    "csrc/fmx_nh_decode.hip",
    "csrc/fmx_nh.cpp",
]

ARCH = os.environ.get("FMX_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in any kernel.
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(ROOT / "include"),
]


# per-source additions. The decode kernels fold MFMA results into their
# accumulators with VALU FMAs: MFMAs that write VGPRs save an accumulator
# register move per value.
EXTRA_FLAGS = {
    "csrc/fmx_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "csrc/fmx_nh_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfmx.so)")


def _compile(cc: str, src: pathlib.Path, obj: pathlib.Path, extra: list) -> tuple[str, int, str]:
    cmd = [cc, "-x", "hip", *CFLAGS, *extra, "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    err = "\n".join(
        ln for ln in p.stderr.splitlines()
        if "packed-fp32-ops" not in ln and "not a recognized feature" not in ln and ln.strip()
    )
    return str(src), p.returncode, err


def build(verbose: bool = False) -> pathlib.Path:
    """Compiles every source and links libfmx.so; raises on any error."""
    cc = hipcc()
    OBJDIR.mkdir(exist_ok=True)
    objs = []
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        for rel in SOURCES:
            src = HERE / rel
            obj = OBJDIR / (src.name + ".o")
            objs.append(obj)
            jobs.append(ex.submit(_compile, cc, src, obj, EXTRA_FLAGS.get(rel, [])))
        failed = []
        for j in jobs:
            src, rc, err = j.result()
            if err and (verbose or rc):
                print(f"[fmx build] {src}:\n{err}", file=sys.stderr)
            if rc:
                failed.append(src)
    if failed:
        raise RuntimeError(f"libfmx build failed: {failed}")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp), "-lpthread"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode:
        raise RuntimeError(f"libfmx link failed:\n{p.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
