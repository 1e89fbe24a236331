"""Builds libzt_hip.so (the gfx950 kernels + host helpers) in-tree.

Each source compiles to an object under ztensor_amd/_build/ in parallel,
then hipcc links the shared library next to this file.  Usable as
``python -m ztensor_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libzt_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]
# Packed-FP32 (v_pk_*_f32) instructions are switched off for device code.
# The first kernel-argument dwords are preloaded into SGPRs at wave launch
# (gfx950 kernarg preload), so a kernel does not wait on an s_load of its
# arguments before it can issue its first memory load: 1238 -> 1171 us for
# the 224-GEMV decode step.  Kernels still carry the s_load fallback entry
# for firmware without preloading.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mllvm", "-amdgpu-kernarg-preload-count=16"]


# Per-source device flags.  The tiled MFMA kernels consume MFMA results in
# VALU right away; the VGPR form of the MFMAs avoids copying each result out
# of the accumulation registers first.
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
EXTRA = {"zt_blockt.hip": _VGPR_MFMA, "zt_q4.hip": _VGPR_MFMA, "zt_q8.hip": _VGPR_MFMA, "zt_w4a16.hip": _VGPR_MFMA,
         "zt_intq.hip": _VGPR_MFMA}


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *COMMON, *(DEVICE if src.suffix == ".hip" else []), *EXTRA.get(src.name, []), "-c", str(src),
           "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
