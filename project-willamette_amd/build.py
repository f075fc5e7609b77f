"""Build libwillamette_hip.so (gfx950) in-tree with hipcc.

    python project-willamette_amd/build.py

Every HIP/C++ source under csrc/ is compiled to an object in _build/ (in
parallel) and linked into project-willamette_amd/libwillamette_hip.so.
Floating point: -ffp-contract=off (no mul+add fusion anywhere: the decode
path reproduces the reference's unfused f32 arithmetic), no fast-math, IEEE
denormals (hipcc's default), packed-fp32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libwillamette_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-value",
    "-Wno-unused-result",
]


# The batched GEMM keeps its MFMA accumulators in VGPRs: with the compiler's
# default (AGPRs) its wave-split-K loop copies them between the two register
# files on every chunk.
# The fused matvecs and decode attention take what their first loads need in
# their leading 16 argument dwords, which the hardware then preloads into
# SGPRs at wave launch instead of each wave fetching them from memory.
PER_FILE = {"k_batch.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
            "k_i2s.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
            "k_attn.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *COMMON, *PER_FILE.get(src.name, [])]
    if src.suffix == ".hip":
        cmd += ["-x", "hip"]
    cmd += ["-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
