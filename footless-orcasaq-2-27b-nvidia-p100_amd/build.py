"""Build libfl355.so (the gfx950 HIP kernels + their C ABI) in-tree with hipcc.

Each ``csrc/*.hip`` compiles to an object under ``_build/`` (in parallel),
then one shared library is linked next to this file. Every HIP compile line
carries ``-Xclang -target-feature -Xclang -packed-fp32-ops``: packed fp32
instructions are kept out of the generated code.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = REPO / "_build" / "fl355"
LIB_PATH = PKG_DIR / "libfl355.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# Per-source extras. attn_prefill: the compiler's MFMAs (the S = K Q^T
# scores) accumulate in VGPRs, where the softmax reads them (the P V
# accumulators are AGPRs held by inline asm); no NaNs and IEEE mode off, so
# the score max is plain v_max / v_max3 without NaN-quieting canonicalisation
# (scores are finite or -inf). attn_decode: its accumulators (scores read by the
# softmax, O rescaled in place) in VGPRs as well. gdn_chunk: the products'
# results are split, scaled and fed back as operands by VALU code; in AGPRs
# each would be copied out first.
FILE_FLAGS = {
    "attn_prefill": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans", "-mno-amdgpu-ieee"],
    "attn_decode": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "gdn_chunk": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libfl355")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.stem, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libfl355.so; returns its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 4) // 2), 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libfl355.so failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
