"""Build libgmhip.so, the package's HIP kernels for gfx950, in-tree.

``python gm-attention_amd/build.py`` (or :func:`build`) compiles every
``csrc/*.hip`` with ``hipcc --offload-arch=gfx950`` into ``_build/`` and links
``gm_attention_amd/_lib/libgmhip.so``.  Packed FP32 instructions are disabled
on every device compile (``-packed-fp32-ops``): hipcc forms them from plain
float code, and some of their forms are not trusted on this hardware.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
LIB = ROOT / "gm_attention_amd" / "_lib" / "libgmhip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


#: Per-source extra flags.  The factored, trunk and depthwise-walk kernels keep
#: their MFMA accumulators in VGPRs: the VALU reads every accumulator (the
#: factored slots, the trunk's SiLU and partial rows, the walk's dC and dh~), so
#: AGPRs would only add copies and registers (the trunk backward: 184 -> 151
#: VGPRs, three waves a SIMD; the paired depthwise backward: 88 AGPR copies an
#: edge tile gone, 28.0 -> 27.0 ms at 256x512, B = 4; the fused feed-forward's
#: backward: 222 + 40 AGPRs -> 254 registers, two waves a SIMD instead of one,
#: 1.41 -> 1.08 ms at the C4 block).
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
EXTRA = {"factored.hip": _VGPR_MFMA, "trunk.hip": _VGPR_MFMA, "depthwise_radial.hip": _VGPR_MFMA,
         "ffn.hip": _VGPR_MFMA}


def _compile(source: Path, verbose: bool) -> Path:
    obj = BUILD / (source.stem + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(source.name, []), "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or result.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + result.stdout + result.stderr)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or result.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + result.stdout + result.stderr)
    if result.returncode != 0:
        raise RuntimeError("linking libgmhip.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
