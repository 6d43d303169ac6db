"""Build step of libseqattn_hip.so (the gfx950 kernels and transfer pipeline).

Compiles stream-attn_amd/csrc/*.hip|*.cpp with hipcc for gfx950 into
stream-attn_amd/seqattn/_lib/libseqattn_hip.so.  The library is built in-tree
so it travels with the source tree; nothing is installed system-wide.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_ROOT.parent
CSRC = PACKAGE_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_DIR = PACKAGE_ROOT / "seqattn" / "_lib"
LIB_PATH = LIB_DIR / "libseqattn_hip.so"
# bench.py's register-only MFMA rate probe; not part of the attention path.
PROBE_LIB_PATH = LIB_DIR / "libseqattn_probe.so"
ARCH = "gfx950"

SOURCES = ("sa_kernels.hip", "sa_pipeline.cpp")
PROBE_SOURCES = ("sa_probe.hip",)

# Device-side flags.  Packed FP32 VALU instructions are disabled for all
# device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # Keep MFMA accumulators in VGPRs: the softmax rescale multiplies them
    # with VALU ops, and AGPR-resident accumulators were copied to VGPRs and
    # back on every tile.
    "-mllvm",
    "--amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; ROCm is required to build libseqattn_hip.so")


def build(verbose: bool = False) -> Path:
    """Compile every source into the attention library and the probe library;
    returns the attention library's path."""
    _link(SOURCES, LIB_PATH, verbose)
    _link(PROBE_SOURCES, PROBE_LIB_PATH, verbose)
    return LIB_PATH


def _link(sources, target: Path, verbose: bool) -> None:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = target.with_suffix(".so.tmp")
    cmd = [
        hipcc(),
        *HIP_FLAGS,
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        "-shared",
        *(str(CSRC / name) for name in sources),
        "-o",
        str(tmp),
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    # The host compilation pass reports the device-only target feature as
    # unknown; that note is expected and not an error.
    stderr = "\n".join(
        line for line in result.stderr.splitlines() if "packed-fp32-ops" not in line
    )
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    os.replace(tmp, target)


if __name__ == "__main__":
    print(build(verbose=True))
