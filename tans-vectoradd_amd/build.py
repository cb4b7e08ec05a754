"""Build libtans_amd.so in-tree: the CPU codec (g++, OpenMP) and the gfx950
HIP kernels and GPU encoder (hipcc), linked into one shared library next to the Python
package (rans_vectoradd/libtans_amd.so).

    python tans-vectoradd_amd/build.py [--asm]

--asm also writes the gfx950 assembly of kernels.hip under _build/ for
inspection.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "rans_vectoradd", "libtans_amd.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# Packed FP32 VALU ops are kept out of every kernel (they have produced
# silent wrong results on these boxes); the host pass ignores the feature.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# The decoders' one atomic is a single lane's LDS add per tile (the pacing
# count).  The atomic optimizer rewrites it for a whole wave (mbcnt, a
# compare and a second exec mask: 6 VALU and 6 SALU per tile), so it is off
# for kernels.hip.
KERNEL_FLAGS = ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]
CXX_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-fopenmp", "-Wall", "-Wextra"]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    # hipcc's host pass warns once per file about the packed-fp32 feature
    noise = "'-packed-fp32-ops' is not a recognized feature"
    for line in (res.stdout + res.stderr).splitlines():
        if line.strip() and noise not in line:
            sys.stderr.write(line + "\n")


def build(asm: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    codec_o = os.path.join(BUILD, "codec.o")
    kern_o = os.path.join(BUILD, "kernels.o")
    enc_o = os.path.join(BUILD, "encode.o")
    _run(["g++", *CXX_FLAGS, "-c", os.path.join(CSRC, "codec.cpp"), "-o", codec_o])
    _run([HIPCC, *HIP_FLAGS, *KERNEL_FLAGS, "-c", os.path.join(CSRC, "kernels.hip"),
          "-o", kern_o])
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, "encode.hip"), "-o", enc_o])
    if asm:
        _run([HIPCC, *HIP_FLAGS, *KERNEL_FLAGS, "--cuda-device-only", "-S",
              os.path.join(CSRC, "kernels.hip"), "-o", os.path.join(BUILD, "kernels.s")])
    tmp = OUT + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, codec_o, kern_o, enc_o,
          "-lgomp"])
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(asm="--asm" in sys.argv))
