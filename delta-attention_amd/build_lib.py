"""Build libdelta_attn.so (the C-ABI library) for gfx950 with hipcc.

Run as a script or call ``build()``. The library lands next to the Python
package (delta_attention/libdelta_attn.so) so that it travels with the tree.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(HERE, "delta_attention", "libdelta_attn.so")
SOURCES = ["attn_kernels.hip", "attn_bwd.hip", "delta_add.hip", "rope.hip", "norm.hip",
           "anchor_cos.hip", "adapt_loop.hip"]
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled: they are not used by hand and must not be
# formed by the compiler either.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMAs the compiler emits keep their accumulators in VGPRs also in the
    # one-wave-per-SIMD kernels (their default there is the AGPR form, whose
    # score tiles the softmax would have to copy out); the accumulators meant
    # for AGPRs are placed there by inline asm
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def build(verbose: bool = False, out: str = OUT) -> str:
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
           *[os.path.join(CSRC, s) for s in SOURCES], "-o", out + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass warns that it does not know the packed-fp32 feature
    warn = "\n".join(l for l in res.stderr.splitlines()
                     if "packed-fp32-ops" not in l and l.strip())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{warn}")
    if warn and verbose:
        print(warn, file=sys.stderr)
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
