"""Builds libexactattn_hip.so in-tree with hipcc for gfx950 (python -m exactattention_amd.build)."""

from __future__ import annotations

import os
import subprocess
import sys

SOURCES = ["ea_hip.hip", "ea_decode.hip", "ea_prefill.hip", "ea_exact_host.cpp", "ea_csr.cpp"]
HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libexactattn_hip.so")

# -packed-fp32-ops: never emit packed fp32 VALU ops (their forms have misbehaved on this pool).
# -fno-gpu-flush-denormals-to-zero: bf16 subnormals convert exactly through fp32.
# -amdgpu-mfma-vgpr-form=1: MFMA operands and accumulators in VGPRs; the prefill kernel's int32
#  accumulators are also read by VALU folds, and the AGPR file then serves as cheap spill space
#  (the AGPR form spills the kernel's working set to scratch).
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
               "-fno-gpu-flush-denormals-to-zero", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-mllvm", "-amdgpu-mfma-vgpr-form=1", "-Wall", "-Wno-unused-function"]


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    gen = os.path.join(CSRC, "gen_tables.py")
    subprocess.run([sys.executable, gen], check=True, stdout=subprocess.DEVNULL)
    tmp = LIB + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-o", tmp] + [os.path.join(CSRC, f) for f in SOURCES]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libexactattn_hip.so")
    if verbose:
        sys.stderr.write(r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
