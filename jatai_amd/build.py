"""Builds libjatai.so (gfx950) in-tree from jatai_amd/csrc with hipcc.

One translation unit (csrc/jatai.hip includes the kernel files), so the device error record is shared by every
kernel. Packed-FP32 instruction selection is disabled (-packed-fp32-ops); the host pass warns that it does not
know the feature, which is harmless. MFMA destinations are kept in VGPRs (-amdgpu-mfma-vgpr-form). Usage: python -m jatai_amd.build
"""
import os
import subprocess
import sys

AQUI = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(AQUI, "csrc")
SAIDA = os.path.join(AQUI, "libjatai.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-mcode-object-version=5",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # MFMA results in VGPRs: the epilogues read every MFMA output, an AGPR->VGPR move each otherwise
         "-mllvm", "-amdgpu-mfma-vgpr-form"]


def build(saida=SAIDA, extra=()):
    tmp = saida + ".tmp"
    cmd = [HIPCC, *FLAGS, *extra, "-o", tmp, os.path.join(CSRC, "jatai.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    erros = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{erros}")
    os.replace(tmp, saida)
    return saida


if __name__ == "__main__":
    print(build(extra=sys.argv[1:]))
