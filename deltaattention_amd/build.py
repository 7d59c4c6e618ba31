"""Build libdeltaattn.so (the C ABI of include/deltaattn.h) for gfx950 with hipcc.

``python -m deltaattention_amd.build`` compiles every ``csrc/*.hip`` into one shared
library next to this file.  The library is built in-tree so that it travels with the
source tree to the GPU machine; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libdeltaattn.so")
ARCH = os.environ.get("DELTAATTN_ARCH", "gfx950")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32.
# -fno-honor-nans: max/min need no NaN canonicalisation (infinities stay honoured; the
# kernels mask with -inf).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-honor-nans",
    # MFMA accumulators in VGPRs: the softmax reads S with VALU instructions, and the
    # AGPR form would copy every S element through v_accvgpr_read
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-result", "-Wno-unused-function",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libdeltaattn.so")
    return exe


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link libdeltaattn.so; returns its path."""
    hipcc = _hipcc()
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="deltaattn_build_") as tmp:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj]
            r = subprocess.run(cmd, capture_output=True, text=True)
            out = (r.stdout + r.stderr).strip()
            # hipcc's host pass warns that it does not know the packed-fp32 feature
            lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(lines))
            if verbose and lines:
                print("\n".join(lines), file=sys.stderr)
            return obj
        with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            objs = list(ex.map(compile_one, srcs))
        tmp_lib = LIB + ".tmp"
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp_lib, *objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
        os.replace(tmp_lib, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
