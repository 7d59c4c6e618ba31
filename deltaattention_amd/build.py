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
# bench.py's on-box ceilings (an MFMA issue loop); not part of the product ABI
DIAG_SRC = os.path.join(HERE, "diag", "peaks.hip")
DIAG_LIB = os.path.join(HERE, "libdeltaattn_diag.so")
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


# Every kernel must run from registers alone: no scratch memory, no VGPR spill, no dynamic
# stack.  The attention kernels issue LDS reads as inline asm whose destination registers
# are written when the data arrives, after the compiler takes them as written; a spill or
# copy of such a register in between would store stale data.  SGPR spills into VGPR lanes
# are register moves and are allowed.  The compiler's per-kernel resource report
# (-Rpass-analysis=kernel-resource-usage) is parsed, printed and checked.
RESOURCE_FLAGS = ["-Rpass-analysis=kernel-resource-usage"]
_RES_KEYS = {
    "Function Name": "name",
    "VGPRs": "vgpr",
    "AGPRs": "agpr",
    "TotalSGPRs": "sgpr",
    "ScratchSize [bytes/lane]": "scratch",
    "Dynamic Stack": "dynamic_stack",
    "VGPRs Spill": "vgpr_spill",
    "SGPRs Spill": "sgpr_spill",
    "LDS Size [bytes/block]": "lds",
}


class ResourceError(RuntimeError):
    """A kernel needs scratch memory, spills VGPRs or uses a dynamic stack."""


def parse_resource_usage(text: str) -> list[dict]:
    """Per-kernel records from the compiler's kernel-resource-usage remarks."""
    kernels, cur = [], None
    for line in text.splitlines():
        if "remark:" not in line or "kernel-resource-usage" not in line:
            continue
        body = line.split("remark:", 1)[1].rsplit("[-Rpass-analysis", 1)[0].strip()
        if ":" not in body:
            continue
        key, val = (x.strip() for x in body.rsplit(":", 1))
        field = _RES_KEYS.get(key)
        if field is None:
            continue
        if field == "name":
            cur = {"name": val}
            kernels.append(cur)
        elif cur is not None:
            cur[field] = val if field == "dynamic_stack" else int(val)
    return kernels


def check_resources(kernels: list[dict], src: str) -> None:
    """Raise ResourceError if any kernel of ``src`` uses scratch, spills VGPRs or has a
    dynamic stack."""
    bad = [k for k in kernels
           if k.get("scratch", 0) or k.get("vgpr_spill", 0) or k.get("dynamic_stack") == "True"]
    if bad:
        lines = [f"  {k['name']}: scratch {k.get('scratch')} B/lane, VGPR spill {k.get('vgpr_spill')}, "
                 f"dynamic stack {k.get('dynamic_stack')}" for k in bad]
        raise ResourceError(f"{os.path.basename(src)}: kernels that do not run from registers alone:\n"
                            + "\n".join(lines))


def resource_line(k: dict) -> str:
    return (f"{k['name'][:60]:60s} VGPR {k.get('vgpr', 0):3d} AGPR {k.get('agpr', 0):3d} "
            f"SGPR {k.get('sgpr', 0):3d} (spilled {k.get('sgpr_spill', 0):3d}) scratch {k.get('scratch', 0)} "
            f"LDS {k.get('lds', 0)}")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libdeltaattn.so")
    return exe


def compile_checked(src: str, obj: str, verbose: bool = False) -> list[dict]:
    """hipcc -c one source with the library's flags; returns its kernels' resource
    records, or raises RuntimeError (compile error) / ResourceError (a kernel that does
    not run from registers alone)."""
    cmd = [_hipcc(), *HIPCC_FLAGS, *RESOURCE_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = (r.stdout + r.stderr).strip()
    kernels = parse_resource_usage(out)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    lines = [ln for ln in out.splitlines()
             if "packed-fp32-ops" not in ln and "kernel-resource-usage" not in ln
             and not ln.lstrip().startswith(("|", "^")) and not ln.strip()[:1].isdigit()]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(lines))
    with open(src) as f:
        has_kernels = "__global__" in f.read()
    if has_kernels and not kernels:
        raise ResourceError(f"{os.path.basename(src)}: no kernel resource report from hipcc")
    check_resources(kernels, src)
    if verbose and lines:
        print("\n".join(lines), file=sys.stderr)
    return kernels


def _link(objs: list[str], lib: str) -> None:
    tmp_lib = lib + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp_lib, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp_lib, lib)


def build_diag(verbose: bool = False) -> str:
    """Compile libdeltaattn_diag.so (the MFMA issue loop bench.py measures the on-box
    bf16 ceiling with), under the same register-only check; returns its path."""
    with tempfile.TemporaryDirectory(prefix="deltaattn_diag_") as tmp:
        obj = os.path.join(tmp, "peaks.o")
        ks = compile_checked(DIAG_SRC, obj, verbose=verbose)
        if verbose:
            for k in ks:
                print(resource_line(k), file=sys.stderr)
        _link([obj], DIAG_LIB)
    return DIAG_LIB


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link libdeltaattn.so (and the diagnostics library);
    returns the product library's path.  Raises
    ResourceError (and links nothing) if any kernel uses scratch memory, spills VGPRs or
    has a dynamic stack; prints one resource line per kernel when ``verbose``."""
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="deltaattn_build_") as tmp:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            return obj, compile_checked(src, obj, verbose=verbose)
        with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            results = list(ex.map(compile_one, srcs))
        objs = [o for o, _ in results]
        if verbose:
            for _, ks in results:
                for k in ks:
                    print(resource_line(k), file=sys.stderr)
        _link(objs, LIB)
    build_diag(verbose=verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
