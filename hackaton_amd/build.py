"""Builds libvarlen_attn.so in-tree with hipcc for gfx950 (no JIT cache, no torch extension).

Usage: python -m hackaton_amd.build   (or hackaton_amd.build.build())
"""

import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libvarlen_attn.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

SOURCES = ["attn_fwd.hip", "attn_bwd.hip", "rope.hip", "plan_device.hip", "noalloc.hip", "probe.hip",
           "api.cpp", "plan.cpp"]
ARCH = os.environ.get("VA_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops off: no packed fp32 VALU instructions are generated.
# -amdgpu-mfma-vgpr-form: MFMA accumulators in VGPRs, so the softmax rescale of O and the
#   reads of S need no accumulation-register moves.
# -amdgpu-kernarg-preload-count: the first kernel arguments arrive in SGPRs at launch instead of
#   through a scalar load, one memory round trip less before a work-group's first loads.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=16",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall",
             "-Wno-unused-function"]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build " + LIB_NAME)
    return path


def build(verbose=False, jobs=None):
    """Compile every source to an object, link the shared library, replace it atomically."""
    cc = hipcc()
    tmp = tempfile.mkdtemp(prefix="va_build_")
    try:
        objs, procs = [], []
        for src in SOURCES:
            obj = os.path.join(tmp, src + ".o")
            lang = ["-x", "hip"] if src.endswith(".hip") else []
            cmd = [cc, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
        failed = []
        for src, p in procs:
            out, _ = p.communicate()
            if p.returncode != 0:
                failed.append((src, out))
            elif verbose and out.strip():
                print(out, flush=True)
        if failed:
            msg = "\n".join(f"--- {s}\n{o}" for s, o in failed)
            raise RuntimeError("hipcc failed:\n" + msg)
        out_tmp = os.path.join(tmp, LIB_NAME)
        cmd = [cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", out_tmp]
        res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if res.returncode != 0:
            raise RuntimeError("link failed:\n" + res.stdout)
        shutil.copy2(out_tmp, LIB_PATH + ".tmp")
        os.replace(LIB_PATH + ".tmp", LIB_PATH)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
