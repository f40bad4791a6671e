"""Builds a copy of the library whose host code (planner, argument checks, launch set-up) carries
AddressSanitizer and UndefinedBehaviorSanitizer, for the CPU test suite; the GPU code is the
ordinary build's (device code is never sanitized here).

Usage:
    python -m hackaton_amd.build_hostsan
    ASAN_OPTIONS=detect_leaks=0 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \\
    LD_PRELOAD=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so) \\
    VA_LIB_PATH=hackaton_amd/libvarlen_attn_hostsan.so python -m pytest tests -m "not gpu"

The sanitizer runtime is preloaded because the Python interpreter itself is not instrumented;
leak detection is off because the interpreter keeps its allocations until exit.
"""

import os
import shutil
import subprocess
import sys
import tempfile

from hackaton_amd import build as B

SAN_LIB = os.path.join(B.HERE, "libvarlen_attn_hostsan.so")
# host-side only (every sanitizer flag behind -Xarch_host); frame pointers for the reports
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]


def build_hostsan():
    cc = B.hipcc()
    tmp = tempfile.mkdtemp(prefix="va_hostsan_")
    try:
        objs, procs = [], []
        for src in B.SOURCES:
            obj = os.path.join(tmp, src + ".o")
            lang = ["-x", "hip"] if src.endswith(".hip") else []
            cmd = [cc, *B.HIP_FLAGS, *HOST_SAN, *lang, "-c", os.path.join(B.CSRC, src), "-o", obj]
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
        failed = [(s, p.communicate()[0]) for s, p in procs]
        failed = [(s, o) for (s, o), (_, p) in zip(failed, procs) if p.returncode != 0]
        if failed:
            raise RuntimeError("hipcc failed:\n" + "\n".join(f"--- {s}\n{o}" for s, o in failed))
        out_tmp = os.path.join(tmp, os.path.basename(SAN_LIB))
        cmd = [cc, "-shared", "-fPIC", f"--offload-arch={B.ARCH}", *HOST_SAN, "-shared-libsan",
               *objs, "-o", out_tmp]
        res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if res.returncode != 0:
            raise RuntimeError("link failed:\n" + res.stdout)
        shutil.copy2(out_tmp, SAN_LIB)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return SAN_LIB


if __name__ == "__main__":
    print(build_hostsan(), file=sys.stdout)
