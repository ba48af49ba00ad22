"""Build the native library in-tree: phonemap_amd/libslipstream_hip.so.

HIP sources are compiled for gfx950 only; host C sources with gcc. Run as
``python -m phonemap_amd.build`` or through ``__graft_entry__.build()``.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libslipstream_hip.so")

HIP_SOURCES = ["ss_gemv.hip", "ss_kernels.hip", "ss_gemm.hip", "ss_flash.hip", "ss_sweep.hip", "ss_sample.hip", "ss_hip.hip"]
C_SOURCES = ["ss_gguf.c", "ss_tokenizer.c", "ss_engine.c", "ss_synth.c"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed fp32 VALU ops are disabled for all device code.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
             "-Wno-unused-value", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
C_FLAGS = ["-O2", "-std=gnu11", "-fPIC", "-Wall", "-Wno-unused-result", "-pthread",
           "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    jobs = []
    for s in HIP_SOURCES:
        jobs.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, s), "-o",
                                           os.path.join(OBJ, s + ".o")])
    for s in C_SOURCES:
        if os.path.exists(os.path.join(CSRC, s)):
            jobs.append(["gcc"] + C_FLAGS + ["-c", os.path.join(CSRC, s), "-o",
                                             os.path.join(OBJ, s + ".o")])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        outs = list(ex.map(_run, jobs))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    objs = [j[-1] for j in jobs]
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread", "-lm"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
