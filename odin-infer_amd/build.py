"""Build the native libraries in-tree.

  liboi_hip.so    the product: gfx950 kernels + the C ABI of include/oi.h
  liboi_synth.so  synthetic GGUF writer and quantizers (include/oi_synth.h)

Usage: python odin-infer_amd/build.py   (also called by __graft_entry__.build)
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(PKG, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed FP32 instructions are disabled for all device code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result", "-I", INCLUDE, "-I", CSRC]

LIB_HIP = os.path.join(PKG, "liboi_hip.so")
LIB_SYNTH = os.path.join(PKG, "liboi_synth.so")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s%s" % (" ".join(cmd), r.stdout, r.stderr))
    return r


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    objs = []
    for src in ["kernels.hip", "gemv.hip", "attn.hip", "gemm.hip", "prefill.hip", "deltanet.hip", "qwen35_attn.hip", "noalloc.hip", "sample.hip", "prefill_hybrid.hip"]:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        jobs.append([HIPCC, "--offload-arch=" + ARCH, *COMMON, *DEVICE_FLAGS, "-x", "hip", "-c",
                     os.path.join(CSRC, src), "-o", obj])
    for src in ["engine.cpp", "gguf.cpp", "oikv.cpp", "state.cpp"]:
        obj = os.path.join(BUILD, src + ".o")
        objs.append(obj)
        jobs.append([HIPCC, *COMMON, "-D__HIP_PLATFORM_AMD__", "-c", os.path.join(CSRC, src), "-o", obj])
    synth_cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-Wall", "-I", INCLUDE,
                 os.path.join(CSRC, "synth", "synth.cpp"), "-o", LIB_SYNTH + ".tmp", "-pthread"]
    with ThreadPoolExecutor(max_workers=4) as ex:
        futs = [ex.submit(_run, j) for j in jobs + [synth_cmd]]
        for f in futs:
            r = f.result()
            if verbose and (r.stdout or r.stderr):
                print(r.stdout + r.stderr)
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", LIB_HIP + ".tmp"])
    os.replace(LIB_HIP + ".tmp", LIB_HIP)
    os.replace(LIB_SYNTH + ".tmp", LIB_SYNTH)
    return LIB_HIP, LIB_SYNTH


if __name__ == "__main__":
    out = build(verbose="-v" in sys.argv)
    print("built:", *out)
