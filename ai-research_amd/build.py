"""Builds the MI355X backend in-tree.

  gh_<family>.hsaco   gfx950 code objects (hipcc --genco), loaded at run time
                      with hipModuleLoad
  libgemma_hip.so     the C-ABI host library (g++ against libamdhip64)

Run:  python ai-research_amd/build.py        (or __graft_entry__.build())
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# Every device code object is built with packed-FP32 instructions disabled:
# hipcc -O3 otherwise forms v_pk_{add,mul,fma}_f32 from plain float code.
DEVICE_FLAGS = ["--offload-arch=gfx950", "--genco", "--no-gpu-bundle-output", "-O3", "-std=c++17",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-I", CSRC, "-I", os.path.join(ROOT, "include")]

KERNEL_FAMILIES = ["gemv", "gemv_norm", "util", "attn", "norm", "prefill"]

# Per-family extra flags.  The prefill GEMMs scale each 32-block's MFMA sum on
# the VALU; in VGPR form the MFMA results need no v_accvgpr_read first.
FAMILY_FLAGS = {"prefill": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

HOST_SOURCES = ["runtime.cpp", "engine.cpp", "model.cpp", "ring.cpp"]
HIP_HOST_SOURCES = ["noalloc.hip"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-pthread", "-ffp-contract=off",
              "-Wall", "-Wno-unused-result", "-D__HIP_PLATFORM_AMD__",
              "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"),
              "-I", CSRC]
HOST_LIBS = ["-L" + os.path.join(ROCM, "lib"), "-Wl,-rpath," + os.path.join(ROCM, "lib"),
             "-lamdhip64", "-ldl"]

LIB_PATH = os.path.join(PKG, "libgemma_hip.so")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError("build step failed: " + " ".join(cmd))
    return r.stdout


def build_kernels():
    jobs = []
    for fam in KERNEL_FAMILIES:
        src = os.path.join(CSRC, "kernels", fam + ".hip")
        if not os.path.exists(src):
            continue
        out = os.path.join(PKG, "gh_%s.hsaco" % fam)
        jobs.append([HIPCC] + DEVICE_FLAGS + FAMILY_FLAGS.get(fam, []) + [src, "-o", out])
    with ThreadPoolExecutor(max_workers=min(8, max(1, len(jobs)))) as ex:
        list(ex.map(_run, jobs))


def build_host():
    srcs = [os.path.join(CSRC, "runtime", s) for s in HOST_SOURCES
            if os.path.exists(os.path.join(CSRC, "runtime", s))]
    # Host sources with device variables of their own (the allocation-free
    # entry point's scratch array) go through hipcc, which embeds their gfx950
    # code object in the library.
    objs = []
    bdir = os.path.join(PKG, "_build")
    os.makedirs(bdir, exist_ok=True)
    for src in HIP_HOST_SOURCES:
        obj = os.path.join(bdir, os.path.splitext(src)[0] + ".o")
        _run([HIPCC, "-c", "-fPIC", "-O2", "-std=c++17", "--offload-arch=gfx950",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-I", os.path.join(ROOT, "include"), "-I", CSRC,
              os.path.join(CSRC, "runtime", src), "-o", obj])
        objs.append(obj)
    tmp = LIB_PATH + ".tmp"
    _run(["g++"] + HOST_FLAGS + srcs + objs + ["-o", tmp] + HOST_LIBS)
    os.replace(tmp, LIB_PATH)


def build():
    build_kernels()
    build_host()


if __name__ == "__main__":
    build()
    print("built", LIB_PATH)
