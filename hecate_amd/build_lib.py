"""Builds libhecate_moe.so (the C ABI of include/hecate_moe.h) in-tree for gfx950 with hipcc.

python -m hecate_amd.build_lib    (or __graft_entry__.build())
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libhecate_moe.so")
SOURCES = ["common.hip", "decode.hip", "router.hip", "norm.hip", "prefill.hip", "cputier_gpu.hip", "shared_gemm.hip"]
HOST_SOURCES = ["cputier.cpp"]                 # host-only C++ (the CPU expert tier), built with the host compiler
CXX = os.environ.get("CXX_HOST", "g++")
# AVX2 / FMA / F16C is the x86-64-v3 level (every AVX2 EPYC and Xeon); no fp contraction, so the q8_0 arithmetic
# rounds exactly as written
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-mavx2", "-mfma", "-mf16c", "-ffp-contract=off", "-pthread", "-Wall",
              f"-I{os.path.join(ROOT, 'include')}"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("HMOE_ARCH", "gfx950")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-Wall", "-Wno-unused-function",
    # no packed-fp32 VALU instructions anywhere in the library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]


# per-source additions: the dense GEMM keeps its MFMA accumulators in VGPRs (with AGPR accumulators the compiler
# copies accumulator tiles between register files at every loop trip); the decode kernels are scheduled for memory
# clauses (the streaming launches' loads kept together: 0.1-0.5 % per decode step at 1-16 rows, same bits)
SOURCE_FLAGS = {"shared_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
                "decode.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]}


def _compile(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + FLAGS + SOURCE_FLAGS.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def _compile_host(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [CXX] + HOST_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{CXX} failed on {src}:\n{r.stdout}{r.stderr}")
    return obj, r.stdout + r.stderr


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, len(SOURCES) + len(HOST_SOURCES))) as ex:
        jobs = [ex.submit(_compile, s) for s in SOURCES] + [ex.submit(_compile_host, s) for s in HOST_SOURCES]
        results = [j.result() for j in jobs]
    for _, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + [o for o, _ in results] + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
