"""Build libmx_encoder.so for gfx950 with hipcc, in-tree.

    python npu-embeddings-xdna1_amd/build.py [--jobs N]

Every library source under csrc/ is compiled with hipcc for gfx950 only and
linked into _build/libmx_encoder.so beside this file. Packed-fp32 instructions are
disabled for all device code (-packed-fp32-ops); hipcc's host pass warns that
it does not know that feature, which is harmless.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(OUT, "libmx_encoder.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the softmax and epilogue VALU read them directly,
    # without accvgpr copies.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", os.path.join(HERE, "..", "include"),
]
SOURCES = ["k_gemm_lds.hip", "k_gemm_i8.hip", "k_elem.hip", "k_gemm.hip", "k_attn.hip",
           "k_front.hip", "k_panel.hip", "k_quant.hip", "k_glu.hip", "mx_abi.cpp", "mx_i8.cpp",
           "mx_encoder.cpp", "mx_npue.cpp", "mx_service.cpp", "mx_host.cpp", "mx_static.hip"]


def _compile(src):
    obj = os.path.join(OUT, src + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    cmd = [HIPCC] + FLAGS + lang + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def build(jobs=None, verbose=False):
    os.makedirs(OUT, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, SOURCES))
    objs = []
    for obj, warn in results:
        objs.append(obj)
        if warn.strip() and verbose:
            print(warn)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    build_abi_check()
    return LIB


ABI_CHECK = os.path.join(OUT, "abi_check")


def build_abi_check():
    """tests/abi_cxx/abi_check.cpp: a C++17 caller of include/mx_gpu_backend.hpp,
    compiled by the host compiler (no HIP) and linked to the library, as the
    reference runtime would build against it."""
    src = os.path.join(HERE, "..", "tests", "abi_cxx", "abi_check.cpp")
    cmd = [os.environ.get("CXX", "g++"), "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror",
           "-I", os.path.join(HERE, "..", "include"), src, "-o", ABI_CHECK + ".tmp", "-L", OUT,
           "-lmx_encoder", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("g++ failed on abi_check.cpp:\n" + r.stdout + r.stderr)
    os.replace(ABI_CHECK + ".tmp", ABI_CHECK)
    return ABI_CHECK


if __name__ == "__main__":
    jobs = None
    if "--jobs" in sys.argv:
        jobs = int(sys.argv[sys.argv.index("--jobs") + 1])
    print(build(jobs, verbose=True))
