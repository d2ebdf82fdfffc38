"""Build libvkv.so (gfx950 HIP kernels + C++ host layer) in-tree.

Usage: python voxtral.cpp_amd/build.py            # builds vkv/libvkv.so
The library is what include/vkv.h declares; it links nothing but the HIP runtime.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "vkv", "libvkv.so")
SOURCES = ["vkv_kernels.hip", "vkv_matvec.hip", "vkv_conv.hip", "vkv_static.hip", "vkv_host.cpp",
           "vkv_gguf.cpp"]
ARCH = os.environ.get("VKV_OFFLOAD_ARCH", "gfx950")


def hipcc_command(out=OUT):
    return [
        "hipcc", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-Wall", "-Wno-unused-function",
        # never let the compiler emit packed fp32 arithmetic
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA accumulators in ordinary VGPRs: the decode kernels rescale and
        # read them with VALU every batch, which the AGPR form turns into
        # accvgpr copies
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-I", os.path.join(ROOT, "include"), "-I", CSRC,
        *[os.path.join(CSRC, s) for s in SOURCES],
        "-o", out,
    ]


def build(verbose=False):
    tmp = OUT + ".tmp"
    cmd = hipcc_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l]
    if res.returncode != 0:
        sys.stderr.write("\n".join(errs) + "\n")
        raise RuntimeError(f"hipcc failed with status {res.returncode}")
    if verbose and errs:
        sys.stderr.write("\n".join(errs) + "\n")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
