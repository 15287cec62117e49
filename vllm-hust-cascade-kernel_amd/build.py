"""Build the gfx950 kernel library and the torch-op library in-tree.

Outputs (git-ignored, shipped with the tree):
  cascade_amd/_lib/libcascade_hip.so    HIP kernels + the C ABI of include/cascade_kernels.h
  cascade_amd/_lib/libcascade_torch.so  torch.ops.npu.* registration, links the one above

Usage: python build.py [--jobs N]   (also called by __graft_entry__.build()).
No CMake / ninja: one hipcc invocation per kernel source (in parallel), one
link, one g++ invocation for the torch layer.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIBDIR = os.path.join(HERE, "cascade_amd", "_lib")
OBJDIR = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

KERNEL_SOURCES = ["abi.hip", "lse_merge.hip", "fa_stage1.hip", "suffix_decode.hip", "cascade.hip",
                  "gateup_swiglu.hip", "add_rms_norm.hip", "probe.hip"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fno-gpu-rdc",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-inline-asm",
    # Packed FP32 ops (v_pk_*_f32) are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def run(cmd, cwd=None):
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # the host pass warns that it does not know the packed-fp32 feature: drop that noise
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


# Per-source code-generation options. The stage-1 kernels keep their score and
# output accumulators in architectural VGPRs (MFMA results written there, not
# to AGPRs): the softmax reads and rescales them with VALU instructions every
# 128 tokens, and AGPR-resident accumulators cost a copy in and out each time.
# suffix_decode.hip holds the fused cascade kernel, whose stage-1 waves run the
# same body. Its cascade epilogue takes the arguments of its first loads as
# leading scalar parameters, which kernarg preloading puts in SGPRs at wave
# launch (kernels whose first parameter is a struct are left as they are).
SOURCE_FLAGS = {"fa_stage1.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
                "suffix_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def compile_hip(src):
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    run([HIPCC] + HIP_FLAGS + SOURCE_FLAGS.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_kernels(jobs):
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_hip, KERNEL_SOURCES))
    out = os.path.join(LIBDIR, "libcascade_hip.so")
    tmp = out + ".tmp"
    run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, out)
    return out


def build_torch_ops():
    import torch
    from torch.utils import cpp_extension
    tdir = os.path.dirname(torch.__file__)
    tlib = os.path.join(tdir, "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in cpp_extension.include_paths()] + [f"-I{ROCM}/include", f"-I{INCLUDE}"]
    out = os.path.join(LIBDIR, "libcascade_torch.so")
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=cascade_torch",
           "-Wno-deprecated-declarations"] + incs + [
        os.path.join(CSRC, "torch_ops.cpp"), "-o", tmp,
        f"-L{LIBDIR}", "-lcascade_hip", f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}"]
    run(cmd)
    os.replace(tmp, out)
    return out


def build(jobs=None):
    if not os.path.exists(HIPCC) and not shutil.which("hipcc"):
        raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")
    jobs = jobs or min(8, os.cpu_count() or 4)
    k = build_kernels(jobs)
    t = build_torch_ops()
    return k, t


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    for p in build(args.jobs):
        print("built", p)
    sys.exit(0)
