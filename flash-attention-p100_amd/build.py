"""Builds the gfx950 kernels and the torch binding in-tree.

    python flash-attention-p100_amd/build.py

Outputs, next to this file:
  libfa_mi355x.so            hipcc, --offload-arch=gfx950: kernels + C ABI
  fa_p100_ext<EXT_SUFFIX>    g++: torch binding over the C ABI (rpath $ORIGIN)

The binding is compiled as plain C++ (no hipify pass, no device code): it
includes torch's HIP stream header only to pick up the current stream.
"""
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

LIB_NAME = "libfa_mi355x.so"
EXT_NAME = "fa_p100_ext"
KERNEL_SOURCES = ["fa_fwd.hip", "fa_bwd.hip", "fa_mask.hip", "fa_capi.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # Packed fp32 VALU ops are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + INCLUDE, "-Wno-unused-result",
]
# Per-file additions (same-box A/B timings, bit-identical output each). The
# forward's kernels schedule for instruction-level parallelism: 2-4% faster
# at D = 64 and D = 96 and on non-causal shapes, neutral at B=1 H=8 N=4096
# D=128 causal and at H=16/8 N=8192 (the backward lost 3-11% with it). The
# backward's scheduler uses the register-pressure trackers: 2.3% faster at
# B=2 H=32/8 N=3001 D=128 dense, neutral at the causal shapes (the forward
# gains nothing from them).
FILE_FLAGS = {
    "fa_fwd.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "fa_bwd.hip": ["-mllvm", "-amdgpu-use-amdgpu-trackers=1"],
}


def lib_path():
    return os.path.join(HERE, LIB_NAME)


def ext_path():
    return os.path.join(HERE, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_kernels(jobs=8):
    os.makedirs(OBJ, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objs = []
    cmds = []
    for src in KERNEL_SOURCES:
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), "-c",
                     os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(jobs, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    tmp = lib_path() + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, lib_path())
    return lib_path()


def build_ext():
    import torch
    from torch.utils import cpp_extension

    py_inc = sysconfig.get_paths()["include"]
    incs = cpp_extension.include_paths() + [py_inc, INCLUDE, os.path.join(ROCM, "include")]
    libdirs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           os.path.join(CSRC, "fa_p100_ext.cpp")]
    cmd += ["-I" + i for i in incs]
    cmd += ["-L" + d for d in libdirs] + ["-Wl,-rpath," + d for d in libdirs]
    cmd += ["-L" + HERE, "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN",
            "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip",
            "-L" + os.path.join(ROCM, "lib"), "-lamdhip64"]
    tmp = ext_path() + ".tmp"
    _run(cmd + ["-o", tmp])
    os.replace(tmp, ext_path())
    return ext_path()


def build(jobs=8):
    build_kernels(jobs)
    build_ext()


if __name__ == "__main__":
    build()
    print("built", lib_path(), ext_path())
    sys.exit(0)
