"""Builds the torch-free driver (test infrastructure) in-tree.

    python tests/driver/build.py

hipcc: tests/driver/fa_driver from fa_driver.cpp, linked to the library
(flash-attention-p100_amd/libfa_mi355x.so, found through an rpath relative to
the binary) and to the C oracle object (oracle/build.py builds it first).
"""
import importlib.util
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
PKG = os.path.join(ROOT, "flash-attention-p100_amd")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def exe_path():
    return os.path.join(HERE, "fa_driver")


def build():
    spec = importlib.util.spec_from_file_location("fa_oracle_build",
                                                  os.path.join(ROOT, "oracle", "build.py"))
    oracle_build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(oracle_build)
    _, obj = oracle_build.build()
    cmd = [os.path.join(ROCM, "bin", "hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17",
           # Packed fp32 VALU ops are kept out of generated code.
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           os.path.join(HERE, "fa_driver.cpp"), "-x", "none", obj, "-L" + PKG, "-lfa_mi355x",
           "-Wl,-rpath,$ORIGIN/../../flash-attention-p100_amd", "-o", exe_path()]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"driver build failed:\n{out}")
    return exe_path()


if __name__ == "__main__":
    print("built", build())
