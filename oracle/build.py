"""Builds the C restatement of the oracle (test infrastructure) in-tree.

    python oracle/build.py

gcc, into oracle/_build/: libattention_ref.so (loaded with ctypes by
tests/test_oracle_c.py) and attention_ref.o (linked into the torch-free
driver, tests/driver/fa_driver). Nothing in the library uses either.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build")
SRC = os.path.join(HERE, "attention_ref.c")


def lib_path():
    return os.path.join(OUT, "libattention_ref.so")


def obj_path():
    return os.path.join(OUT, "attention_ref.o")


def build():
    os.makedirs(OUT, exist_ok=True)
    flags = ["-O2", "-std=c99", "-fPIC", "-Wall", "-Werror"]
    subprocess.run(["gcc", *flags, "-c", SRC, "-o", obj_path()], check=True)
    subprocess.run(["gcc", *flags, "-shared", SRC, "-lm", "-o", lib_path()], check=True)
    return lib_path(), obj_path()


if __name__ == "__main__":
    print("built", *build())
