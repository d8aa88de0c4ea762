"""Build recipe for the CPU oracle (test infrastructure).

* ``oracle/liboracle.so`` - this repository's C++ restatement (oracle.cpp), built with
  ``-O2 -ffp-contract=off`` as the reference builds its CPU twins (CMakeLists.txt:31-34).
* ``oracle/_ref/libref.so`` - the reference's own scalar twins, compiled from their
  sources where they lie under ``/root/reference`` through ``ref_shim.cpp``. Only built
  when that tree is present; nothing is copied out of it.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"

CXXFLAGS = ["-O2", "-ffp-contract=off", "-fPIC", "-shared", "-fopenmp", "-Wall", "-Wextra"]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.check_call(cmd)


def build_oracle():
    out = os.path.join(HERE, "liboracle.so")
    _run(["g++", "-std=c++17", *CXXFLAGS, os.path.join(HERE, "oracle.cpp"), "-o", out])
    return out


def build_ref():
    """Compile the reference's header-only twins; returns the path or None when absent."""
    if not os.path.isdir(os.path.join(REF, "tests", "kernels")):
        return None
    outdir = os.path.join(HERE, "_ref")
    os.makedirs(outdir, exist_ok=True)
    out = os.path.join(outdir, "libref.so")
    _run(["g++", "-std=c++20", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-w",
          "-I" + os.path.join(REF, "src"), "-I" + os.path.join(REF, "tests"),
          os.path.join(HERE, "ref_shim.cpp"), os.path.join(REF, "src", "loader", "lm_head_int8.cc"),
          "-pthread", "-o", out])
    return out


def build_all():
    build_oracle()
    build_ref()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
