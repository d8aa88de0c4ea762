"""Build libmi355x_decode.so in-tree: every csrc/*.hip and *.cpp with hipcc for gfx950,
compiled in parallel, linked into one shared library next to this file."""
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmi355x_decode.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: fused multiply-adds only where the source spells them (the reference's
# rounding discipline). packed-fp32-ops off: no v_pk_*_f32 in the generated code.
COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall",
          "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
HIP_ONLY = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-munsafe-fp-atomics"]


# Per-file code generation options. attn.hip: the attention accumulators live in ordinary
# VGPRs (they are rescaled by the vector ALUs between matrix-core products, which AGPRs would
# turn into copies back and forth). gemv_w4a16.hip: each product's result is scaled into the
# fp32 accumulators by the vector ALUs at once, so it too is kept out of AGPRs (no copies out of
# them: 27B step 4.23 -> 4.13 ms, verify steps at 2..8 rows 0.5-2 % faster).
PER_FILE = {"attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
            "gemv_w4a16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
            # the prefill GEMM and attention: 27B prefill 20.4 -> 21.1 k tokens/s, MoE 69.7 -> 72.0 k
            "prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON]
    if src.endswith(".hip"):
        cmd += ["-x", "hip", *HIP_ONLY, *PER_FILE.get(os.path.basename(src), [])]
    cmd += ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stderr or "").splitlines()
                     if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{errs}")
    return obj


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, srcs))
    cmd = [HIPCC, "-shared", "--offload-arch=gfx950", "-fPIC", *objs, "-o", LIB]
    subprocess.check_call(cmd)
    if verbose:
        print("built", LIB, flush=True)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
