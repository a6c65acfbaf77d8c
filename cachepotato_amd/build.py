"""Build libcachepotato_amd.so in-tree: HIP sources with hipcc for gfx950, C11 engine
sources with gcc, linked by hipcc. Run as `python -m cachepotato_amd.build`.

Every build compiles from scratch (the driver's build check relies on that)."""
import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcachepotato_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

INCLUDES = ["-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
# -packed-fp32-ops: no v_pk_*_f32 in generated code. -ffp-contract=off: a*b+c is never
# fused behind our back; the kernels write fmaf() where they want an FMA.
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function"] + INCLUDES
# per-file additions. prefill.hip: MFMA results in VGPRs, where the per-block scaling reads
# them (the default AGPR form costs a v_accvgpr_read per element, 16 per stage of the
# one-tile GEMM).
FILE_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
C_FLAGS = ["-O2", "-std=c11", "-fPIC", "-Wall", "-Wextra", "-ffp-contract=off"] + INCLUDES


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError("compile failed: " + os.path.basename(cmd[-1]))
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if msg.strip():
        sys.stderr.write(msg + "\n")


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    hip_srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    c_srcs = sorted(glob.glob(os.path.join(CSRC, "engine", "*.c")))
    jobs = []
    for s in hip_srcs:
        o = os.path.join(BUILD, os.path.basename(s) + ".o")
        jobs.append([HIPCC] + HIP_FLAGS + FILE_FLAGS.get(os.path.basename(s), [])
                    + ["-c", "-o", o, s])
    for s in c_srcs:
        o = os.path.join(BUILD, os.path.basename(s) + ".o")
        jobs.append(["gcc"] + C_FLAGS + ["-c", "-o", o, s])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs) or 1)) as ex:
        list(ex.map(_run, jobs))
    objs = [j[j.index("-o") + 1] for j in jobs]
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-Wl,-Bsymbolic", "-o", tmp]
         + objs)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build()
