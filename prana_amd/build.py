"""Build libprana_hip.so (gfx950) in-tree: prana_amd/_build/libprana_hip.so,
plus the host-only fixture-encoder library libprana_synth.so.

Every HIP/C++ source under prana_amd/csrc is compiled with hipcc for gfx950
only, without FMA contraction (the kernels reproduce the reference's f32
evaluation order) and with packed-FP32 instruction selection disabled, then
linked into one shared library exposing the C ABI of include/prana_hip.h.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(OUT, "libprana_hip.so")

ARCH = "gfx950"
COMMON = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]
# Matrix-core results in ordinary VGPRs: the batched GEMMs read every result
# lane in their f32 epilogue, and with accumulation registers each of those
# reads costs a v_accvgpr_read (16 of ~93 VALU instructions per block).
PER_SOURCE = {"gemv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src):
    obj = os.path.join(OUT, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [hipcc()] + COMMON + PER_SOURCE.get(os.path.basename(src), []) + lang + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(OUT, exist_ok=True)
    srcs = sorted(os.path.join(SRC, f) for f in os.listdir(SRC) if f.endswith((".hip", ".cpp")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_synth()
    if verbose:
        print(f"built {LIB} and {SYNTH_LIB}")
    return LIB


SYNTH_SRC = os.path.join(HERE, "synth", "synth.cpp")
SYNTH_LIB = os.path.join(OUT, "libprana_synth.so")


def build_synth():
    """libprana_synth.so: the fixture encoders (host C++ only, no GPU code)."""
    os.makedirs(OUT, exist_ok=True)
    tmp = SYNTH_LIB + ".tmp"
    cmd = ["g++", "-O2", "-fPIC", "-std=c++17", "-shared", "-Wall", "-o", tmp, SYNTH_SRC, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
