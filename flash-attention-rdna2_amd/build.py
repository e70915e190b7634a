"""Build libfable_attn_hip.so (the C-ABI library) for gfx950 in-tree.

    python flash-attention-rdna2_amd/build.py [-j N]

Every .hip file under csrc/ is compiled separately (in parallel) with hipcc for gfx950 only and
linked into fable_attn/libfable_attn_hip.so. Objects go to _build/ (git-ignored).
Flags: -O3, C++17, packed-fp32 VALU ops disabled (a hard rule for this hardware pool), no
fast-math (masking relies on IEEE infinities). The backward kernels keep MFMA accumulators in
architectural VGPRs (-amdgpu-mfma-vgpr-form): the compiler's default there parks the dK/dV
accumulators in AGPRs and copies them back and forth around every MFMA group.
"""
import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "fable_attn", "libfable_attn_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + os.path.join(HERE, "..", "include")]


# per-source extra flags
def _extra(name):
    # the fp16/bf16 backward kernels (bwd_dNN.hip) keep MFMA accumulators in VGPR form
    if name.startswith("bwd_d") and name.endswith(".hip"):
        return ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
    return []


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC] + FLAGS + _extra(os.path.basename(src)) + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs=None, verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    build(a.j)
