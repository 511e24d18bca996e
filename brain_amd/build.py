"""Build libbrain_hip.so (gfx950) in-tree with hipcc.

Each HIP source is compiled to an object in parallel, then linked into
brain_amd/libbrain_hip.so. Flags:
  --offload-arch=gfx950                 MI355X only
  -ffp-contract=off                     (f32(acc)*sx)*sw [+bias] stays unfused
  -fhip-fp32-correctly-rounded-divide-sqrt   1/sx is the IEEE quotient
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-FP32 VALU ops
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libbrain_hip.so")
SOURCES = ["bh_api.hip", "bh_quant.hip", "bh_gemv.hip", "bh_gemm.hip", "bh_qwen3.hip", "bh_q4.hip", "bh_kv8.hip",
           "bh_st.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-inline-asm",
]


# Sources whose code decides the GEMV/tile crossover: the tune store keys its
# tables by a fingerprint of these and of FLAGS (bh_tune_save / bh_tune_load).
FP_SOURCES = ["bh_gemv.hip", "bh_gemm.hip", "bh_common.h"]


def kernel_fingerprint():
    """FNV-1a 64 over the tuned kernels' sources and the compile flags."""
    h = 0xcbf29ce484222325
    data = b"".join(open(os.path.join(CSRC, f), "rb").read() for f in FP_SOURCES) + " ".join(FLAGS).encode()
    for byte in data:
        h = ((h ^ byte) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def _compile(src, fp):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, f"-DBH_KERNEL_FP=0x{fp:016x}ULL", "-c", os.path.join(CSRC, src), "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise.
    err = "\n".join(l for l in p.stderr.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        fp = kernel_fingerprint()
        objs = list(ex.map(lambda src: _compile(src, fp), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
