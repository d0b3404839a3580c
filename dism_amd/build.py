"""Build libdism_hip.so (gfx950) in-tree with hipcc.

Every translation unit is compiled with:
  * -ffp-contract=off, correctly rounded fp32 division/sqrt, fp32 denormals kept: the kernels'
    floating point is a fixed sequence of IEEE operations (explicit fmaf where fused);
  * -Xclang -target-feature -Xclang -packed-fp32-ops: no packed-fp32 VALU instructions.
Objects go to dism_amd/_build/, the shared library to dism_amd/libdism_hip.so.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libdism_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("DISM_OFFLOAD_ARCH", "gfx950")

SOURCES = ["dism_aux.hip", "dism_sort.hip", "dism_msort.hip", "dism_pairs.hip", "dism_scan.hip",
           "dism_packed.hip", "dism_dense.hip", "dism_levels.hip", "dism_prefix.hip", "dism_prefix_rows.hip", "dism_prefix_keys.hip", "dism_decode.hip", "dism_vocab.hip", "dism_capi.cpp"]

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


def _compile(src):
    path = os.path.join(CSRC, src)
    obj = os.path.join(OUT_DIR, src + ".o")
    cmd = [HIPCC, *FLAGS, "-c", path, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose=True):
    """Compile all sources (always) and link libdism_hip.so."""
    os.makedirs(OUT_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    subprocess.check_call([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
