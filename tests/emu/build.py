"""Build the CPU emulation of libdism_hip.so (test infrastructure): every HIP unit of
dism_amd/csrc, compiled as host C++ against
tests/emu/hip/hip_runtime.h with g++ -O0, frame pointers, AddressSanitizer and basic-block
hooks (the lockstep scheduler), linked into libdism_emu.so."""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CLANG = "/opt/rocm/llvm/bin/clang++"
UNITS = ["dism_aux", "dism_sort", "dism_msort", "dism_pairs", "dism_scan", "dism_packed",
         "dism_dense", "dism_levels", "dism_prefix", "dism_prefix_rows", "dism_prefix_keys",
         "dism_decode"]


def build(out_dir, csrc=os.path.join(ROOT, "dism_amd", "csrc")):
    os.makedirs(out_dir, exist_ok=True)
    # -O0: basic blocks stay in source order, which the lowest-code-position scheduling
    # relies on (with -O1 block layout and if-conversion the lockstep order breaks)
    flags = ["-std=c++17", "-O0", "-g", "-fno-omit-frame-pointer", "-fPIC", "-ffp-contract=off",
             "-fno-fast-math", "-fsanitize=address", "-I" + HERE, "-I" + csrc]
    jobs = [(os.path.join(csrc, u + ".hip"),
             ["-x", "c++", "-fsanitize-coverage=trace-pc", "-Wno-attributes"]) for u in UNITS]
    jobs += [(os.path.join(csrc, "dism_capi.cpp"), ["-x", "c++", "-Wno-attributes"]),
             (os.path.join(HERE, "emu.cpp"), ["-Wno-attributes"])]
    # the codebook-label unit's MFMA operands are clang vector types: built with clang (same
    # ASan interface); without clang the stub stands in for it
    if os.path.exists(CLANG):
        jobs.append((os.path.join(csrc, "dism_vocab.hip"),
                     ["-x", "c++", "-fsanitize-coverage=trace-pc", "-Wno-unknown-attributes",
                      "-Wno-unused-command-line-argument"]))
    else:
        jobs.append((os.path.join(HERE, "stubs.cpp"), []))

    def compile_one(job):
        src, extra = job
        obj = os.path.join(out_dir, os.path.basename(src) + ".o")
        cc = CLANG if src.endswith("dism_vocab.hip") else "g++"
        r = subprocess.run([cc, *flags, *extra, "-c", src, "-o", obj], capture_output=True,
                           text=True)
        if r.returncode:
            raise RuntimeError(f"g++ failed for {src}:\n{r.stderr[-4000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(compile_one, jobs))
    lib = os.path.join(out_dir, "libdism_emu.so")
    subprocess.check_call(["g++", "-shared", "-fsanitize=address", "-o", lib, *objs])
    return lib


def asan_env(lib):
    """Environment of a process that loads the emulated library (ASan preloaded)."""
    env = dict(os.environ)
    env["LD_PRELOAD"] = subprocess.check_output(["g++", "-print-file-name=libasan.so"],
                                                text=True).strip()
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["DISM_EMU_LIB"] = lib
    return env


if __name__ == "__main__":
    print(build(sys.argv[1] if len(sys.argv) > 1 else os.path.join(HERE, "_build")))
