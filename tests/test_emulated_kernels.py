"""The HIP kernels themselves, run on the CPU: dism_amd/csrc compiled against a lockstep
emulation of the wave64 execution model (tests/emu/: fibers per lane, basic-block stepping
with reconvergence, wave operations over the lanes that run them together) with
AddressSanitizer on every memory access, driven through the C ABI and compared bit for bit
with the CPU model.  Each scenario runs in its own process (ASan preloaded).  No GPU; the
GPU suite (-m gpu) remains the parity gate on hardware."""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "emu"))


@pytest.fixture(scope="module")
def emu_lib(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ is not available")
    import build
    return build.build(str(tmp_path_factory.mktemp("emu")))


def _run(lib, *names):
    import build
    r = subprocess.run([sys.executable, os.path.join(HERE, "emu", "scenarios.py"), *names],
                       env=build.asan_env(lib), capture_output=True, text=True, timeout=1200)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-6000:])
    for name in names:
        assert f"OK {name}" in r.stdout


def test_fused_forward_backward(emu_lib):
    """dism_hard_forward (both halves of the prepare, the in-scan pair counts, the pair
    kernels) and dism_hard_backward on random 256-symbol rows: bit-exact, no invalid access"""
    _run(emu_lib, "fused_fwd_bwd")


def test_padded_prefill_prefix_rows(emu_lib):
    """dism_hard_prefill on rows padded from 79 to 256 tokens whose real positions form
    prefix rows (the compacted segment list): bit-exact, no invalid access"""
    _run(emu_lib, "prefill_padded")


def test_codebook_labels(emu_lib):
    """dism_vocab_labels on emulated v_mfma_f32_32x32x8_bf16 tiles (operand layouts of the
    instruction), with exact ties rescored in fp64: equal to the exact CPU model"""
    _run(emu_lib, "vocab")
