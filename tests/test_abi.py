"""C-ABI of libdism_hip.so on the CPU: the library loads (HIP runtime present, no device
needed), exports every entry point include/dism_hard.h declares, and its host-side validation
rejects bad arguments with the reference's error texts -- without launching anything."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dism_hard.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dism_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from dism_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libdism_hip.so not built")
    return _lib.load()


def test_header_symbols_exported(lib):
    names = _declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name


def test_python_signatures_cover_header(lib):
    from dism_amd import _lib
    declared = set(_declared())
    special = {"dism_last_error", "dism_abi_version", "dism_layout_check"}
    bound = set(_lib.SIGNATURES) | set(_lib.SIZE_SIGNATURES)
    assert declared - special == bound, declared ^ bound


def test_version_and_workspace(lib):
    assert lib.dism_abi_version() == 7
    assert lib.dism_layout_check() == 0, lib.dism_last_error()
    ws = lib.dism_hard_workspace_bytes(4, 16384, 16, 8, 64, 0)
    assert ws > 4 * 16384 * 16 * 64 * 4  # holds one fp32 readout row per query
    assert ws % 256 == 0
    assert lib.dism_hard_workspace_bytes(4, 16384, 16, 3, 64, 0) == -1   # R unsupported
    assert lib.dism_hard_workspace_bytes(4, 16384, 16, 8, 48, 0) == -1   # DV unsupported
    assert lib.dism_hard_workspace_bytes(0, 16384, 16, 8, 64, 0) == -1   # empty
    assert lib.dism_hard_workspace_bytes(4, 16384, 16, 8, 64, 7) == -1   # dtype
    packed = lib.dism_hard_packed_workspace_bytes(16384, 16, 8, 64, 0)
    assert packed > lib.dism_hard_workspace_bytes(1, 16384, 16, 8, 64, 0)
    assert packed % 256 == 0
    assert lib.dism_hard_packed_workspace_bytes(16384, 16, 8, 48, 0) == -1


def test_host_validation_without_launch(lib):
    from dism_amd import _lib
    # null pointers and unsupported dims fail before any HIP call
    rc = lib.dism_hard_readout(None, None, None, 0, None, None, None, None, 0, None, 257, 1, 256,
                               1, 8, 64, None, 0, None, 0, None, None, None, None)
    assert rc == 1 and b"null pointer" in lib.dism_last_error()
    rc = lib.dism_hard_log_weights(None, 4, 256, None, None)
    assert rc == 1 and b"tau must be contiguous" in lib.dism_last_error()
    rc = lib.dism_hard_boundary(None, None, None, 1, 1, 256, 0, 0, None, None)
    assert rc == 1 and b"null pointer" in lib.dism_last_error()
    dummy = ctypes.c_void_p(16)  # never dereferenced: rejected by the dimension check
    rc = lib.dism_hard_prepare(dummy, dummy, dummy, 0, dummy, dummy, 1, 256, 1, 3, 64, dummy,
                               1 << 20, None)
    assert rc == 2 and b"unsupported R=3" in lib.dism_last_error()
    rc = lib.dism_hard_prepare(dummy, dummy, dummy, 0, dummy, dummy, 1, 256, 1, 8, 64, dummy, 16,
                               None)
    assert rc == 1 and b"workspace too small" in lib.dism_last_error()
    with pytest.raises(RuntimeError, match="tau must be contiguous"):
        _lib.call("dism_hard_log_weights", None, 4, 256, None, None)


def test_python_api_rejects_cpu_tensors():
    """The product path needs the HIP device: CPU tensors are rejected with the reference's
    messages, never computed on the host."""
    import torch
    import dism_amd
    tau = torch.zeros(4)
    with pytest.raises(RuntimeError, match="tau must be contiguous"):
        dism_amd.hard_log_weights(tau, 256)
