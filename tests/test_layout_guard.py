"""A library linked from objects compiled against different layouts of the by-value argument
structs must refuse to run.

The failure this guards against: a kernel unit compiled before a field was added to
``dism::Orders`` (which ``PathArgs`` and ``SortArgs`` embed by value) reads every later field
of its kernel argument at the old offset, so a launch from a relinked library dereferences
pointer fields that hold other fields' values.  The test builds exactly such a library on the
CPU -- ``dism_aux.hip`` recompiled against a copy of ``dism_launch.h`` whose ``Orders`` has
one more pointer, linked with the current objects of every other unit -- and checks that
the per-unit fingerprints differ, that ``dism_layout_check`` names the stale unit, and that
an entry point refuses before launching anything.  No GPU is used."""
import ctypes
import os
import shutil
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from dism_amd import build as B  # noqa: E402


def _objects_present():
    return all(os.path.exists(os.path.join(B.OUT_DIR, s + ".o")) for s in B.SOURCES)


@pytest.fixture(scope="module")
def stale_lib(tmp_path_factory):
    if not os.path.exists(B.HIPCC) or not _objects_present():
        pytest.skip("hipcc or the built objects are missing (run the build first)")
    d = tmp_path_factory.mktemp("stale")
    src = d / "csrc"
    shutil.copytree(B.CSRC, src)
    hdr = src / "dism_launch.h"
    text = hdr.read_text()
    marker = "    int32_t* pxL;"
    assert marker in text
    # the same kind of change as adding a section to the workspace orders: one more pointer
    text = text.replace(marker, marker + "\n    int32_t* stale_test_extra;", 1)
    # the old unit's static size checks would stop it compiling; a stale object predates them
    text = text.replace("static_assert(sizeof(Orders)", "static_assert(true || sizeof(Orders)")
    text = text.replace("static_assert(sizeof(SortArgs)",
                        "static_assert(true || sizeof(SortArgs)")
    text = text.replace("static_assert(sizeof(PathArgs)",
                        "static_assert(true || sizeof(PathArgs)")
    hdr.write_text(text)
    obj = d / "dism_aux.hip.o"
    subprocess.run([B.HIPCC, *B.FLAGS, "-c", str(src / "dism_aux.hip"), "-o", str(obj)],
                   check=True, capture_output=True)
    objs = [str(obj) if s == "dism_aux.hip" else os.path.join(B.OUT_DIR, s + ".o")
            for s in B.SOURCES]
    lib = d / "libdism_stale.so"
    subprocess.run([B.HIPCC, f"--offload-arch={B.ARCH}", "-shared", "-fPIC", "-o", str(lib),
                    *objs], check=True, capture_output=True)
    return str(lib)


def _run(lib_path, body):
    """Load a library in a fresh process (two copies of the HIP runtime state in one process
    are not needed for this) and run ``body`` against it."""
    code = textwrap.dedent(f"""
        import ctypes
        lib = ctypes.CDLL({lib_path!r})
        lib.dism_last_error.restype = ctypes.c_char_p
    """) + textwrap.dedent(body)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout


def test_load_check_names_the_stale_unit(stale_lib):
    out = _run(stale_lib, """
        print(lib.dism_layout_check())
        print(lib.dism_last_error().decode())
    """).split("\n")
    assert out[0] == "1"
    assert "mismatched argument-struct layouts" in out[1] and "dism_aux" in out[1]
    assert "dism_sort" not in out[1]


def test_entry_point_refuses_before_launch(stale_lib):
    # a prepare call with plausible arguments: the layout guard answers before any check
    # that would touch the (dummy) pointers or the device
    out = _run(stale_lib, """
        d = ctypes.c_void_p(256)
        f = lib.dism_hard_prepare
        f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int32] + [ctypes.c_void_p] * 2 + \\
            [ctypes.c_int64] * 3 + [ctypes.c_int32] * 2 + [ctypes.c_void_p, ctypes.c_int64,
            ctypes.c_void_p]
        print(f(d, d, d, 0, d, d, 1, 256, 1, 8, 64, d, 1 << 30, None))
        print(lib.dism_last_error().decode())
    """).split("\n")
    assert out[0] == "1" and "dism_aux" in out[1]


def test_current_library_passes():
    from dism_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libdism_hip.so not built")
    lib = _lib.load()
    assert lib.dism_layout_check() == 0, lib.dism_last_error()
