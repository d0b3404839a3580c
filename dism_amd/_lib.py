"""ctypes binding of libdism_hip.so (C ABI declared in include/dism_hard.h).

The library is loaded from this package directory.  If it is missing the import of the
compute entry points raises: there is no CPU fallback for the hard core.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdism_hip.so")

# name -> argtypes (all return int32 status)
_P, _I32, _I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
SIGNATURES = {
    "dism_sign_labels": [_P, _I32, _I64, _I64, _I64, _I32, _P, _P],
    "dism_hard_log_weights": [_P, _I32, _I64, _P, _P],
    "dism_hard_dlog_weights": [_P, _I32, _I64, _P, _P],
    "dism_hard_summary": [_P, _P, _P, _I64, _I64, _I64, _P, _P],
    "dism_hard_chunk": [_P, _P, _I64, _I64, _P],
    "dism_hard_boundary": [_P, _P, _P, _I64, _I64, _I64, _I32, _I32, _P, _P],
    "dism_hard_prepare": [_P, _P, _P, _I32, _P, _P, _I64, _I64, _I64, _I32, _I32, _P, _I64, _P],
    "dism_hard_forward_noalloc": [_P, _P, _P, _I32, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                  _I32, _I32, _P, _I32, _P, _P, _P, _P],
    "dism_hard_row_modes": [_P, _I64, _I64, _I64, _I64, _I32, _I32, _P, _P],
    "dism_hard_readout": [_P, _P, _P, _I32, _P, _P, _P, _P, _I32, _P, _I64, _I64, _I64, _I64,
                          _I32, _I32, _P, _I64, _P, _I32, _P, _P, _P, _P],
    "dism_hard_forward": [_P, _P, _P, _I32, _P, _P, _P, _P, _I32, _P, _I64, _I64, _I64, _I64,
                          _I32, _I32, _P, _I64, _P, _I32, _P, _P, _P, _P],
    "dism_hard_backward": [_P, _P, _P, _P, _I32, _P, _P, _P, _P, _I32, _P, _P, _I64, _P, _I64,
                           _I64, _I64, _I32, _I32, _P, _I64, _P, _P, _P, _P, _P, _P],
    "dism_hard_backward_row_pairs": [_P, _P, _P, _P, _I32, _P, _P, _P, _P, _I32, _P, _P, _I64,
                                     _P, _I64, _I64, _I64, _I32, _I32, _P, _I64, _P],
    "dism_hard_backward_queries": [_P, _P, _P, _P, _I32, _P, _P, _P, _P, _I32, _P, _P, _I64,
                                   _P, _I64, _I64, _I64, _I32, _I32, _P, _I64, _P, _P, _P],
    "dism_hard_backward_keys": [_P, _P, _P, _P, _I32, _P, _P, _P, _P, _I32, _P, _I64, _P, _I64,
                                _I64, _I64, _I32, _I32, _P, _I64, _P, _P, _P],
    "dism_hard_backward_key_pairs": [_P, _P, _P, _P, _I32, _P, _P, _P, _P, _I32, _P, _I64, _P,
                                     _I64, _I64, _I64, _I32, _I32, _P, _I64, _P, _P, _P],
    "dism_hard_tau_reduce": [_P, _I64, _I64, _I64, _P, _P],
    "dism_hard_packed_prepare": [_P, _P, _P, _I32, _P, _P, _P, _I64, _I64, _I64, _I32, _I32,
                                 _P, _I64, _P],
    "dism_hard_packed_readout": [_P, _P, _P, _I32, _P, _I64, _P, _I64, _I64, _I64, _I64, _I32,
                                 _I32, _P, _I64, _P, _I32, _P, _P, _P, _P],
    "dism_hard_packed_backward": [_P, _P, _P, _P, _I32, _P, _I64, _P, _P, _I64, _I64, _P, _I64,
                                  _I64, _I32, _I32, _P, _I64, _P, _P, _P, _P, _P, _P],
    "dism_vocab_labels": [_P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P],
    "dism_hard_prefill": [_P, _P, _P, _I32, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32,
                          _I32, _P, _I64, _P, _P, _P],
    "dism_decoder_init": [_P, _I64, _I64, _I32, _I32, _I64, _I32, _I32, _P],
    "dism_decoder_prime": [_P, _I64, _I64, _I64, _I32, _I32, _I64, _I32, _I32, _I64, _P, _P,
                           _P, _P, _P, _P, _I64, _P],
    "dism_decoder_step": [_P, _I64, _I64, _I64, _I32, _I32, _I64, _I32, _I32, _I64, _P, _P, _P,
                          _P, _P, _P, _P, _I64, _P, _P, _P],
}

# entry points returning a size (int64, -1 = unsupported) rather than a status
SIZE_SIGNATURES = {
    "dism_hard_workspace_bytes": [_I64, _I64, _I64, _I32, _I32, _I32],
    "dism_hard_packed_workspace_bytes": [_I64, _I64, _I32, _I32, _I32],
    "dism_hard_prefill_workspace_bytes": [_I64, _I64, _I64, _I32, _I32, _I32],
    "dism_decoder_state_bytes": [_I64, _I32, _I32, _I64, _I32, _I32],
    "dism_decoder_prime_workspace_bytes": [_I64, _I64, _I64, _I32, _I32, _I32],
    "dism_hard_forward_noalloc_max_bytes": [],
}

_lib = None


class DismNativeMissing(RuntimeError):
    pass


def load():
    """Load (once) and return the ctypes handle; raise if the HIP library is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DismNativeMissing(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
                " (the hard core has no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int32
        lib.dism_last_error.restype = ctypes.c_char_p
        lib.dism_last_error.argtypes = []
        lib.dism_abi_version.restype = ctypes.c_int32
        lib.dism_abi_version.argtypes = []
        lib.dism_layout_check.restype = ctypes.c_int32
        lib.dism_layout_check.argtypes = []
        if lib.dism_layout_check() != 0:
            raise DismNativeMissing(
                f"{LIB_PATH}: {lib.dism_last_error().decode(errors='replace')}")
        for name, args in SIZE_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int64
        _lib = lib
    return _lib


def call(name, *args):
    """Invoke a C-ABI entry point; translate a non-zero status into RuntimeError."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.dism_last_error().decode(errors="replace")
        raise RuntimeError(f"{name}: {msg}")


def workspace_bytes(B, N, H, R, DV, dtype_code):
    """Bytes of the caller-owned workspace (raises for unsupported dimensions)."""
    nbytes = load().dism_hard_workspace_bytes(B, N, H, R, DV, dtype_code)
    if nbytes < 0:
        raise RuntimeError(f"unsupported hard-core dimensions B={B} N={N} H={H} R={R} DV={DV}")
    return nbytes


def packed_workspace_bytes(N, H, R, DV, dtype_code):
    """Bytes of a packed (varlen) call's workspace (raises for unsupported dimensions)."""
    nbytes = load().dism_hard_packed_workspace_bytes(N, H, R, DV, dtype_code)
    if nbytes < 0:
        raise RuntimeError(f"unsupported packed hard-core dimensions N={N} H={H} R={R} DV={DV}")
    return nbytes


def size(name, *args):
    """Call a size entry point (SIZE_SIGNATURES); raise for unsupported dimensions."""
    nbytes = getattr(load(), name)(*args)
    if nbytes < 0:
        raise RuntimeError(f"{name}: unsupported dimensions {args}")
    return nbytes
