"""Argument validation mirroring the reference's TORCH_CHECK texts (raised as RuntimeError).

Reference messages: dism_v3/src/host/hard_forward.cpp:12-52, hard_backward.cpp:132-153,
hard_summary.cpp:13-25, hard_chunk.cpp:85-128.
"""
import torch

VECTOR_DTYPES = (torch.bfloat16, torch.float32)
DTYPE_CODE = {torch.bfloat16: 0, torch.float32: 1}
READOUT_DIMS = (2, 4, 8, 16, 32)
VALUE_DIMS = (32, 64, 128)


def require(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def check_tensor(t, dtype, shape, name, device):
    dtypes = dtype if isinstance(dtype, tuple) else (dtype,)
    require(isinstance(t, torch.Tensor) and t.device == device and t.dtype in dtypes and
            t.is_contiguous() and tuple(t.shape) == tuple(shape),
            f"{name}: invalid device, dtype, shape or stride")


def check_ctas(ctas):
    require(isinstance(ctas, int) and 0 <= ctas <= 2**31 - 1, "invalid CTA count")


def check_layout(layout):
    if layout is not None:
        from .varlen import VarlenLayout
        require(isinstance(layout, VarlenLayout), "layout must be a VarlenLayout")


def check_graph_choice(choice):
    if choice is not None:
        raise NotImplementedError("_graph_choice routing is not implemented by the MI355X hard core")


def check_length(b, n, h):
    require(b > 0 and h > 0 and n > 0 and n % 256 == 0 and n <= 2**31 - 1024,
            "positive dimensions and 256-aligned length required")


def check_hard(hard, b, h, device, name=None):
    if name is None:
        require(isinstance(hard, torch.Tensor) and hard.device == device and
                hard.dtype == torch.bool and hard.dim() == 2 and hard.shape[0] > 0 and
                hard.shape[1] == h and hard.is_contiguous(),
                "hard must be contiguous bool [training_rows,H]; token-level masks are unsupported")
        require(hard.shape[0] == b, "fixed hard must be [B,H]")
    else:
        check_tensor(hard, torch.bool, (b, h), name, device)


def check_vectors(sq, sk, v, extra=()):
    """Validate SQ/SK/V (+ optional dO) BNHD tensors; returns (B, N, H, R, DV, dtype)."""
    require(isinstance(sq, torch.Tensor) and sq.is_cuda and sq.dim() == 4,
            "SQ must be CUDA [B,N,H,R]")
    b, n, h, r = sq.shape
    check_length(b, n, h)
    require(sq.dtype in VECTOR_DTYPES, "SQ: invalid device, dtype, shape or stride")
    dt = sq.dtype
    require(v.dim() == 4, "V: invalid device, dtype, shape or stride")
    dv = v.shape[3]
    check_tensor(sq, dt, (b, n, h, r), "SQ", sq.device)
    check_tensor(sk, dt, (b, n, h, r), "SK", sq.device)
    check_tensor(v, dt, (b, n, h, dv), "V", sq.device)
    for name, t in extra:
        check_tensor(t, dt, (b, n, h, dv), name, sq.device)
    require(r in READOUT_DIMS, f"unsupported readout dimension R={r} (supported {READOUT_DIMS})")
    require(dv in VALUE_DIMS, f"unsupported value dimension DV={dv} (supported {VALUE_DIMS})")
    return b, n, h, r, dv, dt


def check_labels(iq, ik, b, h, n, device):
    check_tensor(iq, torch.int32, (b, h, n), "query labels", device)
    check_tensor(ik, torch.int32, (b, h, n), "key labels", device)
