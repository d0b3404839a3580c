"""Sign binarizer: the label producer of this build.

labels[b,h,n] = sum_k [x[b,n,h,k] > 0] 2^k.  For the hypercube codebook e_c[k] = 2 bit_k(c) - 1
this is the argmax of x . e_c with the reference's first-index tie rule (x_k == 0 -> bit 0),
i.e. the label producer of dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162 and the
Triton argmax of dism_v3/python/flash_dism/emb_kernel.py:83-108 specialised to hypercube
codebooks.  NaN gives bit 0.
"""
import torch

from . import _lib
from ._checks import DTYPE_CODE, require


@torch.no_grad()
def sign_labels(x):
    """x [B,N,H,d] (bf16 or f32, CUDA, d <= 30) -> int32 labels [B,H,N]."""
    require(isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 4 and x.is_contiguous()
            and x.dtype in DTYPE_CODE, "x must be contiguous CUDA bf16/f32 [B,N,H,d]")
    b, n, h, d = x.shape
    require(b > 0 and n > 0 and h > 0 and 1 <= d <= 30, "invalid label source shape")
    out = torch.empty((b, h, n), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("dism_sign_labels", x.data_ptr(), DTYPE_CODE[x.dtype], b, n, h, d,
                  out.data_ptr(), torch.cuda.current_stream(x.device).cuda_stream)
    return out
