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


@torch.no_grad()
def vocab_labels(x, vocab, *, return_exact_count=False):
    """Codebook argmax labels (the general label producer): x bf16 [B,N,H,D] (CUDA),
    vocab bf16 [H,V,D] or shared [V,D], D in {32, 64, 128} -> int32 [B,H,N] with
    labels[b,h,n] = argmax_v x[b,n,h] . vocab[h,v] in exact arithmetic, first index on ties
    (reference dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162).  Scores run on the
    matrix cores; tokens whose top-two margin lies within the certified fp32 error bound are
    rescored in fp64.  With return_exact_count, also returns how many tokens were rescored."""
    require(isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 4 and x.is_contiguous()
            and x.dtype == torch.bfloat16, "x must be contiguous CUDA bf16 [B,N,H,D]")
    b, n, h, d = x.shape
    require(isinstance(vocab, torch.Tensor) and vocab.device == x.device and
            vocab.dtype == torch.bfloat16 and vocab.is_contiguous() and vocab.dim() in (2, 3),
            "vocabulary must be contiguous CUDA bf16 [H,V,D] or [V,D]")
    require(vocab.shape[-1] == d and (vocab.dim() == 2 or vocab.shape[0] == h) and
            vocab.shape[-2] > 0, "invalid vocabulary/channel size")
    require(d in (32, 64, 128), "invalid vocabulary/channel size")
    v = vocab.shape[-2]
    out = torch.empty((b, h, n), dtype=torch.int32, device=x.device)
    scratch = torch.empty((1 + 2 * h + b * h * n,), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("dism_vocab_labels", x.data_ptr(), vocab.data_ptr(),
                  0 if vocab.dim() == 2 else v * d, b, n, h, v, d, out.data_ptr(),
                  scratch.data_ptr(), torch.cuda.current_stream(x.device).cuda_stream)
    return (out, scratch[:1]) if return_exact_count else out


@torch.library.custom_op("dism_amd::vocab_labels", mutates_args=())
def vocab_labels_op(x: torch.Tensor, vocab: torch.Tensor) -> torch.Tensor:
    """vocab_labels as a torch.library operator (opaque to torch.compile, no autograd: the
    argmax is piecewise constant)."""
    return vocab_labels(x, vocab)


@vocab_labels_op.register_fake
def _vocab_labels_fake(x, vocab):
    b, n, h, _ = x.shape
    return x.new_empty((b, h, n), dtype=torch.int32)


def vocab_argmax_labels(q, k, q_vocab, k_vocab):
    """(idx_q, idx_k) = codebook argmax labels of q against q_vocab and of k against k_vocab,
    the hard labels of dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162."""
    return vocab_labels(q, q_vocab), vocab_labels(k, k_vocab)
