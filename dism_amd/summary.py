"""Integer hard summaries and boundaries on the MI355X library.

Mirrors dism_v3/python/flash_dism/summary.py:5-29 (summarize_hard, hard_chunk_scan) and adds
the fused one-pass ``hard_boundary`` used by the fast path.
"""
import torch

from . import _lib
from ._checks import check_ctas, check_graph_choice, check_layout, require


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_label_pair(idx_q, idx_k):
    require(isinstance(idx_q, torch.Tensor) and idx_q.is_cuda and idx_q.dtype == torch.int32 and
            idx_q.dim() == 3 and idx_q.is_contiguous(),
            "query labels must be contiguous CUDA int32 [B,H,N]")
    b, h, n = idx_q.shape
    require(b > 0 and h > 0 and n > 0 and n % 256 == 0,
            "positive dimensions and 256-aligned sequence length required")
    require(isinstance(idx_k, torch.Tensor) and idx_k.device == idx_q.device and
            idx_k.dtype == torch.int32 and idx_k.shape == idx_q.shape and idx_k.is_contiguous(),
            "invalid key labels")
    return b, h, n


def _check_flags(hard, b, h, device):
    require(isinstance(hard, torch.Tensor) and hard.device == device and
            hard.dtype == torch.bool and hard.dim() == 2 and hard.shape[0] > 0 and
            hard.shape[1] == h and hard.is_contiguous(),
            "hard must be contiguous bool [training_rows,H]; token-level masks are unsupported")
    require(hard.shape[0] == b, "fixed hard must be [B,H]")


def summarize_hard(idx_q, idx_k, hard, *, layout=None, ctas=0, _graph_choice=None):
    """Integer strip-32 hard summary int32 [B,H,(N-1)//32,N].

    R[c,j] is the largest mismatching key coordinate on the diagonal segment ending at
    (32c+31, j) within this 32-row strip, or -1 if none.  Only causal hard entries are
    computed; others are -1.  Reference: dism_v3/python/flash_dism/summary.py:5-17.
    With ``layout`` (B = 1, hard [training_rows, H]) the result is the reference's flat packed
    format [forward_elements * H], each document summarised on its own.
    """
    b, h, n = _check_label_pair(idx_q, idx_k)
    check_ctas(ctas)
    check_layout(layout)
    check_graph_choice(_graph_choice)
    if layout is not None:
        from .varlen import packed_summary
        return packed_summary(idx_q, idx_k, hard, layout)
    _check_flags(hard, b, h, idx_q.device)
    out = torch.empty((b, h, (n - 1) // 32, n), dtype=torch.int32, device=idx_q.device)
    with torch.cuda.device(idx_q.device):
        _lib.call("dism_hard_summary", idx_q.data_ptr(), idx_k.data_ptr(), hard.data_ptr(),
                  b, h, n, out.data_ptr(), _stream(idx_q))
    return out


def hard_chunk_scan(summary, *, layout=None, heads=0, _graph_choice=None, inplace=False):
    """Compose strip-32 R summaries into inclusive boundaries (max with the previous strip's
    value 32 keys earlier; non-causal entries -1).  Returns a new tensor unless inplace.
    Reference: dism_v3/python/flash_dism/summary.py:20-29.
    """
    require(isinstance(summary, torch.Tensor) and summary.is_cuda and
            summary.dtype == torch.int32 and summary.is_contiguous(),
            "hard summary must be contiguous CUDA int32")
    check_layout(layout)
    check_graph_choice(_graph_choice)
    if layout is not None:
        from .varlen import packed_chunk
        return packed_chunk(summary, layout, heads, inplace)
    require(summary.dim() == 4, "fixed hard summary must be [B,H,C,N]")
    bh = summary.shape[0] * summary.shape[1]
    require(0 < bh <= 65535 and (heads == 0 or heads == summary.shape[1]),
            "invalid fixed batch/head count")
    n = summary.shape[3]
    require(n > 0 and n % 256 == 0 and summary.shape[2] == (n - 1) // 32,
            "invalid hard checkpoint shape/alignment")
    out = summary if inplace else torch.empty_like(summary)
    with torch.cuda.device(summary.device):
        _lib.call("dism_hard_chunk", summary.data_ptr(), out.data_ptr(), bh, n, _stream(summary))
    return out


def hard_boundary(idx_q, idx_k, hard, *, strip=32, fill_all=True):
    """Composed boundaries int32 [B,H,(N-1)//strip,N] in one pass:
    boundary[b,h,c,j] = j - L[c*strip+strip-1, j] (causal hard cells), -1 elsewhere when
    fill_all.  strip=32 equals hard_chunk_scan(summarize_hard(...))."""
    b, h, n = _check_label_pair(idx_q, idx_k)
    _check_flags(hard, b, h, idx_q.device)
    require(isinstance(strip, int) and strip >= 1, "boundary strip height must be positive")
    c = (n - 1) // strip
    # fill_all=False leaves non-causal and soft-row cells unwritten (the readout never
    # reads them); fill_all=True writes every cell.
    out = torch.empty((b, h, c, n), dtype=torch.int32, device=idx_q.device)
    if c:
        with torch.cuda.device(idx_q.device):
            _lib.call("dism_hard_boundary", idx_q.data_ptr(), idx_k.data_ptr(), hard.data_ptr(),
                      b, h, n, strip, int(bool(fill_all)), out.data_ptr(), _stream(idx_q))
    return out
