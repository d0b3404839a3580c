"""Packed batch-1 (varlen) layouts of the hard core.

Mirrors dism_v3/python/flash_dism/varlen.py:9-51 (VarlenLayout) and the packed branches of
the hard path: forward_hard / hard_readout / backward_hard / backward_hard_recompute with
``layout=`` (dism_v3/src/host/hard_forward.cpp:55-80, hard_backward.cpp:54-93) and
summarize_hard / hard_chunk_scan with ``layout=`` (hard_summary.cpp:27-58).

A packed call holds documents [cu[d], cu[d+1]) of one sequence (B = 1); matches never cross a
document, every boundary (T included) is 256-aligned, empty documents are allowed.  Hard flags
are per original training row: hard [rows, H] with T/rows tokens each, and no document may
cross a training row.  The library runs its fixed-length kernels on document-tagged labels
(include/dism_hard.h, packed section); this module validates the layout on the host and
allocates the outputs.  Packed strip-32 summaries/boundaries use the reference's flat format:
document s, head h at offset ForwardOffset[s]*H + h*((L-1)//32)*L, a [(L-1)//32, L] block in
document-local coordinates.
"""
import weakref
from dataclasses import dataclass

import torch

from . import _lib
from ._checks import DTYPE_CODE, check_labels, check_tensor, check_vectors, require

# layout table fields (dism_v3/include/varlen/layout.cuh:17-20)
BEGIN, LENGTH, PADDED_BEGIN, PADDED_LENGTH, FORWARD_OFFSET, VERTICAL_OFFSET, BACKWARD_OFFSET = \
    range(7)


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _make_table(offsets, total):
    """Layout table from host offsets (dism_v3/src/frontend.cpp:259-280 semantics and texts)."""
    require(total >= 0 and len(offsets) > 0 and offsets[0] == 0 and offsets[-1] == total,
            "invalid cu_seqlens endpoints")
    rows, lengths = [], []
    f = v = r = 0
    for i, start in enumerate(offsets):
        require(start >= 0 and start % 256 == 0, "all varlen boundaries must be256-token aligned")
        if i == len(offsets) - 1:
            break
        n = offsets[i + 1] - start
        require(0 <= n <= 2**31 - 1 - 255, "cu_seqlens must be monotonic with supported lengths")
        rows.append([start, n, start, n, f, v, r])
        f += ((n - 1) // 32 if n else 0) * n
        v += ((n - 1) // 16 if n else 0) * n
        r += (n + 31) // 32 * n
        lengths.append(n)
    table = torch.tensor(rows, dtype=torch.int64).reshape(-1, 7)
    return table, tuple(lengths), f, v, r


@dataclass(frozen=True)
class VarlenLayout:
    """Reusable validated sequence layout (reference dism_v3/python/flash_dism/varlen.py:9).

    Construction reads cu_seqlens on the host once; reuse the layout across layers and steps
    with the same pack.  ``table`` is CPU int64 [sequences, 7] (begin, length, padded begin,
    padded length, forward/vertical/backward checkpoint offsets).  The device copy of the
    offsets used by the kernels is cached per device.
    """
    table: torch.Tensor
    lengths: tuple
    tokens: int
    padded_tokens: int
    forward_elements: int
    vertical_elements: int
    backward_elements: int
    max_length: int = 0  # nonzero only for an explicitly prepared graph capacity

    def __post_init__(self):
        object.__setattr__(self, "_device_offsets", {})

    @classmethod
    def from_cu_seqlens(cls, cu_seqlens, total_tokens):
        require(isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.dim() == 1 and
                cu_seqlens.dtype == torch.int32 and cu_seqlens.is_contiguous() and
                cu_seqlens.numel() > 0, "cu_seqlens must be contiguous int32 [sequences+1]")
        offsets = [int(x) for x in cu_seqlens.cpu().tolist()]
        table, lengths, f, v, r = _make_table(offsets, int(total_tokens))
        return cls(table, lengths, int(total_tokens), int(total_tokens), f, v, r)

    @classmethod
    def for_graph(cls, table, total_tokens):
        """Layout over a fixed-capacity graph table (make_graph_layout); reference
        varlen.py:28-36.  Capacities (checkpoint elements, LUT length) follow max_seqlen, so
        they stay valid after update_graph_layout rewrites the documents in place.
        ``lengths`` (and ``documents``, which counts the padding rows) describe the table at
        construction; after update_graph_layout, read the current documents from ``spans()``,
        which reads the live table."""
        maximum = graph_layout_maximum(table)
        if not maximum:
            raise ValueError("expected an owned CUDA Graph layout")
        return cls(table, tuple(table[:, 1].tolist()), total_tokens, total_tokens,
                   total_tokens * ((maximum - 1) // 32), total_tokens * ((maximum - 1) // 16),
                   total_tokens * (maximum // 32), maximum)

    @property
    def documents(self):
        return len(self.lengths)

    @property
    def longest(self):
        """Longest document (the log-weight table's maximum length)."""
        return self.max_length or (max(self.lengths) if self.lengths else 0)

    def spans(self):
        """(begin, length) of every non-empty document."""
        return [(int(b), int(n)) for b, n in self.table[:, :2].tolist() if n]

    def offsets(self, device):
        """Device int32 offsets of the non-empty documents, [docs+1] (cached per device)."""
        state = _graph_state(self.table)
        if state is not None:
            return state.device_offsets(torch.device(device))
        key = str(torch.device(device))
        cache = self._device_offsets
        if key not in cache:
            host = [b for b, _ in self.spans()] + [self.tokens]
            cache[key] = torch.tensor(host, dtype=torch.int32, device=device)
        return cache[key]

    def pack(self, tensor, *, vectors):
        """Diagnostic compatibility only (reference varlen.py:42-47, varlen_pack_cuda in
        src/probe/host/varlen_pack.cpp:42-58).  Vectors [1,T,H,C] are returned as the view
        [T,H,C] (no copy).  Per-token metadata [1,H,T] (labels, normalizers) is copied into
        the documents' head-major blocks: for a document at ``begin`` of length ``n``,
        ``out[begin*H + h*n + t] = x[0, h, begin + t]``; the result is flat [T*H].  A
        permutation of whole elements (no arithmetic): a torch gather on the input's device."""
        require(isinstance(tensor, torch.Tensor) and tensor.is_contiguous() and
                tensor.dim() == (4 if vectors else 3) and tensor.shape[0] == 1,
                "expected contiguous CUDA vectors [1,T,H,C] or metadata [1,H,T]")
        require(tensor.shape[1 if vectors else 2] == self.tokens, "packed token count mismatch")
        if vectors:
            return tensor.squeeze(0)
        heads = tensor.shape[1]
        index = torch.empty(self.tokens * heads, dtype=torch.int64)
        for begin, n in self.spans():
            h = torch.arange(heads, dtype=torch.int64).view(-1, 1)
            t = torch.arange(n, dtype=torch.int64).view(1, -1)
            index[begin * heads:(begin + n) * heads] = (h * self.tokens + begin + t).reshape(-1)
        return tensor.reshape(-1)[index.to(tensor.device)]

    def checkpoint_bytes(self, heads):
        return 4 * heads * (self.forward_elements + self.vertical_elements +
                            3 * self.backward_elements)


# ---- fixed-capacity layouts for graph replay (reference dism_v3/src/host/graph_layout.h) ----
#
# A graph captures kernel launches with their pointer arguments, so a layout that changes
# between replays must keep every device buffer at a fixed address and size.  The table is a
# CPU int64 [tokens/256, 7] tensor (the most documents `tokens` can hold): its non-empty
# documents first, then padding rows (begin = tokens, length 0).  The kernels read a device
# int32 offsets array [tokens/256 + 1] built from the begin column plus `tokens`; padding rows
# repeat `tokens`, which the packed kernels read as empty documents.  update_graph_layout
# validates new boundaries, rewrites the table in place and refreshes every device copy in
# place with an async copy on the owning stream, ordered after the previous replay and before
# the next one.  The state hangs off the table's storage: views share it, clones do not.

_GRAPH_STATES = weakref.WeakKeyDictionary()


class _GraphState:
    def __init__(self, tokens, maximum, row_tokens):
        self.tokens, self.maximum, self.row_tokens = tokens, maximum, row_tokens
        self.documents = tokens // 256
        self.storage = None  # weak: set by make_graph_layout
        self.offsets = {}    # device -> int32 [documents + 1]
        self.device_index = -1
        self.stream_id = None

    def rows(self):
        storage = self.storage()
        return torch.empty(0, dtype=torch.int64).set_(storage, 0, (self.documents, 7))

    def host_offsets(self):
        begins = self.rows()[:, BEGIN].to(torch.int32)
        return torch.cat([begins, torch.tensor([self.tokens], dtype=torch.int32)])

    def check_stream(self, device):
        stream = torch.cuda.current_stream(device)
        if self.device_index < 0:
            self.device_index, self.stream_id = device.index, stream.stream_id
        require(self.device_index == device.index and self.stream_id == stream.stream_id,
                "graph metadata must be staged, captured and replayed on its owning stream")

    def device_offsets(self, device):
        if device.type != "cuda":
            return self.host_offsets().to(device)
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.check_stream(device)
        found = self.offsets.get(device.index)
        if found is not None:
            return found
        _outside_capture(device)
        gpu = self.host_offsets().pin_memory().to(device, non_blocking=True)
        self.offsets[device.index] = gpu
        return gpu


def _outside_capture(device):
    with torch.cuda.device(device):
        require(not torch.cuda.is_current_stream_capturing(),
                "prepare/update graph metadata outside CUDA Graph capture")


def _graph_state(table):
    if not isinstance(table, torch.Tensor) or table.device.type != "cpu":
        return None
    return _GRAPH_STATES.get(table.untyped_storage())


def _graph_rows(state, boundaries):
    """Validated table rows for new boundaries (reference graph_layout.h update), or raise
    before anything is changed."""
    require(isinstance(boundaries, torch.Tensor) and boundaries.device.type == "cpu" and
            boundaries.dtype == torch.int32 and boundaries.dim() == 1 and
            boundaries.is_contiguous() and boundaries.numel() >= 2,
            "graph boundaries must be contiguous CPU int32 [documents+1]")
    cu = [int(x) for x in boundaries.tolist()]
    require(cu[0] == 0 and cu[-1] == state.tokens, "invalid graph boundary endpoints")
    rows = []
    f = v = b = 0
    for begin, end in zip(cu[:-1], cu[1:]):
        n = end - begin
        require(begin >= 0 and begin % 256 == 0 and n >= 0 and n % 256 == 0 and
                n <= state.maximum,
                "graph documents must be monotonic, 256-aligned and within max_seqlen")
        if not n:
            continue  # empty documents have no work and no table row
        require(begin // state.row_tokens == (begin + n - 1) // state.row_tokens,
                "document cannot cross a hard training-row boundary")
        require(len(rows) < state.documents, "too many graph documents")
        rows.append([begin, n, begin, n, f, v, b])
        f += (n - 1) // 32 * n
        v += (n - 1) // 16 * n
        b += n // 32 * n
    rows += [[state.tokens, 0, state.tokens, 0, f, v, b]] * (state.documents - len(rows))
    return torch.tensor(rows, dtype=torch.int64)


def make_graph_layout(boundaries, tokens, maximum, row_tokens):
    """Fixed-capacity graph layout table (reference cu.make_graph_layout,
    dism_v3/src/host/graph_layout.h create): tokens, max_seqlen and training-row length are
    256-aligned capacities fixed for the table's life; ``boundaries`` is the first pack."""
    tokens, maximum, row_tokens = int(tokens), int(maximum), int(row_tokens)
    require(0 < tokens <= 2**31 - 1 - 256 and tokens % 256 == 0 and 0 < maximum <= tokens and
            maximum % 256 == 0 and row_tokens > 0 and row_tokens % 256 == 0 and
            tokens % row_tokens == 0 and maximum <= row_tokens,
            "invalid graph token/max_seqlen/training-row capacities")
    # documents are told apart by tagging label ranks with their index: 2 * N * docs <= 2^32
    require(2 * tokens * (tokens // 256) <= 2**32,
            "graph layout tokens exceed the packed core's document-tag range "
            "(2 * tokens * tokens/256 <= 2^32)")
    state = _GraphState(tokens, maximum, row_tokens)
    table = _graph_rows(state, boundaries)
    storage = table.untyped_storage()
    state.storage = weakref.ref(storage)
    _GRAPH_STATES[storage] = state
    return table


def update_graph_layout(table, boundaries):
    """Rewrite a graph layout's documents in place (reference cu.update_graph_layout).  All
    input is validated before anything changes; device copies are refreshed in place on the
    owning stream, so call it between replays, outside capture."""
    state = _graph_state(table)
    require(state is not None, "expected an owned graph layout")
    rows = _graph_rows(state, boundaries)
    for index in state.offsets:
        device = torch.device("cuda", index)
        _outside_capture(device)
        state.check_stream(device)
    state.rows().copy_(rows)
    host = state.host_offsets()
    for index, gpu in state.offsets.items():
        with torch.cuda.device(index):
            gpu.copy_(host.pin_memory(), non_blocking=True)


def graph_layout_maximum(table):
    """max_seqlen of a graph layout table, 0 for any other tensor (reference
    cu.graph_layout_maximum)."""
    state = _graph_state(table)
    return state.maximum if state is not None else 0


def layout_from_table(table, tokens):
    """VarlenLayout from a layout table without any device readback (reference
    hard_training.py:328-340): graph tables keep their fixed capacities."""
    if table is None:
        return None
    table = table.view(-1, 7)
    if graph_layout_maximum(table):
        return VarlenLayout.for_graph(table, tokens)
    lengths = tuple(table[:, 1].tolist())
    return VarlenLayout(table, lengths, tokens, tokens,
                        sum((n - 1) // 32 * n for n in lengths if n),
                        sum((n - 1) // 16 * n for n in lengths if n),
                        sum((n + 31) // 32 * n for n in lengths))


def check_packed_rows(layout, n, hard, h, device):
    """Packed batch-1 preconditions of the reference (hard_forward.cpp:57-75): returns the
    training-row length."""
    require(isinstance(layout, VarlenLayout), "layout must be a VarlenLayout")
    require(isinstance(hard, torch.Tensor) and hard.device == device and
            hard.dtype == torch.bool and hard.dim() == 2 and hard.shape[0] > 0 and
            hard.shape[1] == h and hard.is_contiguous(),
            "hard must be contiguous bool [training_rows,H]; token-level masks are unsupported")
    require(layout.tokens == n, "packed labels/layout length mismatch")
    rows = hard.shape[0]
    require(n % rows == 0 and (n // rows) % 256 == 0,
            "packed hard rows must evenly divide tokens into 256-aligned training rows")
    row_n = n // rows
    state = _graph_state(layout.table)
    require(state is None or state.row_tokens == row_n,
            "packed hard rows must match the graph layout's training-row length")
    for begin, length in layout.spans():
        require(begin // row_n == (begin + length - 1) // row_n,
                "document cannot cross a hard training-row boundary")
    return row_n


def packed_prepare(sq, sk, v, iq, ik, layout):
    """Workspace of a packed call: tagged labels, document starts, orders and pair plans."""
    _, n, h, r, dv, dt = check_vectors(sq, sk, v)
    nbytes = _lib.packed_workspace_bytes(n, h, r, dv, DTYPE_CODE[dt])
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=sq.device)
    cu = layout.offsets(sq.device)
    with torch.cuda.device(sq.device):
        _lib.call("dism_hard_packed_prepare", sq.data_ptr(), sk.data_ptr(), v.data_ptr(),
                  DTYPE_CODE[dt], iq.data_ptr(), ik.data_ptr(), cu.data_ptr(),
                  cu.numel() - 1, n, h, r, dv, ws.data_ptr(), nbytes, _stream(sq))
    return ws


def packed_readout(sq, sk, v, iq, ik, hard, log_weights, layout, out_dtype, matches,
                   workspace=None):
    """Packed readout -> (O, lse2, lmax, jarg, workspace)."""
    b, n, h, r, dv, dt = check_vectors(sq, sk, v)
    require(b == 1, "packed labels/layout length mismatch")
    check_labels(iq, ik, b, h, n, sq.device)
    check_packed_rows(layout, n, hard, h, sq.device)
    longest = layout.longest
    require(isinstance(log_weights, torch.Tensor) and log_weights.device == sq.device and
            log_weights.dtype == torch.float32 and log_weights.dim() == 2 and
            log_weights.shape[0] == h and log_weights.is_contiguous(),
            "invalid hard log-weight table")
    require(log_weights.shape[1] > longest, "hard log-weight table is too short")
    if workspace is None:
        workspace = packed_prepare(sq, sk, v, iq, ik, layout)
    out = torch.empty((b, n, h, dv), dtype=out_dtype, device=sq.device)
    lse2 = torch.empty((b, h, n), dtype=torch.float32, device=sq.device)
    lmax = jarg = None
    if matches:
        lmax = torch.empty((b, h, n), dtype=torch.int32, device=sq.device)
        jarg = torch.empty((b, h, n), dtype=torch.int32, device=sq.device)
    ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
    with torch.cuda.device(sq.device):
        _lib.call("dism_hard_packed_readout", sq.data_ptr(), sk.data_ptr(), v.data_ptr(),
                  DTYPE_CODE[dt], hard.data_ptr(), hard.shape[0], log_weights.data_ptr(),
                  log_weights.shape[1], longest, n, h, r, dv, workspace.data_ptr(),
                  workspace.numel(), out.data_ptr(), DTYPE_CODE[out_dtype], lse2.data_ptr(),
                  ptr(lmax), ptr(jarg), _stream(sq))
    return out, lse2, lmax, jarg, workspace


def packed_backward(sq, sk, v, dout, iq, ik, hard, lse2, lut, dlut, layout, workspace=None):
    """Packed backward -> (dSQ, dSK, dV, dtau), all fp32."""
    b, n, h, r, dv, dt = check_vectors(sq, sk, v, extra=(("dO", dout),))
    require(b == 1, "packed labels/layout length mismatch")
    check_labels(iq, ik, b, h, n, sq.device)
    check_packed_rows(layout, n, hard, h, sq.device)
    check_tensor(lse2, torch.float32, (b, h, n), "log2 normalizer", sq.device)
    longest = layout.longest
    require(isinstance(lut, torch.Tensor) and lut.device == sq.device and
            lut.dtype == torch.float32 and lut.dim() == 2 and lut.shape[0] == h and
            lut.is_contiguous(), "log weight LUT: invalid device, dtype, shape or stride")
    require(lut.shape[1] > longest, "hard log-weight table is too short")
    check_tensor(dlut, torch.float32, tuple(lut.shape), "log weight derivative table",
                 sq.device)
    if workspace is None or workspace.numel() < _lib.packed_workspace_bytes(
            n, h, r, dv, DTYPE_CODE[dt]):
        workspace = packed_prepare(sq, sk, v, iq, ik, layout)
    dsq = torch.empty((b, n, h, r), dtype=torch.float32, device=sq.device)
    dsk = torch.empty((b, n, h, r), dtype=torch.float32, device=sq.device)
    dvv = torch.empty((b, n, h, dv), dtype=torch.float32, device=sq.device)
    rowtau = torch.empty((b, h, n), dtype=torch.float32, device=sq.device)
    dtau = torch.empty((h,), dtype=torch.float32, device=sq.device)
    with torch.cuda.device(sq.device):
        _lib.call("dism_hard_packed_backward", sq.data_ptr(), sk.data_ptr(), v.data_ptr(),
                  dout.data_ptr(), DTYPE_CODE[dt], hard.data_ptr(), hard.shape[0],
                  lut.data_ptr(), dlut.data_ptr(), lut.shape[1], longest, lse2.data_ptr(), n,
                  h, r, dv, workspace.data_ptr(), workspace.numel(), dsq.data_ptr(),
                  dsk.data_ptr(), dvv.data_ptr(), rowtau.data_ptr(), dtau.data_ptr(),
                  _stream(sq))
    return dsq, dsk, dvv, dtau


def packed_summary(idx_q, idx_k, hard, layout):
    """Flat packed strip-32 summary int32 [forward_elements * H] (reference format): each
    non-empty document is summarised on its own (document-local coordinates); soft documents
    and non-causal cells are -1."""
    b, h, n = idx_q.shape
    require(b == 1, "packed labels/layout length mismatch")
    row_n = check_packed_rows(layout, n, hard, h, idx_q.device)
    out = torch.full((layout.forward_elements * h,), -1, dtype=torch.int32,
                     device=idx_q.device)
    for s, (begin, length) in enumerate(layout.table[:, :2].tolist()):
        c = (length - 1) // 32 if length else 0
        if not c:
            continue
        off = int(layout.table[s, FORWARD_OFFSET]) * h
        view = out[off:off + h * c * length]
        q = idx_q[:, :, begin:begin + length].contiguous()
        k = idx_k[:, :, begin:begin + length].contiguous()
        flags = hard[begin // row_n:begin // row_n + 1]
        with torch.cuda.device(idx_q.device):
            _lib.call("dism_hard_summary", q.data_ptr(), k.data_ptr(), flags.data_ptr(), 1, h,
                      length, view.data_ptr(), _stream(idx_q))
    return out


def packed_chunk(summary, layout, heads, inplace):
    """Composition of a flat packed summary, document by document."""
    require(isinstance(heads, int) and heads > 0, "packed hard summary needs the head count")
    require(summary.dim() == 1 and summary.numel() == layout.forward_elements * heads,
            "packed hard summary must be flat int32 [forward_elements*H]")
    out = summary if inplace else torch.empty_like(summary)
    for s, (begin, length) in enumerate(layout.table[:, :2].tolist()):
        c = (length - 1) // 32 if length else 0
        if not c:
            continue
        off = int(layout.table[s, FORWARD_OFFSET]) * heads
        size = heads * c * length
        with torch.cuda.device(summary.device):
            _lib.call("dism_hard_chunk", summary[off:off + size].data_ptr(),
                      out[off:off + size].data_ptr(), heads, length, _stream(summary))
    return out
