"""Full-hard inference on the MI355X library: prefill and incremental decoding.

Mirrors dism_v3/python/flash_dism/inference/ (HardDismPrefill, PreparedHardPrefill:
prefill_batch.py:30-118; HardDismDecoder: api.py:11-105; README.md:229-350) with the same
class names, arguments, shapes, FP32 outputs and ValueError texts.

The reference builds a suffix automaton on the CPU and executes its event streams.  This
build needs neither: the hard readout decomposes into per-label running matrices plus
bigram-pair corrections (see dism_scan.hip / dism_pairs.hip), so
  * prefill is the training forward (dism_hard_prefill) with query resets bounding the
    suffix walks -- any positive length (rows are padded to 256 internally; padding sits
    after every real query and never matches one);
  * the decoder (dism_decoder_step) keeps each row's label table of running matrices and
    key-position lists on the device and appends tokens in O(R*DV) plus the token's bigram
    pairs -- no snapshots and no rebuilds.
Both give, bit for bit, the training forward's fp32 outputs (oracle/dism_cpu_model.c:
orc_forward / orc_forward_reset).  Resets: reset[b,h,i] starts query i's match afresh; stored
keys stay visible (dism_v3/tests/test_sam_inference.py:9-29).
"""
import torch

from . import _lib
from ._checks import DTYPE_CODE
from .hard_forward import hard_log_weights

PAD = 256


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _tau_tensor(tau, heads, device):
    if isinstance(tau, torch.Tensor):
        if tau.shape != (heads,):
            raise ValueError("tau must have shape [H]")
        tau = tau.detach().double().cpu().tolist()
    tau = list(tau)
    if len(tau) != heads:
        raise ValueError("one fixed tau per head")
    return torch.tensor(tau, dtype=torch.float32, device=device)


def _padded_lut(tau, length):
    """log2 weight table covering lengths 0..length (rounded up to 256)."""
    return hard_log_weights(tau, (length + PAD - 1) // PAD * PAD)


class PreparedHardPrefill:
    """Labels, resets and the LUT of one prefill, uploaded to the engine's device; execute()
    runs the readout for vectors of that shape (reference prefill_batch.py:30-62)."""

    def __init__(self, engine, idx_q, idx_k, tau, reset):
        self.device = engine.device
        self.batch, self.heads, self.n = idx_q.shape
        self.stream = torch.cuda.current_stream(self.device)
        n_pad = (self.n + PAD - 1) // PAD * PAD
        self.n_pad = n_pad

        def pad_labels(x):
            out = torch.zeros((self.batch, self.heads, n_pad), dtype=torch.int32,
                              device=self.device)
            out[..., :self.n] = x.to(self.device)
            return out

        self.iq, self.ik = pad_labels(idx_q), pad_labels(idx_k)
        self.reset = None
        if reset is not None:
            self.reset = torch.zeros((self.batch, self.heads, n_pad), dtype=torch.uint8,
                                     device=self.device)
            self.reset[..., :self.n] = reset.to(self.device, torch.uint8)
        self.tau = _tau_tensor(tau, self.heads, self.device)
        self.lut = hard_log_weights(self.tau, n_pad)

    def _pad(self, x):
        if self.n_pad == self.n:
            return x
        out = torch.zeros((x.shape[0], self.n_pad) + tuple(x.shape[2:]), dtype=x.dtype,
                          device=x.device)
        out[:, :self.n] = x
        return out

    def execute(self, sq, sk, value):
        expected = (self.batch, self.n, self.heads)
        if sq.ndim != 4 or sk.shape != sq.shape or value.ndim != 4 or \
                sq.shape[:3] != expected or value.shape[:3] != expected:
            raise ValueError("vectors must be sq/sk [B,N,H,R], value [B,N,H,DV]")
        if any(not x.is_contiguous() for x in (sq, sk, value)):
            raise ValueError("contiguous BNHD vectors required; no implicit transpose")
        if torch.cuda.current_stream(self.device) != self.stream:
            raise ValueError("prepared prefill must execute on its upload stream")
        if sq.dtype not in DTYPE_CODE or sk.dtype != sq.dtype or value.dtype != sq.dtype:
            raise ValueError("vectors must share one dtype (bf16 or fp32)")
        if any(x.device != self.device for x in (sq, sk, value)):
            raise ValueError("vectors must be on the engine device")
        b, n, h, r = sq.shape
        dv = value.shape[3]
        a, c, d = (self._pad(x) for x in (sq, sk, value))
        code = DTYPE_CODE[sq.dtype]
        nbytes = _lib.size("dism_hard_prefill_workspace_bytes", b, self.n_pad, h, r, dv, code)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=self.device)
        out = torch.empty((b, self.n_pad, h, dv), dtype=torch.float32, device=self.device)
        lse2 = torch.empty((b, h, self.n_pad), dtype=torch.float32, device=self.device)
        reset = 0 if self.reset is None else self.reset.data_ptr()
        with torch.cuda.device(self.device):
            _lib.call("dism_hard_prefill", a.data_ptr(), c.data_ptr(), d.data_ptr(), code,
                      self.iq.data_ptr(), self.ik.data_ptr(), reset, self.lut.data_ptr(),
                      self.lut.shape[1], b, self.n_pad, self.n, h, r, dv, ws.data_ptr(), nbytes,
                      out.data_ptr(), lse2.data_ptr(), _stream(self.device))
        self.last_lse2 = lse2[..., :self.n]
        return out[:, :self.n] if self.n_pad != self.n else out

    # one path serves every stream length here
    execute_dispatch = execute

    def statistics(self):
        return dict(batch=self.batch, heads=self.heads, n=self.n, padded=self.n_pad)


class HardDismPrefill:
    """Reusable prefill engine (reference prefill_batch.py:65-118).  Labels int32 [B,H,N] (CPU
    or the engine's device), vectors contiguous BNHD bf16/fp32, FP32 output [B,N,H,DV].
    ``workers``, ``chunk_size``, ``mma_precision`` and ``dispatch_threshold`` are the
    reference's planner/GEMM knobs: validated and accepted; the MI355X path has no CPU planner
    and computes the exact fp32 readout."""

    def __init__(self, *, workers=16, chunk_size=16, mma_precision="bf16", device="cuda",
                 dispatch_threshold=64):
        if chunk_size not in (16, 32, 64):
            raise ValueError("invalid chunk_size")
        if mma_precision not in ("bf16", "tf32x3"):
            raise ValueError("invalid mma_precision")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("CUDA device required")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.workers, self.chunk_size, self.mma_precision = workers, chunk_size, mma_precision
        self.dispatch_threshold = dispatch_threshold

    def prepare(self, idx_q, idx_k, tau, *, reset=None):
        for x in (idx_q, idx_k):
            if not isinstance(x, torch.Tensor) or x.ndim != 3 or x.dtype != torch.int32:
                raise ValueError("labels must be int32 tensors [B,H,N]")
        if idx_q.shape != idx_k.shape or min(idx_q.shape) <= 0 or idx_q.device != idx_k.device:
            raise ValueError("nonempty matching label shapes/devices required")
        if idx_q.device.type != "cpu" and idx_q.device != self.device:
            raise ValueError("labels must be CPU or on the engine CUDA device")
        b, h, n = idx_q.shape
        if b * h * n > 2**31 - 1:
            raise ValueError("flattened row count exceeds int32")
        if reset is not None and (reset.shape != idx_q.shape or reset.dtype != torch.bool or
                                  reset.device != idx_q.device):
            raise ValueError("reset must be bool [B,H,N] on the label device")
        return PreparedHardPrefill(self, idx_q, idx_k, tau, reset)

    def __call__(self, idx_q, idx_k, sq, sk, value, tau, *, reset=None):
        return self.prepare(idx_q, idx_k, tau, reset=reset).execute_dispatch(sq, sk, value)

    def close(self):
        pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class HardDismDecoder:
    """Incremental hard decoder (reference api.py:11-105): ``append`` returns FP32 [B,n,H,DV],
    each new token including its current key; ``prime`` loads a complete prompt history
    (keys only).  ``label_slots`` (power of two >= 64) sizes each row's label table -- at
    least twice the distinct key labels a row will see; the error flag is checked after each
    call.  ``planner_backend`` 'cpu'/'gpu' and the reference's tuning knobs are accepted and
    validated; both backends run the same device decoder."""

    def __init__(self, batch, heads, readout_dim, value_dim, capacity, tau, *, device="cuda",
                 cache_dtype=torch.bfloat16, planner_backend="cpu", summary_backend="native",
                 summary_workspace=None, label_slots=1024, check_errors=True, **tuning):
        self.batch, self.heads, self.r, self.dv = batch, heads, readout_dim, value_dim
        self.capacity, self.position = capacity, 0
        self.dtype = cache_dtype
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        if planner_backend not in ("cpu", "gpu"):
            raise ValueError("planner_backend must be cpu or gpu")
        if summary_backend not in ("native", "persistent") or \
                (summary_backend == "persistent" and planner_backend != "gpu"):
            raise ValueError("persistent summary requires GPU planner")
        if summary_workspace is not None and summary_backend != "persistent":
            raise ValueError("summary workspace requires persistent backend")
        if cache_dtype not in DTYPE_CODE:
            raise ValueError("cache_dtype must be bf16 or fp32")
        if label_slots < 64 or label_slots & (label_slots - 1):
            raise ValueError("label_slots must be a power of two >= 64")
        self.planner_backend, self.summary_backend = planner_backend, summary_backend
        self.tuning = tuning
        self.slots = label_slots
        self.check_errors = check_errors
        self.tau = _tau_tensor(tau, heads, self.device)
        if not bool(torch.isfinite(self.tau).all()) or bool((self.tau < 0).any()):
            raise ValueError("tau must be finite and nonnegative for decoding")
        self.lut = _padded_lut(self.tau, capacity)
        self.rows = batch * heads
        self._code = DTYPE_CODE[cache_dtype]
        nbytes = _lib.size("dism_decoder_state_bytes", self.rows, readout_dim, value_dim,
                           capacity, label_slots, self._code)
        self.state = torch.empty((nbytes,), dtype=torch.uint8, device=self.device)
        with torch.cuda.device(self.device):
            _lib.call("dism_decoder_init", self.state.data_ptr(), nbytes, self.rows,
                      readout_dim, value_dim, capacity, label_slots, self._code,
                      _stream(self.device))

    def _prepare(self, idx_q, idx_k, sk, v, reset):
        if sk.ndim != 4 or sk.shape[0] != self.batch or sk.shape[2:] != (self.heads, self.r):
            raise ValueError("sk must be [B,N,H,R]")
        n = sk.shape[1]
        if n + self.position > self.capacity:
            raise ValueError("cache capacity exceeded")
        if n <= 0 or v.shape != (self.batch, n, self.heads, self.dv):
            raise ValueError("v shape")
        for label in (idx_q, idx_k):
            if label.shape != (self.batch, self.heads, n) or label.dtype != torch.int32:
                raise ValueError("labels must be int32 [B,H,N]; convert bounded vocabulary "
                                 "argmax explicitly")
        if reset is not None and (reset.shape != idx_q.shape or reset.dtype != torch.bool):
            raise ValueError("reset must be bool [B,H,N]")
        if any(x.device != self.device for x in (idx_q, idx_k, sk, v)) or \
                (reset is not None and reset.device != self.device):
            raise ValueError("device changed")
        if sk.dtype != self.dtype or v.dtype != self.dtype:
            raise ValueError("cache payload dtype changed")
        rs = None if reset is None else reset.to(torch.uint8).contiguous()
        return n, idx_q.contiguous(), idx_k.contiguous(), rs

    def _step(self, n, iq, ik, rs, sq, sk, v, out, lse2):
        ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
        with torch.cuda.device(self.device):
            _lib.call("dism_decoder_step", self.state.data_ptr(), self.state.numel(), self.batch,
                      self.heads, self.r, self.dv, self.capacity, self.slots, self._code, n,
                      iq.data_ptr(), ik.data_ptr(), ptr(rs), ptr(sq), sk.data_ptr(),
                      v.data_ptr(), self.lut.data_ptr(), self.lut.shape[1], ptr(out), ptr(lse2),
                      _stream(self.device))
        self.position += n
        if self.check_errors:
            self._check()

    def _check(self):
        meta = self.state[:self.rows * 16].view(torch.int32).view(self.rows, 4)
        if bool(meta[:, 3].any()):
            raise RuntimeError("decoder label table overflow: raise label_slots")

    @torch.no_grad()
    def append(self, idx_q, idx_k, sq, sk, v, *, reset=None):
        """Return FP32 [B,N,H,DV].  Each new token includes its current key.  reset=True
        starts the query's match afresh at that token, without deleting stored keys."""
        if sq.shape != sk.shape or sq.device != self.device or sq.dtype != self.dtype:
            raise ValueError("sq must match sk shape/device/dtype")
        n, iq, ik, rs = self._prepare(idx_q, idx_k, sk, v, reset)
        out = torch.empty((self.batch, n, self.heads, self.dv), dtype=torch.float32,
                          device=self.device)
        self._step(n, iq, ik, rs, sq.contiguous(), sk.contiguous(), v.contiguous(), out, None)
        return out

    @torch.no_grad()
    def prime(self, idx_q, idx_k, sk, v, *, reset=None, serial=False):
        """Initialize from a complete prefill history; compute outputs separately.  The state
        is built in parallel over (row, label) (dism_decoder_prime); serial=True appends the
        prompt's keys one token at a time instead (the same state, for tests)."""
        if self.position:
            raise ValueError("prime requires empty cache")
        n, iq, ik, rs = self._prepare(idx_q, idx_k, sk, v, reset)
        if serial:
            self._step(n, iq, ik, rs, None, sk.contiguous(), v.contiguous(), None, None)
            return
        sk, v = sk.contiguous(), v.contiguous()
        nbytes = _lib.size("dism_decoder_prime_workspace_bytes", self.batch, n, self.heads,
                           self.r, self.dv, self._code)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=self.device)
        with torch.cuda.device(self.device):
            _lib.call("dism_decoder_prime", self.state.data_ptr(), self.state.numel(),
                      self.batch, self.heads, self.r, self.dv, self.capacity, self.slots,
                      self._code, n, iq.data_ptr(), ik.data_ptr(),
                      0 if rs is None else rs.data_ptr(), sk.data_ptr(), v.data_ptr(),
                      ws.data_ptr(), nbytes, _stream(self.device))
        self.position += n
        if self.check_errors:
            self._check()

    def memory_stats(self):
        meta = self.state[:self.rows * 16].view(torch.int32).view(self.rows, 4).cpu()
        return dict(position=self.position, capacity=self.capacity,
                    state_bytes=self.state.numel(), label_slots=self.slots,
                    list_blocks_used=int(meta[:, 1].sum()),
                    planner_backend=self.planner_backend)
