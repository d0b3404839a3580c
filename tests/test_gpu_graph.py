"""The hard core's launches captured into a HIP graph (torch.cuda.CUDAGraph): one forward +
backward step through the C ABI with fixed buffers -- label binarizer, log-weight tables,
dism_hard_forward (its side-stream fork and join inside the capture), the backward entry
points with the key chain on a side stream, the tau reduction -- replayed several times with
the program's own eager work and synchronizations between the replays.  Every replay must
reproduce the eager step bit for bit (no launch of the path records a memset node; a node
that misbehaves on replays after the first would show here).  Row kinds: level rows (alphabet
4), sparse rows (8-bit labels), prefix rows (identical labels), dense tile rows (long runs of
one label with two predecessors)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


class Step:
    def __init__(self, B, T, H, D, DV, pattern, seed):
        import dism_amd
        from dism_amd import _lib
        from dism_amd._checks import DTYPE_CODE
        self.dism_amd, self._lib = dism_amd, _lib
        dev = torch.device("cuda:0")
        g = torch.Generator(device="cpu").manual_seed(seed)
        q = torch.randn(B, T, H, D, generator=g)
        k = torch.randn(B, T, H, D, generator=g)
        if pattern in ("equal", "direct"):
            q = q.abs()
            k = k.abs()
        if pattern == "direct":  # label 255 with two predecessors: a direct dense row
            q[:, ::97, :, 0] *= -1
            k[:, ::89, :, 0] *= -1
        self.tq = q.to(dev, torch.bfloat16).contiguous()
        self.tk = k.to(dev, torch.bfloat16).contiguous()
        self.tv = torch.randn(B, T, H, DV, generator=g).to(dev, torch.bfloat16).contiguous()
        self.tdo = torch.randn(B, T, H, DV, generator=g).to(dev, torch.bfloat16).contiguous()
        self.tau = torch.linspace(-0.4, 0.6, H, device=dev)
        self.hard = torch.ones((B, H), dtype=torch.bool, device=dev)
        self.dims = (B, T, H, D, DV)
        self.code = DTYPE_CODE[torch.bfloat16]
        self.nbytes = _lib.workspace_bytes(B, T, H, D, DV, self.code)
        self.ws = torch.empty((self.nbytes,), dtype=torch.uint8, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.out = torch.empty((B, T, H, DV), **f32)
        self.lse2 = torch.empty((B, H, T), **f32)
        self.dsq = torch.empty((B, T, H, D), **f32)
        self.dsk = torch.empty_like(self.dsq)
        self.dv = torch.empty((B, T, H, DV), **f32)
        self.rowtau = torch.empty((B, H, T), **f32)
        self.dtau = torch.empty((H,), **f32)
        self.side = torch.cuda.Stream(device=dev)
        self.fork, self.join = torch.cuda.Event(), torch.cuda.Event()

    def __call__(self):
        d, L = self.dism_amd, self._lib
        B, T, H, D, DV = self.dims
        stream = torch.cuda.current_stream()
        S = stream.cuda_stream
        iq, ik = d.sign_labels(self.tq), d.sign_labels(self.tk)
        lut = d.hard_log_weights(self.tau, T)
        dlut = d.hard_dlog_weights(self.tau, T + 1)
        vec = (self.tq.data_ptr(), self.tk.data_ptr(), self.tv.data_ptr())
        W, nb, c = self.ws.data_ptr(), self.nbytes, self.code
        base = (iq.data_ptr(), ik.data_ptr(), self.hard.data_ptr(), 0, 0, lut.data_ptr())
        L.call("dism_hard_forward", *vec, c, *base, T + 1, B, T, H, D, DV, W, nb,
               self.out.data_ptr(), 1, self.lse2.data_ptr(), 0, 0, S)
        bw = (*vec, self.tdo.data_ptr(), c, *base)
        self.fork.record(stream)
        L.call("dism_hard_backward_row_pairs", *bw, dlut.data_ptr(), T + 1, self.lse2.data_ptr(),
               B, T, H, D, DV, W, nb, S)
        self.side.wait_event(self.fork)
        ks = self.side.cuda_stream
        L.call("dism_hard_backward_keys", *bw, T + 1, self.lse2.data_ptr(), B, T, H, D, DV, W,
               nb, self.dsk.data_ptr(), self.dv.data_ptr(), ks)
        L.call("dism_hard_backward_key_pairs", *bw, T + 1, self.lse2.data_ptr(), B, T, H, D, DV,
               W, nb, self.dsk.data_ptr(), self.dv.data_ptr(), ks)
        L.call("dism_hard_backward_queries", *bw, dlut.data_ptr(), T + 1, self.lse2.data_ptr(),
               B, T, H, D, DV, W, nb, self.dsq.data_ptr(), self.rowtau.data_ptr(), S)
        L.call("dism_hard_tau_reduce", self.rowtau.data_ptr(), B, H, T, self.dtau.data_ptr(), S)
        self.join.record(self.side)
        stream.wait_event(self.join)

    def results(self):
        return [t.detach().cpu().numpy().copy() for t in
                (self.out, self.lse2, self.dsq, self.dsk, self.dv, self.rowtau, self.dtau)]

    def clear(self):
        for t in (self.out, self.lse2, self.dsq, self.dsk, self.dv, self.rowtau, self.dtau):
            t.fill_(-7.0)


@pytest.mark.parametrize("shape", [(2, 512, 4, 2, 64, "level"), (1, 1024, 4, 8, 64, "sparse"),
                                   (1, 512, 2, 8, 64, "equal"), (1, 512, 2, 8, 64, "direct")])
def test_graph_replays_match_eager(shape):
    *dims, pattern = shape
    print(f"graph replay {shape}", flush=True)
    st = Step(*dims, pattern, seed=11)
    other = Step(*dims, pattern, seed=12)  # eager work between the replays
    st()
    torch.cuda.synchronize()
    want = st.results()
    modes = st.dism_amd.hard_forward.row_modes(st.ws, st.tq, st.tv).cpu().numpy()
    expect = {"level": 3, "sparse": 0, "equal": 4, "direct": 1}[pattern]
    assert (modes == expect).all(), modes
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        st()
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=cs):
        st()
    for rep in range(3):
        st.clear()
        other()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, exp, name in zip(st.results(), want,
                                  ("out", "lse2", "dsq", "dsk", "dv", "rowtau", "dtau")):
            assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (rep, name)
