"""Fixed-capacity graph layouts on the MI355X (reference dism_v3/src/host/graph_layout.h,
varlen.py:28-36, nanochat/nanochat/cuda_graph.py:105-181): one packed forward + backward
captured into a HIP graph (torch.cuda.CUDAGraph) over a graph layout of 2048 tokens; between
replays update_graph_layout rewrites the documents in place and new inputs are copied into
the captured buffers.  Every replay must equal the CPU model's per-document results for that
pack bit for bit.  The library receives tokens / 256 = 8 document slots (padding slots repeat
`tokens`), so the model classifies the rows with that tag multiplier."""
import numpy as np
import pytest
import torch

from tests.test_gpu_packed import HARD, _expected, _inputs
from tests.test_gpu_parity import assert_bits, dev, host

pytestmark = pytest.mark.gpu

N, MAX = 2048, 1024
PACKS = [([0, 0, 256, 512, 1024, 1024, 2048], "random"),
         ([0, 1024, 1280, 2048], "periodic"),
         ([0, 256, 512, 768, 1024, 1280, 1536, 1792, 2048], "alphabet4")]


class _Step:
    """Static buffers and one packed forward + backward on them."""

    def __init__(self, layout):
        self.layout = layout
        self.t = None

    def load(self, x):
        sq, sk, v, do, q, k, tau = x
        new = [dev(a, torch.bfloat16) for a in (sq, sk, v, do)] + [dev(q), dev(k), dev(HARD),
                                                                   dev(tau)]
        if self.t is None:
            self.t = new
        else:
            for dst, src in zip(self.t, new):
                dst.copy_(src)

    def __call__(self):
        import dism_amd
        sq, sk, v, do, iq, ik, th, tt = self.t
        out, lse2, state, m = dism_amd.forward_hard(sq, sk, v, iq, ik, th, tt,
                                                    layout=self.layout, save_state=True,
                                                    return_matches=True,
                                                    out_dtype=torch.float32)
        grads = dism_amd.backward_hard(sq, sk, v, do, iq, ik, th, lse2, state,
                                       layout=self.layout)
        self.res = (out, lse2, m["length"], m["index"]) + tuple(grads)


def _check(res, x, offsets, tag):
    o, l2, lm, ja, g, dtau = _expected(x, offsets, HARD, slots=N // 256)
    for got, want, name in zip(res, (o, l2, lm, ja) + tuple(g) + (dtau,),
                               ("out", "lse2", "lmax", "argmax", "dsq", "dsk", "dv", "dtau")):
        assert_bits(host(got), want, f"{tag} {name}")


def test_graph_layout_replays_follow_updates():
    import dism_amd
    offsets, pattern = PACKS[0]
    table = dism_amd.make_graph_layout(torch.tensor(offsets, dtype=torch.int32), N, MAX, MAX)
    layout = dism_amd.VarlenLayout.for_graph(table, N)
    st = _Step(layout)
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        x = _inputs(N, pattern)
        st.load(x)
        print(f"graph layout eager step offsets={offsets} pattern={pattern}", flush=True)
        st()   # stages the layout's device offsets on cs, outside capture
    torch.cuda.synchronize()
    _check(st.res, x, offsets, "eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        st()
    for rep, (offsets, pattern) in enumerate(PACKS * 2):
        x = _inputs(N, pattern, seed=rep)
        with torch.cuda.stream(cs):
            dism_amd.update_graph_layout(table, torch.tensor(offsets, dtype=torch.int32))
            st.load(x)
            print(f"graph layout replay {rep} offsets={offsets} pattern={pattern}", flush=True)
            g.replay()
        torch.cuda.synchronize()
        _check(st.res, x, offsets, f"replay {rep}")
        # the program's own eager work between replays
        torch.randn(1 << 16, device="cuda").sum().item()
    # updates from a stream other than the owning one are refused
    with pytest.raises(RuntimeError, match="owning stream"):
        dism_amd.update_graph_layout(table, torch.tensor(PACKS[1][0], dtype=torch.int32))
    g.reset()


def test_graph_layout_matches_packed_layout_per_document():
    """A graph layout and an ordinary packed layout of the same pack give the CPU model's
    results, each with its own tag multiplier (8 slots vs the non-empty documents)."""
    import dism_amd
    offsets, pattern = PACKS[2]
    x = _inputs(N, pattern, seed=7)
    table = dism_amd.make_graph_layout(torch.tensor(offsets, dtype=torch.int32), N, MAX, MAX)
    for layout, slots in ((dism_amd.VarlenLayout.for_graph(table, N), N // 256),
                          (dism_amd.VarlenLayout.from_cu_seqlens(
                              torch.tensor(offsets, dtype=torch.int32), N), None)):
        st = _Step(layout)
        st.load(x)
        print(f"graph vs packed layout slots={slots}", flush=True)
        st()
        torch.cuda.synchronize()
        o, l2, lm, ja, g, dtau = _expected(x, offsets, HARD, slots=slots)
        assert_bits(host(st.res[0]), o, f"out slots={slots}")
        assert_bits(host(st.res[5]), g[1], f"dsk slots={slots}")
        assert_bits(host(st.res[7]), dtau, f"dtau slots={slots}")
