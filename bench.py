"""Benchmark: flash_dism hard core on one MI355X (BASELINE.json metric).

Default (the line the driver records): BASELINE.json configs[2] -- B=4, H=16, T=16384,
d_qk=8, d_v=64, bf16, periodic component on 25% of the heads, forward + backward.  A step is
one training pass of the hard DISM op over one synthetic batch:
    labels (sign binarizer, q and k) -> log2 weight table -> forward (dism_hard_forward:
    dense-row classification and position orders, the bigram half of the prepare on a side
    stream overlapping the length-1 label scan, the pair corrections, the dense rows) -> dlog
    table -> row pairs -> query-row scan / dense rows (dSQ, tau terms) -> tau reduction, with
    the key scan / dense keys (dV, dSK) -> key pairs chain on a side stream (--streams 2, the
    default; joined each step).
`--config K` measures BASELINE.json configs[K] instead (0: forward only, fp32, B1 H4 T256;
1: low-entropy d_qk=2 fwd+bwd; 3: one T=65536 sequence with copied spans, forward only;
4: the nanochat-shaped layer, projections + op forward and backward).  Inputs are resident in
HBM before timing.  Prints ONE JSON line.  The timed region records events only around the
roofline candidates' stages (`roofline` uses the dominant one's live duration); `kernel_ms`
comes from a separate instrumented pass with events around every stage (under --streams 2 the
overlapping stages' times include their contention).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12             # bytes/s
FP32_PEAK = 157.3e12          # flop/s, MI355X fp32 (vector)
METRIC = "DISM fwd+bwd tokens/sec (B*H*T/s) at T=16k, 1 GPU"

# BASELINE.json configs (generators as BASELINE.md section 2: seeds 20261201 + index, labels
# by the sign binarizer, sq = q, sk = k, every row hard)
CONFIGS = {
    0: dict(B=1, H=4, T=256, dqk=8, dv=64, dtype="f32", fwd_only=True, gen="plain",
            workload="BASELINE configs[0]: CPU reference path case, forward only, fp32"),
    1: dict(B=2, H=8, T=2048, dqk=2, dv=64, dtype="bf16", fwd_only=False, gen="plain",
            workload="BASELINE configs[1]: low-entropy (d_qk=2, alphabet 4) fwd+bwd"),
    2: dict(B=4, H=16, T=16384, dqk=8, dv=64, dtype="bf16", fwd_only=False, gen="periodic",
            workload="BASELINE configs[2]: hard DISM fwd+bwd, periodic heads"),
    3: dict(B=1, H=16, T=65536, dqk=8, dv=128, dtype="bf16", fwd_only=True, gen="copied",
            workload="BASELINE configs[3]: long single sequence, copied spans, forward only"),
    4: dict(B=8, H=10, T=2048, dqk=8, dv=128, dtype="bf16", fwd_only=False, gen="layer",
            workload="BASELINE configs[4]: nanochat-shaped DISM layer fwd+bwd (d_model 1280)"),
}


def make_inputs(B, T, H, dqk, dv, seed, periodic=True):
    """BASELINE config 3 generator: q, k ~ N(0,1); heads h % 4 == 0 get 2*P[t mod 97] added to
    both q and k (P ~ N(0,1) [97, d_qk] per head); v, dO ~ N(0,1); all rounded to bf16."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, H, dqk), dtype=np.float32)
    k = rng.standard_normal((B, T, H, dqk), dtype=np.float32)
    if periodic:
        for h in range(0, H, 4):
            p = rng.standard_normal((97, dqk), dtype=np.float32)
            rep = p[np.arange(T) % 97]
            q[:, :, h] += 2 * rep
            k[:, :, h] += 2 * rep
    v = rng.standard_normal((B, T, H, dv), dtype=np.float32)
    do = rng.standard_normal((B, T, H, dv), dtype=np.float32)
    return q, k, v, do


def config_inputs(idx):
    """q, k, v, dO float32 arrays of configs[idx] (not rounded)."""
    c = CONFIGS[idx]
    B, T, H, D, DV = c["B"], c["T"], c["H"], c["dqk"], c["dv"]
    seed = 20261201 + idx
    if c["gen"] == "periodic":
        return make_inputs(B, T, H, D, DV, seed)
    if c["gen"] == "layer":  # the core's inputs inside the layer: bf16 projections of x
        import torch
        rnd = lambda a: torch.from_numpy(a).bfloat16().float().numpy()  # noqa: E731
        x, wq, wk, wv, _, do, _ = layer_arrays()
        xb = rnd(x)
        proj = lambda w, d: (xb @ rnd(w)).reshape(B, T, H, d)  # noqa: E731
        return proj(wq, D), proj(wk, D), proj(wv, DV), do
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, H, D), dtype=np.float32)
    k = rng.standard_normal((B, T, H, D), dtype=np.float32)
    if c["gen"] == "copied":
        from tests._data import copied_spans
        copied_spans(q, k)
    v = rng.standard_normal((B, T, H, DV), dtype=np.float32)
    do = rng.standard_normal((B, T, H, DV), dtype=np.float32)
    return q, k, v, do


def valid_pairs(iq, ik):
    """Causal equal-label pairs (j <= i, iq[i] == ik[j]) per (b,h) row, int64 [B*H]."""
    B, H, N = iq.shape
    out = np.zeros(B * H, np.int64)
    for r in range(B * H):
        q, k = iq.reshape(-1, N)[r], ik.reshape(-1, N)[r]
        # per label: for each query, #keys with the label at positions <= i
        order = np.lexsort((np.r_[np.zeros(N, np.int8), np.ones(N, np.int8)],
                            np.r_[np.arange(N), np.arange(N)], np.r_[k, q]))
        lab = np.r_[k, q][order]
        isq = np.r_[np.zeros(N, bool), np.ones(N, bool)][order]
        starts = np.r_[True, lab[1:] != lab[:-1]]
        keys_before = np.cumsum(~isq)
        grp_base = np.maximum.accumulate(np.where(starts, np.arange(2 * N), 0))
        base_keys = np.where(grp_base > 0, keys_before[grp_base - 1], 0)
        out[r] = int((keys_before - base_keys)[isq].sum())
    return out


def causal_counts(qc, kc):
    """Per position of one row: #keys j <= i with kc[j] == qc[i] (query side) and #queries
    i >= j with qc[i] == kc[j] (key side), int64 [N] each."""
    N = qc.shape[0]
    side = np.r_[np.zeros(N, np.int8), np.ones(N, np.int8)]
    pos = np.r_[np.arange(N), np.arange(N)]
    order = np.lexsort((side, pos, np.r_[kc, qc]))
    lab = np.r_[kc, qc][order]
    isq = side[order] == 1
    starts = np.r_[True, lab[1:] != lab[:-1]]
    gid = np.cumsum(starts) - 1
    keys_before = np.cumsum(~isq)
    qs_before = np.cumsum(isq)
    first = np.flatnonzero(starts)
    gk0 = np.where(first > 0, keys_before[first - 1], 0)[gid]
    gq0 = np.where(first > 0, qs_before[first - 1], 0)[gid]
    gq_tot = np.add.reduceat(isq.astype(np.int64), first)[gid]
    qcount = np.zeros(N, np.int64)
    kcount = np.zeros(N, np.int64)
    qcount[pos[order][isq]] = (keys_before - gk0)[isq]
    # queries at positions >= j: the group's queries not counted before the key
    kcount[pos[order][~isq]] = (gq_tot - (qs_before - gq0))[~isq]
    return qcount, kcount


def bigram_pair_counts(iq, ik):
    """Bigram pairs (L >= 2: iq[i] == ik[j] and iq[i-1] == ik[j-1], 1 <= j <= i) over all
    rows: (pairs, query owners with a pair, key owners with a pair)."""
    B, H, N = iq.shape
    pairs = qown = kown = 0
    for r in range(B * H):
        q = iq.reshape(-1, N)[r].astype(np.int64)
        k = ik.reshape(-1, N)[r].astype(np.int64)
        # positions >= 1 carry the bigram (label[p-1], label[p]); a key at 0 has none
        qc = (q[:-1] << 32) | (q[1:] & 0xFFFFFFFF)
        kc = (k[:-1] << 32) | (k[1:] & 0xFFFFFFFF)
        qn, kn = causal_counts(qc, kc)
        pairs += int(qn.sum())
        qown += int((qn > 0).sum())
        kown += int((kn > 0).sum())
    return pairs, qown, kown


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS),
                    help="BASELINE.json configs[K] (default 2, the headline metric)")
    ap.add_argument("--tau", type=float, default=0.5)
    ap.add_argument("--carry-strip", type=int, default=0,
                    help="composed carry boundary strip height (0 = off)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--workload", default="train",
                    choices=("train", "decode", "vocab", "refshape"),
                    help="train: the BASELINE metric (default); decode: prefill + token-by-token "
                         "decoding at the nanochat layer shape; vocab: codebook argmax labels; "
                         "refshape: the reference's own benchmark shape (B16 H6 N2048 R32 DV64, "
                         "random-512 and identical labels, forward and backward timed apart)")
    ap.add_argument("--graph", type=int, default=1, choices=(0, 1),
                    help="1: time the step as a captured HIP graph (replayed --steps times); "
                         "the eager step's time is reported beside it")
    ap.add_argument("--streams", type=int, default=2, choices=(1, 2),
                    help="2: the backward's key chain runs concurrently on a side stream")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run 5 device-to-device copies of BYTES bytes (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (single-GPU boxes); "
              "--gpus > 1 is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        src = torch.empty(args.calibrate_copy, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": args.calibrate_copy}), flush=True)
        return
    if args.workload == "decode":
        return bench_decode(args)
    if args.workload == "vocab":
        return bench_vocab(args)
    if args.workload == "refshape":
        return bench_refshape(args)
    return bench_train(args)


def bench_train(args):
    import torch
    import dism_amd
    from dism_amd import _lib
    from dism_amd._checks import DTYPE_CODE
    from dism_amd.hard_forward import row_modes
    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    B, T, H, D, DV = cfg["B"], cfg["T"], cfg["H"], cfg["dqk"], cfg["dv"]
    fwd_only = cfg["fwd_only"]
    vdt = torch.float32 if cfg["dtype"] == "f32" else torch.bfloat16
    q, k, v, do = config_inputs(args.config)
    put = lambda a: torch.from_numpy(a).to(dev).to(vdt).contiguous()  # noqa: E731
    tq, tk, tv, tdo = put(q), put(k), put(v), put(do)
    tau = torch.full((H,), args.tau, dtype=torch.float32, device=dev)
    hard = torch.ones((B, H), dtype=torch.bool, device=dev)
    stream = torch.cuda.current_stream(dev)
    S = stream.cuda_stream
    strip = args.carry_strip
    n = T
    dsq = torch.empty((B, T, H, D), dtype=torch.float32, device=dev)
    dsk = torch.empty_like(dsq)
    dvv = torch.empty((B, T, H, DV), dtype=torch.float32, device=dev)
    rowtau = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    dtau = torch.empty((H,), dtype=torch.float32, device=dev)
    fused = args.streams == 2
    names = ["labels", "lut", "carry"] + (["forward"] if fused else ["prepare", "readout"])
    if not fwd_only:
        names += ["dlut", "row_pairs", "queries", "keys", "key_pairs", "tau_reduce"]
    side = torch.cuda.Stream(device=dev) if fused and not fwd_only else None
    fork, join = torch.cuda.Event(), torch.cuda.Event()
    out = torch.empty((B, T, H, DV), dtype=vdt, device=dev)
    lse2 = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    code = DTYPE_CODE[vdt]
    nbytes = _lib.workspace_bytes(B, T, H, D, DV, code)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    W = ws.data_ptr()
    hp = hard.data_ptr()

    def step(events=None):
        """One pass.  events: {stage: (start, end)} recorded on the stage's stream.  Runs on the
        current stream (a graph capture's stream while capturing)."""
        stream = torch.cuda.current_stream(dev)
        S = stream.cuda_stream

        def mark(name, which, strm=None):
            if events is not None and name in events:
                events[name][which].record(strm if strm is not None else stream)
        mark("labels", 0)
        iq = dism_amd.sign_labels(tq)
        ik = dism_amd.sign_labels(tk)
        qp, kp = iq.data_ptr(), ik.data_ptr()
        mark("labels", 1)
        mark("lut", 0)
        lut = dism_amd.hard_log_weights(tau, n)
        mark("lut", 1)
        mark("carry", 0)
        carry = dism_amd.hard_boundary(iq, ik, hard, strip=strip, fill_all=False) \
            if strip > 0 else None
        cp = 0 if carry is None else carry.data_ptr()
        mark("carry", 1)
        vec = (tq.data_ptr(), tk.data_ptr(), tv.data_ptr())
        rd = (*vec, code, qp, kp, hp, cp, strip, lut.data_ptr(), n + 1, B, T, H, D, DV, W,
              nbytes, out.data_ptr(), code, lse2.data_ptr(), 0, 0, S)
        if fused:
            mark("forward", 0)
            _lib.call("dism_hard_forward", *rd)
            mark("forward", 1)
        else:
            mark("prepare", 0)
            _lib.call("dism_hard_prepare", *vec, code, qp, kp, B, T, H, D, DV, W, nbytes, S)
            mark("prepare", 1)
            mark("readout", 0)
            _lib.call("dism_hard_readout", *rd)
            mark("readout", 1)
        if fwd_only:
            return out, iq, ik
        bw = (*vec, tdo.data_ptr(), code, qp, kp, hp, cp, strip, lut.data_ptr())
        if side is not None:
            fork.record(stream)  # the forward's outputs are ready
        mark("dlut", 0)
        dlut = dism_amd.hard_dlog_weights(tau, n + 1)
        mark("dlut", 1)
        mark("row_pairs", 0)
        _lib.call("dism_hard_backward_row_pairs", *bw, dlut.data_ptr(), n + 1, lse2.data_ptr(),
                  B, T, H, D, DV, W, nbytes, S)
        mark("row_pairs", 1)
        # the key chain (keys -> key pairs) does not depend on the query-row chain (row pairs
        # -> queries -> tau): with --streams 2 it runs on a side stream (default priority),
        # enqueued after the row pairs so that their persistent grid starts first
        ks = stream
        if side is not None:
            side.wait_event(fork)
            ks = side
        mark("keys", 0, ks)
        _lib.call("dism_hard_backward_keys", *bw, n + 1, lse2.data_ptr(), B, T, H, D, DV, W,
                  nbytes, dsk.data_ptr(), dvv.data_ptr(), ks.cuda_stream)
        mark("keys", 1, ks)
        mark("key_pairs", 0, ks)
        _lib.call("dism_hard_backward_key_pairs", *bw, n + 1, lse2.data_ptr(), B, T, H, D, DV,
                  W, nbytes, dsk.data_ptr(), dvv.data_ptr(), ks.cuda_stream)
        mark("key_pairs", 1, ks)
        mark("queries", 0)
        _lib.call("dism_hard_backward_queries", *bw, dlut.data_ptr(), n + 1, lse2.data_ptr(),
                  B, T, H, D, DV, W, nbytes, dsq.data_ptr(), rowtau.data_ptr(), S)
        mark("queries", 1)
        mark("tau_reduce", 0)
        _lib.call("dism_hard_tau_reduce", rowtau.data_ptr(), B, H, T, dtau.data_ptr(), S)
        mark("tau_reduce", 1)
        if side is not None:
            join.record(side)
            stream.wait_event(join)
        return out, iq, ik

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _, iq_t, ik_t = step()
    torch.cuda.synchronize()
    modes = row_modes(ws, tq, tv).cpu().numpy()
    dense_rows = int((modes == 1).sum())
    level_rows = int((modes == 3).sum())

    def stage_events(only=None):
        return {nm: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for nm in names if only is None or nm in only}
    # roofline candidates: the label scans of the backward (HBM), the dense-row kernels
    # (fp32 VALU: forward, queries, keys) and, forward-only, the forward
    if fwd_only:
        cand = ("forward",) if fused else ("readout",)
    elif dense_rows:
        cand = ("forward", "queries", "keys", "row_pairs", "key_pairs")
    else:
        cand = ("queries", "keys", "row_pairs", "key_pairs")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    live = [stage_events(cand) for _ in range(args.steps)]
    t0 = time.perf_counter()
    start.record(stream)
    for s in range(args.steps):
        step(live[s])
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(end)
    ms_step = gpu_ms / args.steps
    live_ms = {nm: float(np.mean([live[s][nm][0].elapsed_time(live[s][nm][1])
                                  for s in range(args.steps)])) for nm in cand}
    per = [stage_events() for _ in range(args.steps)]
    for s in range(args.steps):
        step(per[s])
    torch.cuda.synchronize()
    kern_ms = {nm: float(np.mean([per[s][nm][0].elapsed_time(per[s][nm][1])
                                  for s in range(args.steps)])) for nm in names}
    eager_ms = ms_step
    graph_ms = None
    if args.graph:
        # the same step captured once into a HIP graph (every launch, the side-stream fork and
        # join included) and replayed: the small configs' steps are bounded by the host's
        # launch rate otherwise.  Inputs, workspace and outputs are the same buffers.
        g = torch.cuda.CUDAGraph()
        cs = torch.cuda.Stream(device=dev)
        cs.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(cs):
            step()
        torch.cuda.current_stream(dev).wait_stream(cs)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=cs):
            step()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        gs, ge = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gs.record()
        for _ in range(args.steps):
            g.replay()
        ge.record()
        torch.cuda.synchronize()
        graph_ms = gs.elapsed_time(ge) / args.steps
        ms_step = graph_ms
    units = B * H * T
    value = units / (ms_step / 1e3)
    esz = 4 if vdt == torch.float32 else 2
    order = 16  # combined-order entry and label of the unit's key and query (4 x 4 B)
    dom = max(cand, key=lambda x: live_ms[x])
    if level_rows and not dense_rows:
        # level rows: a chain of short launches (prepare lists, segment totals, walks,
        # combines); the bound is the whole step's HBM traffic at its minimum -- every input
        # read once, every output written once per (b,h,t) unit
        fwd_b = 2 * D * esz + 2 * DV * esz + 4
        bwd_b = 2 * D * esz + 2 * DV * esz + 4 + 8 * D + 4 * DV + 4
        per_unit = fwd_b + (0 if fwd_only else bwd_b)
        alg_bytes = per_unit * units
        achieved = alg_bytes / (ms_step / 1e3)
        roof = {"kernel": "whole step (level rows: all kernels)", "bound": "hbm",
                "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": achieved / HBM_PEAK, "traffic": None, "alg_bytes_per_unit": per_unit,
                "launch_ms": ms_step}
    elif dense_rows and dom in ("forward", "queries", "keys"):
        # fp32 FMAs of the direct definition per valid pair: forward s, acc (R + DV); query rows
        # s, e, dq (2R + DV); keys s, e, dk, dv (2R + 2DV); over the dense rows' valid pairs
        pairs = valid_pairs(iq_t.cpu().numpy(), ik_t.cpu().numpy())
        vp = float(pairs[(modes.reshape(-1) == 1)].sum())
        fma = {"forward": D + DV, "queries": 2 * D + DV, "keys": 2 * D + 2 * DV}[dom]
        flops = 2.0 * fma * vp
        kern = {"forward": "dense_forward_kernel", "queries": "dense_rows_kernel",
                "keys": "dense_keys_kernel"}[dom]
        achieved = flops / (live_ms[dom] / 1e3)
        roof = {"kernel": kern, "bound": "valu", "achieved": achieved / 1e12,
                "peak": FP32_PEAK / 1e12, "unit": "TFLOP/s", "frac": achieved / FP32_PEAK,
                "traffic": None, "alg_flops_per_launch": flops, "valid_pairs": vp,
                "launch_ms": live_ms[dom]}
    elif dom in ("row_pairs", "key_pairs"):
        # bigram-pair corrections: gathers bound by latency, priced at the bytes they must
        # move once -- per owner its record (16 B), its own rows and its result; per pair the
        # partner's rows and two table entries (LUT, dLUT)
        npairs, qown, kown = bigram_pair_counts(iq_t.cpu().numpy(), ik_t.cpu().numpy())
        if dom == "row_pairs":   # owner: sq, dO, lse2, record (R + 4 floats); partner: sk, v
            own_b = 16 + D * esz + DV * esz + 4 + 4 * (D + 4)
            pair_b = D * esz + DV * esz + 8
            owners = qown
            kern = "pairs_rows_kernel"
        else:                    # owner: sk, v, dSK/dV read+write; partner: sq, dO, lse2
            own_b = 16 + D * esz + DV * esz + 8 * (D + DV)
            pair_b = D * esz + DV * esz + 4 + 8
            owners = kown
            kern = "pairs_keys_kernel"
        alg_bytes = owners * own_b + npairs * pair_b
        achieved = alg_bytes / (live_ms[dom] / 1e3)
        roof = {"kernel": kern, "bound": "hbm", "achieved": achieved / 1e9,
                "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": achieved / HBM_PEAK,
                "traffic": measured_traffic(kern) if args.config == 2 else None,
                "alg_bytes_per_launch": alg_bytes, "owners": owners, "bigram_pairs": npairs,
                "owner_bytes": own_b, "pair_bytes": pair_b, "launch_ms": live_ms[dom],
                "stage": dom}
    else:
        # HBM bytes per B*H*T unit that the stage must read and write once
        per_unit = {
            "queries": 2 * D * esz + 2 * DV * esz + 3 * 4 + 4 * D + 4 + order,
            "keys": 2 * D * esz + 2 * DV * esz + 4 + 4 * D + 4 * DV + order,
            "forward": 2 * D * esz + DV * esz + DV * esz + 4 + order,
            "readout": 2 * D * esz + DV * esz + DV * esz + 4 + order,
        }
        kernel_of = {"queries": "scan_rows_kernel", "keys": "scan_keys_kernel",
                     "forward": "dism_hard_forward (all kernels)",
                     "readout": "dism_hard_readout (all kernels)"}
        alg_bytes = per_unit[dom] * units
        achieved = alg_bytes / (live_ms[dom] / 1e3)
        roof = {"kernel": kernel_of[dom], "bound": "hbm", "achieved": achieved / 1e9,
                "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": achieved / HBM_PEAK,
                "traffic": measured_traffic(kernel_of[dom]) if args.config == 2 else None,
                "alg_bytes_per_unit": per_unit[dom], "launch_ms": live_ms[dom]}
    result = {
        "metric": METRIC,
        "value": value,
        "unit": "B*H*T/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "eager_ms_per_step": eager_ms,
        "graph_ms_per_step": graph_ms,
        "wall_ms_per_step_eager": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"fp32 (int32 labels, {cfg['dtype']} vectors)",
        "data": f"synthetic (BASELINE configs[{args.config}] generator, seed "
                f"{20261201 + args.config})",
        "config": {"workload": cfg["workload"], "B": B, "H": H, "T": T, "d_qk": D, "d_v": DV,
                   "tau": args.tau, "carry_strip": strip, "forward_only": fwd_only,
                   "global_batch": B, "seq_len": T, "parallelism": "single-gpu"},
        "row_modes": {str(m): int((modes == m).sum()) for m in (0, 1, 2, 3, 4)},
        "kernel_ms": kern_ms,
        "roofline": roof,
    }
    # BASELINE.json quotes its metric as a fraction of the integer-VALU roofline of the
    # pairwise match recurrence (2 int32 ops -- compare, length update -- per causal pair per
    # pass, two passes), at 256 CUs x 4 SIMD x 16 lanes x 2.4 GHz = 39.3 T int32 ops/s.  For
    # sparse rows this build does not run that recurrence (label scans + bigram corrections
    # are O(N) per row), so this is the time that recurrence would need at peak over the
    # measured step: an algorithmic speed-up figure, not a hardware efficiency.
    pairs = T * (T + 1) / 2
    int_ops = (2 if fwd_only else 4) * pairs * B * H
    int_peak = 256 * 4 * 16 * 2.4e9
    result["pairwise_equiv"] = {"ops": int_ops, "peak_ops_per_s": int_peak,
                                "t_roof_ms": int_ops / int_peak * 1e3,
                                "ratio": (int_ops / int_peak * 1e3) / ms_step,
                                "note": "time of the pairwise int32 recurrence at the VALU "
                                        "peak over the measured step (not a hardware "
                                        "efficiency; see roofline)"}
    if args.config == 2:
        valu = measured_valu(roof["kernel"])
        if valu is not None:  # the label scans are VALU-issue bound: the second ceiling
            insts, peak = valu
            rate = insts / (live_ms[dom] / 1e3)
            result["valu"] = {"kernel": roof["kernel"], "insts_per_launch": insts,
                              "achieved": rate / 1e9, "peak": peak / 1e9,
                              "unit": "G wave64-instr/s", "frac": rate / peak}
    if args.config == 4:
        # the metric's step for configs[4] is the whole layer (projections, the core, the
        # output projection, forward and backward); the core's own step stays beside it
        layer_ms = layer_step_ms(args)
        result["core_ms_per_step"] = ms_step
        result["ms_per_step"] = layer_ms
        result["value"] = units / (layer_ms / 1e3)
        result["config"]["d_model"] = 1280
        result["data"] += " (core inputs: the layer's bf16 projections)"
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(q, k, v, do, cfg, args)
    print(json.dumps(result), flush=True)


def layer_arrays():
    """configs[4] generator (numpy, seed 20261205): x ~ N(0, 0.02) [B, T, 1280]; projections
    wq, wk [1280, H*8], wv [1280, H*128] ~ N(0, 1/1280); the output projection wo [H*128, 1280]
    ~ N(0, 1/(H*128)); the upstream gradient dy ~ N(0, 1) [B, T, 1280]."""
    c = CONFIGS[4]
    B, T, H, D, DV, DM = c["B"], c["T"], c["H"], c["dqk"], c["dv"], 1280
    rng = np.random.default_rng(20261201 + 4)
    x = rng.standard_normal((B, T, DM), dtype=np.float32) * 0.02
    wq, wk = (rng.standard_normal((DM, H * D), dtype=np.float32) / np.sqrt(DM) for _ in range(2))
    wv = rng.standard_normal((DM, H * DV), dtype=np.float32) / np.sqrt(DM)
    do = rng.standard_normal((B, T, H, DV), dtype=np.float32)
    wo = rng.standard_normal((H * DV, DM), dtype=np.float32) / np.sqrt(H * DV)
    dy = rng.standard_normal((B, T, DM), dtype=np.float32)
    return x, wq, wk, wv, wo, do, dy


def layer_step_ms(args):
    """configs[4] layer step on the GPU: bf16 projections q = x wq, k = x wk, v = x wv (one GEMM
    over the concatenated weights), the
    hard core through autograd (labels by the sign binarizer of q and k, sq = q, sk = k), the
    output projection, and the backward of all of it from dy (weights' and tau's gradients).
    Returns the mean ms per step over args.steps steps after args.warmup."""
    import torch
    import dism_amd
    c = CONFIGS[4]
    B, T, H, D, DV = c["B"], c["T"], c["H"], c["dqk"], c["dv"]
    dev = torch.device("cuda:0")
    x, wq, wk, wv, wo, _, dy = layer_arrays()
    put = lambda a: torch.from_numpy(a).to(dev, torch.bfloat16)  # noqa: E731
    x, dy = put(x), put(dy)
    # the three input projections as one [1280, H*(2*8 + 128)] weight: one GEMM forward and
    # two backward instead of three each (the same products; q, k, v are column blocks)
    wqkv = put(np.concatenate([wq, wk, wv], axis=1)).requires_grad_()
    wout = put(wo).requires_grad_()
    tau = torch.full((H,), args.tau, dtype=torch.float32, device=dev, requires_grad=True)
    hard = torch.ones((B, H), dtype=torch.bool, device=dev)
    nq = H * D

    def step():
        qkv = x @ wqkv
        q = qkv[..., :nq].reshape(B, T, H, D).contiguous()
        k = qkv[..., nq:2 * nq].reshape(B, T, H, D).contiguous()
        v = qkv[..., 2 * nq:].reshape(B, T, H, DV).contiguous()
        iq, ik = dism_amd.sign_labels(q.detach()), dism_amd.sign_labels(k.detach())
        o = dism_amd.dism_core_hard(q, k, v, iq, ik, hard, tau)
        (o.reshape(B, T, H * DV) @ wout).backward(dy)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        step()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / args.steps


def _time(fn, steps, warmup):
    """Mean ms per call of `fn` over `steps` calls between CUDA events, after `warmup` calls."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def _median_ms(fn, calls=20, samples=7, warmup=10):
    """The reference's measure (dism_v3/tools/bench_training.py:39-61): warmup calls, then
    `samples` samples of `calls` calls each between CUDA events; the median sample over
    `calls`, in ms."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    out = []
    for _ in range(samples):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(calls):
            fn()
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e) / calls)
    return float(np.median(out))


# published RTX 5090 numbers for this shape (dism_v3/docs/
# HARD_FORWARD_PLAN.md:245-246, HARD_BACKWARD_QUADRATIC.md:134-135), ms
REF_5090 = {"random": {"forward": 0.4780, "backward": 2.271, "backward_recompute": 2.458},
            "identical": {"forward": 0.4813, "backward": 3.062, "backward_recompute": 3.169}}


def bench_refshape(args):
    """The reference's benchmark shape: B16 H6 N2048 R32 DV64 bf16, tau 0.5, every row hard,
    labels random over 512 symbols or all identical.  Forward = LUT + the one-call forward
    (dism_hard_forward: prepare, label scans, bigram corrections, dense rows); backward = dlog
    table + dism_hard_backward on the forward's workspace and normalizer; backward_recompute =
    forward + backward (the reference's default training route recomputes its boundaries).
    Timed like the reference (10 warmups, median of 7 samples of 20 calls).  Prints one JSON
    line."""
    import torch
    import dism_amd
    from dism_amd import _lib
    from dism_amd._checks import DTYPE_CODE
    from dism_amd.hard_forward import row_modes
    B, H, N, R, DV = 16, 6, 2048, 32, 64
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(20261207)
    x = lambda *sh: torch.randn(*sh, generator=g).to(dev, torch.bfloat16)  # noqa: E731
    sq, sk, v, do = x(B, N, H, R), x(B, N, H, R), x(B, N, H, DV), x(B, N, H, DV)
    tau = torch.full((H,), 0.5, dtype=torch.float32, device=dev)
    hard = torch.ones((B, H), dtype=torch.bool, device=dev)
    code = DTYPE_CODE[torch.bfloat16]
    nbytes = _lib.workspace_bytes(B, N, H, R, DV, code)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    out = torch.empty((B, N, H, DV), dtype=torch.bfloat16, device=dev)
    lse2 = torch.empty((B, H, N), dtype=torch.float32, device=dev)
    dsq = torch.empty((B, N, H, R), dtype=torch.float32, device=dev)
    dsk = torch.empty_like(dsq)
    dvv = torch.empty((B, N, H, DV), dtype=torch.float32, device=dev)
    rowtau = torch.empty((B, H, N), dtype=torch.float32, device=dev)
    dtau = torch.empty((H,), dtype=torch.float32, device=dev)
    S = torch.cuda.current_stream(dev).cuda_stream
    result = {"metric": "hard DISM forward / backward time at the reference's benchmark shape",
              "unit": "ms", "higher_is_better": False,
              "config": {"workload": "reference benchmark shape (HARD_FORWARD_PLAN.md:245)",
                         "B": B, "H": H, "N": N, "R": R, "DV": DV, "tau": 0.5,
                         "labels": "random over 512 symbols | all identical"},
              "data": "synthetic N(0,1) bf16 vectors (seed 20261207)",
              "timing": "10 warmups, median of 7 samples of 20 calls (CUDA events)"}
    for kind in ("random", "identical"):
        if kind == "random":
            lab = torch.randint(0, 512, (B, H, N), generator=g, dtype=torch.int32).to(dev)
        else:
            lab = torch.zeros((B, H, N), dtype=torch.int32, device=dev)
        iq = lab
        ik = lab if kind == "identical" else \
            torch.randint(0, 512, (B, H, N), generator=g, dtype=torch.int32).to(dev)
        state = {}

        def forward():
            lut = dism_amd.hard_log_weights(tau, N)
            state["lut"] = lut
            _lib.call("dism_hard_forward", sq.data_ptr(), sk.data_ptr(), v.data_ptr(), code,
                      iq.data_ptr(), ik.data_ptr(), hard.data_ptr(), 0, 0, lut.data_ptr(),
                      N + 1, B, N, H, R, DV, ws.data_ptr(), nbytes, out.data_ptr(), code,
                      lse2.data_ptr(), 0, 0, S)

        def backward():
            dl = dism_amd.hard_dlog_weights(tau, N + 1)
            _lib.call("dism_hard_backward", sq.data_ptr(), sk.data_ptr(), v.data_ptr(),
                      do.data_ptr(), code, iq.data_ptr(), ik.data_ptr(), hard.data_ptr(), 0, 0,
                      state["lut"].data_ptr(), dl.data_ptr(), N + 1, lse2.data_ptr(), B, N, H,
                      R, DV, ws.data_ptr(), nbytes, dsq.data_ptr(), dsk.data_ptr(),
                      dvv.data_ptr(), rowtau.data_ptr(), dtau.data_ptr(), S)

        def both():
            forward()
            backward()
        f_ms = _median_ms(forward)
        b_ms = _median_ms(backward)
        fb_ms = _median_ms(both)
        modes = row_modes(ws, sq, v).cpu()
        ref = REF_5090[kind]
        result[kind] = {"forward_ms": f_ms, "backward_ms": b_ms, "fwd_bwd_ms": fb_ms,
                        "row_modes": {str(m): int((modes == m).sum()) for m in (0, 1, 2, 3, 4)},
                        "bht_per_s_fwd_bwd": B * H * N / (fb_ms / 1e3),
                        "rtx5090_ms": ref,
                        "speedup_vs_rtx5090": {"forward": ref["forward"] / f_ms,
                                               "backward": ref["backward"] / b_ms,
                                               "fwd_bwd": ref["backward_recompute"] / fb_ms}}
    print(json.dumps(result), flush=True)


def bench_decode(args):
    """Inference at the nanochat layer shape (B=8, H=10, d_qk=8, d_v=128,
    bf16): prefill of a 2048-token prompt, then decoding 256 tokens one at a time after priming
    with the prompt.  Prints one JSON line (decode tokens/s over the B*H rows, prefill time)."""
    import torch
    import dism_amd
    B, H, R, DV, P, G = 8, 10, 8, 128, 2048, 256
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(20261205)
    x = lambda *s: torch.randn(*s, generator=g).to(dev, torch.bfloat16)  # noqa: E731
    sq, sk, v = x(B, P + G, H, R), x(B, P + G, H, R), x(B, P + G, H, DV)
    iq, ik = dism_amd.sign_labels(sq), dism_amd.sign_labels(sk)
    tau = [0.5] * H
    with dism_amd.HardDismPrefill() as engine:
        prep = engine.prepare(iq[..., :P], ik[..., :P], tau)
        psq, psk, pv = (t[:, :P].contiguous() for t in (sq, sk, v))
        pre_ms = _time(lambda: prep.execute(psq, psk, pv), args.steps, args.warmup)
    dec = None
    piq, pik, psk2, pv2 = (t[..., :P].contiguous() if t.dim() == 3 else t[:, :P].contiguous()
                           for t in (iq, ik, sk, v))

    def fresh_prime():
        nonlocal dec
        dec = dism_amd.HardDismDecoder(B, H, R, DV, P + G, tau, label_slots=512,
                                       check_errors=False)
        dec.prime(piq, pik, psk2, pv2)
    prime_ms = _time(fresh_prime, args.steps, args.warmup)  # includes the state's zero fill
    torch.cuda.synchronize()
    # per-token inputs as a model step produces them (fresh contiguous tensors)
    toks = [tuple(x[..., t:t + 1].contiguous() if x.dim() == 3 else x[:, t:t + 1].contiguous()
                  for x in (iq, ik, sq, sk, v)) for t in range(P, P + G)]
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for tk in toks:
        dec.append(*tk)
    e.record()
    torch.cuda.synchronize()
    step_ms = s.elapsed_time(e) / G
    dec._check()
    print(json.dumps({"metric": "hard DISM decode step latency (one token, all B*H rows)",
                      "value": step_ms * 1e3, "unit": "us/token", "higher_is_better": False,
                      "decode_tokens_per_s": B / (step_ms / 1e3),
                      "prefill_ms": pre_ms, "prefill_tokens_per_s": B * P / (pre_ms / 1e3),
                      "prime_ms": prime_ms,
                      "config": {"workload": "BASELINE configs[4] shape, inference", "B": B,
                                 "H": H, "d_qk": R, "d_v": DV, "prompt": P, "decoded": G},
                      "data": "synthetic N(0,1) bf16 vectors, sign labels"}), flush=True)


def bench_vocab(args):
    """Codebook argmax labels (the general label producer) for q at configs[2]'s token count
    (B=4, T=16384, H=16) with D=64, V=512 per-head codebooks."""
    import torch
    import dism_amd
    B, T, H, D, V = 4, 16384, 16, 64, 512
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(20261206)
    x = torch.randn(B, T, H, D, generator=g).to(dev, torch.bfloat16)
    voc = torch.randn(H, V, D, generator=g).to(dev, torch.bfloat16)
    ms = _time(lambda: dism_amd.vocab_labels(x, voc), args.steps, args.warmup)
    flops = 2.0 * B * T * H * V * D
    print(json.dumps({"metric": "codebook argmax labels", "value": B * T * H / (ms / 1e3),
                      "unit": "tokens/s", "ms": ms, "mfma_tflops": flops / (ms / 1e3) / 1e12,
                      "mfma_peak_tflops": 2500.0, "config": {"B": B, "T": T, "H": H, "D": D,
                                                             "V": V},
                      "data": "synthetic N(0,1) bf16"}), flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` on this workload from the committed rocprofv3 PMC
    summary (profiles/traffic.json: FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), or
    None when no measurement is committed."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return t["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def measured_valu(kernel):
    """(VALU wave-instructions per launch of `kernel`, peak issue rate) from the committed
    rocprofv3 PMC summary (profiles/valu.json: SQ_INSTS_VALU), or None."""
    path = os.path.join(ROOT, "profiles", "valu.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return t["kernels"][kernel]["valu_insts"], t["peak_wave_insts_per_s"]
    except (OSError, KeyError, ValueError):
        return None


def _cpu_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return model, os.cpu_count(), avail


def cpu_baseline(q, k, v, do, cfg, args):
    """The CPU model (oracle/dism_cpu_model.c, the fp32 sequence the GPU reproduces: each row
    by the same classification) on the same workload, OpenMP over (b,h) rows.  Threads: the
    host cores allotted to this process (at most 16, the GPU box's CPU share for one GPU);
    also a 1-thread figure.  Method of the reference's measure
    (dism_v3/tools/bench_training.py:39-61): 10 warmup runs, median of 7 timed runs -- on a
    bounded sample of the rows (whole batch entries and heads, the same T), chosen from a
    first timed run so that all the runs take about 10-20 s; the sample is stated."""
    import oracle
    oracle.build()
    from oracle import bf16_round
    f32 = cfg["dtype"] == "f32"
    rnd = (lambda a: np.ascontiguousarray(a, np.float32)) if f32 else bf16_round
    model, nproc, avail = _cpu_info()
    threads = max(1, min(16, avail))
    T = cfg["T"]

    def sample(bs, hs):
        sq, sk, vv, dd = (rnd(a[:bs, :, :hs]) for a in (q, k, v, do))
        iq, ik = oracle.sign_labels(sq), oracle.sign_labels(sk)
        tau = np.full(hs, args.tau, np.float32)
        hard = np.ones((bs, hs), bool)
        lut = oracle.log_weights(tau, T)
        dl = None if cfg["fwd_only"] else oracle.dlog_weights(tau, T)
        return sq, sk, vv, dd, iq, ik, hard, lut, dl

    def run(x, th):
        sq, sk, vv, dd, iq, ik, hard, lut, dl = x
        _, l2, _, _ = oracle.forward(sq, sk, vv, iq, ik, hard, lut, threads=th)
        if dl is not None:
            oracle.backward(sq, sk, vv, dd, iq, ik, hard, lut, dl, l2, threads=th)

    def measure(bs, hs, th, warm, reps):
        x = sample(bs, hs)
        for _ in range(warm):
            run(x, th)
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            run(x, th)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    B, H = cfg["B"], cfg["H"]
    # the sample: whole rows, shrunk until one multi-thread run takes at most ~0.6 s
    bs, hs = B, H
    t1 = measure(bs, hs, threads, 0, 1)
    while t1 > 0.6 and bs * hs > threads:
        if bs > 1:
            bs = (bs + 1) // 2
        else:
            hs = max(1, hs // 2)
        t1 = measure(bs, hs, threads, 0, 1)
    tm = measure(bs, hs, threads, 10, 7)
    # one thread: a single row (or the whole workload if it is one row)
    b1 = 1
    t_one = measure(b1, 1, 1, 3, 3)
    units = bs * hs * T
    return {"value": units / tm, "unit": "B*H*T/s", "cores": threads, "kind": "port",
            "one_thread_value": T / t_one, "nproc": nproc, "cores_allotted": avail,
            "cpu_model": model,
            "sample": f"B={bs} H={hs} of B={B} H={H}, T={T}, "
                      f"{'forward' if cfg['fwd_only'] else 'fwd+bwd'}; median of 7 runs after "
                      f"10 warmups ({tm * 1e3:.1f} ms/run, {threads} threads); one thread: "
                      f"one row, median of 3 ({t_one * 1e3:.1f} ms)"}


if __name__ == "__main__":
    main()
