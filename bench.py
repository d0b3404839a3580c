"""Benchmark: flash_dism hard core fwd+bwd on one MI355X (BASELINE.json metric).

A step is one training pass of the hard DISM op over one synthetic batch of the headline
configuration (B=4, H=16, T=16384, d_qk=8, d_v=64, bf16, periodic
component on 25% of the heads):
    labels (sign binarizer, q and k) -> log2 weight table -> carry boundary -> readout
    -> dlog table -> query sweep (dSQ, tau terms) -> key sweep (dV, dSK) -> tau reduction.
Inputs are resident in HBM before timing.  Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

P_INT = 256 * 2.4e9 * 64      # int32 lane-ops/s (256 CUs x 2.4 GHz x 64 lanes)
HBM_PEAK = 8.0e12             # bytes/s


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--B", type=int, default=4)
    ap.add_argument("--H", type=int, default=16)
    ap.add_argument("--T", type=int, default=16384)
    ap.add_argument("--dqk", type=int, default=8)
    ap.add_argument("--dv", type=int, default=64)
    ap.add_argument("--tau", type=float, default=0.5)
    ap.add_argument("--carry-strip", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-heads", type=int, default=16)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (single-GPU boxes); "
              "--gpus > 1 is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    import dism_amd
    from dism_amd import _lib
    from dism_amd._checks import DTYPE_CODE

    dev = torch.device("cuda:0")
    B, T, H, D, DV = args.B, args.T, args.H, args.dqk, args.dv
    q, k, v, do = make_inputs(B, T, H, D, DV, seed=20261203)
    bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16).contiguous()  # noqa: E731
    tq, tk, tv, tdo = bf(q), bf(k), bf(v), bf(do)
    tau = torch.full((H,), args.tau, dtype=torch.float32, device=dev)
    hard = torch.ones((B, H), dtype=torch.bool, device=dev)
    stream = torch.cuda.current_stream(dev)
    S = stream.cuda_stream
    strip = args.carry_strip
    n = T
    # persistent outputs / scratch (allocated once, outside the timed region)
    dsq = torch.empty((B, T, H, D), dtype=torch.float32, device=dev)
    dsk = torch.empty_like(dsq)
    dvv = torch.empty((B, T, H, DV), dtype=torch.float32, device=dev)
    rowtau = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    dtau = torch.empty((H,), dtype=torch.float32, device=dev)
    names = ["labels", "lut", "carry", "prepare", "forward", "dlut", "bwd_prepare",
             "bwd_queries", "bwd_keys", "tau_reduce"]
    out = torch.empty((B, T, H, DV), dtype=torch.bfloat16, device=dev)
    lse2 = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    code = DTYPE_CODE[torch.bfloat16]
    nbytes = _lib.workspace_bytes(B, T, H, D, DV, code)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    W = ws.data_ptr()

    def step(events=None):
        def mark(i):
            if events is not None:
                events[i].record(stream)
        mark(0)
        iq = dism_amd.sign_labels(tq)
        ik = dism_amd.sign_labels(tk)
        mark(1)
        lut = dism_amd.hard_log_weights(tau, n)
        mark(2)
        carry = dism_amd.hard_boundary(iq, ik, hard, strip=strip, fill_all=False) \
            if strip > 0 else None
        cp = 0 if carry is None else carry.data_ptr()
        mark(3)
        _lib.call("dism_hard_prepare", tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), code,
                  iq.data_ptr(), ik.data_ptr(), B, T, H, D, DV, W, nbytes, S)
        mark(4)
        _lib.call("dism_hard_readout", tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), code,
                  iq.data_ptr(), ik.data_ptr(), hard.data_ptr(), cp, strip, lut.data_ptr(),
                  n + 1, B, T, H, D, DV, W, nbytes, out.data_ptr(), code, lse2.data_ptr(), 0, 0,
                  S)
        mark(5)
        dlut = dism_amd.hard_dlog_weights(tau, n + 1)
        mark(6)
        _lib.call("dism_hard_backward_prepare", tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                  tdo.data_ptr(), code, iq.data_ptr(), ik.data_ptr(), lse2.data_ptr(), B, T, H,
                  D, DV, W, nbytes, S)
        mark(7)
        _lib.call("dism_hard_backward_queries", tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                  tdo.data_ptr(), code, iq.data_ptr(), ik.data_ptr(), hard.data_ptr(), cp, strip,
                  lut.data_ptr(), dlut.data_ptr(), n + 1, lse2.data_ptr(), B, T, H, D, DV, W,
                  nbytes, dsq.data_ptr(), rowtau.data_ptr(), S)
        mark(8)
        _lib.call("dism_hard_backward_keys", tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                  tdo.data_ptr(), code, iq.data_ptr(), ik.data_ptr(), hard.data_ptr(), cp, strip,
                  lut.data_ptr(), n + 1, lse2.data_ptr(), B, T, H, D, DV, W, nbytes,
                  dsk.data_ptr(), dvv.data_ptr(), S)
        mark(9)
        _lib.call("dism_hard_tau_reduce", rowtau.data_ptr(), B, H, T, dtau.data_ptr(), S)
        mark(10)
        return out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per = [[torch.cuda.Event(enable_timing=True) for _ in range(11)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    start.record(stream)
    for s in range(args.steps):
        step(per[s])
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(end)
    ms_step = gpu_ms / args.steps
    kern_ms = {nm: float(np.mean([per[s][i].elapsed_time(per[s][i + 1])
                                  for s in range(args.steps)])) for i, nm in enumerate(names)}
    units = B * H * T
    value = units / (ms_step / 1e3)

    # int-VALU roofline of BASELINE.md: 2 int ops per causal pair per pass, 2 passes
    pairs = T * (T + 1) / 2 * B * H
    t_int = 4 * pairs / P_INT
    # dominant kernel: algorithmic HBM bytes per launch (no O(N^2) state)
    dom = max(("forward", "bwd_queries", "bwd_keys"), key=lambda x: kern_ms[x])
    per_unit = {  # bytes per (b,h,t) unit the kernel must move at minimum
        "forward": 2 * D * 2 + 2 * DV + 2 * DV + 4 + 4 * 2,        # sq,sk,v in; O,lse2 out; labels
        "bwd_queries": 2 * D * 2 + 2 * DV * 2 + 4 + 4 * D + 4 + 4 * 2,
        "bwd_keys": 2 * D * 2 + 2 * DV * 2 + 4 + 4 * D + 4 * DV + 4 * 2,
    }[dom]
    alg_bytes = per_unit * units
    achieved = alg_bytes / (kern_ms[dom] / 1e3)
    result = {
        "metric": "DISM fwd+bwd tokens/sec (B*H*T/s) at T=16k, 1 GPU",
        "value": value,
        "unit": "B*H*T/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "wall_ms_per_step": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32+fp32 (bf16 vectors)",
        "data": "synthetic (BASELINE config 3 generator, seed 20261203)",
        "config": {"workload": "BASELINE configs[2]: hard DISM fwd+bwd, periodic heads",
                   "B": B, "H": H, "T": T, "d_qk": D, "d_v": DV, "tau": args.tau,
                   "carry_strip": strip, "global_batch": B, "seq_len": T,
                   "parallelism": "single-gpu"},
        "kernel_ms": kern_ms,
        "int_valu_roofline": {"t_roof_ms": t_int * 1e3, "frac": t_int / (ms_step / 1e3),
                              "peak_int_ops": P_INT,
                              "note": "BASELINE.md accounting (2 int ops/pair/pass); the "
                                      "bitmask sweep does far fewer ops, so frac may exceed 1"},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": achieved / 1e9,
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": achieved / HBM_PEAK,
                     "traffic": None, "alg_bytes_per_unit": per_unit},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(q, k, v, do, args)
    print(json.dumps(result), flush=True)


def cpu_baseline(q, k, v, do, args):
    """CPU model (oracle/dism_cpu_model.c) fwd+bwd on a bounded sample: batch 0, the first
    `cpu_heads` heads (head 0 carries the periodic component), full T, all host threads."""
    import oracle
    oracle.build()
    from oracle import bf16_round
    hs = slice(0, args.cpu_heads)
    sq = bf16_round(q[:1, :, hs])
    sk = bf16_round(k[:1, :, hs])
    vv = bf16_round(v[:1, :, hs])
    dd = bf16_round(do[:1, :, hs])
    Hs = sq.shape[2]
    iq, ik = oracle.sign_labels(sq), oracle.sign_labels(sk)
    tau = np.full(Hs, args.tau, np.float32)
    hard = np.ones((1, Hs), bool)
    threads = os.cpu_count() or 1
    t0 = time.perf_counter()
    lut = oracle.log_weights(tau, args.T)
    dl = oracle.dlog_weights(tau, args.T)
    _, l2, _, _ = oracle.forward(sq, sk, vv, iq, ik, hard, lut, threads=threads)
    oracle.backward(sq, sk, vv, dd, iq, ik, hard, lut, dl, l2, threads=threads)
    dt = time.perf_counter() - t0
    units = Hs * args.T
    return {"value": units / dt, "unit": "B*H*T/s", "cores": min(threads, Hs), "kind": "port",
            "sample": f"B=1 H={Hs} T={args.T} fwd+bwd, OpenMP over (b,h) rows, {dt:.1f}s",
            "host_threads": threads}


if __name__ == "__main__":
    main()
