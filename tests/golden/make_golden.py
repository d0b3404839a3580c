"""Writes tests/golden/golden.json: SHA-256 digests and sample values of the CPU model's
outputs on the BASELINE configs' generators (configs[0] exactly, configs[1] at reduced size:
level rows) and on identical-label rows at the reference's benchmark row shape (reduced to
T=512: prefix rows).

The reference ships no golden vectors (its tests build inputs from seeds), so these fixtures
come from this build's CPU model (oracle/), which tests/test_oracle.py pins against closed
forms, FP64 dense evaluation, brute force and finite differences.  The digests freeze the
bit pattern of every output so that the oracle and the HIP path (tests/test_golden.py) are
held to the same numbers from run to run.  Regenerate with `python tests/golden/make_golden.py`.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def config_inputs(name):
    """Seeded inputs: numpy PCG64 seed 20261201 + config index, N(0,1) fp32, bf16-rounded
    where the config is bf16; sq = q, sk = k; labels by the sign binarizer."""
    if name == "cfg1":
        rng = np.random.default_rng(20261201 + 0)
        B, T, H, D, DV = 1, 256, 4, 8, 64
        q = rng.standard_normal((B, T, H, D), dtype=np.float32)
        k = rng.standard_normal((B, T, H, D), dtype=np.float32)
        v = rng.standard_normal((B, T, H, DV), dtype=np.float32)
        do = None
    elif name == "cfg2s":  # configs[1] generator at B=1, H=2, T=512 (alphabet 4)
        rng = np.random.default_rng(20261201 + 1)
        B, T, H, D, DV = 1, 512, 2, 2, 64
        q = rng.standard_normal((B, T, H, D), dtype=np.float32)
        k = rng.standard_normal((B, T, H, D), dtype=np.float32)
        v = oracle.bf16_round(rng.standard_normal((B, T, H, DV), dtype=np.float32))
        do = oracle.bf16_round(rng.standard_normal((B, T, H, DV), dtype=np.float32))
    elif name == "prefix_s":  # the reference's identical-label benchmark rows, reduced: B=1,
        # H=2, T=512, R=32, DV=64 with q, k >= 0 (every label 255: prefix rows, mode 4)
        rng = np.random.default_rng(20261207)
        B, T, H, D, DV = 1, 512, 2, 32, 64
        q = oracle.bf16_round(np.abs(rng.standard_normal((B, T, H, D), dtype=np.float32)))
        k = oracle.bf16_round(np.abs(rng.standard_normal((B, T, H, D), dtype=np.float32)))
        v = oracle.bf16_round(rng.standard_normal((B, T, H, DV), dtype=np.float32))
        do = oracle.bf16_round(rng.standard_normal((B, T, H, DV), dtype=np.float32))
    else:
        raise ValueError(name)
    tau = np.linspace(-0.5, 0.5, H).astype(np.float32)
    return q, k, v, do, tau


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def compute(name):
    q, k, v, do, tau = config_inputs(name)
    B, T, H, _ = q.shape
    iq, ik = oracle.sign_labels(q), oracle.sign_labels(k)
    hard = np.ones((B, H), bool)
    lut = oracle.log_weights(tau, T)
    out, lse2, lmax, jarg = oracle.forward(q, k, v, iq, ik, hard, lut)
    res = {"out": out, "lse2": lse2, "lmax": lmax, "jarg": jarg, "labels_q": iq,
           "labels_k": ik}
    if do is not None:
        dl = oracle.dlog_weights(tau, T)
        dsq, dsk, dv, dtau, _ = oracle.backward(q, k, v, do, iq, ik, hard, lut, dl, lse2)
        res.update({"dsq": dsq, "dsk": dsk, "dv": dv, "dtau": dtau})
    return res


def main():
    oracle.build()
    table = {}
    for name in ("cfg1", "cfg2s", "prefix_s"):
        res = compute(name)
        table[name] = {
            "digests": {k: digest(v) for k, v in res.items()},
            "samples": {k: np.asarray(v).reshape(-1)[:8].tolist() for k, v in res.items()},
            "shapes": {k: list(np.asarray(v).shape) for k, v in res.items()},
        }
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(table, f, indent=1, sort_keys=True)
    print("wrote", os.path.join(HERE, "golden.json"))


if __name__ == "__main__":
    main()
