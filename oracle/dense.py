"""Dense FP64 restatement of the reference oracle, hard rows only (numpy).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product path.

Follows /root/reference/dism_v3/python/flash_dism/reference/dism_v3_ref.py:
  * forward  ``dism_ref``  :41-66  -- hard score 0/-inf, +rtau, diagonal softplus
    recurrence (:47-52), causal mask, zmax clamped at 0 (:56), unit fallback (:58,:65),
    numerator-only signed readout (:60-66);
  * backward ``dism_ref_backward`` :91-127 -- P, S, E, dV/dSQ/dSK (:109-117), the local
    dlogM with correction (:118-120) and the reverse diagonal scan (:121-126) whose total
    is dtau.  Like the reference (:100-101) softplus is linearised above 20.
Everything is O(N^2) per (b,h) and meant for N <= ~2048.
"""
import numpy as np

__all__ = ["dense_forward", "dense_backward", "dense_lengths", "softplus"]


def softplus(x):
    """torch.nn.functional.softplus(beta=1, threshold=20) in float64."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        out = np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    return np.where(np.isneginf(x), 0.0, out)


def dense_lengths(iq, ik):
    """L[i,j] for one (b,h) by the row recurrence (test_hard_chunk.py:24-36)."""
    n = iq.shape[0]
    out = np.zeros((n, n), dtype=np.int64)
    prev = np.zeros(n, dtype=np.int64)
    for i in range(n):
        inc = np.concatenate(([0], prev[:-1]))
        prev = np.where(iq[i] == ik, inc + 1, 0)
        out[i] = prev
    return np.tril(out)


def _scores(iq, ik, tau, reset=None):
    """logM + softplus recurrence (dism_v3_ref.py:41-52) for one (b,h).  reset [N] bool: the
    predecessor score of a reset query is -inf (inference oracle,
    dism_v3/tests/test_sam_inference.py:19-21)."""
    n = iq.shape[0]
    logm = np.where(iq[:, None] == ik[None, :], 0.0, -np.inf) + tau
    rows = []
    alphas = []
    prev = np.full(n, -np.inf)
    for i in range(n):
        x = np.concatenate(([-np.inf], prev[:-1]))
        if reset is not None and reset[i]:
            x = np.full(n, -np.inf)
        with np.errstate(over="ignore", invalid="ignore"):
            sig = np.where(x > 20.0, 1.0, 1.0 / (1.0 + np.exp(-x)))
        alphas.append(np.where(np.isneginf(x), 0.0, sig))
        prev = logm[i] + softplus(x)
        rows.append(prev)
    w = np.stack(rows)
    causal = np.tril(np.ones((n, n), dtype=bool))
    return np.where(causal, w, -np.inf), np.stack(alphas)


def _bh_forward(sq, sk, v, iq, ik, tau, reset=None):
    w, _ = _scores(iq, ik, tau, reset)
    zmax = np.maximum(w.max(-1, keepdims=True), 0.0)
    with np.errstate(invalid="ignore"):
        ew = np.exp(w - zmax)
    ew = np.where(np.isneginf(w), 0.0, ew)
    fb = np.exp(-zmax)
    s = sq @ sk.T
    num = (ew * s) @ v
    den = ew.sum(-1, keepdims=True) + fb
    lse2 = (zmax[:, 0] + np.log(den[:, 0])) / np.log(2.0)
    return num / den, lse2


def dense_forward(sq, sk, v, iq, ik, hard, tau, reset=None):
    """sq,sk [B,N,H,R], v [B,N,H,DV] (any float), iq/ik [B,H,N] int, hard [B,H] bool,
    tau [H], optional query resets [B,H,N] bool.  Returns (O [B,N,H,DV] float64,
    lse2 [B,H,N] float64); soft rows are zero."""
    sq, sk, v = (np.asarray(x, dtype=np.float64) for x in (sq, sk, v))
    B, N, H, _ = sq.shape
    out = np.zeros(v.shape, dtype=np.float64)
    lse2 = np.zeros((B, H, N), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            if not hard[b, h]:
                continue
            o, l2 = _bh_forward(sq[b, :, h], sk[b, :, h], v[b, :, h], iq[b, h], ik[b, h],
                                float(tau[h]), None if reset is None else reset[b, h])
            out[b, :, h] = o
            lse2[b, h] = l2
    return out, lse2


def _bh_backward(sq, sk, v, do, iq, ik, tau):
    n = iq.shape[0]
    w, alpha = _scores(iq, ik, tau)
    mx = np.maximum(w.max(-1, keepdims=True), 0.0)
    with np.errstate(invalid="ignore"):
        ew = np.exp(w - mx)
    ew = np.where(np.isneginf(w), 0.0, ew)
    p = ew / (ew.sum(-1, keepdims=True) + np.exp(-mx))
    s = sq @ sk.T
    e = do @ v.T
    ds = p * e
    dv = (p * s).T @ do
    dsq = ds @ sk
    dsk = ds.T @ sq
    out = (p * s) @ v
    corr = (do * out).sum(-1, keepdims=True)
    total = p * (s * e - corr)
    for i in range(n - 1, 0, -1):
        total[i - 1, :-1] += (total[i] * alpha[i])[1:]
    return dsq, dsk, dv, total.sum()


def dense_backward(sq, sk, v, dout, iq, ik, hard, tau):
    """Explicit FP64 backward.  Returns (dSQ, dSK, dV, dtau[H])."""
    sq, sk, v, dout = (np.asarray(x, dtype=np.float64) for x in (sq, sk, v, dout))
    B, N, H, _ = sq.shape
    dsq, dsk, dv = np.zeros_like(sq), np.zeros_like(sk), np.zeros_like(v)
    dtau = np.zeros(H, dtype=np.float64)
    for b in range(B):
        for h in range(H):
            if not hard[b, h]:
                continue
            a, c, d, t = _bh_backward(sq[b, :, h], sk[b, :, h], v[b, :, h], dout[b, :, h],
                                      iq[b, h], ik[b, h], float(tau[h]))
            dsq[b, :, h], dsk[b, :, h], dv[b, :, h] = a, c, d
            dtau[h] += t
    return dsq, dsk, dv, dtau
