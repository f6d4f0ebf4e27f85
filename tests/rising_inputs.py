"""Inputs whose logits rise over the keys, and a chunked online softmax on the CPU.

Shared by the GPU parity test of the kernels' base moves (test_gpu_rescale.py) and the CPU
test that shows those inputs move the base and that a wrong move is visible
(test_rescale_inputs.py).
"""

import numpy as np

RISE = 40.0


def rising(seed, B, Nq, Nk, H, D, rise=RISE):
    """q [B, Nq, H, D], k, v [B, Nk, H, D] (float32) whose logits q.k rise by ~rise over the
    keys: q = q0 + u, k_j = k0_j + rise (j / Nk) u with |u| = 1 and q0, k0 ~ N(0, 1/D).
    Returns (q, k, v, u, rng)."""
    rng = np.random.default_rng(seed)
    u = rng.standard_normal(D)
    u /= np.linalg.norm(u)
    sd = np.float32(D ** -0.5)
    q = rng.standard_normal((B, Nq, H, D), dtype=np.float32) * sd + u.astype(np.float32)
    ramp = (rise * np.arange(Nk) / Nk).astype(np.float32)
    k = rng.standard_normal((B, Nk, H, D), dtype=np.float32) * sd + ramp[None, :, None, None] * u.astype(np.float32)
    v = rng.standard_normal((B, Nk, H, D), dtype=np.float32)
    return q, k, v, u, rng


def online_softmax(s, ds, v, vt, chunk=32, threshold=8.0, plant=None):
    """One query row: scores s [n] (natural units), score tangents ds [n], values v, vt [n, D],
    streamed in chunks with the lazy base of the kernels (base 2; the base moves when a chunk's
    maximum exceeds it by more than ``threshold``, and the sums are rescaled by 2^(old - new)).
    Returns (out, tout, moves after the first chunk). ``plant`` puts a mistake into the moves:
    "no_acc" (the value sums not rescaled), "inverse" (rescaled by 2^(new - old)),
    "no_mu" (the tangent row sum not rescaled)."""
    s2 = np.asarray(s, dtype=np.float64) * np.log2(np.e)
    m = -np.inf
    l = mu = 0.0
    o = np.zeros(v.shape[1])
    a = np.zeros(v.shape[1])
    moves = 0
    for c0 in range(0, len(s2), chunk):
        sl = slice(c0, c0 + chunk)
        cmax = s2[sl].max()
        if cmax > m + threshold:
            if c0 > 0:
                moves += 1
            alpha = 2.0 ** (m - cmax)
            if plant == "inverse" and c0 > 0:
                alpha = 1.0 / alpha
            l *= alpha
            if plant != "no_acc":
                o *= alpha
                a *= alpha
            if plant != "no_mu":
                mu *= alpha
            m = cmax
        p = 2.0 ** (s2[sl] - m)
        l += p.sum()
        mu += (p * ds[sl]).sum()
        o += p @ v[sl]
        a += (p * ds[sl]) @ v[sl] + p @ vt[sl]
    out = o / l
    return out, a / l - (mu / l) * out, moves
