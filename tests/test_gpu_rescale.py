"""GPU parity of the online softmax across key chunks when the running maximum keeps rising.

The inputs of the other parity tests give logits of order one, so a kernel that streams keys
in chunks fixes its base in the first chunk and never moves it again. Here the logits rise
by about RISE (natural units) from the first key to the last: q and every key row share a
unit direction u, with key j's component along u growing linearly in j. Keys are visited in
site order, so every chunked kernel has to move its base (and rescale its sums and
accumulators) several times after the first chunk. Checked against the float64 oracle for
each chunked forward family: the float32 LDS-streaming kernel (fp32, N > 64) and its gated
variant (the trunk's head collapse), the bfloat16 kernels (64-key chunks, with a bias and at
D = 32; 32-query tiles at D = 64 without one; N <= 128), the tangent directions, and the
rectangular kernel with and without the head collapse. A base that is moved wrongly (a sum
or an accumulator not rescaled, or rescaled by the wrong factor) gives errors of order one.
The reverse-mode kernels, which rebuild the weights from the stored lse, are run on the same
inputs: dk, dv and de (dS itself) against the float64 oracle with the uncancelled-magnitude
floors of the other backward tests. dq is left to those tests: dq = sum_j dS_j k_j, and the
keys' component RISE (j / N) u makes its u-component a sum of terms ~RISE times larger than
the result (sum_j dS_j = 0), so its error measures the rounding of dS as an operand (bfloat16:
2^-9 of that sum; float32: scores of magnitude RISE) rather than the weights; dk and de carry
the same rebuilt weights without that amplification.

Tolerances. Scores of magnitude RISE carry RISE times the absolute rounding of scores of order
one, so float32 outputs are held to F32_TOL_RISING = 5e-5 here instead of 1e-5; bfloat16 ones
to the usual 2e-2. The query tangents are drawn orthogonal to u, so the score tangents dS stay
of order one: with qt . u of order one, dS_j would be ~RISE times as large and nearly the same
for the keys that carry the weight, and the tangent output sum_j P_j dS_j (v_j - O) would
cancel to a result some thirty times smaller than its terms (the bfloat16 kernels round the
weights P_j dS_j to bfloat16 before their products, which then shows as 10% of that result).
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O
from oracle import rect_oracle as R
from rising_inputs import RISE, rising

pytestmark = pytest.mark.gpu

F32_TOL_RISING = 5e-5
BF16_TOL = 2e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _bf16_round(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).bfloat16().float().numpy()


def _host(t):
    return None if t is None else t.float().cpu().numpy()


def _dev(x, dtype):
    if x is None:
        return None
    if x.dtype == bool:
        return torch.from_numpy(x).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).to(device="cuda", dtype=dtype)


# name, B, N, H, D, n_phys, bias, T, bf16, generic
CASES = [
    ("fp32_n256_d64_t1", 3, 256, 2, 64, 225, False, 1, False, False),
    ("fp32_n256_d32_t2_bias", 2, 256, 2, 32, 200, True, 2, False, False),
    ("fp32_n256_d64_generic", 2, 256, 2, 64, 230, True, 1, False, True),
    ("bf16_n288_d64_t2_tile32", 2, 288, 2, 64, 260, False, 2, True, False),
    ("bf16_n320_d32_bias_t1", 2, 320, 2, 32, 300, True, 1, True, False),
    ("bf16_n1024_d64_t2_tile32", 1, 1024, 2, 64, 1000, False, 2, True, False),
    ("bf16_n128_d64_t1", 3, 128, 2, 64, 120, False, 1, True, False),
    ("bf16_n256_d64_generic", 2, 256, 2, 64, 250, True, 1, True, True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_rising_logits_fwd_jvp(case):
    from hamiltonzero_amd import kernels

    name, B, N, H, D, n_phys, with_e, T, bf16, generic = case
    _say(f"rising logits {name}")
    q, k, v, u, rng = rising(zlib.crc32(name.encode()) % 1000, B, N, N, H, D)
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        mask[b, np.sort(rng.permutation(N)[:n_phys])] = True
    e = rng.standard_normal((B, N, H, N), dtype=np.float32) * np.float32(0.5) if with_e else None
    qt, kt, vt = (rng.standard_normal((T, B, N, H, D), dtype=np.float32) for _ in range(3))
    qt -= (qt @ u.astype(np.float32))[..., None] * u.astype(np.float32)  # qt . u = 0
    et = rng.standard_normal((T, B, N, H, N), dtype=np.float32) if with_e else None
    arrs = dict(q=q, k=k, v=v, e=e, qt=qt, kt=kt, vt=vt, et=et)
    if bf16:
        arrs = {n: None if x is None else _bf16_round(x) for n, x in arrs.items()}
    dt = torch.bfloat16 if bf16 else torch.float32
    d = {n: _dev(x, dt) for n, x in arrs.items()}
    dmask = _dev(mask, None)
    tol = BF16_TOL if bf16 else F32_TOL_RISING

    out, lse, tout = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], dmask, d["qt"], d["kt"], d["vt"], d["e"],
                                           d["et"], generic=generic)
    torch.cuda.synchronize()
    a = arrs
    ref_out, ref_lse = O.fwd(a["q"], a["k"], a["e"], a["v"], mask)
    # the logits do rise over the keys as the test intends (walker 0, its physical rows)
    s0 = O.scores(a["q"][:1], a["k"][:1], None if a["e"] is None else a["e"][:1], mask[:1])[0]
    s0 = s0[:, mask[0]][:, :, mask[0]]
    assert np.median(s0[..., -1] - s0[..., 0]) > 0.75 * RISE
    assert rel(_host(out), ref_out) <= tol
    assert rel(_host(lse)[mask], ref_lse[mask]) <= tol
    assert np.all(_host(out)[~mask] == 0.0)
    for t in range(T):
        ett = None if a["et"] is None else a["et"][t]
        ref_t = O.jvp(a["q"], a["k"], a["e"], a["v"], mask, a["qt"][t], a["kt"][t], ett, a["vt"][t])
        assert rel(_host(tout)[t], ref_t) <= tol, f"tangent {t}"


# name, B, N, H, D, n_phys, bias, T
GATED_CASES = [
    ("gated_n256_d64_t2_bias", 2, 256, 4, 64, 230, True, 2),
    ("gated_n200_d16_t1", 3, 200, 2, 16, 180, False, 1),
]


@pytest.mark.parametrize("case", GATED_CASES, ids=[c[0] for c in GATED_CASES])
def test_rising_logits_gated(case):
    """The head-collapse forward (fp32, N > 64: the LDS-streaming kernel's gated variant)."""
    from hamiltonzero_amd import kernels

    name, B, N, H, D, n_phys, with_e, T = case
    _say(f"rising logits {name}")
    q, k, v, u, rng = rising(zlib.crc32(name.encode()) % 1000, B, N, N, H, D)
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        mask[b, np.sort(rng.permutation(N)[:n_phys])] = True
    e = rng.standard_normal((B, N, H, N), dtype=np.float32) * np.float32(0.5) if with_e else None
    qt, kt, vt = (rng.standard_normal((T, B, N, H, D), dtype=np.float32) for _ in range(3))
    qt -= (qt @ u.astype(np.float32))[..., None] * u.astype(np.float32)  # qt . u = 0
    et = rng.standard_normal((T, B, N, H, N), dtype=np.float32) if with_e else None
    f = lambda x: _dev(x, torch.float32)
    y, ty = kernels.mhsea_fwd_jvp_gated(f(q), f(k), f(v), _dev(mask, None), f(qt), f(kt), f(vt), f(e), f(et))
    torch.cuda.synchronize()
    for t in range(T):
        ett = None if et is None else et[t]
        ref_y, ref_ty = O.gated_fwd_jvp(q, k, e, v, mask, qt[t], kt[t], ett, vt[t])
        if t == 0:
            assert rel(_host(y), ref_y) <= F32_TOL_RISING
        assert rel(_host(ty)[t], ref_ty) <= F32_TOL_RISING, f"tangent {t}"


# The reverse mode rebuilds every weight from the stored lse, P = 2^(s log2 e - lse log2 e):
# with scores of magnitude RISE the two terms are large and nearly equal for the keys that
# carry the weight. name, B, N, H, D, n_phys, bias, bf16
BWD_CASES = [
    ("bwd_fp32_n64_d32_bias", 4, 64, 2, 32, 50, True, False),
    ("bwd_fp32_n64_d64", 3, 64, 2, 64, 48, False, False),
    ("bwd_fp32_n256_d64_bias", 2, 256, 2, 64, 230, True, False),
    ("bwd_bf16_n64_d64", 4, 64, 2, 64, 48, False, True),
    ("bwd_bf16_n200_d32_bias", 2, 200, 2, 32, 180, True, True),
]


@pytest.mark.parametrize("case", BWD_CASES, ids=[c[0] for c in BWD_CASES])
def test_rising_logits_bwd(case):
    from hamiltonzero_amd import kernels
    from test_gpu_parity import vjp_floors  # uncancelled magnitudes of dq, dk, de

    name, B, N, H, D, n_phys, with_e, bf16 = case
    _say(f"rising logits {name}")
    q, k, v, u, rng = rising(zlib.crc32(name.encode()) % 1000, B, N, N, H, D)
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        mask[b, np.sort(rng.permutation(N)[:n_phys])] = True
    e = rng.standard_normal((B, N, H, N), dtype=np.float32) * np.float32(0.5) if with_e else None
    dout = rng.standard_normal((B, N, H, D), dtype=np.float32)
    a = dict(q=q, k=k, v=v, e=e, dout=dout)
    if bf16:
        a = {n: None if x is None else _bf16_round(x) for n, x in a.items()}
    dt = torch.bfloat16 if bf16 else torch.float32
    d = {n: _dev(x, dt) for n, x in a.items()}
    dmask = _dev(mask, None)
    tol = BF16_TOL if bf16 else F32_TOL_RISING
    out, lse = kernels.mhsea_fwd(d["q"], d["k"], d["v"], dmask, d["e"])
    dq, dk, de, dv = kernels.mhsea_bwd(d["q"], d["k"], d["v"], dmask, lse, out, d["dout"], d["e"], want_de=with_e)
    torch.cuda.synchronize()
    a["mask"] = mask
    opts = dict(scale=1.0, key_mask=False, e_layout="qhk")
    ref = O.vjp(a["q"], a["k"], a["e"], a["v"], mask, a["dout"], **opts)
    floors = vjp_floors(a, opts)
    for nm, got, want in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv), ref):
        if got is None or nm == "dq":
            continue
        g = _host(got).astype(np.float64)
        bound = max(np.max(np.abs(want)), floors[nm])
        assert np.max(np.abs(g - want)) <= tol * bound, nm


# B, Nq, Nk, H, D, n_phys (None: no mask), gated
RECT_CASES = [
    (1, 100, 600, 4, 64, 550, False),
    (2, 64, 257, 8, 32, None, False),
    (1, 80, 500, 8, 64, 480, True),
]


@pytest.mark.parametrize("case", RECT_CASES, ids=lambda c: "B%d_Nq%d_Nk%d_H%d_D%d_n%s_%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], "gated" if c[6] else "plain"))
def test_rising_logits_rect(case):
    from hamiltonzero_amd import kernels

    B, Nq, Nk, H, D, n_phys, gated = case
    _say(f"rising logits rect B={B} Nq={Nq} Nk={Nk} H={H} D={D} n_phys={n_phys} gated={gated}")
    q, k, v, _, rng = rising(17 + Nq + Nk + H + D, B, Nq, Nk, H, D)
    bias = rng.standard_normal((B, Nq, Nk, H), dtype=np.float32) * np.float32(0.5)
    mask = None
    if n_phys is not None:
        mask = np.zeros((B, Nk), dtype=bool)
        for b in range(B):
            mask[b, np.sort(rng.permutation(Nk)[:n_phys])] = True
    got = kernels.rect_attention_fwd(_dev(q, torch.float32), _dev(k, torch.float32), _dev(v, torch.float32),
                                     _dev(bias, torch.float32), None if mask is None else _dev(mask, None),
                                     scale=1.0, gated=gated)
    torch.cuda.synchronize()
    want = (R.rect_gated if gated else R.rect_fwd)(q, k, v, bias, mask, scale=1.0)
    assert rel(_host(got), want) <= F32_TOL_RISING
