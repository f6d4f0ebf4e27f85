"""Seeded random sweep of the C ABI against the float64 oracle (GPU).

Each case draws its shape and options from a fixed-seed generator — walkers, sites (1..300),
heads, head dimension, tangent count, storage dtype, mask mode and pattern (prefix,
scattered, per-walker counts including walkers with no physical site), bias presence and
layout, scale, and the automatic or the forced LDS-streaming kernels — and checks the fused
forward+tangent, the tangent from (out, lse) and the backward (with de) against the oracle.
A second sweep does the same for the rectangular forward. Tolerances as in the fixed-case
parity tests: max-norm relative error <= 1e-5 for float32, <= 2e-2 for bfloat16 storage
(oracle on the bf16-rounded inputs); where the exact cotangent cancels, the denominator is
floored by 1% of the uncancelled magnitude of the same sums.
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O
from oracle import rect_oracle as R

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 2e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b, floor=0.0):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), floor, 1e-30))


def bf16_round(x):
    return torch.from_numpy(x).bfloat16().float().numpy()


def draw_case(i):
    rng = np.random.default_rng(7000 + i)
    bf16 = bool(rng.random() < 0.3)
    N = int(rng.choice([1, 2, 5, 8, 13, 16, 24, 31, 32, 40, 48, 57, 64, 65, 80, 100, 128, 129, 160, 200, 257, 300]))
    D = int(rng.choice([32, 64])) if bf16 else int(rng.choice([8, 16, 32, 64]))
    return dict(seed=7000 + i, B=int(rng.integers(1, 5)), N=N, H=int(rng.integers(1, 5)), D=D,
                T=int(rng.integers(1, 4)), bf16=bf16, key_mask=bool(rng.random() < 0.35),
                mask_kind=str(rng.choice(["prefix", "scattered", "counts"])), with_e=bool(rng.random() < 0.5),
                e_layout=str(rng.choice(["qhk", "qkh"])), scale=float(rng.choice([1.0, 0.5, D ** -0.5])),
                generic=bool(rng.random() < 0.3))


def make(c):
    rng = np.random.default_rng(c["seed"])
    B, N, H, D, T = c["B"], c["N"], c["H"], c["D"], c["T"]
    shape = (B, N, H, D)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(D ** -0.5) for _ in range(3))
    eshape = (B, N, H, N) if c["e_layout"] == "qhk" else (B, N, N, H)
    e = rng.standard_normal(eshape, dtype=np.float32) * np.float32(0.5) if c["with_e"] else None
    qt, kt, vt = (rng.standard_normal((T, *shape), dtype=np.float32) for _ in range(3))
    et = rng.standard_normal((T, *eshape), dtype=np.float32) if c["with_e"] else None
    dout = rng.standard_normal(shape, dtype=np.float32)
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        n = int(rng.integers(0, N + 1)) if c["mask_kind"] == "counts" else max(1, (3 * N) // 4)
        sites = np.arange(n) if c["mask_kind"] == "prefix" else rng.permutation(N)[:n]
        mask[b, sites] = True
    a = dict(q=q, k=k, v=v, e=e, qt=qt, kt=kt, vt=vt, et=et, dout=dout)
    if c["bf16"]:
        a = {n: None if x is None else bf16_round(x) for n, x in a.items()}
    a["mask"] = mask
    return a


def floors(a, opts):
    p = O.probs(a["q"], a["k"], a["e"], a["mask"], **opts)
    out, _ = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"], **opts)
    dout = np.abs(a["dout"].astype(np.float64))
    dp = np.einsum("bihd,bjhd->bhij", dout, np.abs(a["v"].astype(np.float64)))
    delta = np.abs(out * a["dout"]).sum(-1).transpose(0, 2, 1)[..., None]
    ds = p * (dp + delta)
    s = abs(opts["scale"])
    dq = s * np.einsum("bhij,bjhd->bihd", ds, np.abs(a["k"].astype(np.float64)))
    dk = s * np.einsum("bhij,bihd->bjhd", ds, np.abs(a["q"].astype(np.float64)))
    return {"dq": 0.01 * dq.max(), "dk": 0.01 * dk.max(), "de": 0.01 * ds.max(), "dv": 0.0}


CASES = [draw_case(i) for i in range(40)]


def case_id(c):
    return "B{B}_N{N}_H{H}_D{D}_T{T}_{dt}_{m}{km}{e}{g}".format(
        dt="bf16" if c["bf16"] else "f32", m=c["mask_kind"], km="_keymask" if c["key_mask"] else "",
        e="_e" + c["e_layout"] if c["with_e"] else "", g="_generic" if c["generic"] else "", **c)


@pytest.mark.parametrize("c", CASES, ids=[case_id(c) for c in CASES])
def test_random_case(c):
    from hamiltonzero_amd import kernels

    _say("random " + case_id(c))
    a = make(c)
    dt = torch.bfloat16 if c["bf16"] else torch.float32
    tol = BF16_TOL if c["bf16"] else F32_TOL
    d = {n: None if x is None else torch.from_numpy(x).to(device="cuda", dtype=dt) for n, x in a.items() if n != "mask"}
    d["mask"] = torch.from_numpy(a["mask"]).cuda()
    opts = dict(scale=c["scale"], key_mask=c["key_mask"], e_layout=c["e_layout"])
    kopts = dict(opts, generic=c["generic"])
    host = lambda t: t.float().cpu().numpy()  # noqa: E731

    out, lse, tout = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"],
                                           d["et"], **kopts)
    tout2 = kernels.mhsea_jvp(d["q"], d["k"], d["v"], d["mask"], out, lse, d["qt"], d["kt"], d["vt"], d["e"], d["et"],
                              **kopts)
    dq, dk, de, dv = kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], lse, out, d["dout"], d["e"], want_de=True,
                                       **kopts)
    torch.cuda.synchronize()

    ref_out, _ = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"], **opts)
    assert rel(host(out), ref_out) <= tol, "out"
    for t in range(c["T"]):
        et = None if a["et"] is None else a["et"][t]
        ref_t = O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"][t], a["kt"][t], et, a["vt"][t], **opts)
        assert rel(host(tout)[t], ref_t) <= tol, f"fused tangent {t}"
        assert rel(host(tout2)[t], ref_t) <= tol, f"tangent {t} from out, lse"
    fl = floors(a, opts)
    for name, got, ref in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv),
                              O.vjp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["dout"], **opts)):
        assert rel(host(got), ref, fl[name]) <= tol, name
    if not c["key_mask"]:
        m = a["mask"]
        assert np.all(host(out)[~m] == 0.0) and np.all(host(dq)[~m] == 0.0)


def draw_rect(i):
    rng = np.random.default_rng(9000 + i)
    return dict(seed=9000 + i, B=int(rng.integers(1, 4)), Nq=int(rng.integers(1, 301)), Nk=int(rng.integers(1, 301)),
                H=int(rng.integers(1, 10)), D=int(rng.choice([8, 16, 32, 64])),
                mask=str(rng.choice(["none", "prefix", "scattered", "counts"])), bias=bool(rng.random() < 0.8),
                scale=float(rng.choice([1.0, 0.3])))


RECT = [draw_rect(i) for i in range(20)]


@pytest.mark.parametrize("c", RECT, ids=["B{B}_Nq{Nq}_Nk{Nk}_H{H}_D{D}_{mask}{b}".format(b="_bias" if c["bias"] else "", **c)
                                         for c in RECT])
def test_random_rect_case(c):
    from hamiltonzero_amd import kernels

    _say("random rect {}".format(c))
    rng = np.random.default_rng(c["seed"])
    B, Nq, Nk, H, D = c["B"], c["Nq"], c["Nk"], c["H"], c["D"]
    q = rng.standard_normal((B, Nq, H, D), dtype=np.float32)
    k = rng.standard_normal((B, Nk, H, D), dtype=np.float32)
    v = rng.standard_normal((B, Nk, H, D), dtype=np.float32)
    e = rng.standard_normal((B, Nq, Nk, H), dtype=np.float32) if c["bias"] else None
    mask = None
    if c["mask"] != "none":
        mask = np.zeros((B, Nk), dtype=bool)
        for b in range(B):
            n = int(rng.integers(0, Nk + 1)) if c["mask"] == "counts" else max(1, (3 * Nk) // 4)
            mask[b, np.arange(n) if c["mask"] == "prefix" else rng.permutation(Nk)[:n]] = True
    dev = lambda x: None if x is None else torch.from_numpy(x).cuda()  # noqa: E731
    out = kernels.rect_attention_fwd(dev(q), dev(k), dev(v), dev(e), dev(mask), scale=c["scale"])
    torch.cuda.synchronize()
    assert rel(out.cpu().numpy(), R.rect_fwd(q, k, v, e, mask, scale=c["scale"])) <= F32_TOL
