"""GPU parity of the gfx950 MHSEA kernels against the float64 oracle (C ABI via ctypes).

Tolerances (max-norm relative error, ||x - ref||_inf / ||ref||_inf per tensor):
  float32 I/O:                 1e-5
  bfloat16 I/O, fp32 accumulate: 2e-2, against the oracle run on the bf16-rounded inputs.
Integer-like facts (masked rows, determinism) are checked bit-exactly.
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 2e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b, floor=0.0):
    """||a - b||_inf / max(||b||_inf, floor). ``floor`` is the magnitude of the uncancelled
    sums behind ``b`` (used where the exact result cancels to ~0, e.g. dq at N = 1)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = max(np.max(np.abs(b)), floor, 1e-30)
    return float(np.max(np.abs(a - b)) / den)


def vjp_floors(a, opts):
    """Magnitudes of dq, dk, de without cancellation: the cotangent sums evaluated on
    |dP| + |delta| instead of dP - delta (their rounding error scales with these)."""
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


def make_inputs(seed, B, N, H, D, n_phys, *, scattered=False, with_e=False, e_layout="qhk", T=1,
                bf16=False):
    rng = np.random.default_rng(seed)
    shape = (B, N, H, D)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(D ** -0.5) for _ in range(3))
    eshape = (B, N, H, N) if e_layout == "qhk" else (B, N, N, H)
    e = rng.standard_normal(eshape, dtype=np.float32) * np.float32(0.5) if with_e else None
    tan = [rng.standard_normal((T, *shape), dtype=np.float32) for _ in range(3)]
    et = rng.standard_normal((T, *eshape), dtype=np.float32) if with_e else None
    dout = rng.standard_normal(shape, dtype=np.float32)
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        n_b = int(rng.integers(0, N + 1)) if n_phys < 0 else n_phys  # n_phys < 0: per-walker counts
        sites = rng.permutation(N)[:n_b] if scattered else np.arange(n_b)
        mask[b, sites] = True
    arrs = dict(q=q, k=k, v=v, e=e, qt=tan[0], kt=tan[1], vt=tan[2], et=et, dout=dout)
    if bf16:
        arrs = {n: None if a is None else torch.from_numpy(a).bfloat16().float().numpy() for n, a in arrs.items()}
    arrs["mask"] = mask
    return arrs


def to_dev(a, dtype):
    if a is None:
        return None
    if a.dtype == bool:
        return torch.from_numpy(a).cuda()
    return torch.from_numpy(a).to(device="cuda", dtype=dtype)


def host(t):
    return None if t is None else t.float().cpu().numpy()


CASES = [
    # name, B, N, H, D, n_phys, scattered, with_e, e_layout, key_mask, scale, T, bf16
    ("c1_full_fwd", 256, 8, 4, 32, 8, False, False, "qhk", False, 1.0, 1, False),
    ("c2_small", 8, 64, 8, 32, 36, False, False, "qhk", False, 1.0, 1, False),
    ("c2_scattered_bias", 4, 64, 4, 32, 36, True, True, "qhk", False, 1.0, 1, False),
    ("n8_d8_bias", 6, 8, 3, 8, 5, True, True, "qhk", False, 1.0, 1, False),
    ("n16_d16_qkh_keymask", 4, 16, 2, 16, 11, True, True, "qkh", True, 0.25, 1, False),
    ("n96_d64_t2", 3, 96, 2, 64, 90, True, True, "qhk", False, 1.0, 2, False),
    ("n1_d16", 5, 1, 2, 16, 1, False, False, "qhk", False, 1.0, 1, False),
    ("n33_odd", 3, 33, 2, 32, 20, True, True, "qkh", False, 0.7, 1, False),
    ("t3_groups", 2, 64, 2, 16, 40, True, False, "qhk", False, 1.0, 3, False),
    ("c3_small_bf16", 4, 64, 8, 64, 48, False, False, "qhk", False, 1.0, 1, True),
    ("c4_small", 2, 256, 4, 64, 225, False, False, "qhk", False, 1.0, 1, False),
    ("c5_small_bf16", 1, 1024, 2, 64, 1000, False, False, "qhk", False, 1.0, 2, True),
    ("keymask_all_masked", 3, 16, 2, 32, 0, False, True, "qkh", True, 1.0, 1, False),
    ("square_all_masked", 3, 16, 2, 32, 0, False, True, "qhk", False, 1.0, 1, False),
    # 32 < N <= 64, float32: one, two, three and four query tiles per item, and walkers whose
    # site counts differ from item to item
    ("n48_one_qtile_bias", 5, 48, 3, 32, 10, True, True, "qhk", False, 1.0, 1, False),
    ("n64_keymask_d16_t2", 4, 64, 2, 16, 40, True, False, "qhk", True, 1.0, 2, False),
    ("n40_d8_t2_bias", 3, 40, 2, 8, 25, True, True, "qkh", False, 0.5, 2, False),
    ("n64_mixed_counts", 24, 64, 3, 32, -1, True, True, "qhk", False, 1.0, 1, False),
    # bias rows staged whole through LDS (keys contiguous, N a multiple of 4, D <= 16 with
    # tangents), with the key mask, and N = 37, where rows are not 16-byte aligned and each
    # score's bias is read on its own
    ("n64_d16_rows_bias", 4, 64, 4, 16, 36, True, True, "qhk", False, 1.0, 1, False),
    ("n44_d8_t2_rows_bias", 3, 44, 2, 8, 30, True, True, "qhk", False, 0.5, 2, False),
    ("n60_d16_keymask_rows_bias", 3, 60, 2, 16, 20, True, True, "qhk", True, 1.0, 1, False),
    ("n37_d16_unaligned_rows_bias", 3, 37, 2, 16, 25, True, True, "qhk", False, 1.0, 1, False),
    # D = 32 without bias: last query tiles of at most four queries (the 4x4-block remainder
    # path) as tile 0, 1, 2 and, through the fourth tile of n > 48, 3; the key mask with and
    # without physical sites; T = 2; walkers whose site counts differ
    ("n64_d32_rem4_sites1", 4, 64, 2, 32, 1, True, False, "qhk", False, 1.0, 1, False),
    ("n64_d32_rem4_sites20_t2", 4, 64, 2, 32, 20, True, False, "qhk", False, 0.5, 2, False),
    ("n64_d32_rem4_sites34", 4, 64, 3, 32, 34, True, False, "qhk", False, 1.0, 1, False),
    ("n64_d32_rem4_sites50", 3, 64, 2, 32, 50, True, False, "qhk", False, 1.0, 1, False),
    ("n36_d32_keymask_rem4", 3, 36, 2, 32, 20, True, False, "qhk", True, 1.0, 1, False),
    ("n35_d32_keymask_none_rem4", 2, 35, 2, 32, 0, False, False, "qhk", True, 1.0, 2, False),
    ("n64_d32_mixed_counts_nobias", 24, 64, 3, 32, -1, True, False, "qhk", False, 1.0, 1, False),
    # float32 D = 64, N <= 64: one tangent (streaming kernel) and two (LDS-streaming kernel)
    ("n64_d64_t1_fp32", 3, 64, 2, 64, 48, False, False, "qhk", False, 1.0, 1, False),
    ("n64_d64_t2_fp32_bias", 3, 64, 2, 64, 48, True, True, "qkh", False, 0.5, 2, False),
    # N > 128, bfloat16: the 64-key chunk pipeline with one, two, three and more chunks,
    # a partial last chunk, bias in both layouts, the key mask (including no physical
    # site, where every site is a key) and walkers whose site counts differ
    ("n144_bf16_one_chunk", 3, 144, 1, 64, 40, True, False, "qhk", False, 1.0, 1, True),
    ("n160_bf16_keymask_t2", 2, 160, 2, 64, 70, True, True, "qkh", True, 1.0, 2, True),
    ("n200_bf16_d32_bias", 2, 200, 2, 32, 150, True, True, "qhk", False, 0.8, 1, True),
    ("n136_bf16_keymask_none", 2, 136, 1, 32, 0, False, False, "qhk", True, 1.0, 1, True),
    ("n256_bf16_mixed_t2", 6, 256, 2, 32, -1, True, True, "qhk", False, 1.0, 2, True),
    # N > 128, bfloat16, D = 64, no bias: the 32-query-tile kernel (32-key chunks, the last
    # one partial or whole): one, two, an odd and an even number of chunks, a whole last chunk,
    # a scale, the key mask with and without physical sites, walkers whose counts differ
    ("n160_bf16_tile32_one_chunk", 2, 160, 2, 64, 20, True, False, "qkh", True, 1.0, 1, True),
    ("n256_bf16_tile32_two_chunks", 2, 256, 2, 64, 50, True, False, "qhk", False, 1.0, 2, True),
    ("n288_bf16_tile32_scaled_t2", 4, 288, 3, 64, 260, True, False, "qhk", False, 0.125, 2, True),
    ("n192_bf16_tile32_whole_chunks", 3, 192, 2, 64, 160, True, False, "qhk", False, 1.0, 1, True),
    ("n200_bf16_tile32_keymask_none", 2, 200, 2, 64, 0, False, False, "qhk", True, 1.0, 2, True),
    ("n320_bf16_tile32_mixed", 8, 320, 2, 64, -1, True, False, "qhk", False, 1.0, 2, True),
]
IDS = [c[0] for c in CASES]


PATHS = [False, True]
PATH_IDS = ["auto", "generic"]


def _setup(case, generic=False):
    name, B, N, H, D, n_phys, scattered, with_e, e_layout, key_mask, scale, T, bf16 = case
    a = make_inputs(zlib.crc32(name.encode()) % 1000, B, N, H, D, n_phys, scattered=scattered, with_e=with_e,
                    e_layout=e_layout, T=T, bf16=bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    d = {n: to_dev(x, dt) for n, x in a.items()}
    opts = dict(scale=scale, key_mask=key_mask, e_layout=e_layout)
    tol = BF16_TOL if bf16 else F32_TOL
    return a, d, opts, dict(opts, generic=generic), tol, T


@pytest.mark.parametrize("generic", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_fwd_parity(case, generic):
    from hamiltonzero_amd import kernels

    _say(f"fwd {case[0]} generic={generic}")
    a, d, opts, kopts, tol, _ = _setup(case, generic)
    out, lse = kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"], d["e"], **kopts)
    torch.cuda.synchronize()
    ref_out, ref_lse = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"], **opts)
    assert rel(host(out), ref_out) <= tol
    m = a["mask"]
    has_key = m.any(axis=1)
    if not opts["key_mask"]:
        assert np.all(host(out)[~m] == 0.0)
        assert rel(host(lse)[m], ref_lse[m]) <= tol if m.any() else True
        np.testing.assert_allclose(host(lse)[~m], ref_lse[~m], rtol=1e-6)
    else:  # every row, walkers without a physical key included (lse relative to the 1e9 shift)
        assert rel(host(lse), ref_lse) <= tol


@pytest.mark.parametrize("generic", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_fwd_jvp_parity(case, generic):
    from hamiltonzero_amd import kernels

    _say(f"fwd_jvp {case[0]} generic={generic}")
    a, d, opts, kopts, tol, T = _setup(case, generic)
    out, lse, tout = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"],
                                           d["e"], d["et"], **kopts)
    torch.cuda.synchronize()
    ref_out, _ = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"], **opts)
    assert rel(host(out), ref_out) <= tol
    for t in range(T):
        et = None if a["et"] is None else a["et"][t]
        ref_t = O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"][t], a["kt"][t], et, a["vt"][t], **opts)
        got = host(tout)[t]
        assert rel(got, ref_t) <= tol, f"tangent {t}"
        if not opts["key_mask"]:
            assert np.all(got[~a["mask"]] == 0.0)


@pytest.mark.parametrize("generic", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_jvp_given_lse_parity(case, generic):
    from hamiltonzero_amd import kernels

    _say(f"jvp {case[0]} generic={generic}")
    a, d, opts, kopts, tol, T = _setup(case, generic)
    out, lse = kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"], d["e"], **kopts)
    tout = kernels.mhsea_jvp(d["q"], d["k"], d["v"], d["mask"], out, lse, d["qt"], d["kt"], d["vt"],
                             d["e"], d["et"], **kopts)
    torch.cuda.synchronize()
    for t in range(T):
        et = None if a["et"] is None else a["et"][t]
        ref_t = O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"][t], a["kt"][t], et, a["vt"][t], **opts)
        assert rel(host(tout)[t], ref_t) <= tol, f"tangent {t}"


@pytest.mark.parametrize("generic", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_bwd_parity(case, generic):
    from hamiltonzero_amd import kernels

    _say(f"bwd {case[0]} generic={generic}")
    a, d, opts, kopts, tol, _ = _setup(case, generic)
    out, lse = kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"], d["e"], **kopts)
    dq, dk, de, dv = kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], lse, out, d["dout"], d["e"],
                                       want_de=True, **kopts)
    torch.cuda.synchronize()
    ref = O.vjp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["dout"], **opts)
    floors = vjp_floors(a, opts)
    for name, got, want in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv), ref):
        if np.max(np.abs(want)) == 0.0 and floors[name] == 0.0:
            assert np.all(host(got) == 0.0), name
        else:
            assert rel(host(got), want, floors[name]) <= tol, name
    m = a["mask"]
    if not opts["key_mask"]:
        for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
            assert np.all(host(got)[~m] == 0.0), name


def test_deterministic_bitwise():
    from hamiltonzero_amd import kernels

    _say("determinism c2 small")
    a = make_inputs(5, 16, 64, 8, 32, 36, with_e=True)
    d = {n: to_dev(x, torch.float32) for n, x in a.items()}
    r1 = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"], d["et"])
    r2 = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"], d["et"])
    g1 = kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], r1[1], r1[0], d["dout"], d["e"])
    g2 = kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], r1[1], r1[0], d["dout"], d["e"])
    for x, y in zip((*r1, *g1), (*r2, *g2)):
        assert torch.equal(x, y)


def test_bias_row_staging_matches_per_score_loads():
    """32 < N <= 64, float32: bias rows of the [B, N, H, N] layout (a query's keys contiguous)
    are staged whole and gathered through LDS; the [B, N, N, H] layout is read one score at
    a time. The same values in either layout add the same floats in the same order, so the
    outputs are bit-identical, plain and gated (and the staged path matches the oracle)."""
    from hamiltonzero_amd import kernels

    _say("bias rows staged vs per-score loads")
    a = make_inputs(55, 6, 64, 4, 16, 36, scattered=True, with_e=True, e_layout="qhk", T=1)
    d = {n: to_dev(x, torch.float32) for n, x in a.items()}
    e2 = d["e"].permute(0, 1, 3, 2).contiguous()  # [B, N, N, H]
    et2 = d["et"].permute(0, 1, 2, 4, 3).contiguous()
    args = (d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"])
    staged = kernels.mhsea_fwd_jvp(*args, d["e"], d["et"])
    single = kernels.mhsea_fwd_jvp(*args, e2, et2, e_layout="qkh")
    gs = kernels.mhsea_fwd_jvp_gated(*args, e=d["e"], et=d["et"])
    g1 = kernels.mhsea_fwd_jvp_gated(*args, e=e2, et=et2, e_layout="qkh")
    torch.cuda.synchronize()
    for x, y in zip((*staged, *gs), (*single, *g1)):
        assert torch.equal(x, y)
    ref_out, _ = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"])
    ref_t = O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"][0], a["kt"][0], a["et"][0], a["vt"][0])
    assert rel(host(staged[0]), ref_out) <= F32_TOL
    assert rel(host(staged[2])[0], ref_t) <= F32_TOL


@pytest.mark.parametrize("layout", ["qkh", "qhk"])
@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("N,D", [(16, 32), (64, 16), (200, 64)])
def test_keymask_no_physical_key_large_logits(N, D, bf16, layout):
    """Key mask, no physical key, logits of a few hundred: the reference's float32 penalty
    rounds every logit to a multiple of 64 (pallas_attention.py:34-35), so the weights sit on
    the keys of the top multiple. The bias is 64 m + u with integer m in [-3, 3] and |u| <= 20,
    so every logit is at least 10 away from a rounding tie of fl32(s - 1e9). Every entry point
    against the oracle, plus a walker with physical keys in the same batch; both bias layouts
    (at N = 64 the [B, N, H, N] one takes the staged-row path of the forward)."""
    from hamiltonzero_amd import kernels

    _say(f"keymask empty large logits N={N} D={D} bf16={bf16} layout={layout}")
    B, H = 3, 2
    rng = np.random.default_rng(N + D)
    a = make_inputs(int(rng.integers(1000)), B, N, H, D, 0, with_e=True, e_layout=layout, T=2, bf16=bf16)
    a["mask"][1, : N // 2] = True  # walker 1 keeps physical keys
    e = 64.0 * rng.integers(-3, 4, size=a["e"].shape) + rng.uniform(-20.0, 20.0, size=a["e"].shape)
    a["e"] = torch.from_numpy(e.astype(np.float32)).bfloat16().float().numpy() if bf16 else e.astype(np.float32)
    s = O._es("bihd,bjhd->bhij", a["q"].astype(np.float64), a["k"]) + O._e_bhqk(a["e"], layout)
    assert np.abs(s).max() > 150.0
    assert np.min(np.abs((s - 32.0) / 64.0 - np.round((s - 32.0) / 64.0))) * 64.0 > 10.0
    dt = torch.bfloat16 if bf16 else torch.float32
    d = {n: to_dev(x, dt) for n, x in a.items()}
    opts = dict(key_mask=True, e_layout=layout, scale=1.0)
    tol = BF16_TOL if bf16 else F32_TOL
    # Calls that read a stored float32 lse (the tangent from (out, lse), the backward) see P
    # with the relative error of lse's rounding, up to |lse| 2^-24 (~1.2e-5 at |lse| ~ 200,
    # the float32 spacing there): their tolerance adds 4 |lse|_max 2^-24.
    out, lse, tout = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"],
                                           d["et"], **opts)
    out2, lse2 = kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"], d["e"], **opts)
    tout2 = kernels.mhsea_jvp(d["q"], d["k"], d["v"], d["mask"], out2, lse2, d["qt"], d["kt"], d["vt"], d["e"],
                              d["et"], **opts)
    dq, dk, de, dv = kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], lse2, out2, d["dout"], d["e"], **opts)
    torch.cuda.synchronize()
    ref_out, ref_lse = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"], **opts)
    for got in (out, out2):
        assert rel(host(got), ref_out) <= tol
    for got in (lse, lse2):
        assert rel(host(got), ref_lse) <= tol
    tol_lse = tol + 4.0 * np.abs(ref_lse).max() * 2.0 ** -24
    for t in range(2):
        ref_t = O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"][t], a["kt"][t], a["et"][t], a["vt"][t],
                      **opts)
        assert rel(host(tout)[t], ref_t) <= tol
        assert rel(host(tout2)[t], ref_t) <= tol_lse
    ref = O.vjp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["dout"], **opts)
    floors = vjp_floors(a, opts)
    for nm, got, want in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv), ref):
        assert rel(host(got), want, floors[nm]) <= tol_lse, nm


def test_keymask_no_physical_key_gated():
    """The gated collapse in key-mask mode with walkers that have no physical key."""
    from hamiltonzero_amd import kernels

    _say("keymask empty gated")
    a = make_inputs(77, 4, 40, 4, 16, -1, scattered=True, with_e=True, e_layout="qhk", T=2)
    a["mask"][0] = False
    a["mask"][2] = False
    d = {n: to_dev(x, torch.float32) for n, x in a.items()}
    y, ty = kernels.mhsea_fwd_jvp_gated(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"],
                                        d["et"], key_mask=True)
    torch.cuda.synchronize()
    for t in range(2):
        ref_y, ref_ty = O.gated_fwd_jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"][t], a["kt"][t],
                                        a["et"][t], a["vt"][t], key_mask=True)
        assert rel(host(y), ref_y) <= F32_TOL
        assert rel(host(ty)[t], ref_ty) <= F32_TOL


# A null query tangent with a key tangent given: dS = Kt Q^T alone must keep its scale (the
# bfloat16 kernels once zeroed the whole dS in this case). Every forward-kernel family:
NULL_QT_CASES = [
    # name, B, N, H, D, n_phys, with_e, scale, T, bf16
    ("fp32_small_n16", 4, 16, 2, 16, 11, False, 0.5, 1, False),
    ("fp32_pc_n64_d32", 8, 64, 4, 32, 36, False, 1.0, 2, False),
    ("fp32_stream_n64_d64", 3, 64, 2, 64, 48, True, 0.7, 1, False),
    ("fp32_lds_n256_d64", 2, 256, 2, 64, 200, False, 1.0, 1, False),
    ("bf16_small_n64_d64", 4, 64, 2, 64, 48, False, 1.0, 2, True),
    ("bf16_tile32_n256_d64", 2, 256, 2, 64, 230, False, 1.0, 2, True),
    ("bf16_tile32_n256_d64_scaled", 2, 256, 2, 64, 230, False, 0.125, 1, True),
    ("bf16_large_n200_d32_bias", 2, 200, 2, 32, 150, True, 0.8, 1, True),
]


@pytest.mark.parametrize("case", NULL_QT_CASES, ids=[c[0] for c in NULL_QT_CASES])
def test_null_query_tangent(case):
    from hamiltonzero_amd import kernels

    name, B, N, H, D, n_phys, with_e, scale, T, bf16 = case
    _say(f"null qt {name}")
    a = make_inputs(zlib.crc32(name.encode()) % 1000, B, N, H, D, n_phys, scattered=True, with_e=with_e, T=T,
                    bf16=bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    d = {n: to_dev(x, dt) for n, x in a.items()}
    out, _, tout = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], None, d["kt"], d["vt"], d["e"], d["et"],
                                         scale=scale)
    torch.cuda.synchronize()
    tol = BF16_TOL if bf16 else F32_TOL
    zero = np.zeros_like(a["q"])
    for t in range(T):
        et = None if a["et"] is None else a["et"][t]
        ref_t = O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], zero, a["kt"][t], et, a["vt"][t], scale=scale)
        assert rel(host(tout)[t], ref_t) <= tol, f"tangent {t}"


def test_bf16_tile32_matches_large_kernel_full_n():
    """The 32-query-tile kernel (no bias) against the 16-query-wave kernel (reached with an
    all-zero bias, the same mathematics) at c5's N and H, every walker's count different:
    both are bf16 products with fp32 softmax, so they agree to bf16 rounding."""
    from hamiltonzero_amd import kernels

    _say("bf16 32-query tiles vs 16-query kernel N=1024 H=16")
    B, N, H, D, T = 3, 1024, 16, 64, 2
    g = torch.Generator(device="cuda").manual_seed(11)
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g, device="cuda") * sc).to(torch.bfloat16)
    q, k, v = r(B, N, H, D, sc=D ** -0.5), r(B, N, H, D, sc=D ** -0.5), r(B, N, H, D)
    qt, kt, vt = r(T, B, N, H, D), r(T, B, N, H, D), r(T, B, N, H, D)
    mask = torch.zeros(B, N, dtype=torch.bool, device="cuda")
    for b, n in enumerate((1000, 777, 1024)):
        mask[b, torch.randperm(N, generator=g, device="cuda")[:n]] = True
    e0 = torch.zeros(B, N, H, N, dtype=torch.bfloat16, device="cuda")
    o1, l1, t1 = kernels.mhsea_fwd_jvp(q, k, v, mask, qt, kt, vt)
    o2, l2, t2 = kernels.mhsea_fwd_jvp(q, k, v, mask, qt, kt, vt, e0, torch.zeros(T, B, N, H, N, dtype=torch.bfloat16,
                                                                                  device="cuda"))
    torch.cuda.synchronize()
    assert rel(host(o1), host(o2)) <= BF16_TOL
    assert rel(host(l1), host(l2)) <= 1e-3  # the 32-query-tile kernel normalises by its rounded weights
    for t in range(T):
        assert rel(host(t1)[t], host(t2)[t]) <= BF16_TOL, f"tangent {t}"
    m = mask.cpu().numpy()
    assert np.all(host(o1)[~m] == 0.0) and np.all(host(t1)[:, ~m] == 0.0)
