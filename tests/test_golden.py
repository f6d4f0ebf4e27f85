"""Golden fixtures of the MHSEA path (``tests/golden/*.npz``, written by
``tests/golden/make_golden.py``): seeded inputs with the float64 oracle's forward, tangent
and VJP outputs.

CPU: the oracle still reproduces every fixture (a regression guard on the checker itself).
GPU: the HIP path, called through the C ABI, matches the stored outputs without running the
oracle — float32 I/O to 1e-5, bfloat16 I/O to 2e-2 (max-norm relative error per tensor) —
and writes exact zeros on masked rows.
"""

import glob
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
# rect_*.npz belong to the rectangular forward (tests/test_golden_rect.py)
FILES = sorted(f for f in glob.glob(os.path.join(HERE, "golden", "*.npz")) if not os.path.basename(f).startswith("rect_"))
IDS = [os.path.basename(f)[:-4] for f in FILES]

F32_TOL = 1e-5
BF16_TOL = 2e-2


def rel(a, b, floor=0.0):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = max(np.max(np.abs(b)), floor, 1e-30)
    return float(np.max(np.abs(a - b)) / den)


def load(path):
    """Inputs (float32; bfloat16 bit patterns widened), expected outputs, options."""
    z = np.load(path, allow_pickle=False)
    scale, key_mask, qkh, T, bf16 = z["meta"]
    bf16 = bool(bf16)
    a = {}
    for n in ("q", "k", "v", "e", "qt", "kt", "vt", "et", "dout"):
        key = f"in_{n}"
        if key not in z:
            a[n] = None
            continue
        x = z[key]
        a[n] = (x.astype(np.uint32) << 16).view(np.float32) if x.dtype == np.uint16 else x
    a["mask"] = z["in_mask"]
    want = {n[5:]: z[n] for n in z.files if n.startswith("want_")}
    opts = dict(scale=float(scale), key_mask=bool(key_mask), e_layout="qkh" if qkh else "qhk")
    return a, want, opts, int(T), bf16, z["vjp_floors"]


def test_fixtures_present():
    assert len(FILES) >= 6


@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_oracle_reproduces_fixture(path):
    import sys

    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_golden import expected

    a, want, opts, T, _, _ = load(path)
    got = expected(a, opts, T)
    for n, w in want.items():
        assert rel(got[n], w) <= 1e-6, n


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_hip_path_matches_fixture(path):
    import torch

    from hamiltonzero_amd import kernels

    a, want, opts, T, bf16, floors = load(path)
    print(f"[case] golden {os.path.basename(path)}", flush=True)
    dt = torch.bfloat16 if bf16 else torch.float32
    tol = BF16_TOL if bf16 else F32_TOL
    d = {n: None if x is None else torch.from_numpy(x).to(device="cuda", dtype=dt) for n, x in a.items() if n != "mask"}
    d["mask"] = torch.from_numpy(a["mask"]).cuda()
    host = lambda t: t.float().cpu().numpy()  # noqa: E731
    m = a["mask"]

    out, lse, tout = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"],
                                           d["et"], **opts)
    tout2 = kernels.mhsea_jvp(d["q"], d["k"], d["v"], d["mask"], out, lse, d["qt"], d["kt"], d["vt"], d["e"],
                              d["et"], **opts)
    dq, dk, de, dv = kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], lse, out, d["dout"], d["e"], want_de=True,
                                       **opts)
    torch.cuda.synchronize()

    assert rel(host(out), want["out"]) <= tol
    sel = m if not opts["key_mask"] else np.ones_like(m)
    assert rel(host(lse)[sel], want["lse"][sel]) <= tol
    for t in range(T):
        assert rel(host(tout)[t], want["tout"][t]) <= tol, f"fused tangent {t}"
        assert rel(host(tout2)[t], want["tout"][t]) <= tol, f"tangent {t} from out, lse"
    for name, got, floor in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv), floors):
        assert rel(host(got), want[name], floor) <= tol, name
    if not opts["key_mask"]:
        for name, got in (("out", out), ("tout", tout[0]), ("dq", dq), ("dk", dk), ("dv", dv)):
            assert np.all(host(got)[~m] == 0.0), name
