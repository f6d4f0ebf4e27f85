"""GPU parity at the configurations' real item counts (C ABI via ctypes).

The persistent kernels launch a fixed grid (compute units x workgroups per unit) that walks
the (walker, head) items: workgroup L takes items L, L + G, L + 2G, ... and carries state
from one item to the next (double-buffered LDS, site lists published items ahead, register
prefetch of the next item's rows). These cases run whole batches where every workgroup
walks many items — c2 at its full [1024, 64, 8, 32] (8192 items, 16 per workgroup), the c3
backward at [512, 64, 8, 64], the fp32 D = 64 streaming kernels at B * H = 2048 — and compare
walkers spread over every period and every workgroup residue with the float64 oracle
(the oracle is per walker, so evaluating it on a sample equals evaluating it on the batch
and selecting). Rows the reference defines as exact zeros are checked on the whole batch.

Tolerances as everywhere: max-norm relative error <= 1e-5 for float32, <= 2e-2 for bfloat16
storage (oracle on the bf16-rounded inputs); where the exact cotangent cancels the
denominator is floored by 1% of the uncancelled magnitude of the same sums.
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O
from test_gpu_parity import BF16_TOL, F32_TOL, host, make_inputs, rel, to_dev, vjp_floors

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


def sample_walkers(B, n=64):
    """Walkers spread over the batch: n strided picks with a varying offset inside each
    stride (so consecutive periods of a workgroup walk and different workgroup residues are
    both covered), plus the first and last two walkers."""
    step = max(B // n, 1)
    picks = {k * step + (5 * k) % step for k in range(min(n, B))}
    picks |= {0, 1, B - 2, B - 1}
    return np.array(sorted(b for b in picks if 0 <= b < B))


def _sub(a, idx):
    """The inputs of walkers idx (tangents carry the direction axis first)."""
    out = {}
    for name, x in a.items():
        if x is None:
            out[name] = None
        elif name in ("qt", "kt", "vt", "et"):
            out[name] = x[:, idx]
        else:
            out[name] = x[idx]
    return out


def _case(seed, B, N, H, D, n_phys, *, scattered=False, with_e=False, e_layout="qhk", T=1, bf16=False):
    a = make_inputs(seed, B, N, H, D, n_phys, scattered=scattered, with_e=with_e, e_layout=e_layout, T=T,
                    bf16=bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    d = {n: to_dev(x, dt) for n, x in a.items()}
    return a, d, (BF16_TOL if bf16 else F32_TOL)


FWD_JVP_CASES = [
    # name, seed, B, N, H, D, n_phys, scattered, with_e, e_layout, key_mask, T, bf16
    ("c2_full_t1", 101, 1024, 64, 8, 32, 36, False, False, "qhk", False, 1, False),
    ("c2_full_t2", 102, 1024, 64, 8, 32, 36, False, False, "qhk", False, 2, False),
    ("c2_full_counts_bias", 103, 1024, 64, 8, 32, -1, True, True, "qhk", False, 1, False),
    ("c2_full_keymask_counts_qkh", 104, 1024, 64, 8, 32, -1, True, True, "qkh", True, 1, False),
    ("d64_stream_t1", 105, 256, 64, 8, 64, 48, False, False, "qhk", False, 1, False),
    ("d64_stream_counts_t1", 106, 256, 64, 8, 64, -1, True, False, "qhk", False, 1, False),
    ("c3_shape_bf16_fwd_t1", 107, 512, 64, 8, 64, 48, False, False, "qhk", False, 1, True),
]


@pytest.mark.parametrize("case", FWD_JVP_CASES, ids=[c[0] for c in FWD_JVP_CASES])
def test_fwd_jvp_at_item_counts(case):
    from hamiltonzero_amd import kernels

    name, seed, B, N, H, D, n_phys, scattered, with_e, e_layout, key_mask, T, bf16 = case
    _say(f"fwd_jvp items {name} B={B} N={N} H={H} D={D} T={T}")
    a, d, tol = _case(seed, B, N, H, D, n_phys, scattered=scattered, with_e=with_e, e_layout=e_layout, T=T,
                      bf16=bf16)
    opts = dict(key_mask=key_mask, e_layout=e_layout)
    out, lse, tout = kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"],
                                           d["e"], d["et"], **opts)
    tout_l = kernels.mhsea_jvp(d["q"], d["k"], d["v"], d["mask"], out, lse, d["qt"], d["kt"], d["vt"],
                               d["e"], d["et"], **opts)
    torch.cuda.synchronize()
    out_h, lse_h, tout_h, tout_lh = host(out), host(lse), host(tout), host(tout_l)
    m = a["mask"]
    if not key_mask:  # masked rows are exact zeros in out and every tangent, on the whole batch
        assert np.all(out_h[~m] == 0.0)
        assert np.all(tout_h[:, ~m] == 0.0)
        assert np.all(tout_lh[:, ~m] == 0.0)
    idx = sample_walkers(B)
    s = _sub(a, idx)
    ref_out, ref_lse = O.fwd(s["q"], s["k"], s["e"], s["v"], s["mask"], **opts)
    assert rel(out_h[idx], ref_out) <= tol
    sm = s["mask"] if not key_mask else np.ones_like(s["mask"])
    if sm.any():
        assert rel(lse_h[idx][sm], ref_lse[sm]) <= tol
    for t in range(T):
        et = None if s["et"] is None else s["et"][t]
        ref_t = O.jvp(s["q"], s["k"], s["e"], s["v"], s["mask"], s["qt"][t], s["kt"][t], et, s["vt"][t], **opts)
        assert rel(tout_h[t][idx], ref_t) <= tol, f"fused tangent {t}"
        assert rel(tout_lh[t][idx], ref_t) <= tol, f"tangent from (out, lse) {t}"


def test_fwd_only_at_item_counts():
    """The forward-only launch (T = 0 variant) at c2's full shape."""
    from hamiltonzero_amd import kernels

    _say("fwd items c2 full")
    a, d, tol = _case(111, 1024, 64, 8, 32, 36, scattered=True)
    out, lse = kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"])
    torch.cuda.synchronize()
    out_h, lse_h = host(out), host(lse)
    assert np.all(out_h[~a["mask"]] == 0.0)
    idx = sample_walkers(1024)
    s = _sub(a, idx)
    ref_out, ref_lse = O.fwd(s["q"], s["k"], None, s["v"], s["mask"])
    assert rel(out_h[idx], ref_out) <= tol
    assert rel(lse_h[idx][s["mask"]], ref_lse[s["mask"]]) <= tol


BWD_CASES = [
    # name, seed, B, N, H, D, n_phys, scattered, with_e, e_layout, key_mask, bf16
    ("c3_bf16_bwd", 121, 512, 64, 8, 64, 48, False, False, "qhk", False, True),
    ("c3_bf16_bwd_counts_bias", 122, 512, 64, 8, 64, -1, True, True, "qhk", False, True),
    ("d64_stream_bwd_fp32", 123, 256, 64, 8, 64, 48, False, False, "qhk", False, False),
    ("d64_stream_bwd_fp32_bias_qkh", 124, 256, 64, 8, 64, -1, True, True, "qkh", False, False),
    ("c2_full_bwd_fp32", 125, 1024, 64, 8, 32, 36, True, False, "qhk", False, False),
    ("c2_full_bwd_keymask_counts", 126, 1024, 64, 8, 32, -1, True, True, "qkh", True, False),
]


@pytest.mark.parametrize("case", BWD_CASES, ids=[c[0] for c in BWD_CASES])
def test_bwd_at_item_counts(case):
    from hamiltonzero_amd import kernels

    name, seed, B, N, H, D, n_phys, scattered, with_e, e_layout, key_mask, bf16 = case
    _say(f"bwd items {name} B={B} N={N} H={H} D={D}")
    a, d, tol = _case(seed, B, N, H, D, n_phys, scattered=scattered, with_e=with_e, e_layout=e_layout, T=1,
                      bf16=bf16)
    opts = dict(key_mask=key_mask, e_layout=e_layout)
    out, lse = kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"], d["e"], **opts)
    dq, dk, de, dv = kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], lse, out, d["dout"], d["e"],
                                       want_de=with_e, **opts)
    torch.cuda.synchronize()
    got = {"dq": host(dq), "dk": host(dk), "de": host(de), "dv": host(dv)}
    m = a["mask"]
    if not key_mask:
        for nm in ("dq", "dk", "dv"):
            assert np.all(got[nm][~m] == 0.0), nm
    idx = sample_walkers(B)
    s = _sub(a, idx)
    ref = dict(zip(("dq", "dk", "de", "dv"), O.vjp(s["q"], s["k"], s["e"], s["v"], s["mask"], s["dout"], **opts)))
    floors = vjp_floors(s, dict(opts, scale=1.0))
    for nm in ("dq", "dk", "de", "dv"):
        if got[nm] is None:
            continue
        assert rel(got[nm][idx], ref[nm], floors[nm]) <= tol, nm


@pytest.mark.parametrize("seed,H,D", [(131, 8, 32), (132, 32, 16)], ids=["c2_shape", "trunk_shape"])
def test_gated_at_item_counts(seed, H, D):
    """The gated collapse at full batch with per-walker scattered masks and bias: c2's shape
    (bias read per score) and the trunk's [1024, 64, 32, 16] (bias rows staged through LDS,
    16 head pairs per walker, 32 items per workgroup)."""
    from hamiltonzero_amd import kernels

    _say(f"gated items B=1024 H={H} D={D}")
    a, d, tol = _case(seed, 1024, 64, H, D, -1, scattered=True, with_e=True)
    y, ty = kernels.mhsea_fwd_jvp_gated(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"],
                                        d["et"])
    torch.cuda.synchronize()
    y_h, ty_h = host(y), host(ty)
    assert np.all(y_h[~a["mask"]] == 0.0)
    idx = sample_walkers(1024)
    s = _sub(a, idx)
    ref_y, ref_ty = O.gated_fwd_jvp(s["q"], s["k"], s["e"], s["v"], s["mask"], s["qt"][0], s["kt"][0],
                                    s["et"][0], s["vt"][0])
    assert rel(y_h[idx], ref_y) <= tol
    assert rel(ty_h[0][idx], ref_ty) <= tol


def test_device_of_every_operand_is_checked():
    """A host tensor among the operands is a ValueError before anything is enqueued."""
    from hamiltonzero_amd import kernels

    _say("device checks")
    a, d, _ = _case(141, 2, 64, 2, 32, 30, with_e=True)
    cpu = {n: None if x is None else torch.from_numpy(np.ascontiguousarray(x)) for n, x in a.items()}
    with pytest.raises(ValueError, match="e is on cpu"):
        kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"], cpu["e"])
    with pytest.raises(ValueError, match="qt is on cpu"):
        kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], cpu["qt"], d["kt"], d["vt"])
    with pytest.raises(ValueError, match="et is on cpu"):
        kernels.mhsea_fwd_jvp(d["q"], d["k"], d["v"], d["mask"], d["qt"], d["kt"], d["vt"], d["e"], cpu["et"])
    out, lse = kernels.mhsea_fwd(d["q"], d["k"], d["v"], d["mask"])
    with pytest.raises(ValueError, match="lse is on cpu"):
        kernels.mhsea_jvp(d["q"], d["k"], d["v"], d["mask"], out, lse.cpu(), d["qt"])
    with pytest.raises(ValueError, match="dout is on cpu"):
        kernels.mhsea_bwd(d["q"], d["k"], d["v"], d["mask"], lse, out, cpu["dout"])
    bias = torch.zeros((2, 64, 64, 2))
    with pytest.raises(ValueError, match="bias is on cpu"):
        kernels.rect_attention_fwd(d["q"], d["k"], d["v"], bias)
    torch.cuda.synchronize()
