"""GPU parity under the route decoder's masking convention.

``route_pointer.py:2042-2048`` does not pass its mask to the attention: it writes -1e30 into
the pair bias wherever (query i, key j) is invalid — key j masked, or the pair excluded by the
attention mask — passes an all-ones key mask, and afterwards zeroes the output rows of queries
with no valid key (``:2082``, ``has_key``). So the kernels see every site as physical and a
bias whose invalid entries are -1e30, including whole rows of -1e30.

In float32 ``q.k + (-1e30)`` is -1e30 (|q.k| is far below half an ulp of 1e30), so a row with
at least one valid key gives its invalid keys weight exactly 0, and a row with none has equal
scores everywhere. Its softmax is then degenerate (jax.nn.softmax gives uniform weights, the
reference's Pallas primitive exp(S - lse) with lse absorbed into -1e30 gives weight 1 per key)
and the caller discards it, so these tests compare the route's own observable result — the
attention output with no-key rows zeroed, its tangent and its cotangents — with the float64
oracle (all-ones mask, the -1e30 bias) and require every raw output, no-key rows included, to
be finite. Shapes cover the op-level dispatch of ``pallas_attention.py:50-61``: full-AD sizes
(n = 8, 16, 32), the tuned sizes (64, 128, 256) and the jnp fallback (n = 48), through the
reference-named mirror (``mhsea_tuned_edge_attention``) in reverse and forward mode, and the
kernel entry points (fused forward + JVP, the tangent from (out, lse), the backward) directly,
automatic and LDS-streaming. Tolerance: max-norm relative error <= 1e-5 (float32).
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5
NEG = np.float32(-1.0e30)


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a.detach().cpu().numpy() if torch.is_tensor(a) else a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def make_route(seed, B, n, h, d):
    """Route-shaped inputs: q, k, v [B, n, h, d] (unscaled: the op applies d^-1/2), the pair
    bias [B, n, n, h] with -1e30 on invalid pairs, its tangent (zero on invalid pairs, as the
    where() with a constant makes it), tangents of q, k, v, a cotangent, and has_key [B, n].
    Walker 0 has no physical key at all; walker 1 has an attention mask that empties some
    rows; the others draw a key mask (about 70%) and a random attention mask (about 80%)."""
    rng = np.random.default_rng(seed)
    shape = (B, n, h, d)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) for _ in range(3))
    edge = rng.standard_normal((B, n, n, h), dtype=np.float32) * np.float32(0.5)
    key_mask = rng.random((B, n)) < 0.7
    attn = rng.random((B, n, n)) < 0.8
    key_mask[0] = False
    attn[1, ::3] = False  # every third query row of walker 1 has no valid key
    valid = key_mask[:, None, :] & attn
    has_key = valid.any(axis=-1)
    bias = np.where(valid[..., None], edge, NEG).astype(np.float32)
    tans = [rng.standard_normal(shape, dtype=np.float32) for _ in range(3)]
    et = np.where(valid[..., None], rng.standard_normal((B, n, n, h), dtype=np.float32), 0.0).astype(np.float32)
    cot = rng.standard_normal(shape, dtype=np.float32)
    return dict(q=q, k=k, v=v, bias=bias, qt=tans[0], kt=tans[1], vt=tans[2], et=et, cot=cot, has_key=has_key)


def _zero_no_key(x, has_key):
    return np.where(has_key[:, :, None, None], x, 0.0)


def dev(x, grad=False):
    t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    return t.requires_grad_(True) if grad else t


ROUTE_SHAPES = [(8, 16), (16, 32), (32, 16), (64, 16), (64, 32), (128, 32), (256, 16), (48, 32)]


@pytest.mark.parametrize("n,d", ROUTE_SHAPES, ids=[f"n{n}_d{d}" for n, d in ROUTE_SHAPES])
def test_route_convention_reverse_mode(n, d):
    """out = where(has_key, mhsea_tuned_edge_attention(q, k, v, bias, ones), 0) and its
    cotangents for q, k, v and the bias, against the oracle of the same composition."""
    from hamiltonzero_amd import mhsea_tuned_edge_attention

    B, h = 4, 3
    _say(f"route reverse n={n} d={d}")
    a = make_route(900 + n + d, B, n, h, d)
    ones = np.ones((B, n), dtype=np.int32)
    q, k, v, bias = (dev(a[nm], grad=True) for nm in ("q", "k", "v", "bias"))
    raw = mhsea_tuned_edge_attention(q, k, v, bias, dev(ones))
    hk = dev(a["has_key"])
    out = torch.where(hk[:, :, None, None], raw, torch.zeros_like(raw))
    out.backward(dev(a["cot"]))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(raw).all()), "raw output (no-key rows included) must be finite"
    scale = d ** -0.5
    m = np.ones((B, n), dtype=bool)
    want, _ = O.fwd(a["q"], a["k"], a["bias"], a["v"], m, scale=scale, e_layout="qkh")
    assert rel(out, _zero_no_key(want, a["has_key"])) <= TOL, "out"
    cot = _zero_no_key(a["cot"], a["has_key"])  # the transpose of the where()
    dq, dk, de, dv = O.vjp(a["q"], a["k"], a["bias"], a["v"], m, cot, scale=scale, e_layout="qkh")
    for name, got, ref in (("dq", q.grad, dq), ("dk", k.grad, dk), ("dv", v.grad, dv), ("dbias", bias.grad, de)):
        assert bool(torch.isfinite(got).all()), name
        assert rel(got, ref) <= TOL, name


@pytest.mark.parametrize("n,d", ROUTE_SHAPES, ids=[f"n{n}_d{d}" for n, d in ROUTE_SHAPES])
def test_route_convention_forward_mode(n, d):
    """The tangent of the same composition (tangents of q, k, v and of the bias on valid
    pairs), against the oracle's jvp with the no-key rows zeroed."""
    import torch.autograd.forward_ad as fwAD

    from hamiltonzero_amd import mhsea_tuned_edge_attention

    B, h = 4, 2
    _say(f"route forward mode n={n} d={d}")
    a = make_route(950 + n + d, B, n, h, d)
    ones = np.ones((B, n), dtype=np.int32)
    hk = dev(a["has_key"])
    with fwAD.dual_level():
        duals = [fwAD.make_dual(dev(a[p]), dev(a[t])) for p, t in (("q", "qt"), ("k", "kt"), ("v", "vt"),
                                                                   ("bias", "et"))]
        raw = mhsea_tuned_edge_attention(duals[0], duals[1], duals[2], duals[3], dev(ones))
        rp, rt = fwAD.unpack_dual(raw)
        torch.cuda.synchronize()
    assert bool(torch.isfinite(rp).all()) and bool(torch.isfinite(rt).all())
    keep = hk[:, :, None, None]
    scale = d ** -0.5
    m = np.ones((B, n), dtype=bool)
    want, _ = O.fwd(a["q"], a["k"], a["bias"], a["v"], m, scale=scale, e_layout="qkh")
    want_t = O.jvp(a["q"], a["k"], a["bias"], a["v"], m, a["qt"], a["kt"], a["et"], a["vt"], scale=scale,
                   e_layout="qkh")
    assert rel(torch.where(keep, rp, 0.0), _zero_no_key(want, a["has_key"])) <= TOL, "out"
    assert rel(torch.where(keep, rt, 0.0), _zero_no_key(want_t, a["has_key"])) <= TOL, "tangent"


@pytest.mark.parametrize("generic", [False, True], ids=["auto", "generic"])
@pytest.mark.parametrize("n,d,T", [(64, 32, 1), (64, 16, 2), (96, 64, 1), (32, 32, 2), (256, 32, 1)])
def test_route_convention_kernel_entry_points(n, d, T, generic):
    """The C-ABI entry points under the route's bias: fused forward + JVP (T directions), the
    tangent from (out, lse) (the reference's lin primitive) and the backward, bias in the
    [B, n, n, h] layout with its tangents, on the rows that have a valid key; every output
    finite."""
    from hamiltonzero_amd import kernels

    B, h = 5, 2
    _say(f"route kernels n={n} d={d} T={T} generic={generic}")
    a = make_route(1000 + n + d + T, B, n, h, d)
    rng = np.random.default_rng(n * d + T)
    qt, kt, vt = (rng.standard_normal((T, B, n, h, d), dtype=np.float32) for _ in range(3))
    valid = a["bias"][..., 0] > NEG  # [B, n, n]: the same for every head
    et = np.where(valid[None, ..., None], rng.standard_normal((T, B, n, n, h), dtype=np.float32), 0.0)
    et = et.astype(np.float32)
    scale = d ** -0.5
    opts = dict(scale=scale, e_layout="qkh", generic=generic)
    mask = dev(np.ones((B, n), dtype=bool))
    q, k, v, e = (dev(a[nm]) for nm in ("q", "k", "v", "bias"))
    out, lse, tout = kernels.mhsea_fwd_jvp(q, k, v, mask, dev(qt), dev(kt), dev(vt), e, dev(et), **opts)
    tout_l = kernels.mhsea_jvp(q, k, v, mask, out, lse, dev(qt), dev(kt), dev(vt), e, dev(et), **opts)
    cot = _zero_no_key(a["cot"], a["has_key"]).astype(np.float32)
    dq, dk, de, dv = kernels.mhsea_bwd(q, k, v, mask, lse, out, dev(cot), e, want_de=True, **opts)
    torch.cuda.synchronize()
    for name, t in (("out", out), ("tout", tout), ("tout_lin", tout_l), ("dq", dq), ("dk", dk), ("de", de),
                    ("dv", dv)):
        assert bool(torch.isfinite(t).all()), f"{name}: non-finite values"
    m = np.ones((B, n), dtype=bool)
    oo = dict(scale=scale, e_layout="qkh")
    hk = a["has_key"]
    want, want_lse = O.fwd(a["q"], a["k"], a["bias"], a["v"], m, **oo)
    assert rel(_zero_no_key(out.cpu().numpy(), hk), _zero_no_key(want, hk)) <= TOL, "out"
    assert rel(lse.cpu().numpy()[hk], want_lse[hk]) <= TOL, "lse"
    for t in range(T):
        want_t = _zero_no_key(O.jvp(a["q"], a["k"], a["bias"], a["v"], m, qt[t], kt[t], et[t], vt[t], **oo), hk)
        assert rel(_zero_no_key(tout[t].cpu().numpy(), hk), want_t) <= TOL, f"fused tangent {t}"
        assert rel(_zero_no_key(tout_l[t].cpu().numpy(), hk), want_t) <= TOL, f"tangent from (out, lse) {t}"
    ref = O.vjp(a["q"], a["k"], a["bias"], a["v"], m, cot, **oo)
    for name, got, want_g in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv), ref):
        assert rel(got, want_g) <= TOL, name
