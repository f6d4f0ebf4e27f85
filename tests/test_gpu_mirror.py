"""GPU parity of the reference-named Python mirror against the float64 oracle.

Exercises the functions a caller of the reference uses, end to end on the gfx950 kernels:
``mhsea_with_tuned_ad`` in reverse mode (``torch.autograd``, the transpose rule) and forward
mode (``torch.autograd.forward_ad``, the lin primitive), the primitives
``mhsea_tuned_ad`` / ``mhsea_tuned_ad_lin`` / ``mhsea_tuned_ad_lin_transpose``, the batched
tangents of ``mhsea_tuned_jvp``, and the op-level ``mhsea_tuned_edge_attention`` /
``reference_edge_attention`` (per system and batched, a head dimension padded on the host,
and the fallback to the jnp formula). Tolerance: max-norm relative error <= 1e-5 (float32).
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a.detach().cpu().numpy() if torch.is_tensor(a) else a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def make(seed, B, N, H, D, n_phys, with_e=True):
    rng = np.random.default_rng(seed)
    shape = (B, N, H, D)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(D ** -0.5) for _ in range(3))
    e = rng.standard_normal((B, N, H, N), dtype=np.float32) * np.float32(0.5) if with_e else None
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        mask[b, rng.permutation(N)[:n_phys]] = True
    tans = [rng.standard_normal(shape, dtype=np.float32) for _ in range(3)]
    et = rng.standard_normal((B, N, H, N), dtype=np.float32) if with_e else None
    cot = rng.standard_normal(shape, dtype=np.float32)
    return dict(q=q, k=k, v=v, e=e, mask=mask, qt=tans[0], kt=tans[1], vt=tans[2], et=et, cot=cot)


def dev(x, grad=False):
    if x is None:
        return None
    t = torch.from_numpy(x).cuda()
    return t.requires_grad_(True) if grad else t


@pytest.mark.parametrize("N,D,n_phys", [(64, 32, 36), (32, 16, 20), (96, 64, 80)])
def test_with_tuned_ad_reverse_mode(N, D, n_phys):
    from hamiltonzero_amd import mhsea_with_tuned_ad

    _say(f"mirror reverse N={N} D={D}")
    a = make(31, 3, N, 2, D, n_phys)
    q, k, e, v = (dev(a[n], grad=True) for n in ("q", "k", "e", "v"))
    out = mhsea_with_tuned_ad(q, k, e, v, dev(a["mask"]))
    out.backward(dev(a["cot"]))
    torch.cuda.synchronize()
    want_out, _ = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"])
    dq, dk, de, dv = O.vjp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["cot"])
    assert rel(out, want_out) <= TOL
    for name, got, want in (("dq", q.grad, dq), ("dk", k.grad, dk), ("de", e.grad, de), ("dv", v.grad, dv)):
        assert rel(got, want) <= TOL, name


@pytest.mark.parametrize("N,D,n_phys", [(64, 32, 36), (16, 8, 11)])
def test_with_tuned_ad_forward_mode(N, D, n_phys):
    import torch.autograd.forward_ad as fwAD

    from hamiltonzero_amd import mhsea_with_tuned_ad

    _say(f"mirror forward mode N={N} D={D}")
    a = make(32, 2, N, 2, D, n_phys)
    with fwAD.dual_level():
        duals = [fwAD.make_dual(dev(a[p]), dev(a[t])) for p, t in (("q", "qt"), ("k", "kt"), ("e", "et"), ("v", "vt"))]
        out = mhsea_with_tuned_ad(duals[0], duals[1], duals[2], duals[3], dev(a["mask"]))
        primal, tangent = fwAD.unpack_dual(out)
        torch.cuda.synchronize()
    want_out, _ = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"])
    want_t = O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"], a["kt"], a["et"], a["vt"])
    assert rel(primal, want_out) <= TOL
    assert rel(tangent, want_t) <= TOL


def test_primitives_lin_and_transpose():
    from hamiltonzero_amd import mhsea_tuned_ad, mhsea_tuned_ad_lin, mhsea_tuned_ad_lin_transpose

    _say("mirror primitives")
    a = make(33, 2, 64, 3, 32, 40)
    d = {n: dev(x) for n, x in a.items()}
    out, lse = mhsea_tuned_ad(d["q"], d["k"], d["e"], d["v"], d["mask"])
    tout = mhsea_tuned_ad_lin(d["q"], d["k"], d["e"], d["v"], d["mask"], out, lse, d["qt"], d["kt"], d["et"], d["vt"])
    dq, dk, de, dv = mhsea_tuned_ad_lin_transpose(d["cot"], d["q"], d["k"], d["e"], d["v"], d["mask"], out, lse)
    torch.cuda.synchronize()
    want_out, want_lse = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"])
    m = a["mask"]
    assert rel(out, want_out) <= TOL
    assert rel(lse.cpu().numpy()[m], want_lse[m]) <= TOL
    assert rel(tout, O.jvp(a["q"], a["k"], a["e"], a["v"], m, a["qt"], a["kt"], a["et"], a["vt"])) <= TOL
    for got, want in zip((dq, dk, de, dv), O.vjp(a["q"], a["k"], a["e"], a["v"], m, a["cot"])):
        assert rel(got, want) <= TOL


def test_batched_tangent_directions():
    from hamiltonzero_amd import mhsea_tuned_jvp

    _say("mirror batched tangents T=3")
    rng = np.random.default_rng(34)
    a = make(34, 2, 64, 2, 32, 36, with_e=False)
    T = 3
    qt, kt, vt = (rng.standard_normal((T, 2, 64, 2, 32), dtype=np.float32) for _ in range(3))
    out, tout = mhsea_tuned_jvp(dev(a["q"]), dev(a["k"]), None, dev(a["v"]), dev(a["mask"]), dev(qt), dev(kt), None, dev(vt))
    torch.cuda.synchronize()
    for t in range(T):
        want = O.jvp(a["q"], a["k"], None, a["v"], a["mask"], qt[t], kt[t], None, vt[t])
        assert rel(tout[t], want) <= TOL, t


@pytest.mark.parametrize("n,d,batched", [(64, 32, False), (16, 16, True), (64, 12, False), (48, 32, True), (20, 64, False)])
def test_op_level_edge_attention(n, d, batched):
    """Tuned / full-AD shapes (square mask, masked rows zero), a head dimension the kernels
    do not take (12, zero-padded to 16 on the host) and the jnp fallback (n = 48, 20:
    additive key mask, every row computed)."""
    from hamiltonzero_amd import mhsea_tuned_edge_attention, reference_edge_attention

    _say(f"mirror op-level n={n} d={d} batched={batched}")
    rng = np.random.default_rng(35 + n + d)
    B, h = 2, 3
    Q, K, V = (rng.standard_normal((B, n, h, d), dtype=np.float32) for _ in range(3))
    E = rng.standard_normal((B, n, n, h), dtype=np.float32) * np.float32(0.5)
    M = np.zeros((B, n), dtype=bool)
    for b in range(B):
        M[b, rng.permutation(n)[: (3 * n) // 4]] = True
    tuned = d in (8, 16, 32, 64) and ((n >= 64 and n % 32 == 0) or (0 < n < 64 and n & (n - 1) == 0))
    scale = d ** -0.5
    want, _ = O.fwd(Q, K, E, V, M, scale=scale, key_mask=not tuned, e_layout="qkh")
    want_ref, _ = O.fwd(Q, K, E, V, M, scale=scale, key_mask=True, e_layout="qkh")
    if batched:
        got = mhsea_tuned_edge_attention(dev(Q), dev(K), dev(V), dev(E), dev(M))
        got_ref = reference_edge_attention(dev(Q), dev(K), dev(V), dev(E), dev(M))
    else:
        got = torch.stack([mhsea_tuned_edge_attention(dev(Q[b]), dev(K[b]), dev(V[b]), dev(E[b]), dev(M[b])) for b in range(B)])
        got_ref = torch.stack([reference_edge_attention(dev(Q[b]), dev(K[b]), dev(V[b]), dev(E[b]), dev(M[b])) for b in range(B)])
    torch.cuda.synchronize()
    assert rel(got, want) <= TOL
    assert rel(got_ref, want_ref) <= TOL
    assert rel(got_ref[0].cpu().numpy(), O.reference_edge_attention(Q[0], K[0], V[0], E[0], M[0])) <= TOL
