"""Pins the float64 oracle (oracle/mhsea_oracle.py) without the reference's own code.

The reference holds no golden vectors or tests for this path (its only test file is
tests/test_fermionic.py) and JAX is not installed, so each oracle function is pinned by
checks that a plausible mistake (dropped term, wrong sign, wrong index, transposed
operand) fails:
  forward  — explicit Python loops on tiny inputs; closed-form special cases;
             invariances (key permutation, masked-site values, per-row bias shift);
  tangent  — central finite differences of the forward; torch forward-mode autodiff of an
             independent float64 torch formula; closed forms (dV = V, constant dE);
  cotangent— transpose identity <J t, c> = <t, J^T c> against the pinned tangent; torch
             reverse-mode autodiff; sum_k de = 0 on physical rows.
Planted-mistake tests at the end show these checks reject a broken oracle.
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O

MODES = [
    dict(key_mask=False, e_layout="qhk", scale=1.0),
    dict(key_mask=False, e_layout="qkh", scale=0.5),
    dict(key_mask=True, e_layout="qkh", scale=32 ** -0.5),
]


def make(rng, B, N, H, D, n_phys=None, scattered=False, with_e=True, e_layout="qhk"):
    q = rng.standard_normal((B, N, H, D)) / np.sqrt(D)
    k = rng.standard_normal((B, N, H, D)) / np.sqrt(D)
    v = rng.standard_normal((B, N, H, D)) / np.sqrt(D)
    eshape = (B, N, H, N) if e_layout == "qhk" else (B, N, N, H)
    e = rng.standard_normal(eshape) * 0.5 if with_e else None
    mask = np.ones((B, N), dtype=bool)
    if n_phys is not None:
        mask[:] = False
        for b in range(B):
            sites = rng.permutation(N)[:n_phys] if scattered else np.arange(n_phys)
            mask[b, sites] = True
    return q, k, v, e, mask


def rel(a, b):
    return np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300)


# ----------------------------------------------------------------------------- forward
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("n_phys,scattered", [(None, False), (3, False), (3, True)])
def test_fwd_matches_explicit_loops(mode, n_phys, scattered):
    rng = np.random.default_rng(11)
    q, k, v, e, mask = make(rng, 2, 5, 2, 4, n_phys, scattered, e_layout=mode["e_layout"])
    out, lse = O.fwd(q, k, e, v, mask, **mode)
    out_l, lse_l = O.loop_fwd(q, k, e, v, mask, **mode)
    assert rel(out, out_l) < 1e-13
    assert np.max(np.abs(lse - lse_l)) < 1e-9


def test_fwd_single_site_is_v():
    rng = np.random.default_rng(1)
    q, k, v, e, mask = make(rng, 3, 1, 2, 8)
    out, lse = O.fwd(q, k, e, v, mask)
    np.testing.assert_allclose(out, v, rtol=0, atol=1e-15)
    s = np.einsum("bihd,bihd->bih", q, k) + e[..., 0]
    np.testing.assert_allclose(lse, s, atol=1e-14)


def test_fwd_zero_logits_is_mean_of_valid_values():
    rng = np.random.default_rng(2)
    q, k, v, _, mask = make(rng, 2, 7, 3, 16, n_phys=4, scattered=True)
    out, lse = O.fwd(np.zeros_like(q), k, None, v, mask)
    for b in range(2):
        mean = v[b, mask[b]].mean(axis=0)
        np.testing.assert_allclose(out[b, mask[b]], np.broadcast_to(mean, out[b, mask[b]].shape), atol=1e-15)
        assert np.all(out[b, ~mask[b]] == 0.0)
        np.testing.assert_allclose(lse[b, mask[b]], np.log(4.0), atol=1e-14)
        np.testing.assert_allclose(lse[b, ~mask[b]], -1e4 + np.log(7.0), atol=1e-9)


def test_fwd_dominant_logit_selects_value():
    rng = np.random.default_rng(3)
    q, k, v, e, mask = make(rng, 1, 6, 2, 8)
    e[:] = 0.0
    e[0, :, :, 4] = 60.0  # every query attends to key 4
    out, _ = O.fwd(q, k, e, v, mask)
    np.testing.assert_allclose(out[0], np.broadcast_to(v[0, 4], out[0].shape), atol=1e-20 + 1e-12)


@pytest.mark.parametrize("mode", MODES)
def test_fwd_invariances(mode):
    rng = np.random.default_rng(4)
    B, N, H, D = 2, 9, 2, 8
    q, k, v, e, mask = make(rng, B, N, H, D, n_phys=6, scattered=True, e_layout=mode["e_layout"])
    out, _ = O.fwd(q, k, e, v, mask, **mode)
    # permuting all sites permutes the output rows
    perm = rng.permutation(N)
    if mode["e_layout"] == "qhk":
        ep = e[:, perm][:, :, :, perm]
    else:
        ep = e[:, perm][:, :, perm]
    out_p, _ = O.fwd(q[:, perm], k[:, perm], ep, v[:, perm], mask[:, perm], **mode)
    assert rel(out_p, out[:, perm]) < 1e-13
    # values at masked sites do not reach physical rows
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    for x in (q2, k2, v2):
        x[~mask] = rng.standard_normal(x[~mask].shape) * 3
    out2, _ = O.fwd(q2, k2, e, v2, mask, **mode)
    assert rel(out2[mask], out[mask]) < 1e-13
    # a per-(query, head) constant added to the bias leaves the softmax unchanged
    shift = rng.standard_normal((B, N, H))
    es = e + (shift[..., None] if mode["e_layout"] == "qhk" else shift[:, :, None, :])
    out3, _ = O.fwd(q, k, es, v, mask, **mode)
    assert rel(out3, out) < 1e-12


def test_fwd_masked_rows_exactly_zero_in_primitive_mode_only():
    rng = np.random.default_rng(5)
    q, k, v, e, mask = make(rng, 2, 8, 2, 8, n_phys=5, scattered=True)
    out, _ = O.fwd(q, k, e, v, mask)
    assert np.all(out[~mask] == 0.0)
    out_k, _ = O.fwd(q, k, e, v, mask, key_mask=True)
    assert np.all(np.abs(out_k[~mask]) > 0)


def test_reference_edge_attention_matches_formula():
    rng = np.random.default_rng(6)
    n, h, d = 6, 3, 16
    Q, K, V = (rng.standard_normal((n, h, d)) for _ in range(3))
    E = rng.standard_normal((n, n, h))
    mask = np.array([1, 1, 0, 1, 0, 1], dtype=bool)
    logits = np.einsum("ihd,jhd->hij", Q, K) / np.sqrt(d) + E.transpose(2, 0, 1)
    logits = logits + (1.0 - mask)[None, None, :] * -1e9
    alpha = np.exp(logits - logits.max(-1, keepdims=True))
    alpha /= alpha.sum(-1, keepdims=True)
    want = np.einsum("hij,jhd->ihd", alpha, V)
    assert rel(O.reference_edge_attention(Q, K, V, E, mask), want) < 1e-13


def _fp32_literal_edge_attention(Q, K, V, E, mask):
    """pallas_attention.py:30-37 evaluated literally in numpy float32, one operation at a
    time: einsum, * d^-1/2, + e^T, + (1 - mask) * -1e9, softmax as exp(x - max) / sum."""
    Q, K, V, E = (np.asarray(x, dtype=np.float32) for x in (Q, K, V, E))
    sm_scale = np.float32(float(Q.shape[-1]) ** -0.5)
    logits = np.einsum("ihd,jhd->hij", Q, K) * sm_scale
    logits = logits + np.transpose(E, (2, 0, 1))
    logits = logits + (np.float32(1.0) - mask.astype(np.float32))[None, None, :] * np.float32(-1e9)
    assert logits.dtype == np.float32
    ex = np.exp(logits - logits.max(-1, keepdims=True))
    alpha = ex / ex.sum(-1, keepdims=True)
    return np.einsum("hij,jhd->ihd", alpha, V)


def _exact_limit(Q, K, V, E):
    """softmax(s) V over every key: the exact-arithmetic limit of the additive mask when no
    key is physical (what the reference's float32 arithmetic does NOT compute)."""
    logits = np.einsum("ihd,jhd->hij", Q, K) / np.sqrt(Q.shape[-1]) + E.transpose(2, 0, 1)
    a = np.exp(logits - logits.max(-1, keepdims=True))
    return np.einsum("hij,jhd->ihd", a / a.sum(-1, keepdims=True), V)


def test_key_mask_matches_float32_literal_partially_masked():
    rng = np.random.default_rng(21)
    n, h, d = 9, 2, 16
    Q, K, V = (rng.standard_normal((n, h, d)).astype(np.float32) for _ in range(3))
    E = rng.standard_normal((n, n, h)).astype(np.float32)
    mask = np.array([1, 0, 1, 1, 0, 0, 1, 0, 1], dtype=bool)
    assert rel(O.reference_edge_attention(Q, K, V, E, mask), _fp32_literal_edge_attention(Q, K, V, E, mask)) < 1e-5


def test_key_mask_all_masked_small_logits_is_uniform():
    """No physical key, every |logit| < 32: fl32(s - 1e9) = -1e9 for every key, so the
    reference averages all value rows; the exact-arithmetic limit does not."""
    rng = np.random.default_rng(22)
    n, h, d = 8, 3, 32
    Q, K, V = (rng.standard_normal((n, h, d)).astype(np.float32) for _ in range(3))
    E = rng.standard_normal((n, n, h)).astype(np.float32)
    mask = np.zeros(n, dtype=bool)
    lit = _fp32_literal_edge_attention(Q, K, V, E, mask)
    mean_v = np.broadcast_to(V.astype(np.float64).mean(axis=0), (n, h, d))
    assert rel(lit, mean_v) < 1e-6
    got = O.reference_edge_attention(Q, K, V, E, mask)
    assert rel(got, lit) < 1e-6
    assert rel(_exact_limit(Q, K, V, E), lit) > 1e-2  # the test tells the two apart
    _, lse = O.fwd(Q[None], K[None], E[None], V[None], mask[None], scale=d ** -0.5, key_mask=True,
                   e_layout="qkh")
    np.testing.assert_allclose(lse, np.log(n), rtol=0, atol=1e-12)  # shifted logits all 0


def test_key_mask_all_masked_large_logits_rounds_to_multiples_of_64():
    """No physical key, logits of a few hundred: fl32(s - 1e9) keeps s to the nearest
    multiple of 64, so the weights concentrate on the keys of the top multiple."""
    rng = np.random.default_rng(23)
    n, h, d = 12, 2, 16
    Q, K, V = (rng.standard_normal((n, h, d)).astype(np.float32) for _ in range(3))
    Q *= np.float32(12.0)
    K *= np.float32(12.0)
    E = (rng.standard_normal((n, n, h)) * 40.0).astype(np.float32)
    s = np.einsum("ihd,jhd->hij", Q.astype(np.float64), K) / np.sqrt(d) + E.transpose(2, 0, 1)
    assert np.abs(s).max() > 200.0
    assert np.min(np.abs((s - 32.0) / 64.0 - np.round((s - 32.0) / 64.0))) * 64.0 > 0.05  # no tie
    mask = np.zeros(n, dtype=bool)
    lit = _fp32_literal_edge_attention(Q, K, V, E, mask)
    assert rel(O.reference_edge_attention(Q, K, V, E, mask), lit) < 1e-5
    assert rel(_exact_limit(Q, K, V, E), lit) > 1e-2


# ----------------------------------------------------------------------------- tangent
def _tangents(rng, q, e):
    return (
        rng.standard_normal(q.shape),
        rng.standard_normal(q.shape),
        None if e is None else rng.standard_normal(e.shape),
        rng.standard_normal(q.shape),
    )


@pytest.mark.parametrize("mode", MODES)
def test_jvp_matches_central_differences(mode):
    rng = np.random.default_rng(7)
    q, k, v, e, mask = make(rng, 2, 6, 2, 8, n_phys=4, scattered=True, e_layout=mode["e_layout"])
    qt, kt, et, vt = _tangents(rng, q, e)
    tout = O.jvp(q, k, e, v, mask, qt, kt, et, vt, **mode)
    hstep = 1e-6
    plus, _ = O.fwd(q + hstep * qt, k + hstep * kt, e + hstep * et, v + hstep * vt, mask, **mode)
    minus, _ = O.fwd(q - hstep * qt, k - hstep * kt, e - hstep * et, v - hstep * vt, mask, **mode)
    fd = (plus - minus) / (2 * hstep)
    assert rel(tout, fd) < 1e-8


def _torch_fwd(q, k, e, v, mask, scale, key_mask, e_layout):
    """Independent float64 torch formula of the forward (for autodiff cross-checks)."""
    eb = e.permute(0, 2, 1, 3) if e_layout == "qhk" else e.permute(0, 3, 1, 2)
    mk = mask[:, None, None, :]
    if key_mask:
        s = torch.einsum("bihd,bjhd->bhij", q, k) * scale + eb + (~mk).double() * -1e9
        return torch.einsum("bhij,bjhd->bihd", torch.softmax(s, -1), v)
    m4 = mask[:, :, None, None].double()
    s = torch.einsum("bihd,bjhd->bhij", q * m4 * scale, k * m4) + eb
    s = torch.where(mask[:, None, :, None] & mk, s, torch.tensor(-1e4, dtype=torch.float64))
    return torch.einsum("bhij,bjhd->bihd", torch.softmax(s, -1), v * m4) * m4


@pytest.mark.parametrize("mode", MODES)
def test_jvp_matches_torch_forward_autodiff(mode):
    rng = np.random.default_rng(8)
    q, k, v, e, mask = make(rng, 2, 7, 3, 8, n_phys=5, scattered=True, e_layout=mode["e_layout"])
    qt, kt, et, vt = _tangents(rng, q, e)
    T = torch.from_numpy
    fn = lambda a, b, c, d: _torch_fwd(a, b, c, d, T(mask), mode["scale"], mode["key_mask"], mode["e_layout"])  # noqa: E731
    _, tan = torch.func.jvp(fn, (T(q), T(k), T(e), T(v)), (T(qt), T(kt), T(et), T(vt)))
    assert rel(O.jvp(q, k, e, v, mask, qt, kt, et, vt, **mode), tan.numpy()) < 1e-12


def test_jvp_closed_forms():
    rng = np.random.default_rng(9)
    q, k, v, e, mask = make(rng, 2, 6, 2, 8, n_phys=4, scattered=True)
    out, _ = O.fwd(q, k, e, v, mask)
    # dV = V, nothing else: tout = P V = out
    assert rel(O.jvp(q, k, e, v, mask, None, None, None, v), out) < 1e-14
    # dE = per-row constant: softmax is shift invariant -> tout = 0
    et = np.broadcast_to(rng.standard_normal((2, 6, 2, 1)), e.shape).copy()
    assert np.max(np.abs(O.jvp(q, k, e, v, mask, None, None, et, None))) < 1e-14
    # linearity in the tangent
    t1, t2 = _tangents(rng, q, e), _tangents(rng, q, e)
    lin = O.jvp(q, k, e, v, mask, *[2 * a + 3 * b for a, b in zip(t1, t2)])
    sep = 2 * O.jvp(q, k, e, v, mask, *t1) + 3 * O.jvp(q, k, e, v, mask, *t2)
    assert rel(lin, sep) < 1e-12
    # P o (dS - rowsum(P o dS)) form of the north star equals the reference's split form
    qt, kt, et, vt = t1
    p = O.probs(q, k, e, mask)
    mz = lambda x: np.where(mask[:, :, None, None], x, 0.0)  # noqa: E731
    ds = np.einsum("bihd,bjhd->bhij", mz(qt), mz(k)) + np.einsum("bihd,bjhd->bhij", mz(q), mz(kt)) + et.transpose(0, 2, 1, 3)
    ds = np.where(mask[:, None, :, None] & mask[:, None, None, :], ds, 0.0)
    pd = p * (ds - (p * ds).sum(-1, keepdims=True))
    alt = np.einsum("bhij,bjhd->bihd", pd, mz(v)) + np.einsum("bhij,bjhd->bihd", p, mz(vt))
    assert rel(O.jvp(q, k, e, v, mask, qt, kt, et, vt), mz(alt)) < 1e-12


# --------------------------------------------------------------------------- cotangent
@pytest.mark.parametrize("mode", MODES)
def test_vjp_transpose_identity(mode):
    rng = np.random.default_rng(10)
    q, k, v, e, mask = make(rng, 2, 6, 2, 8, n_phys=4, scattered=True, e_layout=mode["e_layout"])
    qt, kt, et, vt = _tangents(rng, q, e)
    cot = rng.standard_normal(q.shape)
    lhs = np.sum(O.jvp(q, k, e, v, mask, qt, kt, et, vt, **mode) * cot)
    dq, dk, de, dv = O.vjp(q, k, e, v, mask, cot, **mode)
    rhs = np.sum(dq * qt) + np.sum(dk * kt) + np.sum(de * et) + np.sum(dv * vt)
    assert abs(lhs - rhs) < 1e-12 * max(1.0, abs(lhs))


@pytest.mark.parametrize("mode", MODES)
def test_vjp_matches_torch_reverse_autodiff(mode):
    rng = np.random.default_rng(12)
    q, k, v, e, mask = make(rng, 2, 7, 2, 16, n_phys=5, scattered=True, e_layout=mode["e_layout"])
    cot = rng.standard_normal(q.shape)
    T = torch.from_numpy
    args = [T(x).requires_grad_() for x in (q, k, e, v)]
    out = _torch_fwd(*args[:3], args[3], T(mask), mode["scale"], mode["key_mask"], mode["e_layout"])
    grads = torch.autograd.grad(out, args, T(cot))
    dq, dk, de, dv = O.vjp(q, k, e, v, mask, cot, **mode)
    for mine, ref in zip((dq, dk, de, dv), grads):
        assert rel(mine, ref.numpy()) < 1e-12


def test_vjp_structure():
    rng = np.random.default_rng(13)
    q, k, v, e, mask = make(rng, 2, 8, 2, 8, n_phys=5, scattered=True)
    cot = rng.standard_normal(q.shape)
    dq, dk, de, dv = O.vjp(q, k, e, v, mask, cot)
    # softmax cotangents sum to zero over keys on every physical row
    assert np.max(np.abs(de.sum(-1)[mask])) < 1e-13
    for x in (dq, dk, dv):
        assert np.all(x[~mask] == 0.0)
    assert np.all(de[~mask] == 0.0)
    assert np.all(de.transpose(0, 3, 2, 1)[~mask] == 0.0)
    # dv = P^T dout
    p = O.probs(q, k, e, mask)
    cz = np.where(mask[:, :, None, None], cot, 0.0)
    assert rel(dv, np.einsum("bhij,bihd->bjhd", p, cz)) < 1e-13


# ------------------------------------------------------------------- planted mistakes
def _fd(q, k, e, v, mask, qt, kt, et, vt):
    h = 1e-6
    p, _ = O.fwd(q + h * qt, k + h * kt, e + h * et, v + h * vt, mask)
    m, _ = O.fwd(q - h * qt, k - h * kt, e - h * et, v - h * vt, mask)
    return (p - m) / (2 * h)


def test_planted_jvp_mistakes_are_caught(monkeypatch):
    rng = np.random.default_rng(14)
    q, k, v, e, mask = make(rng, 1, 6, 2, 8, n_phys=4, scattered=True)
    qt, kt, et, vt = _tangents(rng, q, e)
    fd = _fd(q, k, e, v, mask, qt, kt, et, vt)
    good = O.jvp(q, k, e, v, mask, qt, kt, et, vt)
    assert rel(good, fd) < 1e-8
    # dropped "- mean * out" term: add it back to undo it
    out, _ = O.fwd(q, k, e, v, mask)
    p = O.probs(q, k, e, mask)
    mz = lambda x: np.where(mask[:, :, None, None], x, 0.0)  # noqa: E731
    ds = (
        np.einsum("bihd,bjhd->bhij", mz(qt), mz(k))
        + np.einsum("bihd,bjhd->bhij", mz(q), mz(kt))
        + et.transpose(0, 2, 1, 3)
    ) * (mask[:, None, :, None] & mask[:, None, None, :])
    mean = (p * ds).sum(-1).transpose(0, 2, 1)[..., None]
    assert rel(good + mean * out, fd) > 1e-3
    # swap q/k roles in the tangent score (transposed operand)
    bad = O.jvp(q, k, e, v, mask, kt, qt, et, vt)
    assert rel(bad, fd) > 1e-3
    # wrong sign on the bias tangent
    bad = O.jvp(q, k, e, v, mask, qt, kt, -et, vt)
    assert rel(bad, fd) > 1e-3


def test_planted_vjp_mistake_is_caught():
    rng = np.random.default_rng(15)
    q, k, v, e, mask = make(rng, 1, 6, 2, 8, n_phys=5, scattered=True)
    qt, kt, et, vt = _tangents(rng, q, e)
    cot = rng.standard_normal(q.shape)
    lhs = np.sum(O.jvp(q, k, e, v, mask, qt, kt, et, vt) * cot)
    dq, dk, de, dv = O.vjp(q, k, e, v, mask, cot)
    # dq and dk exchanged (a transposed operand) breaks the transpose identity
    rhs_bad = np.sum(dk * qt) + np.sum(dq * kt) + np.sum(de * et) + np.sum(dv * vt)
    assert abs(lhs - rhs_bad) > 1e-6
    # de transposed over (query, key)
    rhs_bad = np.sum(dq * qt) + np.sum(dk * kt) + np.sum(de.transpose(0, 3, 2, 1) * et) + np.sum(dv * vt)
    assert abs(lhs - rhs_bad) > 1e-6
