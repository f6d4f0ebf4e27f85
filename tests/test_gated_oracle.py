"""Pins the gated head collapse of the oracle (``gate_collapse``, ``gated_fwd_jvp``).

The collapse is the trunk's ``sigmoid(out[:, :H/2]) * out[:, H/2:]`` after the attention call
(trunk.py:134-137); no reference test or fixture covers it. Pinned by:
  collapse — closed forms of the logistic function (gate 0 -> value/2, gate ln 3 -> 3/4 of
             the value, gate -> +-inf -> value / 0) and the head pairing (h with h + H/2);
  tangent  — central finite differences of the float64 composite y(x + h t), independent of
             the product rule in ``gated_fwd_jvp``; linearity in the tangent;
  masking  — masked query rows of y and ydot are exactly zero.
A planted mistake (the derivative sign of sigmoid flipped) fails the difference check.
"""

import numpy as np
import pytest

from oracle import mhsea_oracle as O


def make(seed, B, N, H, D, n_phys):
    rng = np.random.default_rng(seed)
    x = [rng.standard_normal((B, N, H, D)) / np.sqrt(D) for _ in range(3)]
    e = rng.standard_normal((B, N, H, N)) * 0.5
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        mask[b, rng.permutation(N)[:n_phys]] = True
    tans = [rng.standard_normal((B, N, H, D)) for _ in range(3)]
    et = rng.standard_normal((B, N, H, N))
    return x, e, mask, tans, et


def rel(a, b):
    return np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300)


def test_collapse_closed_forms():
    value = np.arange(1.0, 7.0).reshape(1, 1, 1, 6)
    for gate, factor in ((0.0, 0.5), (np.log(3.0), 0.75), (-np.log(3.0), 0.25), (800.0, 1.0), (-800.0, 0.0)):
        out = np.concatenate([np.full((1, 1, 1, 6), gate), value], axis=2)
        assert np.allclose(O.gate_collapse(out), factor * value, rtol=1e-15, atol=0)


def test_collapse_pairs_head_h_with_h_plus_half():
    out = np.zeros((1, 1, 4, 2))
    out[0, 0, 1] = 50.0  # gate of head 3 open, gate of head 2 at 1/2
    out[0, 0, 2] = [2.0, 4.0]
    out[0, 0, 3] = [6.0, 8.0]
    y = O.gate_collapse(out)
    assert y.shape == (1, 1, 2, 2)
    assert np.allclose(y[0, 0, 0], [1.0, 2.0]) and np.allclose(y[0, 0, 1], [6.0, 8.0])


def _y(x, e, mask, **kw):
    out, _ = O.fwd(x[0], x[1], e, x[2], mask, **kw)
    return O.gate_collapse(out)


@pytest.mark.parametrize("key_mask", [False, True])
def test_tangent_matches_central_differences(key_mask):
    x, e, mask, tans, et = make(3, 2, 6, 4, 4, 4)
    kw = dict(scale=0.7, key_mask=key_mask)
    _, ydot = O.gated_fwd_jvp(x[0], x[1], e, x[2], mask, tans[0], tans[1], et, tans[2], **kw)
    h = 1e-6
    plus = _y([x[i] + h * tans[i] for i in range(3)], e + h * et, mask, **kw)
    minus = _y([x[i] - h * tans[i] for i in range(3)], e - h * et, mask, **kw)
    assert rel(ydot, (plus - minus) / (2 * h)) < 1e-7


def test_tangent_is_linear_and_masked_rows_zero():
    x, e, mask, tans, et = make(4, 2, 6, 2, 4, 3)
    _, a = O.gated_fwd_jvp(x[0], x[1], e, x[2], mask, tans[0], tans[1], et, tans[2])
    _, b = O.gated_fwd_jvp(x[0], x[1], e, x[2], mask, 2 * tans[0], 2 * tans[1], 2 * et, 2 * tans[2])
    assert rel(b, 2 * a) < 1e-14
    y, _ = O.gated_fwd_jvp(x[0], x[1], e, x[2], mask, tans[0], tans[1], et, tans[2])
    assert np.all(y[~mask] == 0.0) and np.all(a[~mask] == 0.0)


def test_planted_sign_mistake_fails_differences():
    x, e, mask, tans, et = make(5, 1, 5, 2, 4, 5)
    out, _ = O.fwd(x[0], x[1], e, x[2], mask)
    tout = O.jvp(x[0], x[1], e, x[2], mask, tans[0], tans[1], et, tans[2])
    s = 1.0 / (1.0 + np.exp(-out[:, :, :1]))
    wrong = s * (1.0 + s) * tout[:, :, :1] * out[:, :, 1:] + s * tout[:, :, 1:]
    h = 1e-6
    fd = (_y([x[i] + h * tans[i] for i in range(3)], e + h * et, mask)
          - _y([x[i] - h * tans[i] for i in range(3)], e - h * et, mask)) / (2 * h)
    assert rel(wrong, fd) > 1e-3


def test_out_proj_matches_loops_and_masks_rows():
    rng = np.random.default_rng(40)
    y = rng.standard_normal((2, 3, 2, 4))
    w = rng.standard_normal((8, 5))
    mask = np.array([[1, 0, 1], [0, 1, 1]], dtype=bool)
    got = O.out_proj(y, w, mask)
    for b in range(2):
        for i in range(3):
            flat = [y[b, i, hh, d] for hh in range(2) for d in range(4)]
            want = [sum(flat[k] * w[k, j] for k in range(8)) * mask[b, i] for j in range(5)]
            assert np.allclose(got[b, i], want, rtol=1e-13, atol=1e-13)
    assert np.all(got[~mask] == 0.0)
    assert np.allclose(O.out_proj(y, w), np.einsum("bihd,hdj->bij", y, w.reshape(2, 4, 5)), rtol=1e-13)


def test_gated_vjp_is_the_transpose_of_the_pinned_jvp():
    """<ydot(t), dy> = <t, gated_vjp(dy)> for random tangents t of (q, k, e, v): the reverse
    mode is the adjoint of the forward mode pinned above by central differences."""
    rng = np.random.default_rng(43)
    B, N, H, D = 2, 7, 4, 8
    q, k, v, qt, kt, vt = (rng.standard_normal((B, N, H, D)) * 0.5 for _ in range(6))
    e, et = (rng.standard_normal((B, N, H, N)) * 0.5 for _ in range(2))
    mask = rng.random((B, N)) < 0.7
    mask[:, 0] = True
    dy = rng.standard_normal((B, N, H // 2, D))
    _, ydot = O.gated_fwd_jvp(q, k, e, v, mask, qt, kt, et, vt, scale=0.3)
    dq, dk, de, dv = O.gated_vjp(q, k, e, v, mask, dy, scale=0.3)
    lhs = np.sum(ydot * dy)
    rhs = np.sum(dq * qt) + np.sum(dk * kt) + np.sum(de * et) + np.sum(dv * vt)
    assert abs(lhs - rhs) <= 1e-10 * max(1.0, abs(lhs))
