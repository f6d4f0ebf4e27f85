"""Pins the compiled-executor oracle (oracle/executor_oracle.py) without the reference's code.

The reference holds no tests or vectors for these products (its only test file is
tests/test_fermionic.py) and JAX is not installed, so each function is pinned by checks a
plausible mistake (a transposed operand, a wrong index, a dropped conditioner) fails:
explicit loops on tiny inputs, closed forms, bilinearity / linearity, the (k, l) exchange
symmetry of the merge and the conditioner scaling of the apply. A planted mistake at the end
shows the loop check rejects a transposed T.
"""

import numpy as np
import pytest

from oracle import executor_oracle as X


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a) - np.asarray(b))) / max(np.max(np.abs(b)), 1e-300))


def _merge_inputs(rng, B=3, G=2, R=4):
    T = rng.standard_normal((G, R, R, R))
    a = rng.standard_normal((B, G * R))
    b = rng.standard_normal((B, G * R))
    return T, a, b


def test_merge_matches_explicit_loops():
    rng = np.random.default_rng(0)
    T, a, b = _merge_inputs(rng)
    assert rel(X.quadrilinear_merge(T, a, b), X.loop_quadrilinear_merge(T, a, b)) < 1e-13


def test_merge_leading_axes_and_single_row():
    rng = np.random.default_rng(1)
    T, _, _ = _merge_inputs(rng, G=3, R=4)
    a = rng.standard_normal((2, 5, 12))
    b = rng.standard_normal((2, 5, 12))
    out = X.quadrilinear_merge(T, a, b)
    assert out.shape == (2, 5, 12)
    flat = X.quadrilinear_merge(T, a.reshape(10, 12), b.reshape(10, 12))
    assert rel(out.reshape(10, 12), flat) < 1e-14
    # the reference's unbatched path (_custom_lap_primitives.py:39-44) on one row
    assert rel(X.quadrilinear_merge(T, a[0, 0], b[0, 0]), out[0, 0]) < 1e-14


def test_merge_closed_form_copy_tensor():
    """T[i, j, k, l] = delta(j, k) delta(l, 0): out[., i, j] = a[., i, j] * b[., i, 0]."""
    rng = np.random.default_rng(2)
    G, R = 3, 5
    T = np.zeros((G, R, R, R))
    for j in range(R):
        T[:, j, j, 0] = 1.0
    a = rng.standard_normal((4, G * R))
    b = rng.standard_normal((4, G * R))
    want = (a.reshape(4, G, R) * b.reshape(4, G, R)[:, :, :1]).reshape(4, G * R)
    assert rel(X.quadrilinear_merge(T, a, b), want) < 1e-14


def test_merge_bilinear_and_exchange_symmetric():
    rng = np.random.default_rng(3)
    T, a, b = _merge_inputs(rng, B=4, G=2, R=6)
    a2 = rng.standard_normal(a.shape)
    lin = X.quadrilinear_merge(T, 2.0 * a - 3.0 * a2, b)
    sep = 2.0 * X.quadrilinear_merge(T, a, b) - 3.0 * X.quadrilinear_merge(T, a2, b)
    assert rel(lin, sep) < 1e-12
    # exchanging the operands is the same as exchanging T's last two indices
    Tx = T.transpose(0, 1, 3, 2)
    assert rel(X.quadrilinear_merge(Tx, b, a), X.quadrilinear_merge(T, a, b)) < 1e-13


def test_apply_matches_explicit_loops():
    rng = np.random.default_rng(4)
    M, d_in, R, d_out = 5, 6, 4, 7
    x = rng.standard_normal((M, d_in))
    V = rng.standard_normal((d_in, R))
    U = rng.standard_normal((R, d_out))
    h = rng.standard_normal((M, R))
    assert rel(X.factorized_apply(V, U, h, x), X.loop_factorized_apply(V, U, h, x)) < 1e-13


def test_apply_closed_forms_and_linearity():
    rng = np.random.default_rng(5)
    W, d_in, R, d_out = 4, 6, 5, 3
    x = rng.standard_normal((2, W, d_in))
    V = rng.standard_normal((d_in, R))
    U = rng.standard_normal((R, d_out))
    h = rng.standard_normal((W, R))
    ones = np.ones((W, R))
    # h = 1: the product of the two factors
    assert rel(X.factorized_apply(V, U, ones, x), x @ (V @ U)) < 1e-13
    # U = I, h = 1: x V
    assert rel(X.factorized_apply(V, np.eye(R), ones, x), x @ V) < 1e-13
    # linear in x, and scaling the conditioner scales the result
    x2 = rng.standard_normal(x.shape)
    assert rel(X.factorized_apply(V, U, h, x + 2 * x2),
               X.factorized_apply(V, U, h, x) + 2 * X.factorized_apply(V, U, h, x2)) < 1e-12
    assert rel(X.factorized_apply(V, U, 3.0 * h, x), 3.0 * X.factorized_apply(V, U, h, x)) < 1e-13
    # one conditioner row per node, broadcast over the walker axis
    per_row = np.stack([X.factorized_apply(V, U, h[w], x[:, w]) for w in range(W)], axis=1)
    assert rel(X.factorized_apply(V, U, h, x), per_row) < 1e-13


def test_merge_level_gate_and_rescale():
    rng = np.random.default_rng(6)
    G, R, Rm, W = 2, 4, 3, 4
    T = rng.standard_normal((G, R, R, R)) / R
    V = rng.standard_normal((G * R, Rm))
    U = rng.standard_normal((Rm, G * R))
    h = rng.standard_normal((W, Rm))
    u = rng.standard_normal((2, 2 * W, G * R))
    s = rng.standard_normal((2, 2 * W))
    ops = np.array([X.MERGE, X.CARRY_LEFT, X.CARRY_RIGHT, X.EMPTY])
    u2, s2 = X.merge_level(T, V, U, h, 1e-6, u, s, ops)
    # carries copy their side, empty nodes are zero
    assert np.array_equal(u2[:, 1], u[:, 2]) and np.array_equal(s2[:, 1], s[:, 2])
    assert np.array_equal(u2[:, 2], u[:, 5]) and np.array_equal(s2[:, 2], s[:, 5])
    assert np.all(u2[:, 3] == 0) and np.all(s2[:, 3] == 0)
    # merged nodes have unit RMS (up to eps) and carry the log of the scale
    raw = X.quadrilinear_merge(T, u[:, 0], u[:, 1])
    out = raw + X.factorized_apply(V, U, h[0], raw)
    sc = np.sqrt(np.mean(out ** 2, axis=-1) + 1e-6)
    assert rel(u2[:, 0], out / sc[:, None]) < 1e-13
    assert rel(s2[:, 0], s[:, 0] + s[:, 1] + np.log(sc)) < 1e-13


def test_planted_transposed_T_is_caught(monkeypatch):
    rng = np.random.default_rng(7)
    T, a, b = _merge_inputs(rng)
    good = X.quadrilinear_merge

    def bad(T_, ua, ub):
        return good(T_.transpose(0, 1, 3, 2), ua, ub)

    monkeypatch.setattr(X, "quadrilinear_merge", bad)
    assert rel(X.quadrilinear_merge(T, a, b), X.loop_quadrilinear_merge(T, a, b)) > 1e-3


def test_cpu_baseline_level_matches_oracle():
    """bench.py's CPU leg for the merge level (torch-CPU float32) agrees with the float64
    oracle's merge followed by the residual apply."""
    import torch

    from oracle import cpu_baseline

    rng = np.random.default_rng(5)
    G, R, Rm, W, B = 3, 32, 40, 4, 2
    T = (rng.standard_normal((G, R, R, R)) / R).astype(np.float32)
    ul = rng.standard_normal((B * W, G * R)).astype(np.float32)
    ur = rng.standard_normal((B * W, G * R)).astype(np.float32)
    V = (rng.standard_normal((G * R, Rm)) / np.sqrt(G * R)).astype(np.float32)
    U = (rng.standard_normal((Rm, G * R)) / np.sqrt(Rm)).astype(np.float32)
    h = rng.standard_normal((W, Rm)).astype(np.float32)
    got = cpu_baseline.executor_level(*(torch.from_numpy(x) for x in (T, ul, ur, V, U, h))).numpy()
    raw = X.quadrilinear_merge(T, ul, ur)
    want = raw + X.factorized_apply(V, U, h, raw.reshape(B, W, -1)).reshape(raw.shape)
    assert rel(got, want) < 1e-5
