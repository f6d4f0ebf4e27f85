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


def _wavefn_inputs(seed, B=3, n=8, d_q=4, d_z=6, R_leaf=10, G=2, R=4, R_merge=9, R_out=5):
    rng = np.random.default_rng(seed)
    dm = G * R
    w = lambda i, o: rng.standard_normal((i, o)) / np.sqrt(i)  # noqa: E731
    p = dict(q=rng.standard_normal((B, n, d_q)), q_weight=w(d_q, d_z), leaf_V=w(d_z, R_leaf), leaf_U=w(R_leaf, dm),
             leaf_h=rng.standard_normal((n, R_leaf)), merge_T=rng.standard_normal((G, R, R, R)) / R,
             merge_V=w(dm, R_merge), merge_U=w(R_merge, dm), readout_V=w(dm, R_out), readout_U=w(R_out, 2),
             readout_h=rng.standard_normal(R_out), merge_eps=1e-6)
    p["merge_h"] = [rng.standard_normal((n >> (l + 1), R_merge)) for l in range(int(np.log2(n)))]
    return p


def _leaf_only(p, leaf):
    """log|psi| and phase of a tree that carries one leaf to the root: its normalised
    carrier goes straight to the readout (no merge, no level rescale)."""
    z = p["q"][:, leaf] @ p["q_weight"]
    u_raw = ((z @ p["leaf_V"]) * p["leaf_h"][leaf]) @ p["leaf_U"]
    rms = np.sqrt(np.mean(u_raw ** 2, axis=-1) + 1e-30)
    psi = ((u_raw / rms[:, None]) @ p["readout_V"] * p["readout_h"]) @ p["readout_U"]
    return 0.5 * np.log(psi[:, 0] ** 2 + psi[:, 1] ** 2) + np.log(rms), np.arctan2(psi[:, 1], psi[:, 0])


@pytest.mark.parametrize("op,leaf", [(X.CARRY_LEFT, 0), (X.CARRY_RIGHT, 7)])
def test_wavefunction_of_carries_is_one_leaf(op, leaf):
    p = _wavefn_inputs(30)
    ops = [np.full(len(h), op, dtype=np.uint8) for h in p["merge_h"]]
    la, ph = X.execute_wavefunction(opcodes=ops, **p)
    want_la, want_ph = _leaf_only(p, leaf)
    assert rel(la, want_la) < 1e-12 and rel(ph, want_ph) < 1e-12


def test_wavefunction_of_merges_is_homogeneous_in_the_leaf_scale():
    """psi is multilinear in the n leaf carriers: q_to_odd scaled by a adds n log a to
    log|psi| and leaves the phase (every level rescales its carriers)."""
    p = _wavefn_inputs(31)
    ops = [np.full(len(h), X.MERGE, dtype=np.uint8) for h in p["merge_h"]]
    la, ph = X.execute_wavefunction(opcodes=ops, **p)
    la2, ph2 = X.execute_wavefunction(opcodes=ops, **dict(p, q_weight=2.5 * p["q_weight"]))
    assert np.allclose(la2 - la, 8 * np.log(2.5), atol=1e-10)
    assert np.allclose(ph2, ph, atol=1e-10)


def test_wavefunction_composes_the_pinned_pieces():
    p = _wavefn_inputs(32, n=4)
    ops = X.classify_opcodes([True, False, True, True])
    assert [o.tolist() for o in ops] == [[X.CARRY_LEFT, X.MERGE], [X.MERGE]]
    la, ph = X.execute_wavefunction(opcodes=ops, **p)
    B, n = p["q"].shape[:2]
    z = (p["q"] @ p["q_weight"]).reshape(B * n, -1)
    u_raw = X.loop_factorized_apply(p["leaf_V"], p["leaf_U"], np.tile(p["leaf_h"], (B, 1)), z).reshape(B, n, -1)
    u, s = X.normalize_leaf_carriers(u_raw)
    for h, o in zip(p["merge_h"], ops):
        u, s = X.merge_level(p["merge_T"], p["merge_V"], p["merge_U"], h, p["merge_eps"], u, s, o)
    psi = X.loop_factorized_apply(p["readout_V"], p["readout_U"], np.tile(p["readout_h"], (B, 1)), u[:, 0])
    assert rel(la, 0.5 * np.log(psi[:, 0] ** 2 + psi[:, 1] ** 2) + s[:, 0]) < 1e-12
    assert rel(ph, np.arctan2(psi[:, 1], psi[:, 0])) < 1e-12


def test_wavefunction_empty_root_and_leaf_normalisation():
    p = _wavefn_inputs(33, n=2)
    la, ph = X.execute_wavefunction(opcodes=[np.array([X.EMPTY], np.uint8)], **p)
    assert np.all(np.isneginf(la)) and np.all(ph == 0.0)
    u, s = X.normalize_leaf_carriers(np.array([[3.0, 4.0]]))
    assert np.allclose(u, [[3 / np.sqrt(12.5), 4 / np.sqrt(12.5)]]) and np.allclose(s, 0.5 * np.log(12.5))


def test_planted_swapped_carry_is_caught(monkeypatch):
    p = _wavefn_inputs(34)
    ops = [np.full(len(h), X.CARRY_LEFT, dtype=np.uint8) for h in p["merge_h"]]
    real = X.merge_level

    def swapped(T, V, U, h, eps, u, s, o):
        o = np.where(o == X.CARRY_LEFT, X.CARRY_RIGHT, np.where(o == X.CARRY_RIGHT, X.CARRY_LEFT, o))
        return real(T, V, U, h, eps, u, s, o)

    monkeypatch.setattr(X, "merge_level", swapped)
    la, _ = X.execute_wavefunction(opcodes=ops, **p)
    want, _ = _leaf_only(p, 0)
    assert rel(la, want) > 1e-3


def test_cpu_baseline_wavefunction_matches_oracle():
    """bench.py's CPU leg for the wavefunction (torch-CPU float32, packed per-level storage)
    agrees with the float64 oracle."""
    import torch

    from oracle import cpu_baseline

    p = _wavefn_inputs(35, B=3, n=8, G=2, R=32)
    ops = X.classify_opcodes([True, True, False, True, True, True, True, False])
    la, ph = X.execute_wavefunction(opcodes=ops, **p)
    L, half, Rm = len(p["merge_h"]), 4, p["merge_h"][0].shape[1]
    mh = np.zeros((L, half, Rm))
    oc = np.full((L, half), X.EMPTY, np.uint8)
    for lv, (h, o) in enumerate(zip(p["merge_h"], ops)):
        mh[lv, : len(h)], oc[lv, : len(o)] = h, o
    t = lambda x: torch.from_numpy(np.asarray(x, np.float32))  # noqa: E731
    packed = {k: t(p[k]) for k in ("q", "q_weight", "leaf_V", "leaf_U", "leaf_h", "merge_T", "merge_V", "merge_U",
                                   "readout_V", "readout_U", "readout_h")}
    packed["merge_h"], packed["opcodes"] = t(mh), torch.from_numpy(oc)
    r = cpu_baseline.time_wavefunction_walkers_per_s(packed, p["merge_eps"], budget_s=0.05, threads=2)
    assert rel(r["log_abs"].numpy(), la) < 1e-4 and rel(r["phase"].numpy(), ph) < 1e-4
