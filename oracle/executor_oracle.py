"""CPU oracle of the compiled executor's products — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may use this module, and only as
the checker / the timed CPU baseline; the product (``hamiltonzero_amd``) never imports it.

float64 numpy restatements of the two products the compiled per-walker executor runs
at every tree level (paths relative to ``src/hamiltonzero/``):

* ``quadrilinear_merge`` — ``quadrilinear_merge_p``'s impl
  (``model/_custom_lap_primitives.py:36-50``) and ``_compiled_quadrilinear_merge``
  (``compiled/execute.py:34-52``): ``out[B, i, j] = sum_{k,l} T[i, j, k, l] u_a[B, i, k]
  u_b[B, i, l]`` over G groups of rank R, inputs and output flattened to ``[..., G * R]``.
* ``factorized_apply`` — ``_factorized_apply`` (``compiled/execute.py:24-31``):
  ``((x V) * h) U``, with the conditioner h broadcast over the leading (walker) axes the
  way the executor passes it (one row of h per tree node).
* ``merge_level`` — one level of ``execute_wavefunction`` (``compiled/execute.py:98-113``):
  the merge, its residual factorized apply, the RMS rescale and the opcode gate.
* ``normalize_leaf_carriers`` — ``model/model.py:31-37``.
* ``execute_wavefunction`` — the whole per-walker forward
  (``CompiledFinetuneWaveFunction._forward_plain``, ``compiled/model.py:143-180``): leaf,
  every level, readout, (log|psi|, phase).
* ``classify_opcodes`` — the opcodes of a tree over a leaf_real mask
  (``compiled/tree.py:344-360``): MERGE where both children hold a real leaf, CARRY_LEFT /
  CARRY_RIGHT where one does, EMPTY where neither.

How each function is pinned (tests/test_executor_oracle.py): explicit Python loops on tiny
inputs, closed forms (a T that copies one operand, the identity factors), bilinearity and
the (k, l) exchange symmetry of the merge, linearity and the conditioner scaling of the
apply; for the whole wavefunction, trees of carries only (the root is then the first or the
last leaf, whose log|psi| needs no merge at all), the homogeneity of a tree of merges
(scaling q_to_odd by a adds n log a to log|psi| and leaves the phase), an EMPTY root
(psi = 0) and planted mistakes. No function here is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

# compiled/types.py:15-25
MERGE, CARRY_LEFT, CARRY_RIGHT, EMPTY = 0, 1, 2, 3


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def quadrilinear_merge(T, u_a, u_b):
    """``einsum("ijkl,Bik,Bil->Bij", T, u_a, u_b)`` over ``[..., G * R]`` rows
    (_custom_lap_primitives.py:45-50; the unbatched case :39-44 is the same on one row)."""
    T, u_a, u_b = _f64(T), _f64(u_a), _f64(u_b)
    G, R = T.shape[0], T.shape[1]
    lead = u_a.shape[:-1]
    a = u_a.reshape(-1, G, R)
    b = u_b.reshape(-1, G, R)
    out = np.einsum("ijkl,Bik,Bil->Bij", T, a, b, optimize=True)
    return out.reshape(*lead, G * R)


def factorized_apply(V, U, h, x):
    """``((x @ V) * h) @ U`` (execute.py:24-31), h broadcast against ``x @ V``."""
    return ((_f64(x) @ _f64(V)) * _f64(h)) @ _f64(U)


def merge_level(T, V, U, h_level, eps, u, s, opcodes):
    """One tree level of execute_wavefunction (execute.py:98-113): u [..., 2w, G R],
    s [..., 2w], h_level [w, R_merge], opcodes [w] -> (u', s') of width w."""
    u, s = _f64(u), _f64(s)
    u_left, u_right = u[..., 0::2, :], u[..., 1::2, :]
    s_left, s_right = s[..., 0::2], s[..., 1::2]
    raw = quadrilinear_merge(T, u_left, u_right)
    out = raw + factorized_apply(V, U, h_level, raw)
    scale = np.sqrt(np.mean(out * out, axis=-1) + eps)
    cand_u = out / scale[..., None]
    cand_s = s_left + s_right + np.log(scale)
    op = np.asarray(opcodes)
    both, left, right = (op == MERGE).astype(np.float64), (op == CARRY_LEFT).astype(np.float64), (
        op == CARRY_RIGHT).astype(np.float64)
    u_new = both[:, None] * cand_u + left[:, None] * u_left + right[:, None] * u_right
    s_new = both * cand_s + left * s_left + right * s_right
    return u_new, s_new


def normalize_leaf_carriers(u):
    """(u / rms, log rms) with rms = sqrt(mean(u^2) + 1e-30) over the last axis
    (model/model.py:31-37)."""
    u = _f64(u)
    rms = np.sqrt(np.mean(u * u, axis=-1, keepdims=True) + 1e-30)
    return u / rms, np.log(rms)[..., 0]


def execute_wavefunction(q, q_weight, leaf_V, leaf_U, leaf_h, merge_T, merge_V, merge_U, merge_h, opcodes,
                         readout_V, readout_U, readout_h, merge_eps):
    """(log|psi|, phase) per walker (compiled/model.py:143-180). q [..., n, d_q]; merge_h and
    opcodes are per-level sequences ([w, R_merge], [w]) for widths n/2, ..., 1."""
    z = _f64(q) @ _f64(q_weight)
    u, s = normalize_leaf_carriers(factorized_apply(leaf_V, leaf_U, leaf_h, z))
    for h_level, ops in zip(merge_h, opcodes):
        u, s = merge_level(merge_T, merge_V, merge_U, h_level, merge_eps, u, s, ops)
    psi = factorized_apply(readout_V, readout_U, readout_h, u[..., 0, :])
    re, im = psi[..., 0], psi[..., 1]
    with np.errstate(divide="ignore"):
        log_abs = 0.5 * np.log(re * re + im * im) + s[..., 0]
    return log_abs, np.arctan2(im, re)


def classify_opcodes(leaf_real):
    """Per-level opcodes of the pairwise tree over a [n] leaf_real mask (compiled/tree.py:344-360)."""
    real = np.asarray(leaf_real, dtype=bool)
    levels = []
    while real.shape[0] > 1:
        left, right = real[0::2], real[1::2]
        ops = np.full(left.shape, EMPTY, dtype=np.uint8)
        ops[left & right] = MERGE
        ops[left & ~right] = CARRY_LEFT
        ops[~left & right] = CARRY_RIGHT
        levels.append(ops)
        real = left | right
    return levels


def loop_quadrilinear_merge(T, u_a, u_b):
    """Element-by-element restatement of ``quadrilinear_merge`` (tiny inputs)."""
    T = _f64(T)
    G, R = T.shape[0], T.shape[1]
    a = _f64(u_a).reshape(-1, G, R)
    b = _f64(u_b).reshape(-1, G, R)
    out = np.zeros_like(a)
    for n in range(a.shape[0]):
        for i in range(G):
            for j in range(R):
                acc = 0.0
                for k in range(R):
                    for l in range(R):
                        acc += T[i, j, k, l] * a[n, i, k] * b[n, i, l]
                out[n, i, j] = acc
    return out.reshape(np.shape(u_a))


def loop_factorized_apply(V, U, h, x):
    """Element-by-element restatement of ``factorized_apply`` for x [M, d_in], h [M, R]."""
    V, U, h, x = _f64(V), _f64(U), _f64(h), _f64(x)
    M, d_in = x.shape
    R, d_out = U.shape
    y = np.zeros((M, d_out))
    for m in range(M):
        z = [sum(x[m, d] * V[d, r] for d in range(d_in)) * h[m, r] for r in range(R)]
        for o in range(d_out):
            y[m, o] = sum(z[r] * U[r, o] for r in range(R))
    return y
