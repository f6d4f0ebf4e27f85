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

How each function is pinned (tests/test_executor_oracle.py): explicit Python loops on tiny
inputs, closed forms (a T that copies one operand, the identity factors), bilinearity and
the (k, l) exchange symmetry of the merge, linearity and the conditioner scaling of the
apply. No function here is "parity unpinned".
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
