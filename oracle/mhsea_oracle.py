"""CPU oracle of the reference MHSEA attention path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
use this module, and only as the checker / the timed CPU baseline. The product
(``hamiltonzero_amd``) never imports it.

A float64 numpy restatement of what the reference computes, with each function citing
the reference lines it follows (paths relative to ``src/hamiltonzero/model/``). Layout
is the reference's: ``q, k, v: [B, N, H, D]``, ``e: [B, N, H, N]`` (query, head, key)
or ``[B, N, N, H]`` (``e_layout="qkh"``), ``mask: [B, N]`` bool, ``lse: [B, N, H]``.

Two mask modes:

* ``key_mask=False`` — the primitive (``_pallas_attn/mhsea.py:14-31``): scores of pairs
  outside ``mask_q & mask_k`` are replaced by -1e4 (``_pallas_attn/utils.py:51-52``),
  masked q/k/v rows are zeroed before use, and masked query rows of the output and of
  the tangent are zero (``_pallas_attn/mhsea_tuned.py:91``,
  ``_pallas_attn/mhsea_tuned_jvp.py:88-91``).
* ``key_mask=True`` — ``reference_edge_attention`` (``pallas_attention.py:22-37``): an
  additive ``-1e9 * (1 - mask_k)`` on the logits, nothing zeroed. The reference adds the
  penalty in float32 (``:34-35``), so a masked key's logit is ``fl32(s - 1e9)``: a multiple
  of 64 (the float32 spacing at 1e9). While one key is physical this only means that
  masked keys get weight exactly 0; when no key of a walker is physical the softmax runs
  over these rounded logits (uniform weights when every ``|s| < 32``). This oracle
  evaluates that penalty in float32 and, for a walker with no physical key, reports its
  scores and lse shifted back by the constant 1e9 (``fl32(s - 1e9) + 1e9``, exact), which
  the softmax ignores.

How each function is pinned (tests/test_oracle.py): the forward by explicit loops on
tiny inputs and closed-form special cases; the tangent by central finite differences of
the forward and by torch forward-mode autodiff of an independent float64 formula; the
cotangent by the transpose identity <J t, c> = <t, J^T c> against the pinned tangent and
by torch reverse-mode autodiff. No function here is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

MASK_SCORE = -10000.0  # _pallas_attn/utils.py:51-52 (big_number)
KEY_MASK_PENALTY = -1e9  # pallas_attention.py:34


def _f64(x):
    return None if x is None else np.asarray(x, dtype=np.float64)


def _es(spec, a, b):
    """float64 contraction of two operands. The three attention patterns run as batched
    matrix products over (walker, head), which numpy hands to BLAS (its einsum cannot with
    two batch axes, and is ~20x slower at N = 1024); any other spec goes to einsum."""
    if spec == "bihd,bjhd->bhij":  # q k^T
        return np.matmul(a.transpose(0, 2, 1, 3), b.transpose(0, 2, 3, 1))
    if spec == "bhij,bjhd->bihd":  # P v
        return np.matmul(a, b.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3)
    if spec == "bhij,bihd->bjhd":  # P^T dout
        return np.matmul(a.transpose(0, 1, 3, 2), b.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3)
    return np.einsum(spec, a, b, optimize=True)


def _penalised(s, mask):
    """Logits of the additive key mask as the reference's float32 arithmetic forms them
    (pallas_attention.py:34-35): physical keys keep ``s``; a masked key's logit is
    ``fl32(fl32(s) - 1e9)``. For a walker with no physical key the result is shifted back by
    the constant 1e9 (exact: the rounded values are integers), which softmax ignores."""
    pen = (s.astype(np.float32) + np.float32(KEY_MASK_PENALTY)).astype(np.float64)
    out = np.where(mask[:, None, None, :], s, pen)
    empty = ~mask.any(axis=1)
    out[empty] -= KEY_MASK_PENALTY
    return out


def _e_bhqk(e, e_layout):
    """Bias as [B, H, Nq, Nk] (the transpose in pallas_attention.py:33 / :65)."""
    if e is None:
        return 0.0
    e = _f64(e)
    if e_layout == "qhk":
        return e.transpose(0, 2, 1, 3)
    if e_layout == "qkh":
        return e.transpose(0, 3, 1, 2)
    raise ValueError(e_layout)


def _e_back(g_bhqk, e_layout):
    """Inverse of _e_bhqk for cotangents."""
    if e_layout == "qhk":
        return g_bhqk.transpose(0, 2, 1, 3)
    return g_bhqk.transpose(0, 2, 3, 1)


def _zero_rows(x, mask):
    """jnp.where(mask[:, None], x, 0) over [B, N, H, D] (mhsea.py:19-22)."""
    return np.where(mask[:, :, None, None], x, 0.0)


def _valid(mask, key_mask):
    """[B, 1, Nq, Nk] boolean of pairs whose score tangent / cotangent is kept.

    Square mask: valid pairs only (mhsea_tuned_jvp.py:74, custom_gradients.py:276).
    Additive key mask: every pair; the -1e9 penalty is a constant whose weight
    exp(-1e9 - lse) already removes masked keys, exactly as autodiff of the jnp op does.
    """
    if key_mask:
        return np.ones((mask.shape[0], 1, mask.shape[1], mask.shape[1]), dtype=bool)
    return mask[:, None, :, None] & mask[:, None, None, :]


def scores(q, k, e, mask, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """S [B, H, Nq, Nk] as the softmax sees it.

    Primitive: ``where(mq & mk, q k^T + e, -1e4)`` with masked q/k zeroed (mhsea.py:18-25).
    reference_edge_attention: ``q k^T * scale + e^T + (1 - mask_k) * -1e9`` (:31-35).
    """
    q, k = _f64(q), _f64(k)
    mask = np.asarray(mask, dtype=bool)
    if key_mask:
        s = _es("bihd,bjhd->bhij", q, k) * scale + _e_bhqk(e, e_layout)
        return _penalised(s, mask)
    q = _zero_rows(q, mask)
    k = _zero_rows(k, mask)
    s = _es("bihd,bjhd->bhij", q * scale, k) + _e_bhqk(e, e_layout)
    return np.where(_valid(mask, False), s, MASK_SCORE)


def fwd(q, k, e, v, mask, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """(out [B,N,H,D], lse [B,N,H]).

    lse = max + log(sum(exp(S - max))), P = exp(S - lse), out = P v (mhsea.py:26-31);
    masked rows of out zeroed (mhsea_tuned.py:91) unless ``key_mask``.
    """
    out, lse, _ = _forward(q, k, e, v, mask, scale, key_mask, e_layout)
    return out, lse


def _forward(q, k, e, v, mask, scale, key_mask, e_layout):
    """(out, lse, P) of ``fwd``, P [B, H, Nq, Nk] the softmax weights."""
    mask = np.asarray(mask, dtype=bool)
    s = scores(q, k, e, mask, scale=scale, key_mask=key_mask, e_layout=e_layout)
    m = s.max(axis=-1, keepdims=True)
    lse = m + np.log(np.exp(s - m).sum(axis=-1, keepdims=True))
    p = np.exp(s - lse)
    v = _f64(v) if key_mask else _zero_rows(_f64(v), mask)
    out = _es("bhij,bjhd->bihd", p, v)
    if not key_mask:
        out = _zero_rows(out, mask)
    return out, lse[..., 0].transpose(0, 2, 1), p


def probs(q, k, e, mask, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """Softmax weights P [B, H, Nq, Nk]."""
    s = scores(q, k, e, mask, scale=scale, key_mask=key_mask, e_layout=e_layout)
    m = s.max(axis=-1, keepdims=True)
    w = np.exp(s - m)
    return w / w.sum(axis=-1, keepdims=True)


def jvp(q, k, e, v, mask, qt, kt, et, vt, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """Tangent of ``fwd``'s out (mhsea_tuned_jvp.py:51-91).

    dS = where(valid, scale (qt k^T + q kt^T) + et, 0), mean = sum_j P dS,
    tout = (P o dS) v + P vt - mean * out, masked rows zero. ``None`` tangents are zero.
    """
    mask = np.asarray(mask, dtype=bool)
    q, k, v = _f64(q), _f64(k), _f64(v)
    z = np.zeros_like(q)
    qt = z if qt is None else _f64(qt)
    kt = z if kt is None else _f64(kt)
    vt = z if vt is None else _f64(vt)
    out, _, p = _forward(q, k, e, v, mask, scale, key_mask, e_layout)
    if not key_mask:
        q, k, v, qt, kt, vt = (_zero_rows(x, mask) for x in (q, k, v, qt, kt, vt))
    ds = scale * (_es("bihd,bjhd->bhij", qt, k) + _es("bihd,bjhd->bhij", q, kt))
    if et is not None:
        ds = ds + _e_bhqk(et, e_layout)
    ds = np.where(_valid(mask, key_mask), ds, 0.0)
    pds = p * ds
    mean = pds.sum(axis=-1)  # [B, H, Nq]
    tout = (
        _es("bhij,bjhd->bihd", pds, v)
        + _es("bhij,bjhd->bihd", p, vt)
        - mean.transpose(0, 2, 1)[..., None] * out
    )
    if not key_mask:
        tout = _zero_rows(tout, mask)
    return tout


def vjp(q, k, e, v, mask, dout, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """Cotangents (dq, dk, de, dv) of ``fwd``'s out for cotangent ``dout``.

    Follows mhsea_q_vjp_kernel / mhsea_kv_vjp_kernel (custom_gradients.py:249-285,
    :307-347): dS = (dout v^T - rowsum(out o dout)) o P o valid, dq = scale dS k,
    dk = scale dS^T q, dv = P^T dout, de = dS; masked dout rows are ignored.
    """
    mask = np.asarray(mask, dtype=bool)
    q, k, v, dout = _f64(q), _f64(k), _f64(v), _f64(dout)
    out, _, p = _forward(q, k, e, v, mask, scale, key_mask, e_layout)
    if not key_mask:
        q, k, v, dout = (_zero_rows(x, mask) for x in (q, k, v, dout))
    dp = _es("bihd,bjhd->bhij", dout, v)
    delta = (out * dout).sum(axis=-1).transpose(0, 2, 1)[..., None]  # [B, H, Nq, 1]
    ds = (dp - delta) * p * _valid(mask, key_mask)
    dq = scale * _es("bhij,bjhd->bihd", ds, k)
    dk = scale * _es("bhij,bihd->bjhd", ds, q)
    dv = _es("bhij,bihd->bjhd", p, dout)
    if not key_mask:
        dv = _zero_rows(dv, mask)
    return dq, dk, _e_back(ds, e_layout), dv


def gate_collapse(out):
    """The trunk's sigmoid-gate head collapse after the attention call (trunk.py:134-137):
    head h < H/2 of ``out [B, N, H, D]`` gates head h + H/2,
    ``y = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:]`` of shape [B, N, H/2, D]."""
    out = _f64(out)
    hh = out.shape[2] // 2
    return out[:, :, hh:] / (1.0 + np.exp(-out[:, :, :hh]))


def gated_fwd_jvp(q, k, e, v, mask, qt, kt, et, vt, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """(y, ydot): ``gate_collapse`` of ``fwd``'s out and its forward-mode tangent along
    (qt, kt, et, vt), ``ydot = s (1 - s) gdot value + s vdot`` with ``s = sigmoid(gate)`` and
    (gdot, vdot) the gate / value heads of ``jvp``'s tangent (the chain rule through
    trunk.py:136)."""
    out, _ = fwd(q, k, e, v, mask, scale=scale, key_mask=key_mask, e_layout=e_layout)
    tout = jvp(q, k, e, v, mask, qt, kt, et, vt, scale=scale, key_mask=key_mask, e_layout=e_layout)
    hh = out.shape[2] // 2
    s = 1.0 / (1.0 + np.exp(-out[:, :, :hh]))
    y = s * out[:, :, hh:]
    ydot = s * (1.0 - s) * tout[:, :, :hh] * out[:, :, hh:] + s * tout[:, :, hh:]
    return y, ydot


def gated_vjp(q, k, e, v, mask, dy, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """(dq, dk, de, dv): reverse mode of ``gate_collapse`` after ``fwd``, for the cotangent
    ``dy [B, N, H/2, D]`` of y: the collapse's cotangent per head (gate: dy v s (1 - s), value:
    dy s, s = sigmoid(gate), trunk.py:136) fed to ``vjp``."""
    out, _ = fwd(q, k, e, v, mask, scale=scale, key_mask=key_mask, e_layout=e_layout)
    hh = out.shape[2] // 2
    s = 1.0 / (1.0 + np.exp(-out[:, :, :hh]))
    dy = _f64(dy)
    dout = np.concatenate([dy * out[:, :, hh:] * s * (1.0 - s), dy * s], axis=2)
    return vjp(q, k, e, v, mask, dout, scale=scale, key_mask=key_mask, e_layout=e_layout)


def out_proj(y, w_o, mask=None):
    """The attention block's output projection after the collapse: ``y_flat @ w_o``
    (trunk.py:138-144), times ``mask_q`` when a site mask is given (tree.py:1479-1488).
    y [B, N, H/2, D] or [B, N, d_attn] -> [B, N, d_e]."""
    y = _f64(y)
    out = y.reshape(y.shape[0], y.shape[1], -1) @ _f64(w_o)
    if mask is not None:
        out = np.asarray(mask, dtype=np.float64)[:, :, None] * out
    return out


def reference_edge_attention(Q, K, V, edge_bias, mask):
    """Per-system jnp op (pallas_attention.py:22-37): [n,h,d], [n,n,h], [n] -> [n,h,d]."""
    d = np.asarray(Q).shape[-1]
    out, _ = fwd(
        np.asarray(Q)[None], np.asarray(K)[None], np.asarray(edge_bias)[None], np.asarray(V)[None],
        np.asarray(mask, dtype=bool)[None], scale=float(d) ** -0.5, key_mask=True, e_layout="qkh",
    )
    return out[0]


def loop_fwd(q, k, e, v, mask, *, scale=1.0, key_mask=False, e_layout="qhk"):
    """Element-by-element restatement of ``fwd`` with Python loops and ``math`` (tiny inputs).

    Written independently of the vectorised code above: it walks the reference kernel's
    steps (mhsea.py:18-31) for one (walker, head, query) at a time.
    """
    import math

    q, k, v = _f64(q), _f64(k), _f64(v)
    mask = np.asarray(mask, dtype=bool)
    B, N, H, D = q.shape
    e = None if e is None else _f64(e)
    out = np.zeros((B, N, H, D))
    lse = np.zeros((B, N, H))
    for b in range(B):
        for h in range(H):
            for i in range(N):
                row = []
                for j in range(N):
                    dot = 0.0
                    for d in range(D):
                        qi = q[b, i, h, d] if (key_mask or mask[b, i]) else 0.0
                        kj = k[b, j, h, d] if (key_mask or mask[b, j]) else 0.0
                        dot += qi * scale * kj
                    bias = 0.0
                    if e is not None:
                        bias = e[b, i, h, j] if e_layout == "qhk" else e[b, i, j, h]
                    if key_mask and mask[b, j]:
                        sij = dot + bias
                    elif key_mask:  # float32 penalty; shifted back by 1e9 if no key is physical
                        sij = float(np.float32(np.float32(dot + bias) + np.float32(KEY_MASK_PENALTY)))
                        if not mask[b].any():
                            sij -= KEY_MASK_PENALTY
                    else:
                        sij = dot + bias if (mask[b, i] and mask[b, j]) else MASK_SCORE
                    row.append(sij)
                mx = max(row)
                tot = sum(math.exp(x - mx) for x in row)
                lse[b, i, h] = mx + math.log(tot)
                if not key_mask and not mask[b, i]:
                    continue
                for j in range(N):
                    pij = math.exp(row[j] - lse[b, i, h])
                    vj = v[b, j, h] if (key_mask or mask[b, j]) else np.zeros(D)
                    out[b, i, h] += pij * vj
    return out, lse
