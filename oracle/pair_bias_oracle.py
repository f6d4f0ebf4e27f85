"""Float64 restatement of the trunk attention's coupling-bias producer — TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg as the checker; never part of the product path.

Per site pair (i, j) of a walker the reference computes (``model/trunk.py:89-105``)

    y    = ln_edge(edge[i, j, :])        eqx-style RMS:  x * (w * rsqrt(mean(x^2) + eps))
                                           (``model/tree.py:339-375``, ``odd_ops.py:183-215``)
    bias = bias_mlp(y)                   UnnormalizedMLP, one block (``odd_ops.py:279-316``):
             h0 = y W_in + b_in
             h1 = h0 + gain * (silu(h0 W_1 + b_1) W_2 + b_2)      silu(u) = u * sigmoid(u)
             out = h1 W_out + b_out
    e    = bias / sqrt(d_head)            (``trunk.py:103-105``)

with ``gain = n_layers ** -0.5`` (``trunk.py:55-62``) and eps = 1e-5 (``odd_ops.py:185``),
all in float32 in the reference (``model/fp32.py:7-8``: compute_dtype is float32). The
result is the op-level ``coup_bias [n, n, H]`` that ``reference_edge_attention`` /
``mhsea_tuned_edge_attention`` consume (``trunk.py:111,133``).

``coupling_bias_jvp`` is its forward-mode derivative with respect to ``edge`` (the parameters
held fixed), written out by the chain rule: the RMS's rsqrt derivative -0.5 r / v times
d mean(x^2) = 2 mean(x xdot), silu' = s + u s (1 - s).

``loop_coupling_bias`` is a scalar-loop restatement used to pin the vectorised form.

The second half of the module restates the MLP-class producer of the tree, readout and
large-N callers (the normalised ``MLP`` with RMS norms and the LCA-ALiBi term): ``mlp_bias``,
its tangent ``mlp_bias_jvp`` and the scalar-loop ``loop_mlp_bias``.
"""

from __future__ import annotations

import numpy as np


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def ln_edge(x, w, eps=1e-5):
    """RMS normalisation over the last axis, eqx style (``tree.py:355-375``)."""
    x = _f64(x)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * (_f64(w) * r)


def _sigmoid(u):
    return 1.0 / (1.0 + np.exp(-u))


def bias_mlp(y, params, gain):
    """UnnormalizedMLP with one residual block (``odd_ops.py:306-316``)."""
    p = {k: _f64(v) for k, v in params.items()}
    h0 = y @ p["w_in"] + p["b_in"]
    u = h0 @ p["w_1"] + p["b_1"]
    h1 = h0 + gain * ((u * _sigmoid(u)) @ p["w_2"] + p["b_2"])
    return h1 @ p["w_out"] + p["b_out"]


def coupling_bias(edge, params, gain, d_head, eps=1e-5):
    """coup_bias [..., H] from edge [..., C] (``trunk.py:89-105``)."""
    y = ln_edge(edge, params["ln_w"], eps)
    return bias_mlp(y, params, gain) / np.sqrt(float(d_head))


def coupling_bias_jvp(edge, edge_t, params, gain, d_head, eps=1e-5):
    """(e, e_dot): coup_bias and its derivative along ``edge_t`` (same shape as edge)."""
    p = {k: _f64(v) for k, v in params.items()}
    x, xd = _f64(edge), _f64(edge_t)
    C = x.shape[-1]
    v = np.mean(x * x, axis=-1, keepdims=True) + eps
    r = 1.0 / np.sqrt(v)
    rd = (2.0 * np.sum(x * xd, axis=-1, keepdims=True) / C) * (-0.5 * r / v)
    y = x * (p["ln_w"] * r)
    yd = p["ln_w"] * (xd * r + x * rd)
    h0 = y @ p["w_in"] + p["b_in"]
    h0d = yd @ p["w_in"]
    u = h0 @ p["w_1"] + p["b_1"]
    ud = h0d @ p["w_1"]
    s = _sigmoid(u)
    a = u * s
    ad = ud * (s + u * s * (1.0 - s))
    h1 = h0 + gain * (a @ p["w_2"] + p["b_2"])
    h1d = h0d + gain * (ad @ p["w_2"])
    div = np.sqrt(float(d_head))
    return (h1 @ p["w_out"] + p["b_out"]) / div, (h1d @ p["w_out"]) / div


def loop_coupling_bias(edge, params, gain, d_head, eps=1e-5):
    """Scalar loops over pairs, channels and features (tiny inputs only)."""
    p = {k: _f64(v) for k, v in params.items()}
    x = _f64(edge)
    lead = x.shape[:-1]
    C = x.shape[-1]
    Hd = p["w_in"].shape[1]
    H = p["w_out"].shape[1]
    out = np.zeros(lead + (H,))
    for idx in np.ndindex(*lead):
        row = x[idx]
        ms = 0.0
        for k in range(C):
            ms += row[k] * row[k]
        r = 1.0 / np.sqrt(ms / C + eps)
        y = [row[k] * (p["ln_w"][k] * r) for k in range(C)]
        h0 = [sum(y[k] * p["w_in"][k, f] for k in range(C)) + p["b_in"][f] for f in range(Hd)]
        act = []
        for f in range(Hd):
            u = sum(h0[k] * p["w_1"][k, f] for k in range(Hd)) + p["b_1"][f]
            act.append(u / (1.0 + np.exp(-u)))
        h1 = [h0[f] + gain * (sum(act[k] * p["w_2"][k, f] for k in range(Hd)) + p["b_2"][f]) for f in range(Hd)]
        for h in range(H):
            out[idx + (h,)] = (sum(h1[k] * p["w_out"][k, h] for k in range(Hd)) + p["b_out"][h]) / np.sqrt(float(d_head))
    return out


def to_attention_layout(bias):
    """coup_bias [B, N(query), N(key), H] -> the primitive's e layout [B, N, H, N]."""
    return np.ascontiguousarray(np.swapaxes(_f64(bias), 2, 3))


def init_params(rng, C, hidden, H, *, scale_bias=0.1):
    """Parameters of the reference's shapes and init scales (``odd_ops.py:78-87,286-304``):
    normal(0, fan_in^-1/2) weights; biases drawn small and nonzero (the reference starts them
    at zero; nonzero biases exercise every term); RMS weight near one."""
    def w(i, o):
        return (rng.standard_normal((i, o)) * i ** -0.5).astype(np.float32)

    def b(o):
        return (rng.standard_normal(o) * scale_bias).astype(np.float32)

    return {
        "ln_w": (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32),
        "w_in": w(C, hidden), "b_in": b(hidden),
        "w_1": w(hidden, hidden), "b_1": b(hidden),
        "w_2": w(hidden, hidden), "b_2": b(hidden),
        "w_out": w(hidden, H), "b_out": b(H),
    }


# ---------------------------------------------------------------------------------------------
# The MLP-class producer with the LCA-ALiBi term: the tree's LevelEdgeAttn
# (model/tree.py:1392-1456), the readout context's _attend (model/readout_leaf_context.py:
# 694-712) and the large-N sequence trunk (evaluation/sequence_trunk.py:962-972).
#
#   h    = x W_in + b_in                                (in_proj; the readout's x = [edge, dir])
#   h   += gain * (silu(rms_k(h) W_1[k] + b_1[k]) W_2[k] + b_2[k])        (MLP.__call__,
#            odd_ops.py:256-276; rms_k = _RMS with weight norm_w[k], tree.py:339-375)
#   e    = rms_out(h) W_out + b_out                     (out_norm, out_proj)
#   bias = e / sqrt(d_head) + alibi,  alibi[i, j, h] = -(slope[h] * lca_level(pos_i, pos_j))
#            (lca_alibi_bias, readout_leaf_context.py:161-163, transposed (1, 2, 0))
#
# lca_level counts the thresholds 2^t, t < 13, that pos_i ^ pos_j reaches
# (readout_leaf_context.py:140-148); lca_fixed_slopes(H) = 1.5 * 2^(-4 h / max(H - 1, 1))
# (:166-169). Pinned in tests/test_pair_bias_oracle.py.
# ---------------------------------------------------------------------------------------------

LCA_MAX_LEVELS = 13  # readout_leaf_context.py:131


def lca_level(pos_q, pos_k):
    """[len(pos_q), len(pos_k)] int: sum_t [ (pos_q ^ pos_k) >= 2^t ], t < 13 (literally)."""
    x = np.bitwise_xor(np.asarray(pos_q, dtype=np.int64)[:, None], np.asarray(pos_k, dtype=np.int64)[None, :])
    thresholds = (2 ** np.arange(LCA_MAX_LEVELS)).astype(np.int64)
    return (x[..., None] >= thresholds).sum(axis=-1)


def lca_fixed_slopes(n_heads):
    """lca_fixed_slopes (readout_leaf_context.py:166-169), in float32 as the reference."""
    head = np.arange(n_heads, dtype=np.float32)
    den = np.maximum(np.float32(n_heads - 1), np.float32(1.0))
    return (np.float32(1.5) * np.exp2(-(head * np.float32(4.0) / den))).astype(np.float32)


def rms(x, w, eps=1e-5):
    """_RMS over the last axis: x * (w * rsqrt(mean(x^2) + eps)) (tree.py:355-375)."""
    x = _f64(x)
    return x * (_f64(w) * (1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)))


def _mlp_input(edge, extra):
    x = _f64(edge)
    if extra is None:
        return x
    return np.concatenate([x, _f64(extra)[..., None]], axis=-1)


def mlp(x, params, gain, eps=1e-5):
    """The normalised MLP (odd_ops.py:218-276) over the last axis, float64."""
    p = {k: _f64(v) for k, v in params.items()}
    h = x @ p["w_in"] + p["b_in"]
    for k in range(p["w_1"].shape[0]):
        u = rms(h, p["norm_w"][k], eps) @ p["w_1"][k] + p["b_1"][k]
        h = h + gain * ((u * _sigmoid(u)) @ p["w_2"][k] + p["b_2"][k])
    return rms(h, p["out_norm_w"], eps) @ p["w_out"] + p["b_out"]


def alibi(Nq, Nk, slopes, row_offset=0):
    """[Nq, Nk, H]: -(slope[h] * lca_level(row_offset + i, j)), float64 of the float32 slopes."""
    lvl = lca_level(np.arange(Nq) + row_offset, np.arange(Nk)).astype(np.float64)
    return -(lvl[:, :, None] * _f64(slopes)[None, None, :])


def mlp_bias(edge, params, gain, d_head, *, extra=None, slopes=None, row_offset=0, eps=1e-5):
    """bias [B, Nq, Nk, H] (the reference's layout) from edge [B, Nq, Nk, C] (and extra
    [B, Nq, Nk])."""
    e = mlp(_mlp_input(edge, extra), params, gain, eps) / np.sqrt(float(d_head))
    if slopes is not None:
        e = e + alibi(e.shape[1], e.shape[2], slopes, row_offset)[None]
    return e


def mlp_bias_jvp(edge, edge_t, params, gain, d_head, *, extra=None, extra_t=None, slopes=None, row_offset=0,
                 eps=1e-5):
    """(bias, bias_dot): the bias and its derivative along (edge_t, extra_t), by the chain rule
    (RMS: d(x r) = xdot r + x rdot, rdot = -r mean(x xdot) / (mean(x^2) + eps); silu' = s + u s
    (1 - s)); the ALiBi term is constant."""
    p = {k: _f64(v) for k, v in params.items()}
    x = _mlp_input(edge, extra)
    xd = _mlp_input(edge_t, None if extra is None else (np.zeros_like(_f64(extra)) if extra_t is None else extra_t))

    def rms_jvp(h, hd, w):
        v = np.mean(h * h, axis=-1, keepdims=True) + eps
        r = 1.0 / np.sqrt(v)
        rd = -r * np.mean(h * hd, axis=-1, keepdims=True) / v
        return h * (w * r), w * (hd * r + h * rd)

    h = x @ p["w_in"] + p["b_in"]
    hd = xd @ p["w_in"]
    for k in range(p["w_1"].shape[0]):
        n, nd = rms_jvp(h, hd, p["norm_w"][k])
        u = n @ p["w_1"][k] + p["b_1"][k]
        ud = nd @ p["w_1"][k]
        s = _sigmoid(u)
        h = h + gain * ((u * s) @ p["w_2"][k] + p["b_2"][k])
        hd = hd + gain * ((ud * (s + u * s * (1.0 - s))) @ p["w_2"][k])
    n, nd = rms_jvp(h, hd, p["out_norm_w"])
    div = np.sqrt(float(d_head))
    e = (n @ p["w_out"] + p["b_out"]) / div
    if slopes is not None:
        e = e + alibi(e.shape[1], e.shape[2], slopes, row_offset)[None]
    return e, (nd @ p["w_out"]) / div


def loop_mlp_bias(edge, params, gain, d_head, *, extra=None, slopes=None, row_offset=0, eps=1e-5):
    """Scalar loops (tiny inputs only): independent restatement of ``mlp_bias``."""
    import math

    p = {k: _f64(v) for k, v in params.items()}
    x = _mlp_input(edge, extra)
    B, Nq, Nk, Cin = x.shape
    Hd = p["w_in"].shape[1]
    H = p["w_out"].shape[1]

    def rms_list(v, w):
        ms = sum(a * a for a in v) / len(v)
        r = 1.0 / math.sqrt(ms + eps)
        return [v[f] * w[f] * r for f in range(len(v))]

    out = np.zeros((B, Nq, Nk, H))
    for b in range(B):
        for i in range(Nq):
            for j in range(Nk):
                row = x[b, i, j]
                h = [sum(row[c] * p["w_in"][c, f] for c in range(Cin)) + p["b_in"][f] for f in range(Hd)]
                for k in range(p["w_1"].shape[0]):
                    n = rms_list(h, p["norm_w"][k])
                    act = []
                    for f in range(Hd):
                        u = sum(n[q] * p["w_1"][k, q, f] for q in range(Hd)) + p["b_1"][k, f]
                        act.append(u / (1.0 + math.exp(-u)))
                    h = [h[f] + gain * (sum(act[q] * p["w_2"][k, q, f] for q in range(Hd)) + p["b_2"][k, f])
                         for f in range(Hd)]
                n = rms_list(h, p["out_norm_w"])
                xr = (row_offset + i) ^ j
                level = sum(1 for t in range(LCA_MAX_LEVELS) if xr >= 2 ** t)
                for hh in range(H):
                    val = (sum(n[q] * p["w_out"][q, hh] for q in range(Hd)) + p["b_out"][hh]) / math.sqrt(d_head)
                    if slopes is not None:
                        val -= float(slopes[hh]) * level
                    out[b, i, j, hh] = val
    return out


def init_mlp_params(rng, C, hidden, H, n_blocks=1, *, extra=False, scale_bias=0.1):
    """Parameters of the MLP's shapes and init scales (odd_ops.py:78-87, 230-248): normal(0,
    fan_in^-1/2) weights; biases small and nonzero (the reference starts them at zero); RMS
    weights near one. With ``extra``, w_in has C + 1 rows (the readout's direction channel)."""
    cin = C + (1 if extra else 0)

    def w(*shape):
        return (rng.standard_normal(shape) * shape[-2] ** -0.5).astype(np.float32)

    def b(*shape):
        return (rng.standard_normal(shape) * scale_bias).astype(np.float32)

    return {
        "w_in": w(cin, hidden), "b_in": b(hidden),
        "norm_w": (1.0 + 0.1 * rng.standard_normal((n_blocks, hidden))).astype(np.float32),
        "w_1": w(n_blocks, hidden, hidden), "b_1": b(n_blocks, hidden),
        "w_2": w(n_blocks, hidden, hidden), "b_2": b(n_blocks, hidden),
        "out_norm_w": (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32),
        "w_out": w(hidden, H), "b_out": b(H),
    }
