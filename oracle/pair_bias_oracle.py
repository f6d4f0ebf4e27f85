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
