"""Pins the coupling-bias oracle (oracle/pair_bias_oracle.py) without the reference's code.

The reference holds no tests or vectors for ln_edge / bias_mlp and JAX is not installed, so
the oracle is pinned by checks that a plausible mistake fails: scalar loops on tiny inputs,
an independent torch float64 implementation (torch.nn.functional.rms_norm, silu, linear)
with torch.func.jvp for the tangent, central differences, closed forms (zero weights,
no residual branch, scale invariance of the RMS) and planted mistakes that must be caught.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import pair_bias_oracle as X

GAIN = 8 ** -0.5
D_HEAD = 16


def rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _inputs(seed, lead=(2, 3, 3), C=8, Hd=6, H=4):
    rng = np.random.default_rng(seed)
    params = X.init_params(rng, C, Hd, H, scale_bias=0.3)
    edge = rng.standard_normal(lead + (C,)).astype(np.float32)
    edge_t = rng.standard_normal(lead + (C,)).astype(np.float32)
    return params, edge, edge_t


def _torch_bias(edge, p, gain=GAIN, d_head=D_HEAD, eps=1e-5):
    """Independent float64 torch statement of trunk.py:89-105."""
    y = F.rms_norm(edge, (edge.shape[-1],), weight=p["ln_w"], eps=eps)
    h0 = F.linear(y, p["w_in"].T, p["b_in"])
    h1 = h0 + gain * F.linear(F.silu(F.linear(h0, p["w_1"].T, p["b_1"])), p["w_2"].T, p["b_2"])
    return F.linear(h1, p["w_out"].T, p["b_out"]) / d_head ** 0.5


def _t(p):
    return {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in p.items()}


def test_vectorised_matches_scalar_loops():
    params, edge, _ = _inputs(0)
    assert rel(X.coupling_bias(edge, params, GAIN, D_HEAD), X.loop_coupling_bias(edge, params, GAIN, D_HEAD)) < 1e-12


def test_matches_independent_torch_implementation():
    params, edge, edge_t = _inputs(1, lead=(3, 5, 5), C=16, Hd=12, H=8)
    want = _torch_bias(torch.from_numpy(edge.astype(np.float64)), _t(params)).numpy()
    assert rel(X.coupling_bias(edge, params, GAIN, D_HEAD), want) < 1e-12


def test_jvp_matches_torch_forward_mode():
    params, edge, edge_t = _inputs(2, lead=(2, 4, 4), C=16, Hd=12, H=8)
    tp = _t(params)
    e_ref, et_ref = torch.func.jvp(lambda x: _torch_bias(x, tp), (torch.from_numpy(edge.astype(np.float64)),),
                                   (torch.from_numpy(edge_t.astype(np.float64)),))
    e, et = X.coupling_bias_jvp(edge, edge_t, params, GAIN, D_HEAD)
    assert rel(e, e_ref.numpy()) < 1e-12
    assert rel(et, et_ref.numpy()) < 1e-12


def test_jvp_matches_central_differences():
    params, edge, edge_t = _inputs(3)
    h = 1e-6
    x = edge.astype(np.float64)
    fd = (X.coupling_bias(x + h * edge_t, params, GAIN, D_HEAD) - X.coupling_bias(x - h * edge_t, params, GAIN, D_HEAD)) / (2 * h)
    e, et = X.coupling_bias_jvp(edge, edge_t, params, GAIN, D_HEAD)
    assert rel(e, X.coupling_bias(edge, params, GAIN, D_HEAD)) < 1e-14
    assert rel(et, fd) < 1e-7


def test_closed_forms():
    params, edge, _ = _inputs(4)
    # zero weights: every pair's bias is b_out / sqrt(d_head)
    z = {k: (np.zeros_like(v) if k.startswith("w_") else v) for k, v in params.items()}
    out = X.coupling_bias(edge, z, GAIN, D_HEAD)
    assert np.allclose(out, np.broadcast_to(params["b_out"] / 4.0, out.shape), rtol=0, atol=1e-15)
    # no residual branch (W_2 = 0, b_2 = 0): an affine map of the normalised edge
    nr = dict(params, w_2=np.zeros_like(params["w_2"]), b_2=np.zeros_like(params["b_2"]))
    y = X.ln_edge(edge, params["ln_w"])
    want = ((y @ params["w_in"].astype(np.float64) + params["b_in"]) @ params["w_out"].astype(np.float64)
            + params["b_out"]) / 4.0
    assert rel(X.coupling_bias(edge, nr, GAIN, D_HEAD), want) < 1e-13
    # eps = 0: the RMS normalisation is invariant to the scale of the edge features and
    # gives unit mean square after dividing out the weight
    y0 = X.ln_edge(edge, params["ln_w"], eps=0.0)
    assert rel(X.ln_edge(3.7 * edge.astype(np.float64), params["ln_w"], eps=0.0), y0) < 1e-14
    assert np.allclose(np.mean((y0 / params["ln_w"]) ** 2, axis=-1), 1.0, atol=1e-13)


def test_attention_layout_is_query_head_key():
    rng = np.random.default_rng(5)
    b = rng.standard_normal((2, 3, 4, 5))
    e = X.to_attention_layout(b)
    assert e.shape == (2, 3, 5, 4)
    assert e[1, 2, 3, 0] == b[1, 2, 0, 3]


@pytest.mark.parametrize("plant", ["sigmoid_sign", "residual_gain", "rms_mean"])
def test_planted_mistakes_are_caught(monkeypatch, plant):
    params, edge, edge_t = _inputs(6, lead=(2, 3, 3), C=16, Hd=12, H=8)
    want = _torch_bias(torch.from_numpy(edge.astype(np.float64)), _t(params)).numpy()
    if plant == "sigmoid_sign":
        monkeypatch.setattr(X, "_sigmoid", lambda u: 1.0 / (1.0 + np.exp(u)))
        got = X.coupling_bias(edge, params, GAIN, D_HEAD)
    elif plant == "residual_gain":
        got = X.coupling_bias(edge, params, 1.0, D_HEAD)
    else:
        monkeypatch.setattr(X, "ln_edge", lambda x, w, eps=1e-5: np.asarray(x, np.float64) * w
                            / np.sqrt(np.sum(np.asarray(x, np.float64) ** 2, axis=-1, keepdims=True) + eps))
        got = X.coupling_bias(edge, params, GAIN, D_HEAD)
    assert rel(got, want) > 1e-3


def test_cpu_baseline_trunk_matches_oracle_chain():
    """bench.py's CPU leg for the trunk config (torch-CPU float32, torch.func.jvp) agrees
    with the oracle's coupling bias followed by the gated attention's forward + JVP."""
    from oracle import cpu_baseline
    from oracle import mhsea_oracle as O

    rng = np.random.default_rng(17)
    B, N, H, D, C = 2, 12, 16, 16, 32
    params = X.init_params(rng, C, 64, H)
    edge, edge_t = (rng.standard_normal((B, N, N, C)).astype(np.float32) for _ in range(2))
    q, k, v, qt, kt, vt = (rng.standard_normal((B, N, H, D)).astype(np.float32) * np.float32(0.25) for _ in range(6))
    mask = np.zeros((B, N), bool)
    mask[0, :7] = True
    mask[1, rng.permutation(N)[:10]] = True
    t = torch.from_numpy
    r = cpu_baseline.time_trunk_walkers_per_s(
        {"q": t(q), "k": t(k), "v": t(v), "qt": t(qt), "kt": t(kt), "vt": t(vt), "edge": t(edge), "edge_t": t(edge_t)},
        t(mask), {n: t(x) for n, x in params.items()}, GAIN, D, budget_s=0.05, threads=2)
    eb, ebt = X.coupling_bias_jvp(edge, edge_t, params, GAIN, D)
    wy, wty = O.gated_fwd_jvp(q, k, X.to_attention_layout(eb), v, mask, qt, kt, X.to_attention_layout(ebt), vt)
    assert rel(r["y"].numpy(), wy) < 1e-5
    assert rel(r["ty"].numpy(), wty) < 1e-5


# ---- the MLP-class producer (tree / readout / large-N) ----------------------------------------

def _mlp_inputs(seed, B=2, Nq=3, Nk=5, C=8, Hd=6, H=4, nb=2, extra=True):
    rng = np.random.default_rng(seed)
    params = X.init_mlp_params(rng, C, Hd, H, nb, extra=extra, scale_bias=0.3)
    edge = rng.standard_normal((B, Nq, Nk, C)).astype(np.float32)
    edge_t = rng.standard_normal((B, Nq, Nk, C)).astype(np.float32)
    ex = rng.standard_normal((B, Nq, Nk)).astype(np.float32) if extra else None
    ex_t = rng.standard_normal((B, Nq, Nk)).astype(np.float32) if extra else None
    return params, edge, edge_t, ex, ex_t


def _torch_mlp_bias(edge, extra, p, gain, d_head, eps=1e-5):
    """Independent float64 torch statement of MLP.__call__ (odd_ops.py:256-276) / d_head^1/2."""
    x = edge if extra is None else torch.cat([edge, extra[..., None]], dim=-1)
    h = F.linear(x, p["w_in"].T, p["b_in"])
    for k in range(p["w_1"].shape[0]):
        n = F.rms_norm(h, (h.shape[-1],), weight=p["norm_w"][k], eps=eps)
        h = h + gain * F.linear(F.silu(F.linear(n, p["w_1"][k].T, p["b_1"][k])), p["w_2"][k].T, p["b_2"][k])
    n = F.rms_norm(h, (h.shape[-1],), weight=p["out_norm_w"], eps=eps)
    return F.linear(n, p["w_out"].T, p["b_out"]) / d_head ** 0.5


def test_mlp_bias_matches_loops_and_torch():
    params, edge, _, ex, _ = _mlp_inputs(31)
    sl = X.lca_fixed_slopes(4)
    got = X.mlp_bias(edge, params, 0.6, 16, extra=ex, slopes=sl, row_offset=3)
    assert rel(got, X.loop_mlp_bias(edge, params, 0.6, 16, extra=ex, slopes=sl, row_offset=3)) < 1e-13
    t = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in params.items()}
    tb = _torch_mlp_bias(torch.from_numpy(edge.astype(np.float64)), torch.from_numpy(ex.astype(np.float64)), t, 0.6,
                         16).numpy()
    alibi = X.alibi(3, 5, sl, 3)[None]
    assert rel(got, tb + alibi) < 1e-13


def test_mlp_bias_tangent_against_torch_jvp_and_differences():
    params, edge, edge_t, ex, ex_t = _mlp_inputs(32)
    e, ed = X.mlp_bias_jvp(edge, edge_t, params, 0.6, 16, extra=ex, extra_t=ex_t, slopes=X.lca_fixed_slopes(4))
    assert rel(e, X.mlp_bias(edge, params, 0.6, 16, extra=ex, slopes=X.lca_fixed_slopes(4))) < 1e-14
    t = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in params.items()}
    f64 = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float64))  # noqa: E731
    _, td = torch.func.jvp(lambda a, b: _torch_mlp_bias(a, b, t, 0.6, 16), (f64(edge), f64(ex)), (f64(edge_t), f64(ex_t)))
    assert rel(ed, td.numpy()) < 1e-12
    h = 1e-6
    e64, et64, x64, xt64 = (np.asarray(a, dtype=np.float64) for a in (edge, edge_t, ex, ex_t))
    fd = (X.mlp_bias(e64 + h * et64, params, 0.6, 16, extra=x64 + h * xt64)
          - X.mlp_bias(e64 - h * et64, params, 0.6, 16, extra=x64 - h * xt64)) / (2 * h)
    assert rel(ed, fd) < 1e-7


def test_lca_level_and_slopes():
    """lca_level: 0 on the diagonal, the bit length of i ^ j otherwise, capped at 13; the
    fixed slopes: 1.5 at head 0 and 1.5 / 16 at the last head (H > 1), 1.5 for H = 1."""
    lv = X.lca_level(np.arange(20), np.arange(20))
    for i in range(20):
        for j in range(20):
            assert lv[i, j] == (i ^ j).bit_length()
    assert X.lca_level([0], [8191])[0, 0] == 13 and X.lca_level([0], [1 << 20])[0, 0] == 13
    s = X.lca_fixed_slopes(16)
    assert s.dtype == np.float32 and s[0] == np.float32(1.5) and abs(s[-1] - 1.5 / 16) < 1e-7
    assert np.all(np.diff(s) < 0) and X.lca_fixed_slopes(1)[0] == np.float32(1.5)


def test_mlp_bias_closed_forms():
    """Zero out_proj weights: b_out / sqrt(d) + ALiBi whatever the input; zero W_2 and b_2: the
    blocks vanish and the result is out_proj(rms(in_proj(x))); with W_2 = 0 and eps = 0 the
    output is invariant under a positive scaling of W_in and b_in together (the RMS)."""
    params, edge, _, ex, _ = _mlp_inputs(33)
    z = dict(params, w_out=np.zeros_like(params["w_out"]))
    got = X.mlp_bias(edge, z, 0.6, 16, extra=ex, slopes=X.lca_fixed_slopes(4), row_offset=2)
    want = np.broadcast_to(params["b_out"] / 4.0, got.shape) + X.alibi(3, 5, X.lca_fixed_slopes(4), 2)[None]
    assert rel(got, want) < 1e-14
    nob = dict(params, w_2=np.zeros_like(params["w_2"]), b_2=np.zeros_like(params["b_2"]))
    x = np.concatenate([edge, ex[..., None]], axis=-1).astype(np.float64)
    h = x @ params["w_in"].astype(np.float64) + params["b_in"]
    direct = X.rms(h, params["out_norm_w"]) @ params["w_out"].astype(np.float64) + params["b_out"]
    assert rel(X.mlp_bias(edge, nob, 0.6, 16, extra=ex), direct / 4.0) < 1e-13
    scaled = dict(nob, w_in=params["w_in"] * 4.0, b_in=params["b_in"] * 4.0)  # exact in float32
    assert rel(X.mlp_bias(edge, scaled, 0.6, 16, extra=ex, eps=0.0), X.mlp_bias(edge, nob, 0.6, 16, extra=ex, eps=0.0)) < 1e-13


@pytest.mark.parametrize("kind", ["norm_weight_dropped", "alibi_sign", "extra_ignored", "row_offset_ignored"])
def test_mlp_bias_planted_mistakes_are_caught(kind):
    params, edge, _, ex, _ = _mlp_inputs(34)
    sl = X.lca_fixed_slopes(4)
    want = X.loop_mlp_bias(edge, params, 0.6, 16, extra=ex, slopes=sl, row_offset=6)
    if kind == "norm_weight_dropped":
        bad = X.mlp_bias(edge, dict(params, norm_w=np.ones_like(params["norm_w"])), 0.6, 16, extra=ex, slopes=sl,
                         row_offset=6)
    elif kind == "alibi_sign":
        bad = X.mlp_bias(edge, params, 0.6, 16, extra=ex, slopes=-sl, row_offset=6)
    elif kind == "extra_ignored":
        bad = X.mlp_bias(edge, params, 0.6, 16, extra=np.zeros_like(ex), slopes=sl, row_offset=6)
    else:
        bad = X.mlp_bias(edge, params, 0.6, 16, extra=ex, slopes=sl, row_offset=0)
    assert rel(bad, want) > 1e-4
