"""Pins the rectangular-attention oracle (oracle/rect_oracle.py) without the reference.

Each check fixes a fact of the reference's computation (src/hamiltonzero/evaluation/
pallas_mha.py:43-161, sequence_parallel.py:59-90) independently of the oracle's own
formula: explicit loops, closed forms, the float32 arithmetic of the -1e30 mask, the
already-pinned square oracle, and invariances. Planted mistakes in a copy of the oracle
show that these checks catch the plausible errors.
"""

import numpy as np
import pytest

from oracle import mhsea_oracle as O
from oracle import rect_oracle as R


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def make(rng, B, Nq, Nk, H, D, n_phys=None, scattered=False):
    q = rng.standard_normal((B, Nq, H, D))
    k = rng.standard_normal((B, Nk, H, D))
    v = rng.standard_normal((B, Nk, H, D))
    bias = rng.standard_normal((B, Nq, Nk, H))
    mask = np.zeros((B, Nk), dtype=bool)
    for b in range(B):
        n = Nk if n_phys is None else n_phys
        sites = rng.permutation(Nk)[:n] if scattered else np.arange(n)
        mask[b, sites] = True
    return q, k, v, bias, mask


@pytest.mark.parametrize("scattered", [False, True])
def test_matches_explicit_loops(scattered):
    rng = np.random.default_rng(0)
    q, k, v, bias, mask = make(rng, 2, 3, 5, 2, 4, n_phys=3, scattered=scattered)
    want = R.rect_fwd_loops(q, k, v, bias, mask, scale=0.7)
    assert rel(R.rect_fwd(q, k, v, bias, mask, scale=0.7), want) < 1e-13


def test_single_key_returns_its_value():
    rng = np.random.default_rng(1)
    q, k, v, bias, mask = make(rng, 2, 4, 1, 3, 8)
    out = R.rect_fwd(q, k, v, bias, mask, scale=0.3)
    np.testing.assert_allclose(out, np.broadcast_to(v[:, :1], out.shape), atol=1e-15)


def test_dominant_bias_selects_that_value_row():
    rng = np.random.default_rng(2)
    q, k, v, bias, mask = make(rng, 1, 5, 6, 2, 8)
    bias[:] = 0.0
    bias[0, :, 3, :] = 80.0  # every query, every head attends to key 3
    out = R.rect_fwd(q, k, v, bias, mask)
    np.testing.assert_allclose(out[0], np.broadcast_to(v[0, 3], out[0].shape), atol=1e-12)


def test_zero_scores_average_the_physical_values():
    rng = np.random.default_rng(3)
    q, k, v, _, mask = make(rng, 2, 3, 9, 2, 8, n_phys=4, scattered=True)
    out = R.rect_fwd(np.zeros_like(q), k, v, None, mask)
    for b in range(2):
        mean = v[b, mask[b]].mean(axis=0)
        np.testing.assert_allclose(out[b], np.broadcast_to(mean, out[b].shape), atol=1e-15)


def test_all_masked_follows_float32_arithmetic():
    """Every key masked: the reference's float32 logits q.k + (-1e30) all round to -1e30
    (pallas_mha.py:68-71), so each weight is 1 and out is the mean of all value rows.
    Evaluated here literally in float32, independently of the oracle's special case."""
    rng = np.random.default_rng(4)
    B, Nq, Nk, H, D = 1, 3, 7, 2, 8
    q, k, v, bias, _ = make(rng, B, Nq, Nk, H, D)
    q32, k32, b32 = (x.astype(np.float32) for x in (q, k, bias))
    logits = np.einsum("bihd,bjhd->bhij", q32, k32).astype(np.float32)
    masked_bias = np.where(np.zeros((B, 1, Nk, 1), dtype=bool), b32, np.float32(-1e30))
    logits = (logits + masked_bias.transpose(0, 3, 1, 2)) * np.float32(np.log2(np.e))
    w = np.exp2(logits - logits.max(-1, keepdims=True))
    assert np.all(w == 1.0)
    w = w.astype(np.float64)
    want = np.einsum("bhij,bjhd->bihd", w / w.sum(-1, keepdims=True), v)
    out = R.rect_fwd(q, k, v, bias, np.zeros((B, Nk), dtype=bool))
    assert rel(out, want) < 1e-13
    np.testing.assert_allclose(out[0, 0, 0], v[0, :, 0].mean(axis=0), atol=1e-14)


def test_square_case_equals_pinned_key_mask_oracle():
    """Nq = Nk: the -1e30 replacement and reference_edge_attention's additive -1e9 give the
    same result whenever a key is physical (both weights underflow to exactly 0)."""
    rng = np.random.default_rng(5)
    B, N, H, D = 3, 10, 2, 16
    q, k, v, bias, mask = make(rng, B, N, N, H, D, n_phys=6, scattered=True)
    scale = D ** -0.5
    want, _ = O.fwd(q, k, bias, v, mask, scale=scale, key_mask=True, e_layout="qkh")
    assert rel(R.rect_fwd(q, k, v, bias, mask, scale=scale), want) < 1e-13


def test_sequence_parallel_rows_of_the_square_problem():
    """A rank's local query rows against all keys equal those rows of the full problem
    (the decomposition sequence_trunk.py uses around this op)."""
    rng = np.random.default_rng(6)
    B, N, H, D = 2, 12, 2, 8
    q, k, v, bias, mask = make(rng, B, N, N, H, D, n_phys=9, scattered=True)
    full = R.rect_fwd(q, k, v, bias, mask, scale=0.4)
    for lo, hi in ((0, 4), (4, 8), (8, 12)):
        part = R.rect_fwd(q[:, lo:hi], k, v, bias[:, lo:hi], mask, scale=0.4)
        assert rel(part, full[:, lo:hi]) < 1e-14


def test_invariances():
    rng = np.random.default_rng(7)
    B, Nq, Nk, H, D = 2, 5, 11, 3, 8
    q, k, v, bias, mask = make(rng, B, Nq, Nk, H, D, n_phys=7, scattered=True)
    out = R.rect_fwd(q, k, v, bias, mask, scale=0.5)
    perm = rng.permutation(Nk)
    out_p = R.rect_fwd(q, k[:, perm], v[:, perm], bias[:, :, perm], mask[:, perm], scale=0.5)
    assert rel(out_p, out) < 1e-13
    k2, v2, b2 = k.copy(), v.copy(), bias.copy()
    for b in range(B):
        k2[b, ~mask[b]] = rng.standard_normal(k2[b, ~mask[b]].shape) * 5
        v2[b, ~mask[b]] = rng.standard_normal(v2[b, ~mask[b]].shape) * 5
        b2[b, :, ~mask[b]] = np.nan
    assert rel(R.rect_fwd(q, k2, v2, b2, mask, scale=0.5), out) < 1e-14
    # the per-(query, head) constant added to the bias cancels in the softmax
    shift = rng.standard_normal((B, Nq, 1, H))
    assert rel(R.rect_fwd(q, k, v, bias + shift, mask, scale=0.5), out) < 1e-12


def _planted(kind):
    def f(q, k, v, bias, mask, *, scale=1.0):
        if kind == "bias_transposed":  # read bias as [B, Nk, Nq, H]
            bias = np.swapaxes(bias, 1, 2)
            return R.rect_fwd(q, k, v, bias, mask, scale=scale)
        if kind == "mask_ignored":
            return R.rect_fwd(q, k, v, bias, None, scale=scale)
        if kind == "scale_on_bias_too":
            return R.rect_fwd(q, k, v, bias * scale, mask, scale=scale)
        raise ValueError(kind)

    return f


@pytest.mark.parametrize("kind", ["bias_transposed", "mask_ignored", "scale_on_bias_too"])
def test_planted_mistakes_are_caught(kind):
    rng = np.random.default_rng(8)
    q, k, v, bias, mask = make(rng, 2, 6, 6, 2, 8, n_phys=4, scattered=True)
    bad = _planted(kind)(q, k, v, bias, mask, scale=0.5)
    want = R.rect_fwd_loops(q, k, v, bias, mask, scale=0.5)
    assert rel(bad, want) > 1e-3


def _gated_loops(q, k, v, bias, mask, w_o, row_mask, scale):
    """y and the masked projection by explicit loops over the element-loop forward: head h
    of y is sigmoid(head h) times head h + H/2 (H/2 = the module's n_heads)."""
    import math

    out = R.rect_fwd_loops(q, k, v, bias, mask, scale=scale)
    B, Nq, H, D = out.shape
    hh = H // 2
    y = np.zeros((B, Nq, hh, D))
    for b in range(B):
        for i in range(Nq):
            for h in range(hh):
                for d in range(D):
                    y[b, i, h, d] = out[b, i, h + hh, d] / (1.0 + math.exp(-out[b, i, h, d]))
    proj = np.zeros((B, Nq, w_o.shape[1]))
    for b in range(B):
        for i in range(Nq):
            if not row_mask[b, i]:
                continue
            flat = y[b, i].reshape(-1)
            for o in range(w_o.shape[1]):
                proj[b, i, o] = sum(flat[f] * w_o[f, o] for f in range(flat.size))
    return y, proj


def test_gated_and_projection_against_loops():
    """rect_gated / sequence_attention_output against explicit loops; swapping the gate and
    value halves (a planted mistake) fails."""
    rng = np.random.default_rng(9)
    B, Nq, Nk, H, D = 2, 5, 7, 4, 8
    q, k, v, bias, mask = make(rng, B, Nq, Nk, H, D, n_phys=5, scattered=True)
    w_o = rng.standard_normal((H // 2 * D, 6))
    row_mask = rng.random((B, Nq)) < 0.6
    y_loop, proj_loop = _gated_loops(q, k, v, bias, mask, w_o, row_mask, 0.5)
    assert rel(R.rect_gated(q, k, v, bias, mask, scale=0.5), y_loop) < 1e-12
    assert rel(R.sequence_attention_output(q, k, v, bias, mask, w_o, row_mask, scale=0.5), proj_loop) < 1e-12
    out = R.rect_fwd(q, k, v, bias, mask, scale=0.5)
    swapped = out[:, :, : H // 2] / (1.0 + np.exp(-out[:, :, H // 2:]))  # gate and value exchanged
    assert rel(swapped, y_loop) > 1e-3
