"""GPU parity of the rectangular large-N attention kernel against the float64 oracle.

Calls the C ABI (hz_rect_attention_fwd) through the torch wrapper and the reference-named
mirror (pallas_rectangular_edge_attention, noncausal_bias_mha). Tolerance: max-norm
relative error ||out - ref||_inf / ||ref||_inf <= 1e-5 (float32). Determinism is checked
bit-exactly. Cases cover every head grouping (H % 4 == 0, H % 2 == 0, odd H), both
query-block sizes, D in {8, 16, 32, 64}, Nq != Nk, lengths that are not multiples of the
key chunk or query block, prefix / scattered / absent / all-masked key masks, a zero bias
and several systems per call.
"""

import numpy as np
import pytest
import torch

from oracle import rect_oracle as R

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def make(seed, B, Nq, Nk, H, D, n_phys=None, scattered=False, bias=True):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Nq, H, D), dtype=np.float32)
    k = rng.standard_normal((B, Nk, H, D), dtype=np.float32)
    v = rng.standard_normal((B, Nk, H, D), dtype=np.float32)
    e = rng.standard_normal((B, Nq, Nk, H), dtype=np.float32) * np.float32(D ** -0.5) if bias else None
    mask = None
    if n_phys is not None:
        mask = np.zeros((B, Nk), dtype=bool)
        for b in range(B):
            n = int(rng.integers(0, Nk + 1)) if n_phys < 0 else n_phys
            sites = rng.permutation(Nk)[:n] if scattered else np.arange(n)
            mask[b, sites] = True
    return q, k, v, e, mask


def dev(x):
    return None if x is None else torch.from_numpy(x).cuda()


def run(q, k, v, e, mask, scale):
    from hamiltonzero_amd import kernels

    out = kernels.rect_attention_fwd(dev(q), dev(k), dev(v), dev(e), dev(mask), scale=scale)
    torch.cuda.synchronize()
    return out.cpu().numpy()


CASES = [
    # B, Nq, Nk, H, D, n_phys, scattered, bias
    (1, 64, 64, 4, 32, None, False, True),
    (2, 100, 75, 4, 64, 60, True, True),
    (1, 256, 1024, 16, 64, 1000, False, True),  # a sequence-parallel rank's share at c5's width
    (3, 33, 47, 2, 16, 20, True, True),  # H % 4 != 0: two heads per workgroup
    (2, 17, 40, 3, 8, -1, True, True),  # odd H: one head per workgroup, per-system key counts
    (1, 7, 5, 8, 32, 5, False, True),
    (4, 128, 96, 8, 16, 80, True, False),  # no bias
    (2, 96, 130, 4, 64, 0, False, True),  # every key masked: mean of all values
    (1, 300, 33, 8, 64, None, False, True),  # no mask, four query tiles per workgroup
    (16, 64, 64, 8, 32, 36, False, True),  # many systems: the four-tile variant
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B%d_Nq%d_Nk%d_H%d_D%d_n%s_%s_%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], "scat" if c[6] else "pre", "bias" if c[7] else "nobias"))
def test_rect_parity(case):
    B, Nq, Nk, H, D, n_phys, scattered, bias = case
    _say(f"rect B={B} Nq={Nq} Nk={Nk} H={H} D={D} n_phys={n_phys} scattered={scattered} bias={bias}")
    q, k, v, e, mask = make(1000 + Nq + Nk + H + D, B, Nq, Nk, H, D, n_phys, scattered, bias)
    scale = D ** -0.5
    got = run(q, k, v, e, mask, scale)
    want = R.rect_fwd(q, k, v, e, mask, scale=scale)
    err = rel(got, want)
    assert err <= F32_TOL, err


def test_rect_all_masked_is_mean_of_values():
    _say("rect all keys masked")
    q, k, v, e, _ = make(7, 2, 40, 50, 4, 16)
    mask = np.zeros((2, 50), dtype=bool)
    got = run(q, k, v, e, mask, 0.25)
    want = np.broadcast_to(v.astype(np.float64).mean(axis=1, keepdims=True), got.shape)
    assert rel(got, want) <= F32_TOL


def test_rect_masked_keys_never_read():
    """Values of masked keys (k, v, bias; NaN in the bias) do not change the result."""
    _say("rect masked keys never read")
    q, k, v, e, mask = make(8, 2, 70, 90, 4, 32, n_phys=50, scattered=True)
    base = run(q, k, v, e, mask, 0.2)
    k2, v2, e2 = k.copy(), v.copy(), e.copy()
    for b in range(2):
        k2[b, ~mask[b]] = 7.0
        v2[b, ~mask[b]] = -3.0
        e2[b, :, ~mask[b]] = np.nan
    assert np.array_equal(run(q, k2, v2, e2, mask, 0.2), base)


def test_rect_deterministic():
    _say("rect determinism")
    q, k, v, e, mask = make(9, 2, 200, 300, 8, 64, n_phys=280, scattered=True)
    a = run(q, k, v, e, mask, 0.125)
    b = run(q, k, v, e, mask, 0.125)
    assert np.array_equal(a, b)


def test_reference_named_wrappers():
    """pallas_rectangular_edge_attention on one system and noncausal_bias_mha on a batch."""
    from hamiltonzero_amd import rect_attention as RA

    _say("rect reference-named wrappers")
    q, k, v, e, mask = make(10, 1, 128, 512, 8, 32, n_phys=500, scattered=False)
    out = RA.pallas_rectangular_edge_attention(dev(q[0]), dev(k[0]), dev(v[0]), dev(e[0]), dev(mask[0]))
    torch.cuda.synchronize()
    want = R.rect_fwd(q, k, v, e, mask, scale=32 ** -0.5)[0]
    assert rel(out.cpu().numpy(), want) <= F32_TOL

    q, k, v, e, _ = make(11, 2, 256, 128, 4, 64)
    out = RA.noncausal_bias_mha(dev(q), dev(k), dev(v), dev(e))
    torch.cuda.synchronize()
    assert rel(out.cpu().numpy(), R.rect_fwd(q, k, v, e, None, scale=1.0)) <= F32_TOL


GATED_CASES = [
    # B, Nq, Nk, H, D, n_phys, scattered, bias
    (1, 64, 64, 4, 32, None, False, True),       # H/2 even: two gate + two value heads per workgroup
    (2, 100, 75, 8, 64, 60, True, True),
    (1, 256, 1024, 16, 64, 1000, False, True),   # the large-N shape, four query tiles per workgroup
    (3, 33, 47, 6, 16, 20, True, True),          # H/2 odd: one gate + one value head per workgroup
    (2, 17, 40, 2, 8, -1, True, True),           # a single head pair, per-system key counts
    (4, 128, 96, 8, 16, 80, True, False),        # no bias
    (2, 96, 130, 4, 64, 0, False, True),         # every key masked
    (1, 300, 33, 16, 32, None, False, True),
]


@pytest.mark.parametrize("case", GATED_CASES, ids=lambda c: "B%d_Nq%d_Nk%d_H%d_D%d_n%s_%s_%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], "scat" if c[6] else "pre", "bias" if c[7] else "nobias"))
def test_rect_gated_parity(case):
    """hz_rect_attention_fwd_gated: y = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:] against the
    oracle, and against the ungated kernel followed by the collapse in torch."""
    from hamiltonzero_amd import kernels

    B, Nq, Nk, H, D, n_phys, scattered, bias = case
    _say(f"rect gated B={B} Nq={Nq} Nk={Nk} H={H} D={D} n_phys={n_phys} scattered={scattered} bias={bias}")
    q, k, v, e, mask = make(2000 + Nq + Nk + H + D, B, Nq, Nk, H, D, n_phys, scattered, bias)
    scale = D ** -0.5
    y = kernels.rect_attention_fwd(dev(q), dev(k), dev(v), dev(e), dev(mask), scale=scale, gated=True)
    out = kernels.rect_attention_fwd(dev(q), dev(k), dev(v), dev(e), dev(mask), scale=scale)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (B, Nq, H // 2, D)
    assert rel(y.cpu().numpy(), R.rect_gated(q, k, v, e, mask, scale=scale)) <= F32_TOL
    unfused = torch.sigmoid(out[:, :, : H // 2]) * out[:, :, H // 2:]
    assert rel(y.cpu().numpy(), unfused.cpu().numpy()) <= F32_TOL


def test_sequence_attention_output():
    """The large-N attention tail (sequence_trunk.py:973-984) through the mirror: gated
    rectangular attention, then W_O with the row mask, on one system; masked rows zero."""
    from hamiltonzero_amd import rect_attention as RA

    _say("rect gated + W_O mirror")
    rng = np.random.default_rng(12)
    q, k, v, e, mask = make(13, 1, 192, 256, 16, 16, n_phys=240, scattered=True)
    w_o = (rng.standard_normal((8 * 16, 64)) / np.sqrt(128)).astype(np.float32)
    row_mask = rng.random((1, 192)) < 0.7
    got = RA.sequence_attention_output(dev(q[0]), dev(k[0]), dev(v[0]), dev(e[0]), dev(mask[0]), dev(w_o),
                                       dev(row_mask[0]))
    y = RA.gated_rectangular_edge_attention(dev(q[0]), dev(k[0]), dev(v[0]), dev(e[0]), dev(mask[0]))
    torch.cuda.synchronize()
    want = R.sequence_attention_output(q, k, v, e, mask, w_o, row_mask, scale=16 ** -0.5)[0]
    assert rel(got.cpu().numpy(), want) <= F32_TOL
    assert np.all(got.cpu().numpy()[~row_mask[0]] == 0.0)
    assert rel(y.cpu().numpy(), R.rect_gated(q, k, v, e, mask, scale=16 ** -0.5)[0]) <= F32_TOL


def test_rect_gated_rejects_odd_heads():
    from hamiltonzero_amd import kernels

    q, k, v, e, _ = make(14, 1, 16, 16, 3, 8)
    with pytest.raises(ValueError, match="H must be even"):
        kernels.rect_attention_fwd(dev(q), dev(k), dev(v), dev(e), None, gated=True)
