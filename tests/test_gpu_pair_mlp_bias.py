"""GPU parity of the MLP-class coupling-bias producer (hz_pair_mlp_bias) against the float64
oracle (oracle/pair_bias_oracle.py: mlp_bias / mlp_bias_jvp, pinned in
tests/test_pair_bias_oracle.py).

Cases follow the three callers: the tree's LevelEdgeAttn (edge channels 96, hidden 128, one
block, 16 heads, LCA-ALiBi on positions 0..n-1; model/tree.py:1392-1456), the readout context
(hidden 32, the direction as an extra input channel; model/readout_leaf_context.py:694-712)
and the large-N trunk (rectangular Nq x Nk, a global row offset for the ALiBi positions;
evaluation/sequence_trunk.py:962-972), plus two-block MLPs, 32 heads, both output layouts, the
square and the key mask (an empty walker included) and T = 0 / 1. Only the pairs the attention
reads are compared (the others are not written); tolerance: max-norm relative error <= 1e-5
(float32).
"""

import numpy as np
import pytest
import torch

from oracle import pair_bias_oracle as X
from oracle import rect_oracle as R

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


CASES = [
    # name, B, Nq, Nk, C, hidden, H, n_blocks, T, extra, alibi, row_offset, mask ("none"/"square"/"key"), layout
    ("tree", 4, 64, 64, 96, 128, 16, 1, 1, False, True, 0, "square", "qkh"),
    ("tree_t0_qhk", 3, 48, 48, 96, 128, 16, 1, 0, False, True, 0, "square", "qhk"),
    ("readout", 3, 40, 40, 96, 32, 16, 1, 1, True, True, 0, "key", "qkh"),
    ("large_n", 1, 100, 300, 96, 128, 16, 1, 0, False, True, 1000, "key", "qkh"),
    ("large_n_t1_nomask", 1, 37, 130, 64, 128, 32, 1, 1, False, True, 4090, "none", "qkh"),
    ("two_blocks_h32", 2, 33, 33, 64, 64, 32, 2, 0, False, False, 0, "none", "qhk"),
    ("two_blocks_tan", 2, 24, 24, 32, 64, 16, 2, 1, True, True, 0, "square", "qhk"),
    ("hidden32_empty_walker", 3, 20, 20, 32, 32, 32, 1, 1, False, False, 0, "square_empty", "qhk"),
    ("c128_h128", 2, 16, 16, 128, 128, 32, 1, 1, False, True, 0, "key_empty", "qkh"),
]


def _make(name, B, Nq, Nk, C, hidden, H, nb, T, extra, mask_kind, seed):
    rng = np.random.default_rng(seed)
    params = X.init_mlp_params(rng, C, hidden, H, nb, extra=extra, scale_bias=0.2)
    edge = rng.standard_normal((B, Nq, Nk, C)).astype(np.float32)
    edge_t = rng.standard_normal((B, Nq, Nk, C)).astype(np.float32) if T else None
    ex = rng.standard_normal((B, Nq, Nk)).astype(np.float32) if extra else None
    ex_t = rng.standard_normal((B, Nq, Nk)).astype(np.float32) if (extra and T) else None
    mask = None
    if mask_kind != "none":
        mask = rng.random((B, Nk)) < 0.7
        if mask_kind.endswith("empty"):
            mask[0] = False
    return params, edge, edge_t, ex, ex_t, mask


def _read_pairs(mask, B, Nq, Nk, square):
    """[B, Nq, Nk] bool: the pairs the attention reads (all without a mask)."""
    if mask is None:
        return np.ones((B, Nq, Nk), dtype=bool)
    keys = mask.copy()
    if not square:
        keys[~mask.any(axis=1)] = True  # key-mask mode: a walker with no physical key uses every key
        return np.broadcast_to(keys[:, None, :], (B, Nq, Nk)).copy()
    return mask[:, :, None] & mask[:, None, :]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_pair_mlp_bias_matches_oracle(case):
    from hamiltonzero_amd import pair_bias

    name, B, Nq, Nk, C, hidden, H, nb, T, extra, alibi, row_offset, mask_kind, layout = case
    _say(f"pair mlp bias {case}")
    params, edge, edge_t, ex, ex_t, mask = _make(name, B, Nq, Nk, C, hidden, H, nb, T, extra, mask_kind,
                                                  sum(map(ord, name)))
    square = mask_kind.startswith("square")
    slopes = X.lca_fixed_slopes(H) if alibi else None
    d_head = 16
    res = pair_bias.mlp_bias(dev(edge), {k: dev(v) for k, v in params.items()}, d_head=d_head, inner_gain=0.7,
                             extra=dev(ex), alibi_slopes=dev(slopes), row_offset=row_offset, mask=dev(mask),
                             key_mask=not square, e_layout=layout, edge_t=dev(edge_t), extra_t=dev(ex_t))
    torch.cuda.synchronize()
    e, e_t = (res, None) if T == 0 else res
    if T:
        want, want_t = X.mlp_bias_jvp(edge, edge_t, params, 0.7, d_head, extra=ex, extra_t=ex_t, slopes=slopes,
                                      row_offset=row_offset)
    else:
        want = X.mlp_bias(edge, params, 0.7, d_head, extra=ex, slopes=slopes, row_offset=row_offset)
    to_ref = (lambda a: a) if layout == "qkh" else (lambda a: np.swapaxes(a, 2, 3))  # -> [B, Nq, Nk, H]
    read = _read_pairs(mask, B, Nq, Nk, square)
    got = to_ref(e.cpu().numpy())
    assert rel(got[read], want[read]) <= TOL, "e"
    if mask is not None and Nk <= 256:  # beyond 256 keys the producer computes every pair
        assert np.all(got[~read] == 0.0), "pairs the attention never reads are left untouched (zeros here)"
    if T:
        assert rel(to_ref(e_t.cpu().numpy())[read], want_t[read]) <= TOL, "e_t"


def test_pair_mlp_bias_feeds_the_gated_rect_attention():
    """The large-N chain (sequence_trunk.py:962-984): the producer's bias with a global row
    offset, then the gated rectangular attention, against the oracle's chain."""
    from hamiltonzero_amd import kernels, pair_bias

    _say("pair mlp bias -> gated rect")
    rng = np.random.default_rng(5)
    Nq, Nk, H, D, C = 96, 200, 16, 32, 96
    params = X.init_mlp_params(rng, C, 128, H, 1, scale_bias=0.2)
    edge = rng.standard_normal((1, Nq, Nk, C)).astype(np.float32)
    q = rng.standard_normal((1, Nq, H, D)).astype(np.float32)
    k, v = (rng.standard_normal((1, Nk, H, D)).astype(np.float32) for _ in range(2))
    mask = rng.random((1, Nk)) < 0.9
    slopes = X.lca_fixed_slopes(H)
    bias = pair_bias.mlp_bias(dev(edge), {n: dev(x) for n, x in params.items()}, d_head=D, inner_gain=1.0,
                              alibi_slopes=dev(slopes), row_offset=512, mask=dev(mask), key_mask=True)
    y = kernels.rect_attention_fwd(dev(q), dev(k), dev(v), bias, dev(mask), scale=D ** -0.5, gated=True)
    torch.cuda.synchronize()
    want_bias = X.mlp_bias(edge, params, 1.0, D, slopes=slopes, row_offset=512)
    want = R.rect_gated(q, k, v, want_bias, mask, scale=D ** -0.5)
    assert rel(y.cpu().numpy(), want) <= TOL


def test_pair_mlp_bias_rejects_bad_arguments():
    from hamiltonzero_amd import _native, pair_bias

    rng = np.random.default_rng(6)
    params = X.init_mlp_params(rng, 96, 128, 16, 2)
    edge = dev(rng.standard_normal((1, 8, 8, 96)).astype(np.float32))
    with pytest.raises(_native.HzError, match="n_blocks"):
        pair_bias.mlp_bias(edge, {k: dev(v) for k, v in params.items()}, d_head=16)
    p1 = X.init_mlp_params(rng, 96, 48, 16, 1)
    with pytest.raises(ValueError, match="hidden width"):
        pair_bias.mlp_bias(edge, {k: dev(v) for k, v in p1.items()}, d_head=16)
