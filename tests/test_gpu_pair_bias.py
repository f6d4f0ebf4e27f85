"""GPU parity of the coupling-bias producer (hz_pair_bias) against the float64 oracle
(oracle/pair_bias_oracle.py, pinned in tests/test_pair_bias_oracle.py), through the C ABI.

Covers every channel count and head count the kernel instantiates, both output layouts, the
tangent, the square-mask pair compaction (only the pairs the attention reads are written;
other entries keep their previous contents), the key-mask mode (every query row; a walker
with no physical site gets every pair), a batch where every wave walks several (walker,
part) items, and the producer feeding the trunk's gated attention (fwd + JVP) against the
oracle's chain. Tolerance: max-norm relative error <= 1e-5 (float32 products and
accumulation, as the reference computes this path).
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O
from oracle import pair_bias_oracle as X

pytestmark = pytest.mark.gpu

TOL = 1e-5
GAIN = 8 ** -0.5
SENTINEL = 7.25


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _run(edge, edge_t, mask, params, d_head, key_mask=False, layout="qhk"):
    """The raw C ABI on outputs pre-filled with a sentinel; returns host (e, e_t) in the
    oracle's [B, N(query), N(key), H] layout."""
    from hamiltonzero_amd import _native

    lib = _native.lib()
    B, N, _, C = edge.shape
    H = params["w_out"].shape[1]
    eshape = (B, N, H, N) if layout == "qhk" else (B, N, N, H)
    e = torch.full(eshape, SENTINEL, dtype=torch.float32, device="cuda")
    et = torch.full(eshape, SENTINEL, dtype=torch.float32, device="cuda") if edge_t is not None else None
    d = {n: dev(params[n]) for n in params}
    m = dev(mask.astype(np.uint8)) if mask is not None else None
    ed, etd = dev(edge), dev(edge_t)
    flags = (_native.HZ_FLAG_KEY_MASK if key_mask else 0) | (_native.HZ_FLAG_E_QKH if layout == "qkh" else 0)
    args = [torch.cuda.current_stream().cuda_stream, ed.data_ptr(), None if etd is None else etd.data_ptr(),
            None if m is None else m.data_ptr()]
    args += [d[n].data_ptr() for n in ("ln_w", "w_in", "b_in", "w_1", "b_1", "w_2", "b_2", "w_out", "b_out")]
    args += [e.data_ptr(), None if et is None else et.data_ptr(), B, N, C, 64, H, 0 if edge_t is None else 1,
             GAIN, 1e-5, float(np.sqrt(np.float32(d_head))), flags]
    _native.check(lib.hz_pair_bias(*args))
    torch.cuda.synchronize()

    def back(t):
        if t is None:
            return None
        a = t.cpu().numpy()
        return np.swapaxes(a, 2, 3) if layout == "qhk" else a

    return back(e), back(et)


def _inputs(seed, B, N, C, H, tangent):
    rng = np.random.default_rng(seed)
    params = X.init_params(rng, C, 64, H)
    edge = rng.standard_normal((B, N, N, C), dtype=np.float32)
    edge_t = rng.standard_normal((B, N, N, C), dtype=np.float32) if tangent else None
    return params, edge, edge_t


def _computed_pairs(mask, key_mask):
    """[B, N, N] bool: the pairs hz_pair_bias writes for this mask."""
    B, N = mask.shape
    rows = np.ones((B, N), bool) if key_mask else mask
    w = rows[:, :, None] & mask[:, None, :]
    if key_mask:
        w[~mask.any(axis=1)] = True
    return w


@pytest.mark.parametrize("C", [32, 64, 96, 128])
@pytest.mark.parametrize("H", [16, 32, 64])
@pytest.mark.parametrize("tangent", [False, True])
def test_all_pairs_match_oracle(C, H, tangent):
    _say(f"pair bias C={C} H={H} tangent={tangent}")
    B, N = 3, 11
    params, edge, edge_t = _inputs(C + H + tangent, B, N, C, H, tangent)
    e, et = _run(edge, edge_t, None, params, 16)
    if tangent:
        want, want_t = X.coupling_bias_jvp(edge, edge_t, params, GAIN, 16)
        assert rel(et, want_t) <= TOL
    else:
        want = X.coupling_bias(edge, params, GAIN, 16)
    assert rel(e, want) <= TOL


@pytest.mark.parametrize("layout", ["qhk", "qkh"])
@pytest.mark.parametrize("key_mask", [False, True])
def test_masked_pairs_compacted(layout, key_mask):
    _say(f"pair bias mask layout={layout} key_mask={key_mask}")
    rng = np.random.default_rng(7)
    B, N, C, H = 6, 64, 96, 32
    params, edge, edge_t = _inputs(8, B, N, C, H, True)
    mask = np.zeros((B, N), bool)
    for b in range(B):
        mask[b, rng.permutation(N)[: [36, 0, 64, 1, 17, 50][b]]] = True
    e, et = _run(edge, edge_t, mask, params, 16, key_mask=key_mask, layout=layout)
    want, want_t = X.coupling_bias_jvp(edge, edge_t, params, GAIN, 16)
    w = _computed_pairs(mask, key_mask)
    assert rel(e[w], want[w]) <= TOL
    assert rel(et[w], want_t[w]) <= TOL
    assert np.all(e[~w] == SENTINEL) and np.all(et[~w] == SENTINEL)


def test_large_n_without_compaction():
    """N above the compaction limit (256): every pair is computed even with a mask."""
    _say("pair bias N=260 mask")
    B, N, C, H = 1, 260, 32, 16
    params, edge, _ = _inputs(9, B, N, C, H, False)
    mask = np.zeros((B, N), bool)
    mask[0, :100] = True
    e, _ = _run(edge, None, mask, params, 16)
    assert rel(e, X.coupling_bias(edge, params, GAIN, 16)) <= TOL


def test_many_items_per_wave():
    """64 walkers of 64 sites (36 physical, scattered per walker): several (walker, part)
    items per wave, at the trunk's channel and head counts."""
    _say("pair bias B=64 N=64 C=96 H=32 mask")
    rng = np.random.default_rng(10)
    B, N, C, H = 64, 64, 96, 32
    params, edge, edge_t = _inputs(11, B, N, C, H, True)
    mask = np.zeros((B, N), bool)
    for b in range(B):
        mask[b, rng.permutation(N)[:36]] = True
    e, et = _run(edge, edge_t, mask, params, 16)
    want, want_t = X.coupling_bias_jvp(edge, edge_t, params, GAIN, 16)
    w = _computed_pairs(mask, False)
    assert rel(e[w], want[w]) <= TOL
    assert rel(et[w], want_t[w]) <= TOL


def test_mirror_zero_fills_and_matches():
    from hamiltonzero_amd import pair_bias

    _say("pair bias torch mirror")
    rng = np.random.default_rng(12)
    B, N, C, H = 2, 16, 64, 16
    params, edge, edge_t = _inputs(13, B, N, C, H, True)
    mask = np.zeros((B, N), bool)
    mask[0, :9] = True
    mask[1, rng.permutation(N)[:5]] = True
    e, et = pair_bias.coupling_bias(dev(edge), {n: dev(v) for n, v in params.items()}, d_head=16, inner_gain=GAIN,
                                    mask=dev(mask), edge_t=dev(edge_t), e_layout="qkh")
    torch.cuda.synchronize()
    want, want_t = X.coupling_bias_jvp(edge, edge_t, params, GAIN, 16)
    w = _computed_pairs(mask, False)
    assert rel(e.cpu().numpy()[w], want[w]) <= TOL
    assert rel(et.cpu().numpy()[w], want_t[w]) <= TOL
    assert np.all(e.cpu().numpy()[~w] == 0.0)


def test_producer_feeds_gated_attention():
    """The trunk's attention call with its learned bias (trunk.py:89-137): the producer's
    (e, e_t) into hz_mhsea_fwd_jvp_gated, against the oracle's coupling bias + gated fwd/JVP."""
    from hamiltonzero_amd import kernels, pair_bias

    _say("pair bias -> gated attention, [8, 64, 32, 16], 36/64")
    rng = np.random.default_rng(14)
    B, N, H, D, C = 8, 64, 32, 16, 96
    params, edge, edge_t = _inputs(15, B, N, C, H, True)
    mask = np.zeros((B, N), bool)
    for b in range(B):
        mask[b, rng.permutation(N)[:36]] = True
    q, k, v, qt, kt, vt = (rng.standard_normal((B, N, H, D), dtype=np.float32) * np.float32(0.25) for _ in range(6))
    e, et = pair_bias.coupling_bias(dev(edge), {n: dev(x) for n, x in params.items()}, d_head=D, inner_gain=GAIN,
                                    mask=dev(mask), edge_t=dev(edge_t))
    y, ty = kernels.mhsea_fwd_jvp_gated(dev(q), dev(k), dev(v), dev(mask), dev(qt[None]), dev(kt[None]),
                                        dev(vt[None]), e=e, et=et[None], scale=D ** -0.5)
    torch.cuda.synchronize()
    eb, ebt = X.coupling_bias_jvp(edge, edge_t, params, GAIN, D)
    wy, wty = O.gated_fwd_jvp(q, k, X.to_attention_layout(eb), v, mask, qt, kt, X.to_attention_layout(ebt), vt,
                              scale=D ** -0.5)
    assert rel(y.cpu().numpy(), wy) <= TOL
    assert rel(ty[0].cpu().numpy(), wty) <= TOL


POISON_ROUTES = [
    # name, N, D, dtype, key_mask, generic
    ("fwd_small", 24, 16, torch.float32, False, False),
    ("fwd_pc", 64, 32, torch.float32, False, False),
    ("fwd_jvp_pc", 64, 32, torch.float32, False, False),
    ("fwd_jvp_generic", 64, 32, torch.float32, False, True),
    ("fwd_jvp_large_n", 100, 32, torch.float32, False, False),
    ("fwd_jvp_keymask", 64, 32, torch.float32, True, False),
    ("gated", 64, 16, torch.float32, False, False),
    ("bwd_stream", 64, 32, torch.float32, False, False),
    ("bwd_large_n", 100, 16, torch.float32, False, False),
    ("fwd_jvp_bf16", 64, 64, torch.bfloat16, False, False),
    ("fwd_jvp_bf16_large", 160, 64, torch.bfloat16, False, False),
    ("bwd_bf16", 64, 64, torch.bfloat16, False, False),
]


@pytest.mark.parametrize("route", POISON_ROUTES, ids=[r[0] for r in POISON_ROUTES])
def test_attention_never_reads_uncomputed_bias(route):
    """Every attention kernel family gives bit-identical results whether the bias entries
    hz_pair_bias leaves unwritten (masked pairs) hold zeros or NaN: those entries are never
    read, so the producer need not fill them."""
    from hamiltonzero_amd import kernels

    name, N, D, dtype, key_mask, generic = route
    _say(f"uncomputed bias entries never read: {name}")
    rng = np.random.default_rng(16)
    B, H = 5, 4
    mask = np.zeros((B, N), bool)
    for b in range(B):
        mask[b, rng.permutation(N)[: [N // 2, 1, N, (5 * N) // 8, 3][b]]] = True
    w = _computed_pairs(mask, key_mask)                            # [B, Nq, Nk]
    poison = np.broadcast_to(~w[:, :, None, :], (B, N, H, N))      # e layout [B, N, H, N]

    def t(shape, scale=1.0):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).cuda().to(dtype)

    q, k, v = t((B, N, H, D), D ** -0.5), t((B, N, H, D), D ** -0.5), t((B, N, H, D))
    qt, kt, vt, dout = t((1, B, N, H, D)), t((1, B, N, H, D)), t((1, B, N, H, D)), t((B, N, H, D))
    e0, et0 = t((B, N, H, N), 0.5), t((1, B, N, H, N))
    pz = torch.from_numpy(np.ascontiguousarray(poison)).cuda()
    m = dev(mask)

    def run(fill):
        e = torch.where(pz, torch.full_like(e0, fill), e0)
        et = torch.where(pz[None], torch.full_like(et0, fill), et0)
        kw = dict(scale=D ** -0.5, key_mask=key_mask, generic=generic)
        if name.startswith("fwd_jvp"):
            out, lse, tout = kernels.mhsea_fwd_jvp(q, k, v, m, qt, kt, vt, e=e, et=et, **kw)
            res = [out, lse, tout]
        elif name.startswith("fwd"):
            res = list(kernels.mhsea_fwd(q, k, v, m, e=e, **kw))
        elif name == "gated":
            res = list(kernels.mhsea_fwd_jvp_gated(q, k, v, m, qt, kt, vt, e=e, et=et, scale=D ** -0.5))
        else:
            out, lse = kernels.mhsea_fwd(q, k, v, m, e=e, **kw)
            dq, dk, de, dv = kernels.mhsea_bwd(q, k, v, m, lse, out, dout, e=e, **kw)
            de = torch.where(pz, torch.zeros_like(de), de)  # the cotangent of an unread entry is not compared
            res = [out, lse, dq, dk, de, dv]
        torch.cuda.synchronize()
        return [r.float().cpu().numpy() for r in res]

    clean, poisoned = run(0.0), run(float("nan"))
    for a, b in zip(clean, poisoned):
        assert np.array_equal(a, b, equal_nan=False), name
