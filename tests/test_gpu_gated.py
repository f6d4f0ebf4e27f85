"""GPU parity of the gated head collapse (hz_mhsea_fwd_jvp_gated) against the float64 oracle.

The fused kernel's y = sigmoid(gate) * value and its tangents are compared with
``oracle.mhsea_oracle.gated_fwd_jvp`` (pinned in tests/test_gated_oracle.py) on seeded
inputs, over T in {0, 1, 2}, D in {8, 16, 32, 64}, prefix / scattered / empty masks, the key-mask
mode, bias in both layouts, the kernel's own two-direction variant (D <= 16) and the two-pass
route (D = 32), and grids where one workgroup walks several head pairs; and
against the unfused composition (hz_mhsea_fwd_jvp, then the collapse in torch) at c2's shape.
Tolerance: max-norm relative error <= 1e-5 (float32).
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def make(seed, B, N, H, D, T, mask_kind, with_e, e_layout):
    rng = np.random.default_rng(seed)
    shape = (B, N, H, D)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(D ** -0.5) for _ in range(3))
    eshape = (B, N, H, N) if e_layout == "qhk" else (B, N, N, H)
    e = rng.standard_normal(eshape, dtype=np.float32) * np.float32(0.5) if with_e else None
    tq, tk, tv = (rng.standard_normal((max(T, 1), *shape), dtype=np.float32) for _ in range(3))
    te = rng.standard_normal((max(T, 1), *eshape), dtype=np.float32) if with_e else None
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        n = int(rng.integers(0, N + 1)) if mask_kind == "counts" else max(1, (9 * N) // 16)
        mask[b, np.arange(n) if mask_kind == "prefix" else rng.permutation(N)[:n]] = True
    return q, k, v, e, mask, tq, tk, tv, te


CASES = [
    # seed, B, N, H, D, T, mask, key_mask, e, e_layout
    (1, 64, 64, 8, 32, 1, "prefix", False, False, "qhk"),
    (2, 37, 64, 8, 32, 2, "scattered", False, True, "qhk"),
    (3, 20, 40, 4, 16, 1, "counts", False, True, "qkh"),
    (4, 50, 64, 2, 8, 0, "scattered", False, False, "qhk"),
    (5, 9, 17, 6, 32, 2, "counts", True, True, "qhk"),
    (6, 300, 64, 8, 32, 1, "scattered", False, False, "qhk"),
    (7, 3, 8, 4, 16, 1, "prefix", False, True, "qhk"),
    (8, 11, 64, 4, 32, 0, "counts", True, False, "qhk"),
    (9, 40, 64, 4, 16, 2, "scattered", False, True, "qkh"),
    (10, 13, 33, 2, 8, 2, "counts", False, False, "qhk"),
    (11, 25, 64, 8, 8, 1, "prefix", True, True, "qhk"),
    # the trunk's own call: n_heads 16 doubled for the gate, d_head 256 / 16 (config.py:20,26)
    (12, 48, 64, 32, 16, 2, "prefix", False, True, "qkh"),
    # N > 64 and D = 64: the LDS-streaming kernel (gate head, then value head, per block)
    (13, 6, 100, 4, 32, 2, "scattered", False, True, "qhk"),
    (14, 3, 256, 2, 64, 1, "counts", False, True, "qkh"),
    (15, 4, 130, 8, 16, 2, "prefix", True, True, "qhk"),
    (16, 5, 96, 6, 8, 0, "scattered", False, False, "qhk"),
    (17, 2, 300, 4, 64, 2, "scattered", False, False, "qhk"),
    (18, 7, 64, 4, 64, 1, "prefix", False, True, "qhk"),
]


@pytest.mark.parametrize("case", CASES, ids=["s{}_B{}_N{}_H{}_D{}_T{}_{}{}{}{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], "_keymask" if c[7] else "", "_e" if c[8] else "", c[9] if c[8] else "")
    for c in CASES])
def test_gated_matches_oracle(case):
    from hamiltonzero_amd import kernels

    seed, B, N, H, D, T, mask_kind, key_mask, with_e, e_layout = case
    _say(f"gated {case}")
    q, k, v, e, mask, tq, tk, tv, te = make(seed, B, N, H, D, T, mask_kind, with_e, e_layout)
    dev = lambda x: None if x is None else torch.from_numpy(x).cuda()  # noqa: E731
    scale = D ** -0.5
    kw = dict(scale=scale, key_mask=key_mask, e_layout=e_layout)
    if T == 0:
        y, ty = kernels.mhsea_fwd_jvp_gated(dev(q), dev(k), dev(v), dev(mask), e=dev(e), **kw)
        assert ty is None
    else:
        y, ty = kernels.mhsea_fwd_jvp_gated(dev(q), dev(k), dev(v), dev(mask), dev(tq[:T]), dev(tk[:T]), dev(tv[:T]),
                                            e=dev(e), et=None if te is None else dev(te[:T]), **kw)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (B, N, H // 2, D)
    for t in range(max(T, 1)):
        ey, eyd = O.gated_fwd_jvp(q, k, e, v, mask, tq[t], tk[t], None if te is None else te[t], tv[t], **kw)
        if t == 0:
            assert rel(y.cpu().numpy(), ey) <= TOL, "y"
            if not key_mask:
                assert np.all(y.cpu().numpy()[~mask] == 0.0)
        if T:
            assert rel(ty[t].cpu().numpy(), eyd) <= TOL, f"ydot {t}"


def test_gated_equals_unfused_composition_at_c2_shape():
    from hamiltonzero_amd import kernels

    _say("gated vs unfused at [1024, 64, 8, 32], 36/64")
    B, N, H, D = 1024, 64, 8, 32
    g = torch.Generator(device="cuda").manual_seed(1)
    q, k, v = (torch.randn(B, N, H, D, device="cuda", generator=g) * D ** -0.5 for _ in range(3))
    qt, kt, vt = (torch.randn(B, N, H, D, device="cuda", generator=g) for _ in range(3))
    mask = torch.zeros(B, N, dtype=torch.bool, device="cuda")
    mask[:, :36] = True
    y, ty = kernels.mhsea_fwd_jvp_gated(q, k, v, mask, qt, kt, vt, scale=D ** -0.5)
    out, _, tout = kernels.mhsea_fwd_jvp(q, k, v, mask, qt, kt, vt, scale=D ** -0.5)
    s = torch.sigmoid(out[:, :, : H // 2])
    want_y = s * out[:, :, H // 2:]
    want_ty = s * (1 - s) * tout[:, :, : H // 2] * out[:, :, H // 2:] + s * tout[:, :, H // 2:]
    torch.cuda.synchronize()
    assert rel(y.cpu().numpy(), want_y.cpu().numpy()) <= TOL
    assert rel(ty.cpu().numpy(), want_ty.cpu().numpy()) <= TOL


@pytest.mark.parametrize("with_e", [False, True])
def test_gated_edge_attention_autograd(with_e):
    """``gated_edge_attention``: reverse mode (recomputed out, lse; attention backward on the
    collapse's cotangent) against the float64 oracle's VJP of the composite, and forward mode
    (the fused kernel's tangent) against ``gated_fwd_jvp``."""
    import torch.autograd.forward_ad as fwAD

    from hamiltonzero_amd import gated_edge_attention

    _say(f"gated autograd e={with_e}")
    B, N, H, D = 3, 64, 4, 16
    q, k, v, e, mask, tq, tk, tv, te = make(21, B, N, H, D, 1, "scattered", with_e, "qhk")
    rng = np.random.default_rng(22)
    dy = rng.standard_normal((B, N, H // 2, D), dtype=np.float32)
    dev = lambda x, g=False: None if x is None else torch.from_numpy(x).cuda().requires_grad_(g)  # noqa: E731
    scale = D ** -0.5
    qd, kd, ed, vd = dev(q, True), dev(k, True), dev(e, with_e), dev(v, True)
    y = gated_edge_attention(qd, kd, ed, vd, dev(mask), scale=scale)
    y.backward(dev(dy))
    torch.cuda.synchronize()
    out, _ = O.fwd(q, k, e, v, mask, scale=scale)
    s = 1.0 / (1.0 + np.exp(-out[:, :, : H // 2]))
    dout = np.concatenate([dy * out[:, :, H // 2:] * s * (1 - s), dy * s], axis=2)
    want = O.vjp(q, k, e, v, mask, dout, scale=scale)
    assert rel(y.detach().cpu().numpy(), O.gate_collapse(out)) <= TOL
    for name, got, ref in (("dq", qd.grad, want[0]), ("dk", kd.grad, want[1]), ("dv", vd.grad, want[3])):
        assert rel(got.cpu().numpy(), ref) <= TOL, name
    if with_e:
        assert rel(ed.grad.cpu().numpy(), want[2]) <= TOL, "de"
    with fwAD.dual_level():
        duals = [fwAD.make_dual(dev(x), dev(t[0])) for x, t in ((q, tq), (k, tk), (v, tv))]
        ee = fwAD.make_dual(dev(e), dev(te[0])) if with_e else None
        yd = gated_edge_attention(duals[0], duals[1], ee, duals[2], dev(mask), scale=scale)
        _, ty = fwAD.unpack_dual(yd)
        torch.cuda.synchronize()
        _, want_t = O.gated_fwd_jvp(q, k, e, v, mask, tq[0], tk[0], te[0] if with_e else None, tv[0], scale=scale)
        assert rel(ty.cpu().numpy(), want_t) <= TOL


@pytest.mark.parametrize("T,masked,shape", [(0, False, (3, 17, 2, 8, 5)), (1, True, (64, 64, 16, 16, 512)),
                                            (2, True, (5, 33, 3, 8, 70)), (1, True, (7, 37, 4, 16, 132)),
                                            (1, True, (3, 40, 3, 4, 20))])
def test_gated_out_proj(T, masked, shape):
    """W_O after the collapse (trunk.py:138-144), with the tree's site mask
    (tree.py:1479-1488) and the tangents, against the float64 oracle."""
    from hamiltonzero_amd import kernels

    B, N, hh, D, d_e = shape
    _say(f"out proj T={T} masked={masked} {shape}")
    rng = np.random.default_rng(sum(shape) + T)
    y = rng.standard_normal((B, N, hh, D), dtype=np.float32)
    ty = rng.standard_normal((max(T, 1), B, N, hh, D), dtype=np.float32)
    w = (rng.standard_normal((hh * D, d_e)) / np.sqrt(hh * D)).astype(np.float32)
    mask = rng.random((B, N)) < 0.6 if masked else None
    dev = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    delta, dt = kernels.gated_out_proj(dev(y), dev(w), ty=dev(ty[:T]) if T else None, mask=dev(mask))
    torch.cuda.synchronize()
    assert rel(delta.cpu().numpy(), O.out_proj(y, w, mask)) <= TOL
    if masked:
        assert np.all(delta.cpu().numpy()[~mask] == 0.0)
    for t in range(T):
        assert rel(dt[t].cpu().numpy(), O.out_proj(ty[t], w, mask)) <= TOL


def test_out_proj_masked_row_compaction():
    """The masked projection compacts each workgroup's physical rows (256 rows per workgroup):
    workgroups with every row masked, every row physical, one physical row, and a partial
    last workgroup, against the float64 oracle; masked rows are exact zeros."""
    from hamiltonzero_amd import kernels

    _say("out proj row compaction")
    B, N, hh, D, d_e = 13, 64, 16, 16, 512  # M = 832: three full workgroups and one of 64 rows
    rng = np.random.default_rng(7)
    y = rng.standard_normal((B, N, hh, D), dtype=np.float32)
    ty = rng.standard_normal((1, B, N, hh, D), dtype=np.float32)
    w = (rng.standard_normal((hh * D, d_e)) / np.sqrt(hh * D)).astype(np.float32)
    flat = np.zeros(B * N, dtype=bool)
    flat[256:512] = True              # workgroup 1: every row physical
    flat[512 + 77] = True             # workgroup 2: one physical row
    flat[768:] = rng.random(64) < 0.5  # workgroup 3 (partial): scattered
    mask = flat.reshape(B, N)         # workgroup 0: every row masked
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    delta, dt = kernels.gated_out_proj(dev(y), dev(w), ty=dev(ty), mask=dev(mask))
    torch.cuda.synchronize()
    assert rel(delta.cpu().numpy(), O.out_proj(y, w, mask)) <= TOL
    assert rel(dt[0].cpu().numpy(), O.out_proj(ty[0], w, mask)) <= TOL
    assert np.all(delta.cpu().numpy()[~mask] == 0.0) and np.all(dt[0].cpu().numpy()[~mask] == 0.0)


def test_gated_then_out_proj_at_the_trunk_shape():
    """The trunk's attention tail: gated fwd+JVP at [48, 64, 32, 16] with bias, then W_O
    [256, 512] on y and ydot, against the oracle's chain."""
    from hamiltonzero_amd import kernels

    _say("gated -> out proj, trunk shape")
    q, k, v, e, mask, tq, tk, tv, te = make(41, 48, 64, 32, 16, 1, "prefix", True, "qhk")
    rng = np.random.default_rng(42)
    w = (rng.standard_normal((256, 512)) / 16.0).astype(np.float32)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    y, ty = kernels.mhsea_fwd_jvp_gated(dev(q), dev(k), dev(v), dev(mask), dev(tq[:1]), dev(tk[:1]), dev(tv[:1]),
                                        e=dev(e), et=dev(te[:1]), scale=0.25)
    delta, dt = kernels.gated_out_proj(y, dev(w), ty=ty)
    torch.cuda.synchronize()
    wy, wty = O.gated_fwd_jvp(q, k, e, v, mask, tq[0], tk[0], te[0], tv[0], scale=0.25)
    assert rel(delta.cpu().numpy(), O.out_proj(wy, w)) <= TOL
    assert rel(dt[0].cpu().numpy(), O.out_proj(wty, w)) <= TOL



@pytest.mark.parametrize("case", [(21, 9, 64, 8, 32, 2, "scattered", False, True, "qhk"),
                                  (22, 20, 40, 4, 16, 2, "counts", True, True, "qkh"),
                                  (23, 300, 64, 4, 8, 1, "prefix", False, False, "qhk")])
def test_gated_forced_generic_matches_oracle(case):
    """HZ_FLAG_GENERIC routes shapes the producer/consumer kernel serves to the LDS-streaming
    gated kernel; same oracle, same tolerance."""
    from hamiltonzero_amd import kernels

    seed, B, N, H, D, T, mask_kind, key_mask, with_e, e_layout = case
    _say(f"gated generic {case}")
    q, k, v, e, mask, tq, tk, tv, te = make(seed, B, N, H, D, T, mask_kind, with_e, e_layout)
    dev = lambda x: None if x is None else torch.from_numpy(x).cuda()  # noqa: E731
    kw = dict(scale=D ** -0.5, key_mask=key_mask, e_layout=e_layout, generic=True)
    y, ty = kernels.mhsea_fwd_jvp_gated(dev(q), dev(k), dev(v), dev(mask), dev(tq[:T]), dev(tk[:T]), dev(tv[:T]),
                                        e=dev(e), et=None if te is None else dev(te[:T]), **kw)
    torch.cuda.synchronize()
    kw.pop("generic")
    for t in range(T):
        ey, eyd = O.gated_fwd_jvp(q, k, e, v, mask, tq[t], tk[t], None if te is None else te[t], tv[t], **kw)
        if t == 0:
            assert rel(y.cpu().numpy(), ey) <= TOL
            if not key_mask:
                assert np.all(y.cpu().numpy()[~mask] == 0.0)
        assert rel(ty[t].cpu().numpy(), eyd) <= TOL


@pytest.mark.parametrize("case", [(31, 16, 64, 8, 32, "scattered", False, True, "qhk"),
                                  (32, 6, 100, 4, 16, "counts", True, True, "qkh"),
                                  (33, 48, 64, 32, 16, "prefix", False, False, "qhk")])
def test_gated_bwd_matches_oracle(case):
    """hz_mhsea_bwd_gated (the collapse's cotangent on the GPU, then the attention backward)
    against the oracle's gated_vjp, pinned as the adjoint of the pinned forward mode."""
    from hamiltonzero_amd import kernels

    seed, B, N, H, D, mask_kind, key_mask, with_e, e_layout = case
    _say(f"gated bwd {case}")
    q, k, v, e, mask, *_ = make(seed, B, N, H, D, 0, mask_kind, with_e, e_layout)
    dy = np.random.default_rng(seed + 1).standard_normal((B, N, H // 2, D), dtype=np.float32)
    dev = lambda x: None if x is None else torch.from_numpy(x).cuda()  # noqa: E731
    kw = dict(scale=D ** -0.5, key_mask=key_mask, e_layout=e_layout)
    out, lse = kernels.mhsea_fwd(dev(q), dev(k), dev(v), dev(mask), dev(e), **kw)
    dq, dk, de, dv = kernels.mhsea_bwd_gated(dev(q), dev(k), dev(v), dev(mask), lse, out, dev(dy), dev(e),
                                             want_de=with_e, **kw)
    torch.cuda.synchronize()
    want = O.gated_vjp(q, k, e, v, mask, dy, **kw)
    for name, got, ref in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv), want):
        if got is None:
            continue
        assert rel(got.cpu().numpy(), ref) <= TOL, name


@pytest.mark.parametrize("T,N,with_e", [(0, 64, False), (2, 64, True), (1, 130, True), (2, 96, False)])
def test_gated_key_mask_empty_walkers_d64(T, N, with_e):
    """Key-mask mode at D = 64 with walkers that have no physical site (forced, not drawn):
    the fix-up kernel for those walkers is instantiated per head dimension, so it must write
    exactly their rows at D = 64 and leave every other walker's y and ydot as the main kernel
    wrote them. Both checked against the float64 oracle, per walker group."""
    from hamiltonzero_amd import kernels

    B, H, D = 7, 4, 64
    _say(f"gated key-mask empty walkers D=64 T={T} N={N} e={with_e}")
    q, k, v, e, mask, tq, tk, tv, te = make(60 + T + N, B, N, H, D, T, "scattered", with_e, "qhk")
    empty = np.array([1, 4, 6])
    mask[empty] = False
    full = np.setdiff1d(np.arange(B), empty)
    dev = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    kw = dict(scale=D ** -0.5, key_mask=True, e_layout="qhk")
    if T == 0:
        y, ty = kernels.mhsea_fwd_jvp_gated(dev(q), dev(k), dev(v), dev(mask), e=dev(e), **kw)
    else:
        y, ty = kernels.mhsea_fwd_jvp_gated(dev(q), dev(k), dev(v), dev(mask), dev(tq[:T]), dev(tk[:T]), dev(tv[:T]),
                                            e=dev(e), et=None if te is None else dev(te[:T]), **kw)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    for t in range(max(T, 1)):
        ey, eyd = O.gated_fwd_jvp(q, k, e, v, mask, tq[t], tk[t], None if te is None else te[t], tv[t], **kw)
        if t == 0:
            assert rel(y[full], ey[full]) <= TOL, "y of walkers with a physical site"
            assert rel(y[empty], ey[empty]) <= TOL, "y of walkers with no physical site"
        if T:
            got = ty[t].cpu().numpy()
            assert rel(got[full], eyd[full]) <= TOL, f"ydot {t}, walkers with a physical site"
            assert rel(got[empty], eyd[empty]) <= TOL, f"ydot {t}, walkers with no physical site"


def test_gated_bwd_key_mask_empty_walkers_d64():
    """The gated reverse mode at D = 64 in key-mask mode with forced empty walkers, against
    the oracle's gated_vjp (dq, dk, de, dv over the whole batch)."""
    from hamiltonzero_amd import kernels

    B, N, H, D = 5, 64, 4, 64
    _say("gated bwd key-mask empty walkers D=64")
    q, k, v, e, mask, *_ = make(71, B, N, H, D, 0, "scattered", True, "qhk")
    mask[[0, 3]] = False
    dy = np.random.default_rng(72).standard_normal((B, N, H // 2, D), dtype=np.float32)
    dev = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    kw = dict(scale=D ** -0.5, key_mask=True, e_layout="qhk")
    out, lse = kernels.mhsea_fwd(dev(q), dev(k), dev(v), dev(mask), dev(e), **kw)
    dq, dk, de, dv = kernels.mhsea_bwd_gated(dev(q), dev(k), dev(v), dev(mask), lse, out, dev(dy), dev(e),
                                             want_de=True, **kw)
    torch.cuda.synchronize()
    want = O.gated_vjp(q, k, e, v, mask, dy, **kw)
    for name, got, ref in zip(("dq", "dk", "de", "dv"), (dq, dk, de, dv), want):
        assert rel(got.cpu().numpy(), ref) <= TOL, name
