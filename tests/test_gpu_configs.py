"""GPU parity of the benchmark configurations c3, c4 and c5 at their full BASELINE workloads.

Each case runs the configuration's whole batch through the C ABI exactly as ``bench.py``
launches it — c3: ``hz_mhsea_fwd`` then ``hz_mhsea_bwd`` over [4096, 64, 8, 64] bfloat16;
c4: ``hz_mhsea_fwd_jvp`` as 32 launches of 16 walkers at the bench's base offsets over
[512, 256, 8, 64] float32; c5: one ``hz_mhsea_fwd_jvp`` with T = 2 over [128, 1024, 16, 64]
bfloat16 — and compares walkers sampled from the first, middle and last workgroups (and, for
c4, launches) with the float64 oracle. The oracle is per walker and per head, so evaluating
it on a sample of walkers (c5: and of heads) equals evaluating it on the batch and selecting.
Masked rows, which the reference defines as exact zeros (``mhsea_tuned.py:91``,
``mhsea_tuned_jvp.py:88-91``, ``custom_gradients.py:254-276,313-335``), are checked on the
whole batch, on the device.

Inputs: the configurations' shapes, masks (physical sites first, the same count for every
walker) and scalings (q, k, v ~ N(0, 1)/sqrt(D); tangents and cotangent N(0, 1)), drawn on the
device from a seeded torch generator (the batch is 0.5-4.5 GB, which a host draw would spend
most of the test's time on); bfloat16 configurations round the float32 draws on the device and
the oracle runs on the rounded values. Tolerances: max-norm relative error <= 1e-5 for float32,
<= 2e-2 for bfloat16 storage; the cotangents of dq, dk use the cancellation floor of
``vjp_floors``.
"""

import numpy as np
import pytest
import torch

from oracle import mhsea_oracle as O
from test_gpu_parity import BF16_TOL, F32_TOL, rel, vjp_floors

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _draw(gen, shape, scale, dtype):
    x = torch.randn(shape, device="cuda", generator=gen, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(dtype).contiguous()


def _prefix_mask(B, N, n_phys):
    m = torch.zeros((B, N), dtype=torch.uint8, device="cuda")
    m[:, :n_phys] = 1
    return m


def _host(t, idx, axis=0):
    idx_t = torch.as_tensor(idx, device=t.device)
    return t.index_select(axis, idx_t).float().cpu().numpy()


def _walkers(B, picks):
    return np.array(sorted({b for b in picks if 0 <= b < B}))


def _lib():
    from hamiltonzero_amd import _native

    return _native, _native.lib()


def test_c3_full_fwd_bwd_bf16():
    """c3: [4096, 64, 8, 64] bfloat16, 48/64 sites, forward then backward (no de), as the
    bench runs it. The backward's persistent grid walks 64 items per workgroup here."""
    _native, lib = _lib()
    B, N, H, D, n_phys = 4096, 64, 8, 64, 48
    _say(f"c3 full B={B} N={N} H={H} D={D} n_phys={n_phys}")
    gen = torch.Generator(device="cuda").manual_seed(2)
    shape = (B, N, H, D)
    q, k, v = (_draw(gen, shape, D ** -0.5, torch.bfloat16) for _ in range(3))
    dout = _draw(gen, shape, 1.0, torch.bfloat16)
    mask = _prefix_mask(B, N, n_phys)
    out = torch.empty_like(q)
    lse = torch.empty((B, N, H), dtype=torch.float32, device="cuda")
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    s = torch.cuda.current_stream().cuda_stream
    bf = _native.HZ_DTYPE_BF16
    _native.check(lib.hz_mhsea_fwd(s, q.data_ptr(), k.data_ptr(), None, v.data_ptr(), mask.data_ptr(),
                                   out.data_ptr(), lse.data_ptr(), B, N, H, D, bf, 1.0, 0))
    _native.check(lib.hz_mhsea_bwd(s, q.data_ptr(), k.data_ptr(), None, v.data_ptr(), mask.data_ptr(),
                                   lse.data_ptr(), out.data_ptr(), dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), None,
                                   dv.data_ptr(), B, N, H, D, bf, 1.0, 0))
    torch.cuda.synchronize()
    for name, t in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert int(torch.count_nonzero(t[:, n_phys:])) == 0, f"{name}: masked rows not zero"
        assert bool(torch.isfinite(t).all()), f"{name}: non-finite values"
    idx = _walkers(B, [0, 1, 2, 63, 64, 255, 511, 1023, 1024, 2047, 2048, 2049, 3071, 4093, 4094, 4095]
                   + [int(x) for x in np.linspace(0, B - 1, 16)])
    a = {nm: _host(t, idx) for nm, t in (("q", q), ("k", k), ("v", v), ("dout", dout))}
    a["e"] = None
    a["mask"] = _host(mask, idx).astype(bool)
    ref_out, ref_lse = O.fwd(a["q"], a["k"], None, a["v"], a["mask"])
    assert rel(_host(out, idx), ref_out) <= BF16_TOL, "out"
    m = a["mask"]
    assert rel(_host(lse, idx)[m], ref_lse[m]) <= BF16_TOL, "lse"
    ref = dict(zip(("dq", "dk", "de", "dv"), O.vjp(a["q"], a["k"], None, a["v"], m, a["dout"])))
    floors = vjp_floors(a, dict(scale=1.0))
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert rel(_host(t, idx), ref[name], floors[name]) <= BF16_TOL, name


def test_c4_full_fwd_jvp_in_chunks_of_16():
    """c4: [512, 256, 8, 64] float32, 225/256 sites, T = 1, as 32 launches of 16 walkers at
    base offsets 0, 16, ..., 496 (pointer offsets into the whole-batch buffers, tangents with
    their one direction), exactly the bench's launch pattern."""
    _native, lib = _lib()
    B, N, H, D, n_phys, chunk = 512, 256, 8, 64, 225, 16
    _say(f"c4 full B={B} N={N} H={H} D={D} n_phys={n_phys} chunks of {chunk}")
    gen = torch.Generator(device="cuda").manual_seed(3)
    shape = (B, N, H, D)
    q, k, v = (_draw(gen, shape, D ** -0.5, torch.float32) for _ in range(3))
    qt, kt, vt = (_draw(gen, (1, *shape), 1.0, torch.float32) for _ in range(3))
    mask = _prefix_mask(B, N, n_phys)
    out = torch.empty_like(q)
    tout = torch.empty_like(qt)
    s = torch.cuda.current_stream().cuda_stream
    row = N * H * D * 4
    for b0 in range(0, B, chunk):
        off = b0 * row
        _native.check(lib.hz_mhsea_fwd_jvp(
            s, q.data_ptr() + off, k.data_ptr() + off, None, v.data_ptr() + off, mask.data_ptr() + b0 * N,
            qt.data_ptr() + off, kt.data_ptr() + off, None, vt.data_ptr() + off, 1, out.data_ptr() + off, None,
            tout.data_ptr() + off, chunk, N, H, D, _native.HZ_DTYPE_F32, 1.0, 0))
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(out[:, n_phys:])) == 0
    assert int(torch.count_nonzero(tout[:, :, n_phys:])) == 0
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(tout).all())
    # first, second, middle and last walker of launches 0, 1, 15, 16, 30, 31, plus a spread
    picks = [c * chunk + w for c in (0, 1, 15, 16, 30, 31) for w in (0, 1, 7, 15)]
    idx = _walkers(B, picks + [int(x) for x in np.linspace(0, B - 1, 8)])
    a = {nm: _host(t, idx) for nm, t in (("q", q), ("k", k), ("v", v))}
    tan = {nm: _host(t[0], idx) for nm, t in (("qt", qt), ("kt", kt), ("vt", vt))}
    m = _host(mask, idx).astype(bool)
    ref_out, _ = O.fwd(a["q"], a["k"], None, a["v"], m)
    assert rel(_host(out, idx), ref_out) <= F32_TOL, "out"
    ref_t = O.jvp(a["q"], a["k"], None, a["v"], m, tan["qt"], tan["kt"], None, tan["vt"])
    assert rel(_host(tout[0], idx), ref_t) <= F32_TOL, "tout"


def test_c5_full_fwd_two_jvp_bf16():
    """c5: [128, 1024, 16, 64] bfloat16, 1000/1024 sites, two tangent directions, one launch.
    Walkers from the first, middle and last query-block workgroups, each against the oracle
    on four of its 16 heads (first, two middle, last), both directions."""
    _native, lib = _lib()
    B, N, H, D, n_phys, T = 128, 1024, 16, 64, 1000, 2
    _say(f"c5 full B={B} N={N} H={H} D={D} n_phys={n_phys} T={T}")
    gen = torch.Generator(device="cuda").manual_seed(4)
    shape = (B, N, H, D)
    q, k, v = (_draw(gen, shape, D ** -0.5, torch.bfloat16) for _ in range(3))
    qt, kt, vt = (_draw(gen, (T, *shape), 1.0, torch.bfloat16) for _ in range(3))
    mask = _prefix_mask(B, N, n_phys)
    out = torch.empty_like(q)
    tout = torch.empty_like(qt)
    s = torch.cuda.current_stream().cuda_stream
    _native.check(lib.hz_mhsea_fwd_jvp(s, q.data_ptr(), k.data_ptr(), None, v.data_ptr(), mask.data_ptr(),
                                       qt.data_ptr(), kt.data_ptr(), None, vt.data_ptr(), T, out.data_ptr(), None,
                                       tout.data_ptr(), B, N, H, D, _native.HZ_DTYPE_BF16, 1.0, 0))
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(out[:, n_phys:])) == 0
    assert int(torch.count_nonzero(tout[:, :, n_phys:])) == 0
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(tout).all())
    idx = np.array([0, 64, 127])
    heads = np.array([0, 5, 10, 15])

    def sub(t):  # walkers idx, heads `heads`
        return _host(t, idx)[:, :, heads]

    a = {nm: sub(t) for nm, t in (("q", q), ("k", k), ("v", v))}
    m = _host(mask, idx).astype(bool)
    ref_out, _ = O.fwd(a["q"], a["k"], None, a["v"], m)
    assert rel(sub(out), ref_out) <= BF16_TOL, "out"
    for t in range(T):
        tan = {nm: sub(x[t]) for nm, x in (("qt", qt), ("kt", kt), ("vt", vt))}
        ref_t = O.jvp(a["q"], a["k"], None, a["v"], m, tan["qt"], tan["kt"], None, tan["vt"])
        assert rel(sub(tout[t]), ref_t) <= BF16_TOL, f"tout {t}"
