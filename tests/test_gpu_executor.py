"""GPU parity of the compiled executor's products (hz_quadrilinear_merge, hz_factorized_apply)
against the float64 oracle (oracle/executor_oracle.py), through the C ABI.

Tolerance: max-norm relative error <= 1e-5 (float32 inputs, float32 matrix-core products
and accumulation). Shapes cover the fine-tune model's (merge_dim 1536 = 48 groups of rank
32, merge_rank 1024, config.py:21-29,189-190) at reduced walker counts, row counts that are
not multiples of the tiles, one conditioner row per node and the readout's two outputs.
"""

import types

import numpy as np
import pytest
import torch

from oracle import executor_oracle as X

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


@pytest.mark.parametrize("M,G", [(5, 2), (256, 48), (1000, 3), (2 * 32, 48)])
def test_quadrilinear_merge(M, G):
    from hamiltonzero_amd import executor

    _say(f"merge M={M} G={G}")
    rng = np.random.default_rng(M + G)
    R = 32
    T = (rng.standard_normal((G, R, R, R)) / R).astype(np.float32)
    a = rng.standard_normal((M, G * R)).astype(np.float32)
    b = rng.standard_normal((M, G * R)).astype(np.float32)
    got = executor.quadrilinear_merge(dev(T), dev(a), dev(b))
    torch.cuda.synchronize()
    assert rel(got.cpu().numpy(), X.quadrilinear_merge(T, a, b)) <= TOL


def test_quadrilinear_merge_leading_axes():
    from hamiltonzero_amd import executor

    _say("merge [walkers, nodes, G R]")
    rng = np.random.default_rng(11)
    G, R = 4, 32
    T = (rng.standard_normal((G, R, R, R)) / R).astype(np.float32)
    a = rng.standard_normal((3, 16, G * R)).astype(np.float32)
    b = rng.standard_normal((3, 16, G * R)).astype(np.float32)
    got = executor._compiled_quadrilinear_merge(dev(T), dev(a), dev(b))
    torch.cuda.synchronize()
    assert got.shape == (3, 16, G * R)
    assert rel(got.cpu().numpy(), X.quadrilinear_merge(T, a, b)) <= TOL


@pytest.mark.parametrize(
    "walkers,nodes,d_in,R,d_out,residual",
    [
        (2, 32, 96, 64, 48, False),         # small, tile remainders everywhere
        (8, 32, 1536, 1024, 1536, True),    # a merge level at the fine-tune ranks
        (3, 7, 130, 66, 18, False),         # sizes that are not multiples of 4
        (37, 1, 1536, 1024, 2, False),      # the readout: one conditioner row, psi = (re, im)
        (4, 64, 64, 1536, 1536, False),     # the leaf apply shape (rank 1536)
    ],
)
def test_factorized_apply(walkers, nodes, d_in, R, d_out, residual):
    from hamiltonzero_amd import executor

    _say(f"apply walkers={walkers} nodes={nodes} d_in={d_in} R={R} d_out={d_out} residual={residual}")
    rng = np.random.default_rng(walkers * 7 + nodes)
    x = rng.standard_normal((walkers, nodes, d_in)).astype(np.float32)
    V = (rng.standard_normal((d_in, R)) / np.sqrt(d_in)).astype(np.float32)
    U = (rng.standard_normal((R, d_out)) / np.sqrt(R)).astype(np.float32)
    h = rng.standard_normal((nodes, R)).astype(np.float32)
    res = rng.standard_normal((walkers, nodes, d_out)).astype(np.float32) if residual else None
    factor = types.SimpleNamespace(V=dev(V), U=dev(U))
    got = executor._factorized_apply(factor, dev(h), dev(x), None if res is None else dev(res))
    torch.cuda.synchronize()
    want = X.factorized_apply(V, U, h, x) + (0.0 if res is None else res)
    assert rel(got.cpu().numpy(), want) <= TOL


def test_merge_level_products_compose():
    """One tree level's products as the executor chains them: merge, then the residual apply
    (execute.py:103-104), checked against the oracle's level up to the RMS rescale."""
    from hamiltonzero_amd import executor

    _say("merge level")
    rng = np.random.default_rng(21)
    G, R, Rm, W, B = 48, 32, 1024, 16, 4
    T = (rng.standard_normal((G, R, R, R)) / R).astype(np.float32)
    V = (rng.standard_normal((G * R, Rm)) / np.sqrt(G * R)).astype(np.float32)
    U = (rng.standard_normal((Rm, G * R)) / np.sqrt(Rm)).astype(np.float32)
    h = rng.standard_normal((W, Rm)).astype(np.float32)
    u = rng.standard_normal((B, 2 * W, G * R)).astype(np.float32)
    ul, ur = u[:, 0::2], u[:, 1::2]
    raw = executor.quadrilinear_merge(dev(T), dev(ul), dev(ur))
    out = executor.factorized_apply(types.SimpleNamespace(V=dev(V), U=dev(U)), dev(h), raw, raw)
    torch.cuda.synchronize()
    raw_ref = X.quadrilinear_merge(T, ul, ur)
    want = raw_ref + X.factorized_apply(V, U, h, raw_ref)
    assert rel(out.cpu().numpy(), want) <= TOL


def _wavefn_case(seed, B, n, d_q, d_z, R_leaf, G, R_merge, R_out, real):
    rng = np.random.default_rng(seed)
    R, dm = 32, G * 32
    f32 = lambda x: np.asarray(x, dtype=np.float32)  # noqa: E731
    w = lambda i, o: f32(rng.standard_normal((i, o)) / np.sqrt(i))  # noqa: E731
    if real == "all":
        leaf_real = np.ones(n, bool)
    else:
        leaf_real = rng.random(n) < (0.8 if real == "random" else 0.3)
        leaf_real[rng.integers(n)] = True
    p = dict(q=f32(rng.standard_normal((B, n, d_q))), q_weight=w(d_q, d_z), leaf_V=w(d_z, R_leaf),
             leaf_U=w(R_leaf, dm), leaf_h=f32(rng.standard_normal((n, R_leaf))),
             merge_T=f32(rng.standard_normal((G, R, R, R)) / R), merge_V=w(dm, R_merge), merge_U=w(R_merge, dm),
             readout_V=w(dm, R_out), readout_U=w(R_out, 2), readout_h=f32(rng.standard_normal(R_out)),
             merge_eps=1e-6)
    p["merge_h"] = [f32(rng.standard_normal((n >> (l + 1), R_merge))) for l in range(int(np.log2(n)))]
    p["opcodes"] = X.classify_opcodes(leaf_real) if n > 1 else []
    return p


def _readout_condition(p):
    """kappa_b = sum_r |m_r| (|U_r0| + |U_r1|) / |psi_b| from the oracle's root carriers."""
    z = np.asarray(p["q"], np.float64) @ p["q_weight"]
    u, s = X.normalize_leaf_carriers(X.factorized_apply(p["leaf_V"], p["leaf_U"], p["leaf_h"], z))
    for h, o in zip(p["merge_h"], p["opcodes"]):
        u, s = X.merge_level(p["merge_T"], p["merge_V"], p["merge_U"], h, p["merge_eps"], u, s, o)
    m = (u[:, 0] @ np.asarray(p["readout_V"], np.float64)) * p["readout_h"]
    U = np.asarray(p["readout_U"], np.float64)
    psi = m @ U
    return (np.abs(m) @ np.abs(U)).sum(axis=1) / np.hypot(psi[:, 0], psi[:, 1])


def _namespaces(p):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    fac = lambda V, U: types.SimpleNamespace(V=t(V), U=t(U))  # noqa: E731
    kernel = types.SimpleNamespace(q_to_odd=types.SimpleNamespace(weight=t(p["q_weight"])),
                                   leaf_factors=(fac(p["leaf_V"], p["leaf_U"]),), merge_T=t(p["merge_T"]),
                                   merge_factors=(fac(p["merge_V"], p["merge_U"]),),
                                   readout_factors=(fac(p["readout_V"], p["readout_U"]),), merge_eps=p["merge_eps"])
    tree = types.SimpleNamespace(leaf_h=(t(p["leaf_h"]),), readout_h=(t(p["readout_h"]),), leaf_combiner_h=(),
                                 readout_combiner_h=(), merge_h=tuple(t(h) for h in p["merge_h"]),
                                 opcodes=tuple(t(o) for o in p["opcodes"]))
    return kernel, tree, t(p["q"])


@pytest.mark.parametrize(
    "B,n,d_q,d_z,R_leaf,G,R_merge,R_out,real",
    [
        (16, 64, 4, 32, 1536, 48, 1024, 64, "random"),  # the fine-tune sizes (config.py:21-29,189-190)
        (5, 8, 4, 40, 24, 4, 96, 8, "all"),
        (7, 16, 3, 30, 66, 2, 50, 6, "sparse"),          # sizes off the 4-float staging path
        (3, 1, 4, 32, 64, 3, 32, 16, "all"),             # one site: no merge level
        (300, 4, 4, 32, 128, 8, 64, 64, "random"),       # many walkers, shallow tree
    ],
)
def test_compiled_wavefunction_matches_oracle(B, n, d_q, d_z, R_leaf, G, R_merge, R_out, real):
    from hamiltonzero_amd import executor

    _say(f"wavefunction B={B} n={n} G={G} R_leaf={R_leaf} R_merge={R_merge} R_out={R_out} {real}")
    p = _wavefn_case(B * 3 + n, B, n, d_q, d_z, R_leaf, G, R_merge, R_out, real)
    kernel, tree, q = _namespaces(p)
    la, ph = executor.execute_wavefunction(kernel, tree, q)
    torch.cuda.synchronize()
    want_la, want_ph = X.execute_wavefunction(**p)
    # log|psi| and the phase carry psi's relative error. Where the readout's sum cancels,
    # kappa = sum_r |m_r| (|U_r0| + |U_r1|) / |psi| (m the conditioned readout row), that is
    # kappa times the float32 error of its terms (about 2e-7 kappa measured), so each walker
    # is allowed 1e-6 kappa on top of the max-norm bound.
    kappa = _readout_condition(p)
    dla = np.abs(la.cpu().numpy().astype(np.float64) - want_la)
    assert np.all(dla <= TOL * np.max(np.abs(want_la)) + 1e-6 * kappa), (dla.max(), kappa[np.argmax(dla)])
    dphi = np.abs(np.angle(np.exp(1j * (ph.cpu().numpy().astype(np.float64) - want_ph))))
    assert np.all(dphi <= TOL * np.pi + 1e-6 * kappa), (dphi.max(), kappa[np.argmax(dphi)])
    assert np.median(kappa) < 10  # most walkers are well conditioned: the bound is mostly the max-norm one


def test_compiled_wavefunction_structure_errors():
    from hamiltonzero_amd import executor

    _say("wavefunction structure errors")
    p = _wavefn_case(1, 2, 8, 4, 32, 64, 2, 32, 8, "all")
    kernel, tree, q = _namespaces(p)
    with pytest.raises(ValueError, match="one entry per tree level"):
        executor.execute_wavefunction(kernel, types.SimpleNamespace(**dict(vars(tree), opcodes=tree.opcodes[:-1])), q)
    with pytest.raises(ValueError, match="incompatible shrinking shape"):
        executor.execute_wavefunction(kernel, tree, q[:, :4])
    with pytest.raises(ValueError, match="does not accept combiners"):
        executor.execute_wavefunction(kernel, types.SimpleNamespace(**dict(vars(tree), leaf_combiner_h=(1,))), q)
