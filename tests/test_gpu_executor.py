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
