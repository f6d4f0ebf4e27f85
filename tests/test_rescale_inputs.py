"""The rising-logit inputs of the GPU base-move test do move a chunked online softmax's base,
and a wrong move shows at that test's tolerances (CPU).

The chunked online softmax here (tests/rising_inputs.py) is the kernels' lazy scheme: 32-key
chunks, base 2, a move when a chunk's maximum exceeds the base by more than 8. Run correctly
on the rising inputs it equals the float64 oracle; with a mistake planted in its moves (the
value sums not rescaled, the factor inverted, the tangent row sum not rescaled) the result is
off by far more than the GPU test allows.
"""

import numpy as np
import pytest

from oracle import mhsea_oracle as O
from rising_inputs import RISE, online_softmax, rising


def _rel(a, b):
    return float(np.max(np.abs(np.asarray(a) - np.asarray(b))) / max(np.max(np.abs(b)), 1e-30))


@pytest.fixture(scope="module")
def case():
    B, N, H, D = 1, 256, 1, 64
    q, k, v, u, rng = rising(5, B, N, N, H, D)
    qt, kt, vt = (rng.standard_normal((B, N, H, D), dtype=np.float32) for _ in range(3))
    qt -= (qt @ u.astype(np.float32))[..., None] * u.astype(np.float32)
    mask = np.ones((B, N), dtype=bool)
    out, _ = O.fwd(q, k, None, v, mask)
    tout = O.jvp(q, k, None, v, mask, qt, kt, None, vt)
    f = lambda x: x.astype(np.float64)[0, :, 0]
    s = f(q) @ f(k).T  # [queries, keys]
    ds = f(qt) @ f(k).T + f(q) @ f(kt).T
    return dict(s=s, ds=ds, v=f(v), vt=f(vt), out=out[0, :, 0], tout=tout[0, :, 0])


def _run(c, rows, plant=None):
    res = [online_softmax(c["s"][i], c["ds"][i], c["v"], c["vt"], plant=plant) for i in rows]
    return np.array([r[0] for r in res]), np.array([r[1] for r in res]), [r[2] for r in res]


ROWS = list(range(0, 256, 17))


def test_rising_logits_span(case):
    rise = case["s"][:, -1] - case["s"][:, 0]
    assert np.median(rise) > 0.75 * RISE


def test_chunked_online_softmax_matches_oracle_and_moves_the_base(case):
    out, tout, moves = _run(case, ROWS)
    assert min(moves) >= 3  # every row moves its base at least three times after the first chunk
    assert _rel(out, case["out"][ROWS]) <= 1e-12
    assert _rel(tout, case["tout"][ROWS]) <= 1e-12


@pytest.mark.parametrize("plant", ["no_acc", "inverse", "no_mu"])
def test_wrong_base_move_is_visible(case, plant):
    out, tout, _ = _run(case, ROWS, plant)
    err = max(_rel(out, case["out"][ROWS]), _rel(tout, case["tout"][ROWS]))
    assert err > 1e-2  # at least the GPU test's bfloat16 tolerance; float32's is 5e-5
