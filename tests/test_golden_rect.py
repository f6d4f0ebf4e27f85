"""Golden fixtures of the rectangular large-N forward (``tests/golden/rect_*.npz``, written by
``tests/golden/make_golden_rect.py``): seeded inputs with the float64 oracle's output.

CPU: the oracle still reproduces every fixture. GPU: ``hz_rect_attention_fwd`` (through the
torch wrapper) matches the stored output without running the oracle, max-norm relative
error <= 1e-5 (float32).
"""

import glob
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = sorted(glob.glob(os.path.join(HERE, "golden", "rect_*.npz")))
IDS = [os.path.basename(f)[:-4] for f in FILES]
F32_TOL = 1e-5


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def load(path):
    z = np.load(path, allow_pickle=False)
    a = {n: (z[f"in_{n}"] if f"in_{n}" in z else None) for n in ("q", "k", "v", "bias", "key_mask")}
    return a, z["want_out"], float(z["meta"][0])


def test_rect_fixtures_present():
    assert len(FILES) >= 3


@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_oracle_reproduces_rect_fixture(path):
    from oracle import rect_oracle as R

    a, want, scale = load(path)
    got = R.rect_fwd(a["q"], a["k"], a["v"], a["bias"], a["key_mask"], scale=scale)
    assert rel(got, want) <= 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=IDS)
def test_hip_rect_matches_fixture(path):
    import torch

    from hamiltonzero_amd import kernels

    a, want, scale = load(path)
    print(f"[case] golden {os.path.basename(path)}", flush=True)
    d = {n: None if x is None else torch.from_numpy(x).cuda() for n, x in a.items()}
    out = kernels.rect_attention_fwd(d["q"], d["k"], d["v"], d["bias"], d["key_mask"], scale=scale)
    torch.cuda.synchronize()
    assert rel(out.cpu().numpy(), want) <= F32_TOL
