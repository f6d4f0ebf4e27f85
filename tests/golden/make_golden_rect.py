"""Write the golden fixtures of the rectangular large-N forward: small seeded inputs and the
float64 oracle's output, one ``rect_*.npz`` per case.

The reference has no golden vectors for this path (``src/hamiltonzero/evaluation/
pallas_mha.py``, ``sequence_parallel.py``) and its Pallas code cannot run here, so the expected
outputs come from ``oracle/rect_oracle.py`` (pinned by ``tests/test_rect_oracle.py``).
``tests/test_golden_rect.py`` checks that the oracle still reproduces them (CPU) and that the
HIP path matches them (GPU) without running the oracle.

Run from the repository root:  python tests/golden/make_golden_rect.py
"""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import rect_oracle as R  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

# name, seed, B, Nq, Nk, H, D, n_phys (None: no mask; -1: per-system counts), scattered, bias, scale
CASES = [
    ("rect_q24_k40_h4_d16_mask", 21, 2, 24, 40, 4, 16, 29, True, True, 0.25),    # four heads per workgroup
    ("rect_q70_k33_h2_d32_nomask", 22, 1, 70, 33, 2, 32, None, False, True, 1.0),  # noncausal_bias_mha
    ("rect_q9_k20_h3_d8_counts", 23, 3, 9, 20, 3, 8, -1, True, True, 0.35),      # odd H, varied masks
]


def make_case(seed, B, Nq, Nk, H, D, n_phys, scattered, bias):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Nq, H, D), dtype=np.float32)
    k = rng.standard_normal((B, Nk, H, D), dtype=np.float32)
    v = rng.standard_normal((B, Nk, H, D), dtype=np.float32)
    e = rng.standard_normal((B, Nq, Nk, H), dtype=np.float32) if bias else None
    mask = None
    if n_phys is not None:
        mask = np.zeros((B, Nk), dtype=bool)
        for b in range(B):
            n = int(rng.integers(0, Nk + 1)) if n_phys < 0 else n_phys
            sites = rng.permutation(Nk)[:n] if scattered else np.arange(n)
            mask[b, sites] = True
    return dict(q=q, k=k, v=v, bias=e, key_mask=mask)


def main():
    for name, seed, B, Nq, Nk, H, D, n_phys, scattered, bias, scale in CASES:
        a = make_case(seed, B, Nq, Nk, H, D, n_phys, scattered, bias)
        want = R.rect_fwd(a["q"], a["k"], a["v"], a["bias"], a["key_mask"], scale=scale)
        arrays = {f"in_{n}": x for n, x in a.items() if x is not None}
        arrays["want_out"] = want.astype(np.float32)
        arrays["meta"] = np.array([scale])
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
