"""Write the golden fixtures of the MHSEA path: small seeded inputs and the float64 oracle's
outputs (forward, T tangents, VJP), one ``.npz`` per case.

The reference has no golden vectors or known-answer tests for this path, and its code
(JAX 0.11 / Pallas) cannot run here, so the expected outputs come from the oracle in
``oracle/mhsea_oracle.py`` (a restatement of the reference math, pinned by the closed forms,
finite differences and autodiff checks of ``tests/test_oracle.py``). The fixtures freeze
those outputs: ``tests/test_golden.py`` checks the oracle still reproduces them (CPU) and
the HIP path matches them (GPU) without running the oracle.

Run from the repository root:  python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import mhsea_oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

# name, seed, B, N, H, D, n_phys (-1: per-walker counts), scattered, with_e, e_layout,
# key_mask, scale, T, bf16 (inputs rounded to bfloat16) — one case per kernel family
CASES = [
    ("n8_d32_keymask_bias", 11, 2, 8, 2, 32, 5, True, True, "qkh", True, 0.5, 2, False),     # small
    ("n40_d16_square_bias", 12, 2, 40, 1, 16, 23, True, True, "qhk", False, 1.0, 1, False),  # pc
    ("n64_d32_first_sites", 13, 1, 64, 1, 32, 36, False, False, "qhk", False, 1.0, 1, False),  # pc (c2 head)
    ("n48_d16_mixed_counts", 14, 3, 48, 1, 16, -1, True, False, "qhk", False, 1.0, 1, False),  # pc, varied masks
    ("n80_d16_generic", 15, 1, 80, 1, 16, 70, True, True, "qhk", False, 0.7, 1, False),       # N > 64
    ("n130_d32_bf16", 16, 1, 130, 1, 32, 121, False, False, "qhk", False, 1.0, 1, True),      # bf16, N > 128
]


def bf16_round(x):
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def make_case(seed, B, N, H, D, n_phys, scattered, with_e, e_layout, T, bf16):
    rng = np.random.default_rng(seed)
    shape = (B, N, H, D)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(D ** -0.5) for _ in range(3))
    eshape = (B, N, H, N) if e_layout == "qhk" else (B, N, N, H)
    e = rng.standard_normal(eshape, dtype=np.float32) * np.float32(0.5) if with_e else None
    qt, kt, vt = (rng.standard_normal((T, *shape), dtype=np.float32) for _ in range(3))
    et = rng.standard_normal((T, *eshape), dtype=np.float32) if with_e else None
    dout = rng.standard_normal(shape, dtype=np.float32)
    mask = np.zeros((B, N), dtype=bool)
    for b in range(B):
        n_b = int(rng.integers(0, N + 1)) if n_phys < 0 else n_phys
        sites = rng.permutation(N)[:n_b] if scattered else np.arange(n_b)
        mask[b, sites] = True
    a = dict(q=q, k=k, v=v, e=e, qt=qt, kt=kt, vt=vt, et=et, dout=dout)
    if bf16:
        a = {n: None if x is None else bf16_round(x) for n, x in a.items()}
    a["mask"] = mask
    return a


def vjp_floors(a, opts):
    """Magnitudes of dq, dk, de without cancellation (see tests/test_gpu_parity.py)."""
    p = O.probs(a["q"], a["k"], a["e"], a["mask"], **opts)
    out, _ = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"], **opts)
    dout = np.abs(a["dout"].astype(np.float64))
    dp = np.einsum("bihd,bjhd->bhij", dout, np.abs(a["v"].astype(np.float64)))
    delta = np.abs(out * a["dout"]).sum(-1).transpose(0, 2, 1)[..., None]
    ds = p * (dp + delta)
    s = abs(opts["scale"])
    dq = s * np.einsum("bhij,bjhd->bihd", ds, np.abs(a["k"].astype(np.float64)))
    dk = s * np.einsum("bhij,bihd->bjhd", ds, np.abs(a["q"].astype(np.float64)))
    return np.array([0.01 * dq.max(), 0.01 * dk.max(), 0.01 * ds.max(), 0.0])


def expected(a, opts, T):
    out, lse = O.fwd(a["q"], a["k"], a["e"], a["v"], a["mask"], **opts)
    tout = np.stack([O.jvp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["qt"][t], a["kt"][t],
                           None if a["et"] is None else a["et"][t], a["vt"][t], **opts) for t in range(T)])
    dq, dk, de, dv = O.vjp(a["q"], a["k"], a["e"], a["v"], a["mask"], a["dout"], **opts)
    return dict(out=out, lse=lse, tout=tout, dq=dq, dk=dk, de=de, dv=dv)


def main():
    for name, seed, B, N, H, D, n_phys, scattered, with_e, e_layout, key_mask, scale, T, bf16 in CASES:
        a = make_case(seed, B, N, H, D, n_phys, scattered, with_e, e_layout, T, bf16)
        opts = dict(scale=scale, key_mask=key_mask, e_layout=e_layout)
        want = expected(a, opts, T)
        # bf16-rounded inputs are stored as their bfloat16 bit patterns (uint16)
        arrays = {f"in_{n}": ((x.view(np.uint32) >> 16).astype(np.uint16) if bf16 and x.dtype == np.float32 else x)
                  for n, x in a.items() if x is not None}
        arrays.update({f"want_{n}": x.astype(np.float32) for n, x in want.items()})
        arrays["vjp_floors"] = vjp_floors(a, opts)
        arrays["meta"] = np.array([scale, float(key_mask), float(e_layout == "qkh"), float(T), float(bf16)])
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
