"""hz_factorized_apply_noalloc (workspace in a static device array) against
hz_factorized_apply (caller-owned workspace), through the C ABI: bit-identical results
(both run the same GEMM kernels per row), on two calls in a row, the second smaller, so the
second reuses the array the first left filled.

The first call spans two row chunks (R = 1024: 8192 rows per chunk) with a conditioner
period (7 node rows) that does not divide the chunk, and a residual; the second is the
readout shape (one conditioner row, d_out = 2) with a rank that is not a multiple of 4.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _apply_both(walkers, nodes, d_in, R, d_out, residual, seed):
    from hamiltonzero_amd import _native

    lib = _native.lib()
    rng = np.random.default_rng(seed)
    dev = torch.device("cuda:0")

    def t(shape, scale=1.0):
        return torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(dev)

    M = walkers * nodes
    x = t((M, d_in))
    V = t((d_in, R), d_in ** -0.5)
    h = t((nodes, R))
    U = t((R, d_out), R ** -0.5)
    res = t((M, d_out)) if residual else None
    y_ws = torch.empty((M, d_out), dtype=torch.float32, device=dev)
    y_na = torch.full((M, d_out), float("nan"), dtype=torch.float32, device=dev)
    work = torch.empty((M, R), dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    rp = None if res is None else res.data_ptr()
    _native.check(lib.hz_factorized_apply(s, x.data_ptr(), V.data_ptr(), h.data_ptr(), U.data_ptr(), rp,
                                          y_ws.data_ptr(), work.data_ptr(), M, d_in, R, d_out, nodes))
    _native.check(lib.hz_factorized_apply_noalloc(s, x.data_ptr(), V.data_ptr(), h.data_ptr(), U.data_ptr(), rp,
                                                  y_na.data_ptr(), M, d_in, R, d_out, nodes))
    torch.cuda.synchronize()
    return y_ws.cpu(), y_na.cpu()


def test_noalloc_apply_matches_workspace_apply_twice():
    _say("noalloc call 1: M=12292 (1756 walkers x 7 nodes), d_in=256, R=1024, d_out=96, residual")
    ws1, na1 = _apply_both(1756, 7, 256, 1024, 96, True, seed=1)
    assert torch.isfinite(ws1).all()
    assert torch.equal(ws1, na1)
    _say("noalloc call 2: M=300 (300 walkers x 1 node), d_in=64, R=3001, d_out=2, no residual")
    ws2, na2 = _apply_both(300, 1, 64, 3001, 2, False, seed=2)
    assert torch.isfinite(ws2).all()
    assert torch.equal(ws2, na2)
