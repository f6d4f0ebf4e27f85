"""The compacted physical-pair bias layout (HZ_FLAG_E_COMPACT) on the CPU: the torch helper
kernels.compact_bias against a loop restatement of the layout in include/hz_mhsea.h (block
(b, h) of [B, H, N, ceil4(N)] holds walker b's n x n physical pairs, sites ascending, as n
rows of stride ceil4(n)), for both source layouts, odd N and walkers with no or every site
physical; and the shape helper kernels.e_shape."""

import numpy as np
import pytest
import torch

from hamiltonzero_amd import kernels


def compact_np(e_qhk, mask):
    """Loop restatement of the layout: e [B, N(query), H, N(key)] -> [B, H, N, ceil4(N)]."""
    B, N, H, _ = e_qhk.shape
    n4_all = (N + 3) // 4 * 4
    out = np.zeros((B, H, N * n4_all), dtype=e_qhk.dtype)
    for b in range(B):
        s = np.flatnonzero(mask[b])
        n = len(s)
        n4 = (n + 3) // 4 * 4
        for h in range(H):
            for i in range(n):
                out[b, h, i * n4:i * n4 + n] = e_qhk[b, s[i], h, s]
    return out.reshape(B, H, N, n4_all)


@pytest.mark.parametrize("N", [1, 5, 37, 64])
def test_compact_bias_matches_the_loop_restatement(N):
    rng = np.random.default_rng(N)
    B, H = 5, 3
    e = rng.standard_normal((B, N, H, N)).astype(np.float32)
    mask = rng.random((B, N)) < 0.6
    mask[0] = False
    mask[1] = True
    want = compact_np(e, mask)
    got = kernels.compact_bias(torch.from_numpy(e), torch.from_numpy(mask))
    got_qkh = kernels.compact_bias(torch.from_numpy(np.ascontiguousarray(np.swapaxes(e, 2, 3))),
                                   torch.from_numpy(mask), "qkh")
    assert got.shape == kernels.e_shape(B, N, H, "compact")
    assert np.array_equal(got.numpy(), want)
    assert np.array_equal(got_qkh.numpy(), want)


def test_compact_rows_are_the_physical_pairs_in_order():
    """A planted bias e[b, i, h, j] = 1000 i + j + 0.5 h: the compacted rows must read back the
    physical sites' values in ascending order, each row at stride ceil4(n)."""
    B, N, H = 2, 10, 2
    i, h, j = np.meshgrid(np.arange(N), np.arange(H), np.arange(N), indexing="ij")
    e = np.broadcast_to((1000.0 * i + j + 0.5 * h).astype(np.float32), (B, N, H, N)).copy()
    mask = np.zeros((B, N), dtype=bool)
    mask[0, [1, 4, 5, 9, 2]] = True  # n = 5, row stride 8
    mask[1, :] = True  # n = 10, row stride 12
    got = kernels.compact_bias(torch.from_numpy(e), torch.from_numpy(mask)).numpy().reshape(B, H, -1)
    sites = [1, 2, 4, 5, 9]
    for r, si in enumerate(sites):
        for c, sj in enumerate(sites):
            assert got[0, 1, r * 8 + c] == 1000.0 * si + sj + 0.5
    assert got[1, 0, 3 * 12 + 7] == 1000.0 * 3 + 7
    assert got[0, 0, 5 * 8:].max() == 0.0  # past the n rows: never read, left zero


def test_e_shape():
    assert kernels.e_shape(2, 37, 4, "qhk") == (2, 37, 4, 37)
    assert kernels.e_shape(2, 37, 4, "qkh") == (2, 37, 37, 4)
    assert kernels.e_shape(2, 37, 4, "compact") == (2, 4, 37, 40)
    with pytest.raises(ValueError, match="e_layout"):
        kernels.e_shape(2, 37, 4, "khq")
