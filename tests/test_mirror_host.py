"""Host-side behaviour of the reference-named Python mirror that needs no GPU: the shape
dispatch and argument checks of ``mhsea_with_tuned_ad`` and friends
(``src/hamiltonzero/model/_pallas_attn/mhsea_tuned.py:29-69,206-211,243-255``) and the
op-level selection between the tuned primitive and the jnp fallback
(``src/hamiltonzero/model/pallas_attention.py:16-19,40-67``). Every check runs before any
device work, so CPU tensors reach them."""

import pytest
import torch

from hamiltonzero_amd import edge_attention as EA
from hamiltonzero_amd import mhsea_tuned as MT


def prim(B=2, N=64, H=2, D=32, dtype=torch.float32, e=True):
    q, k, v = (torch.zeros(B, N, H, D, dtype=dtype) for _ in range(3))
    ee = torch.zeros(B, N, H, N, dtype=dtype) if e else None
    return q, k, ee, v, torch.ones(B, N, dtype=torch.bool)


@pytest.mark.parametrize("N,D,tuned,full", [(64, 32, True, False), (96, 16, True, False), (80, 32, False, False),
                                            (32, 32, False, True), (8, 8, False, True), (48, 32, False, False),
                                            (64, 24, False, False), (16, 128, False, False)])
def test_shape_classes(N, D, tuned, full):
    q = torch.zeros(1, N, 1, D)
    assert MT._supports_tuned_shape(q) == tuned
    assert MT._supports_full_ad_shape(q) == full


@pytest.mark.parametrize("N,D", [(48, 32), (64, 24), (100, 32)])
def test_unsupported_shapes_raise_value_error(N, D):
    with pytest.raises(ValueError, match="power-of-two N"):
        MT.mhsea_with_tuned_ad(*prim(N=N, D=D))


def test_validate_primals_assertions():
    q, k, e, v, m = prim()
    with pytest.raises(AssertionError, match="k shape"):
        MT.mhsea_tuned_ad(q, k[:, :32], e, v, m)
    with pytest.raises(AssertionError, match="requires Vdim"):
        MT.mhsea_tuned_ad(q, k, e, v[..., :16], m)
    with pytest.raises(AssertionError, match="e shape"):
        MT.mhsea_tuned_ad(q, k, e[..., :32], v, m)
    with pytest.raises(AssertionError, match="mask shape"):
        MT.mhsea_tuned_ad(q, k, e, v, m[:, :32])
    with pytest.raises(AssertionError, match="share one storage dtype"):
        MT.mhsea_tuned_ad(q, k.double(), e, v, m)
    with pytest.raises(AssertionError, match="requires float32"):
        MT.mhsea_tuned_ad(*prim(dtype=torch.bfloat16))


def test_zero_cotangent_transposes_to_zeros():
    assert MT.mhsea_tuned_ad_lin_transpose(None, *prim(), None, None) == (None, None, None, None)


def test_op_level_requires_float32():
    Q = torch.zeros(8, 2, 16, dtype=torch.float64)
    with pytest.raises(TypeError, match="float32"):
        EA.reference_edge_attention(Q, Q, Q, torch.zeros(8, 8, 2, dtype=torch.float64), torch.ones(8))
    with pytest.raises(TypeError, match="float32"):
        EA.mhsea_tuned_edge_attention(Q, Q, Q, torch.zeros(8, 8, 2, dtype=torch.float64), torch.ones(8))


@pytest.mark.parametrize("n,d,want_key_mask", [(64, 32, False), (96, 16, False), (16, 32, False), (8, 8, False),
                                               (48, 32, True), (64, 24, True), (100, 32, True)])
def test_op_level_selection(monkeypatch, n, d, want_key_mask):
    """Tuned / full-AD shapes take the primitive (square mask); the rest fall back to the
    jnp formula (additive key mask), as pallas_attention.py:56-61 selects."""
    seen = {}

    def fake_attend(Q, K, V, E, M, *, key_mask):
        seen["key_mask"] = key_mask
        return Q

    monkeypatch.setattr(EA, "_attend", fake_attend)
    Q = torch.zeros(n, 2, d)
    EA.mhsea_tuned_edge_attention(Q, Q, Q, torch.zeros(n, n, 2), torch.ones(n))
    assert seen["key_mask"] == want_key_mask
