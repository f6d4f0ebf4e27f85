"""Host-side behaviour of the rectangular-attention mirror that needs no GPU: the input
checks and messages of the reference's wrappers (src/hamiltonzero/evaluation/
sequence_parallel.py:13-56, pallas_mha.py:101-118) run before any device work."""

import pytest
import torch

from hamiltonzero_amd import rect_attention as RA


def _sys(r=8, n=16, h=4, d=8, dtype=torch.float32):
    return (torch.zeros(r, h, d, dtype=dtype), torch.zeros(n, h, d, dtype=dtype), torch.zeros(n, h, d, dtype=dtype),
            torch.zeros(r, n, h, dtype=dtype), torch.ones(n, dtype=torch.bool))


@pytest.mark.parametrize(
    "mutate,exc,needle",
    [
        (lambda a: (a[0][None], *a[1:]), ValueError, "must have shapes [sequence, heads, head_dim]"),
        (lambda a: (a[0][:0], *a[1:]), ValueError, "must both be positive"),
        (lambda a: (a[0], a[1], a[2][:8], *a[3:]), ValueError, "k and v shapes must match"),
        (lambda a: (a[0], a[1][:, :2], a[2][:, :2], *a[3:]), ValueError, "same head count"),
        (lambda a: (*a[:3], a[3][:, :8], a[4]), ValueError, "edge bias must have shape"),
        (lambda a: (*a[:4], a[4][:8]), ValueError, "key mask must have shape"),
        (lambda a: (a[0].double(), *a[1:]), TypeError, "fp32-only"),
    ],
)
def test_rectangular_wrapper_validation(mutate, exc, needle):
    with pytest.raises(exc) as err:
        RA.pallas_rectangular_edge_attention(*mutate(_sys()))
    assert needle in str(err.value)


def test_rectangular_wrapper_block_size_check():
    with pytest.raises(ValueError, match="block size must be positive"):
        RA.pallas_rectangular_edge_attention(*_sys(), block_k=0)


def test_rectangular_wrapper_needs_gpu_tensors():
    with pytest.raises(ValueError, match="GPU tensors"):
        RA.pallas_rectangular_edge_attention(*_sys())


def test_noncausal_bias_mha_validation():
    q = torch.zeros(1, 256, 4, 8)
    k = torch.zeros(1, 192, 4, 8)
    with pytest.raises(ValueError, match="same head dimension"):
        RA.noncausal_bias_mha(q, k, torch.zeros(1, 192, 4, 16), torch.zeros(1, 256, 192, 4))
    with pytest.raises(ValueError, match=r"bias must have shape \[batch, query, key, heads\]"):
        RA.noncausal_bias_mha(q, k, k, torch.zeros(1, 256, 4, 192))
    with pytest.raises(ValueError, match="must be a multiple of block_k"):
        RA.noncausal_bias_mha(q, k, k, torch.zeros(1, 256, 192, 4))
    assert RA.BlockSizes.get_default() == RA.BlockSizes(128, 128)


def test_dividing_block_size():
    assert RA._dividing_block_size(1000, None) == 8
    assert RA._dividing_block_size(1024, None) == 128
    assert RA._dividing_block_size(96, 64) == 32
    assert RA._dividing_block_size(5, None) == 5
