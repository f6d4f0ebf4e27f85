"""Drop-in for the reference's large-N evaluation attention.

Mirrors ``src/hamiltonzero/evaluation/pallas_mha.py`` (``BlockSizes``,
``noncausal_bias_mha``) and ``src/hamiltonzero/evaluation/sequence_parallel.py``
(``pallas_rectangular_edge_attention`` and its input checks) with the same names,
argument meanings and errors, running on the gfx950 kernel ``hz_rect_attention_fwd``.

Differences that change no result: the block sizes are validated as in the reference but
do not steer the kernel (it streams keys in its own chunks and handles any length); the
``-1e30`` masking of ``sequence_parallel.py:79-83`` and the ``D**-0.5`` pre-scaling of the
queries (``:72,85``) are applied inside the kernel instead of as separate passes over the
bias and the queries.
"""

from __future__ import annotations

import dataclasses

import torch

from . import kernels

Tensor = torch.Tensor


@dataclasses.dataclass(frozen=True)
class BlockSizes:
    """``BlockSizes`` (pallas_mha.py:33-40)."""

    block_q: int
    block_k: int

    @classmethod
    def get_default(cls):
        return cls(block_q=128, block_k=128)


def noncausal_bias_mha(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, *, block_sizes: BlockSizes = BlockSizes.get_default()) -> Tensor:
    """softmax_j(q_i . k_j + bias[b, i, j, h]) v_j (pallas_mha.py:92-161).

    ``q [B, Nq, H, D]``, ``k, v [B, Nk, H, D]``, ``bias [B, Nq, Nk, H]``. The checks and
    their messages follow ``:101-118``.
    """
    batch_size, q_seq_len, num_heads, head_dim = q.shape
    kv_seq_len = k.shape[1]
    block_q = min(block_sizes.block_q, q_seq_len)
    block_k = min(block_sizes.block_k, kv_seq_len)
    if (q.shape[-1] != k.shape[-1]) or (q.shape[-1] != v.shape[-1]):
        raise ValueError(
            "This kernel expects q, k, and v to have the same head dimension, "
            f"but found {tuple(q.shape)=}, {tuple(k.shape)=}, {tuple(v.shape)=}."
        )
    if tuple(bias.shape) != (batch_size, q_seq_len, kv_seq_len, num_heads):
        raise ValueError(f"bias must have shape [batch, query, key, heads]; got {tuple(bias.shape)}")
    if q_seq_len % block_q != 0:
        raise ValueError(f"{q_seq_len=} must be a multiple of {block_q=}")
    if kv_seq_len % block_k != 0:
        raise ValueError(f"{kv_seq_len=} must be a multiple of {block_k=}")
    return kernels.rect_attention_fwd(q, k, v, bias, None, scale=1.0)


def _validate_rectangular_attention_inputs(q_local, k_global, v_global, edge_bias_local, key_mask) -> None:
    """``_validate_rectangular_attention_inputs`` (sequence_parallel.py:13-47)."""
    if q_local.dim() != 3 or k_global.dim() != 3 or v_global.dim() != 3:
        raise ValueError("q, k, and v must have shapes [sequence, heads, head_dim]")
    q_len, n_heads, head_dim = q_local.shape
    kv_len = k_global.shape[0]
    if q_len < 1 or kv_len < 1:
        raise ValueError("query and key sequence lengths must both be positive")
    if k_global.shape != v_global.shape:
        raise ValueError(f"k and v shapes must match; got {tuple(k_global.shape)} and {tuple(v_global.shape)}")
    if tuple(k_global.shape[1:]) != (n_heads, head_dim):
        raise ValueError(
            "q, k, and v must have the same head count and head dimension; "
            f"got {tuple(q_local.shape)}, {tuple(k_global.shape)}, and {tuple(v_global.shape)}"
        )
    if tuple(edge_bias_local.shape) != (q_len, kv_len, n_heads):
        raise ValueError(
            "edge bias must have shape [local_queries, global_keys, heads]; "
            f"got {tuple(edge_bias_local.shape)}, expected {(q_len, kv_len, n_heads)}"
        )
    if tuple(key_mask.shape) != (kv_len,):
        raise ValueError(f"key mask must have shape {(kv_len,)}, got {tuple(key_mask.shape)}")
    arrays = (q_local, k_global, v_global, edge_bias_local)
    if any(value.dtype != torch.float32 for value in arrays):
        raise TypeError(
            "large-N rectangular attention is fp32-only; got " + ", ".join(str(value.dtype) for value in arrays)
        )


def _dividing_block_size(length: int, requested: int | None) -> int:
    """``_dividing_block_size`` (sequence_parallel.py:50-56)."""
    block = min(length, 128 if requested is None else requested)
    if block < 1:
        raise ValueError(f"block size must be positive, got {block}")
    while length % block:
        block //= 2
    return block


def pallas_rectangular_edge_attention(
    q_local: Tensor,
    k_global: Tensor,
    v_global: Tensor,
    edge_bias_local: Tensor,
    key_mask: Tensor,
    *,
    block_k: int | None = None,
) -> Tensor:
    """One system's local queries against all keys (sequence_parallel.py:59-90).

    ``q_local [r, h, d]``, ``k_global, v_global [n, h, d]``, ``edge_bias_local [r, n, h]``,
    ``key_mask [n]``. Returns ``[r, h, d]``.
    """
    _validate_rectangular_attention_inputs(q_local, k_global, v_global, edge_bias_local, key_mask)
    sm_scale = float(q_local.shape[-1]) ** -0.5
    _dividing_block_size(q_local.shape[0], None)
    _dividing_block_size(k_global.shape[0], block_k)
    out = kernels.rect_attention_fwd(
        q_local[None], k_global[None], v_global[None], edge_bias_local[None], key_mask[None], scale=sm_scale
    )
    return out[0]


def gated_rectangular_edge_attention(
    q_local: Tensor,
    k_global: Tensor,
    v_global: Tensor,
    edge_bias_local: Tensor,
    key_mask: Tensor,
    *,
    block_k: int | None = None,
) -> Tensor:
    """The large-N caller's attention and head collapse in one kernel
    (``_sequence_level_edge_attention``, sequence_trunk.py:973-981):
    ``sigmoid(out[:, :h/2]) * out[:, h/2:]`` of :func:`pallas_rectangular_edge_attention`'s
    ``out``, with the same operands and checks. Returns ``[r, h/2, d]``; the attention
    output itself is never written."""
    _validate_rectangular_attention_inputs(q_local, k_global, v_global, edge_bias_local, key_mask)
    sm_scale = float(q_local.shape[-1]) ** -0.5
    _dividing_block_size(q_local.shape[0], None)
    _dividing_block_size(k_global.shape[0], block_k)
    y = kernels.rect_attention_fwd(
        q_local[None], k_global[None], v_global[None], edge_bias_local[None], key_mask[None], scale=sm_scale,
        gated=True,
    )
    return y[0]


def sequence_attention_output(
    q_local: Tensor,
    k_global: Tensor,
    v_global: Tensor,
    edge_bias_local: Tensor,
    key_mask: Tensor,
    w_o: Tensor,
    row_mask: Tensor,
    *,
    block_k: int | None = None,
) -> Tensor:
    """``proposal_attn = row_mask[:, None] * (y.reshape(r, -1) @ w_o)`` with ``y`` from
    :func:`gated_rectangular_edge_attention` (sequence_trunk.py:973-984): two launches, the
    gated attention and the site-masked W_O (rows with ``row_mask`` 0 are written as zeros
    without being multiplied). ``w_o [h/2 * d, d_c]``, ``row_mask [r]``; returns ``[r, d_c]``."""
    y = gated_rectangular_edge_attention(q_local, k_global, v_global, edge_bias_local, key_mask, block_k=block_k)
    delta, _ = kernels.gated_out_proj(y[None], w_o, mask=row_mask[None])
    return delta[0]


__all__ = ["BlockSizes", "gated_rectangular_edge_attention", "noncausal_bias_mha", "pallas_rectangular_edge_attention",
           "sequence_attention_output"]
