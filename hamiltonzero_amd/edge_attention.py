"""Op-level drop-in for ``src/hamiltonzero/model/pallas_attention.py``.

``mhsea_tuned_edge_attention(Q, K, V, edge_bias, mask)`` and
``reference_edge_attention(Q, K, V, edge_bias, mask)`` keep the reference's per-system
signatures ``Q, K, V: [n, h, d]``, ``edge_bias: [n, n, h]``, ``mask: [n]`` and also accept
a leading batch axis (``[B, n, h, d]``, ``[B, n, n, h]``, ``[B, n]``), which is what a
``vmap`` over systems hands to the primitive.

Both run on the gfx950 kernels; neither adds a pass over the data:

* the ``D**-0.5`` pre-scaling of Q (``pallas_attention.py:62``) is applied inside the
  kernel to the Q fragment in registers;
* ``edge_bias`` is read in its ``[n(query), n(key), h]`` layout (``HZ_FLAG_E_QKH``), so the
  transpose to ``[n, h, n]`` (``:65``) disappears, and its gradient comes back in the same
  layout.

Selection between the tuned primitive and the fallback follows ``:50-61``.
``reference_edge_attention`` is the reference's jnp formula (``:22-37``): keys masked by
an additive -1e9, masked query rows computed like the others. Head dimensions outside
{8, 16, 32, 64} (below 64) are zero-padded on the host to the next supported size, which
leaves every dot product unchanged.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .mhsea_tuned import mhsea_ad

Tensor = torch.Tensor

_SUPPORTED_MHSEA_HEAD_DIMS = frozenset((8, 16, 32, 64))


def _require_fp32(*values: Tensor) -> None:
    """``_require_fp32`` (pallas_attention.py:16-19)."""
    for value in values:
        if value.dtype != torch.float32:
            raise TypeError(f"attention tensors must be float32, got {value.dtype}")


def _batched(Q, K, V, edge_bias, mask):
    if Q.dim() == 3:
        return True, Q[None], K[None], V[None], edge_bias[None], mask[None]
    if Q.dim() == 4:
        return False, Q, K, V, edge_bias, mask
    raise ValueError(f"Q must be [n, h, d] or [B, n, h, d], got shape {tuple(Q.shape)}")


def _attend(Q, K, V, edge_bias, mask, *, key_mask: bool):
    squeeze, Q4, K4, V4, E4, M = _batched(Q, K, V, edge_bias, mask)
    d = Q4.shape[-1]
    scale = float(d) ** -0.5
    pad = 0
    if d not in _SUPPORTED_MHSEA_HEAD_DIMS:
        target = next((s for s in sorted(_SUPPORTED_MHSEA_HEAD_DIMS) if s >= d), None)
        if target is None:
            raise ValueError(f"head dimension {d} exceeds the largest supported (64)")
        pad = target - d
        Q4, K4, V4 = (F.pad(x, (0, pad)) for x in (Q4, K4, V4))
    out, _lse = mhsea_ad(Q4, K4, E4, V4, M.to(torch.bool), scale=scale, key_mask=key_mask, e_layout="qkh")
    if pad:
        out = out[..., :d]
    return out[0] if squeeze else out


def reference_edge_attention(Q: Tensor, K: Tensor, V: Tensor, edge_bias: Tensor, mask: Tensor) -> Tensor:
    """softmax(Q K^T / sqrt(d) + E^T - 1e9 (1 - mask_k)) V (pallas_attention.py:22-37)."""
    _require_fp32(Q, K, V, edge_bias)
    return _attend(Q, K, V, edge_bias, mask, key_mask=True)


def mhsea_tuned_edge_attention(Q: Tensor, K: Tensor, V: Tensor, edge_bias: Tensor, mask: Tensor) -> Tensor:
    """Tuned MHSEA with the reference's shape-based fallback (pallas_attention.py:40-67)."""
    _require_fp32(Q, K, V, edge_bias)
    _n, _n_heads, d_head = Q.shape[-3:]
    lead = Q.shape[:-3]
    square = (
        K.shape == Q.shape
        and V.shape == Q.shape
        and tuple(edge_bias.shape) == (*lead, _n, _n, _n_heads)
        and tuple(mask.shape) == (*lead, _n)
    )
    supports_tuned = square and _n >= 64 and _n % 32 == 0
    supports_full_ad = square and 0 < _n < 64 and not (_n & (_n - 1))
    if d_head not in _SUPPORTED_MHSEA_HEAD_DIMS or not (supports_tuned or supports_full_ad):
        return reference_edge_attention(Q, K, V, edge_bias, mask)
    return _attend(Q, K, V, edge_bias, mask, key_mask=False)


__all__ = ["mhsea_tuned_edge_attention", "reference_edge_attention"]
