"""Primitive-level drop-in for the reference's ``mhsea_with_tuned_ad``.

Mirrors ``src/hamiltonzero/model/_pallas_attn/mhsea_tuned.py`` on torch tensors, with
the gfx950 kernels of :mod:`hamiltonzero_amd.kernels` doing all computation:

* ``mhsea_tuned_ad(q, k, e, v, mask) -> (out, lse)`` — the primal primitive
  ``mhsea_tuned_ad_p`` (``mhsea_tuned.py:72-101``).
* ``mhsea_tuned_ad_lin(q, k, e, v, mask, primal_out, lse, qt, kt, et, vt) -> tout`` — the
  linear primitive ``mhsea_tuned_ad_lin_p`` (``:175-203``), 11 operands in the same order.
* ``mhsea_tuned_ad_lin_transpose(cot, q, k, e, v, mask, primal_out, lse)`` — its
  transpose rule (``:206-221``), returning ``(dq, dk, de, dv)``; a ``None`` cotangent
  returns four ``None`` (the reference's ``ad.Zero`` results).
* ``mhsea_with_tuned_ad(q, k, e, v, mask) -> out`` — the public entry (``:243-255``),
  differentiable in reverse mode (``torch.autograd``) and forward mode
  (``torch.autograd.forward_ad``): the forward-mode rule runs the lin primitive and the
  reverse-mode rule runs its transpose, exactly the reference's JVP/transpose pairing
  (``_outer_jvp``, ``:104-118``).
* ``mhsea_tuned_jvp(q, k, e, v, mask, qt, kt, et, vt) -> (out, tout)`` — the batched
  tangent path. Tangents may carry a leading direction axis T; the kernel forms P once
  and reuses it for every direction, where the reference's batching rule broadcasts the
  primals and recomputes P per direction (``:144-148``, ``:224-229``).

``e`` may be ``None`` (no edge bias, the zero tensor in the reference). Argument errors
follow the reference: ``ValueError`` for an unsupported N or head dimension
(``:244-248``), ``AssertionError`` for inconsistent shapes or dtypes (``:29-50``).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import kernels

Tensor = torch.Tensor

_SUPPORTED_TUNED_HEAD_DIMS = frozenset((8, 16, 32, 64))


def _validate_primals(q, k, e, v, mask) -> None:
    """Shape / dtype assertions of ``_validate_primals`` (mhsea_tuned.py:29-50)."""
    assert q.ndim == k.ndim == v.ndim == 4
    assert e is None or e.ndim == 4
    assert mask.ndim == 2
    assert q.dtype == k.dtype == v.dtype and (e is None or e.dtype == q.dtype), (
        f"mhsea_tuned_ad requires q/k/e/v to share one storage dtype; got {q.dtype}, {k.dtype}, "
        f"{None if e is None else e.dtype}, {v.dtype}"
    )
    assert q.dtype == torch.float32, (
        f"mhsea_tuned_ad currently requires float32 public tensors; got {q.dtype}"
    )
    batch_len, seq_len, num_heads, head_len = q.shape
    assert k.shape == q.shape, f"k shape {tuple(k.shape)} != q shape {tuple(q.shape)}"
    assert v.shape == q.shape, (
        "mhsea_tuned_ad currently requires Vdim == q/k head dim and matching leading "
        f"dimensions; got v={tuple(v.shape)}, q={tuple(q.shape)}"
    )
    if e is not None:
        assert tuple(e.shape) == (batch_len, seq_len, num_heads, seq_len), (
            f"e shape {tuple(e.shape)} != ({batch_len}, {seq_len}, {num_heads}, {seq_len})"
        )
    assert tuple(mask.shape) == (batch_len, seq_len), (
        f"mask shape {tuple(mask.shape)} != ({batch_len}, {seq_len})"
    )
    assert head_len == v.shape[-1]


def _supports_tuned_shape(q) -> bool:
    """``_supports_tuned_shape`` (mhsea_tuned.py:53-59): N >= 64, N % 32 == 0."""
    return (
        q.dtype == torch.float32
        and q.shape[1] >= 64
        and q.shape[1] % 32 == 0
        and q.shape[-1] in _SUPPORTED_TUNED_HEAD_DIMS
    )


def _supports_full_ad_shape(q) -> bool:
    """``_supports_full_ad_shape`` (mhsea_tuned.py:62-69): N a power of two below 64."""
    seq_len = q.shape[1]
    return (
        q.dtype == torch.float32
        and 0 < seq_len < 64
        and not (seq_len & (seq_len - 1))
        and q.shape[-1] in _SUPPORTED_TUNED_HEAD_DIMS
    )


class _MhseaAD(torch.autograd.Function):
    """(out, lse) = MHSEA(q, k, e, v, mask) with the lin primitive as its JVP and the
    lin primitive's transpose as its VJP. ``opts`` = (scale, key_mask, e_layout)."""

    @staticmethod
    def forward(q, k, e, v, mask, opts):
        scale, key_mask, e_layout = opts
        out, lse = kernels.mhsea_fwd(q, k, v, mask, e, scale=scale, key_mask=key_mask, e_layout=e_layout)
        return out, lse

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, e, v, mask, opts = inputs
        out, lse = output
        ctx.opts = opts
        ctx.has_e = e is not None
        ctx.mark_non_differentiable(lse)
        saved = (q, k, e, v, mask, out, lse)
        ctx.save_for_backward(*saved)
        ctx.save_for_forward(*saved)

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, e, v, mask, out, lse = ctx.saved_tensors
        scale, key_mask, e_layout = ctx.opts
        dq, dk, de, dv = kernels.mhsea_bwd(
            q, k, v, mask, lse, out, dout, e,
            want_de=bool(ctx.needs_input_grad[2]), scale=scale, key_mask=key_mask, e_layout=e_layout,
        )
        return dq, dk, de, dv, None, None

    @staticmethod
    def jvp(ctx, qt, kt, et, vt, _mask_t, _opts_t):
        q, k, e, v, mask, out, lse = ctx.saved_tensors
        scale, key_mask, e_layout = ctx.opts
        tout = kernels.mhsea_jvp(
            q, k, v, mask, out, lse, qt, kt, vt, e, et,
            scale=scale, key_mask=key_mask, e_layout=e_layout,
        )
        return tout, None


class _GatedAD(torch.autograd.Function):
    """y = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:] of MHSEA(q, k, e, v, mask), the trunk's
    head collapse (trunk.py:134-137). The forward and forward mode run the fused kernel
    (``hz_mhsea_fwd_jvp_gated``); reverse mode recomputes (out, lse) and runs
    ``hz_mhsea_bwd_gated`` (the collapse's cotangent formed on the GPU, then the attention
    backward)."""

    @staticmethod
    def forward(q, k, e, v, mask, opts):
        scale, key_mask, e_layout = opts
        y, _ = kernels.mhsea_fwd_jvp_gated(q, k, v, mask, e=e, scale=scale, key_mask=key_mask, e_layout=e_layout)
        return y

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, e, v, mask, opts = inputs
        ctx.opts = opts
        ctx.save_for_backward(q, k, e, v, mask)
        ctx.save_for_forward(q, k, e, v, mask)

    @staticmethod
    def backward(ctx, dy):
        q, k, e, v, mask = ctx.saved_tensors
        scale, key_mask, e_layout = ctx.opts
        out, lse = kernels.mhsea_fwd(q, k, v, mask, e, scale=scale, key_mask=key_mask, e_layout=e_layout)
        dq, dk, de, dv = kernels.mhsea_bwd_gated(
            q, k, v, mask, lse, out, dy.contiguous(), e,
            want_de=bool(ctx.needs_input_grad[2]), scale=scale, key_mask=key_mask, e_layout=e_layout,
        )
        return dq, dk, de, dv, None, None

    @staticmethod
    def jvp(ctx, qt, kt, et, vt, _mask_t, _opts_t):
        q, k, e, v, mask = ctx.saved_tensors
        scale, key_mask, e_layout = ctx.opts
        y, ty = kernels.mhsea_fwd_jvp_gated(q, k, v, mask, qt, kt, vt, e=e, et=et, scale=scale, key_mask=key_mask,
                                            e_layout=e_layout)
        return torch.zeros_like(y) if ty is None else ty


def gated_edge_attention(q, k, e, v, mask, *, scale: float = 1.0, key_mask: bool = False, e_layout: str = "qhk"):
    """Differentiable head-collapsed attention ``sigmoid(gate) * value`` (trunk.py:130-137 for
    the tuned path): ``[B, N, H, D]`` operands with H = 2 * n_heads, result ``[B, N, H/2, D]``.
    Serves what ``hz_mhsea_fwd_jvp_gated`` serves (fp32, any N and head dimension, even H)."""
    return _GatedAD.apply(q, k, e, v, mask, (float(scale), bool(key_mask), e_layout))


def mhsea_ad(q, k, e, v, mask, *, scale: float = 1.0, key_mask: bool = False, e_layout: str = "qhk"):
    """Differentiable (out, lse) with explicit scale / mask mode / bias layout."""
    return _MhseaAD.apply(q, k, e, v, mask, (float(scale), bool(key_mask), e_layout))


def mhsea_tuned_ad(q, k, e, v, mask) -> Tuple[Tensor, Tensor]:
    """The primal primitive ``mhsea_tuned_ad_p.bind`` (mhsea_tuned.py:72-101)."""
    _validate_primals(q, k, e, v, mask)
    return mhsea_ad(q, k, e, v, mask)


def mhsea_tuned_ad_lin(q, k, e, v, mask, primal_out, lse, qt, kt, et, vt) -> Tensor:
    """The linear primitive ``mhsea_tuned_ad_lin_p.bind`` (mhsea_tuned.py:175-203)."""
    _validate_primals(q, k, e, v, mask)
    return kernels.mhsea_jvp(q, k, v, mask, primal_out, lse, qt, kt, vt, e, et)


def mhsea_tuned_ad_lin_transpose(cot, q, k, e, v, mask, primal_out, lse):
    """Transpose of the linear primitive (``_inner_transpose``, mhsea_tuned.py:206-221)."""
    if cot is None:
        return (None, None, None, None)
    _validate_primals(q, k, e, v, mask)
    return kernels.mhsea_bwd(q, k, v, mask, lse, primal_out, cot, e, want_de=True)


def mhsea_with_tuned_ad(q, k, e, v, mask) -> Tensor:
    """Public entry ``mhsea_with_tuned_ad`` (mhsea_tuned.py:243-255).

    Masked query rows of the result are exact zeros, for both the tuned (N >= 64,
    N % 32 == 0) and the full-AD (power-of-two N < 64) shape classes
    (mhsea_tuned.py:91, :252); one kernel family serves both.
    """
    if not _supports_tuned_shape(q):
        if not _supports_full_ad_shape(q):
            raise ValueError(
                "mhsea requires a power-of-two N and head dimension in "
                f"{sorted(_SUPPORTED_TUNED_HEAD_DIMS)}"
            )
    _validate_primals(q, k, e, v, mask)
    out, _lse = mhsea_ad(q, k, e, v, mask)
    return out


def mhsea_tuned_jvp(q, k, e, v, mask, qt=None, kt=None, et=None, vt=None):
    """Primal and tangent(s) in one fused pass; tangents may have a leading axis T."""
    _validate_primals(q, k, e, v, mask)
    out, _lse, tout = kernels.mhsea_fwd_jvp(q, k, v, mask, qt, kt, vt, e, et, with_lse=False)
    return out, tout


__all__ = [
    "mhsea_ad",
    "mhsea_tuned_ad",
    "mhsea_tuned_ad_lin",
    "mhsea_tuned_ad_lin_transpose",
    "mhsea_tuned_jvp",
    "mhsea_with_tuned_ad",
]
