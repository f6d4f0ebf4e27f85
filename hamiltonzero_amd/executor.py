"""The compiled per-walker executor's products on the gfx950 library (torch mirror).

Reference: ``src/hamiltonzero/compiled/execute.py`` and
``src/hamiltonzero/model/_custom_lap_primitives.py``. The functions keep the reference's
names and argument meaning; they run ``hz_quadrilinear_merge`` / ``hz_factorized_apply``
(``include/hz_executor.h``) on torch's current stream and allocate outputs with torch. There
is no CPU fallback: the HIP library is required and every operand must be a float32 CUDA
tensor on one device.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native

Tensor = torch.Tensor


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _check(name: str, t: Tensor, device: torch.device) -> Tensor:
    if t.dtype != torch.float32:
        raise TypeError(f"{name}.dtype must be float32, got {t.dtype}")
    if not t.is_cuda or t.device != device:
        raise ValueError(f"{name} is on {t.device}: every operand must be on {device}")
    return t.contiguous()


def _compiled_quadrilinear_merge(T: Tensor, u_a: Tensor, u_b: Tensor) -> Tensor:
    """``einsum("ijkl,Bik,Bil->Bij", T, u_a, u_b)`` over ``[..., G * d_r]`` rows
    (``compiled/execute.py:34-52``; ``_custom_lap_primitives.py:36-50``)."""
    if T.dim() != 4 or T.shape[1] != T.shape[2] or T.shape[1] != T.shape[3]:
        raise ValueError(f"T must be [G, d_r, d_r, d_r], got {tuple(T.shape)}")
    G, d_r = T.shape[0], T.shape[1]
    if u_a.shape != u_b.shape or u_a.shape[-1] != G * d_r:
        raise ValueError(f"u_a and u_b must share a shape [..., {G * d_r}], got {tuple(u_a.shape)}, {tuple(u_b.shape)}")
    dev = T.device
    T, u_a, u_b = _check("T", T, dev), _check("u_a", u_a, dev), _check("u_b", u_b, dev)
    M = u_a.numel() // (G * d_r)
    out = torch.empty_like(u_a)
    if M == 0:
        return out
    _native.check(_native.lib().hz_quadrilinear_merge(torch.cuda.current_stream(dev).cuda_stream, _ptr(T), _ptr(u_a),
                                                      _ptr(u_b), _ptr(out), M, G, d_r))
    return out


quadrilinear_merge = _compiled_quadrilinear_merge


def _factorized_apply(factor, h: Tensor, x: Tensor, residual: Optional[Tensor] = None) -> Tensor:
    """``((x @ factor.V) * h) @ factor.U`` (``compiled/execute.py:24-31``), plus ``residual``.

    ``x`` is ``[..., nodes, d_in]`` (or ``[..., d_in]`` with ``h`` one row), ``h`` is
    ``[nodes, R]`` or ``[R]``, broadcast over the leading (walker) axes as in the executor."""
    V, U = factor.V, factor.U
    d_in, R = V.shape
    R2, d_out = U.shape
    if R2 != R or x.shape[-1] != d_in:
        raise ValueError(f"shapes disagree: x {tuple(x.shape)}, V {tuple(V.shape)}, U {tuple(U.shape)}")
    h2 = h.reshape(1, R) if h.dim() == 1 else h
    if h2.dim() != 2 or h2.shape[1] != R:
        raise ValueError(f"h must be [R] or [nodes, R], got {tuple(h.shape)}")
    h_rows = h2.shape[0]
    if h_rows > 1 and (x.dim() < 2 or x.shape[-2] != h_rows):
        raise ValueError(f"h has {h_rows} node rows but x is {tuple(x.shape)}")
    dev = x.device
    x, V, U, h2 = _check("x", x, dev), _check("V", V, dev), _check("U", U, dev), _check("h", h2, dev)
    M = x.numel() // d_in
    y = torch.empty((*x.shape[:-1], d_out), dtype=torch.float32, device=dev)
    if residual is not None:
        if tuple(residual.shape) != tuple(y.shape):
            raise ValueError(f"residual must have shape {tuple(y.shape)}, got {tuple(residual.shape)}")
        residual = _check("residual", residual, dev)
    if M == 0:
        return y
    work = torch.empty((M, R), dtype=torch.float32, device=dev)
    _native.check(_native.lib().hz_factorized_apply(torch.cuda.current_stream(dev).cuda_stream, _ptr(x), _ptr(V),
                                                    _ptr(h2), _ptr(U), _ptr(residual), _ptr(y), _ptr(work), M, d_in, R,
                                                    d_out, h_rows))
    return y


factorized_apply = _factorized_apply
