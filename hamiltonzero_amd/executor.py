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


def _single(values, name: str):
    """Exactly one entry (``compiled/execute.py:16-21``)."""
    if len(values) != 1:
        raise ValueError(f"compiled HT executor requires exactly one {name}; got {len(values)}")
    return values[0]


def execute_wavefunction(kernel, tree, q_routed: Tensor) -> tuple[Tensor, Tensor]:
    """(log|psi|, phase) of every walker (``compiled/execute.py:79-125``), all on the GPU in
    one ``hz_compiled_wavefunction`` call.

    ``kernel`` and ``tree`` have the reference's structure (``compiled/types.py``):
    ``kernel.q_to_odd.weight``, ``kernel.leaf_factors`` / ``merge_factors`` /
    ``readout_factors`` (one factor each, with ``V`` and ``U``), ``kernel.merge_T``,
    ``kernel.merge_eps``; ``tree.leaf_h``, ``tree.readout_h`` (one entry each),
    ``tree.merge_h`` and ``tree.opcodes`` (one entry per level). ``q_routed`` is
    ``[..., n_sites, d_q]``. The structure checks raise the reference's errors."""
    if len(getattr(tree, "leaf_combiner_h", ())) != 0 or len(getattr(tree, "readout_combiner_h", ())) != 0:
        raise ValueError("single-head compiled HT executor does not accept combiners")
    if len(tree.merge_h) != len(tree.opcodes):
        raise ValueError("merge_h and opcodes must have one entry per tree level")
    leaf = _single(kernel.leaf_factors, "leaf factor")
    merge = _single(kernel.merge_factors, "merge factor")
    readout = _single(kernel.readout_factors, "readout factor")
    leaf_h = _single(tree.leaf_h, "leaf conditioner")
    readout_h = _single(tree.readout_h, "readout conditioner").reshape(-1)
    n = q_routed.shape[-2]
    width = n
    for h_level in tree.merge_h:
        if width != 2 * h_level.shape[-2]:
            raise ValueError("compiled merge level has incompatible shrinking shape")
        width //= 2
    if width != 1:
        raise ValueError("compiled tree did not reduce to one root")
    dev = q_routed.device
    q_weight = kernel.q_to_odd.weight
    T = kernel.merge_T
    G, d_r = T.shape[0], T.shape[1]
    d_q, d_z = q_weight.shape
    R_leaf, d_m = leaf.U.shape
    R_merge = merge.V.shape[1]
    R_out = readout.V.shape[1]
    lead = q_routed.shape[:-2]
    B = 1
    for s in lead:
        B *= s
    ops = [_check("q_routed", q_routed.reshape(B, n, d_q), dev), _check("q_to_odd.weight", q_weight, dev),
           _check("leaf V", leaf.V, dev), _check("leaf U", leaf.U, dev), _check("leaf_h", leaf_h, dev),
           _check("merge_T", T, dev), _check("merge V", merge.V, dev), _check("merge U", merge.U, dev)]
    levels = len(tree.merge_h)
    half = max(n // 2, 1)
    # the reference's packed per-level storage (compiled/model.py:58-90): rows past a level's
    # width are zero conditioners with EMPTY opcodes
    merge_h = torch.zeros((max(levels, 1), half, R_merge), dtype=torch.float32, device=dev)
    opcodes = torch.full((max(levels, 1), half), 3, dtype=torch.uint8, device=dev)
    for level, (h_level, op_level) in enumerate(zip(tree.merge_h, tree.opcodes)):
        w = h_level.shape[-2]
        merge_h[level, :w] = _check("merge_h", h_level, dev)
        opcodes[level, :w] = op_level.to(device=dev, dtype=torch.uint8)
    ops += [merge_h, opcodes, _check("readout V", readout.V, dev), _check("readout U", readout.U, dev),
            _check("readout_h", readout_h, dev)]
    log_abs = torch.empty(B, dtype=torch.float32, device=dev)
    phase = torch.empty(B, dtype=torch.float32, device=dev)
    lib = _native.lib()
    nbytes = lib.hz_compiled_wavefunction_workspace(B, n, d_z, R_leaf, d_m, R_merge, R_out)
    if nbytes < 0:
        raise ValueError("every size of the compiled wavefunction must be >= 1")
    work = torch.empty(nbytes // 4 + 64, dtype=torch.float32, device=dev)
    _native.check(lib.hz_compiled_wavefunction(
        torch.cuda.current_stream(dev).cuda_stream, *(_ptr(t) for t in ops), _ptr(log_abs), _ptr(phase), _ptr(work),
        nbytes, B, n, d_q, d_z, R_leaf, G, d_r, R_merge, R_out, float(kernel.merge_eps)))
    return log_abs.reshape(lead), phase.reshape(lead)
