"""Torch-tensor entry points of the gfx950 MHSEA kernels.

Thin, allocation-owning wrappers over the C ABI (``include/hz_mhsea.h``): they check
shapes, dtypes and devices, allocate outputs with torch on the inputs' device and
enqueue the kernels on torch's current stream. No computation happens here; the HIP
library is required.

Layouts follow the reference primitives (``_pallas_attn/utils.py:21-36``):
``q, k, v: [B, N, H, D]``, ``e: [B, N, H, N]`` (or ``[B, N, N, H]`` with
``e_layout="qkh"``, or the compacted physical-pair layout ``[B, H, N, ceil4(N)]`` with
``e_layout="compact"``: ``compact_bias``), ``mask: [B, N]`` bool, ``lse: [B, N, H]`` float32,
tangents ``[T, B, N, H, D]`` or a single ``[B, N, H, D]`` direction.

Every call takes ``generic=True`` to force the LDS-streaming kernels (``HZ_FLAG_GENERIC``)
instead of the automatic choice, for testing and comparison.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native

Tensor = torch.Tensor

_DTYPES = {torch.float32: _native.HZ_DTYPE_F32, torch.bfloat16: _native.HZ_DTYPE_BF16}
SUPPORTED_HEAD_DIMS = (8, 16, 32, 64)


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


E_LAYOUTS = ("qhk", "qkh", "compact")


def e_shape(B: int, N: int, H: int, e_layout: str) -> tuple:
    """Shape of the bias in ``e_layout``: ``[B, N, H, N]`` (query, head, key), ``[B, N, N, H]``
    (``"qkh"``) or ``[B, H, N, ceil4(N)]`` (``"compact"``, see ``compact_bias``)."""
    if e_layout == "qhk":
        return (B, N, H, N)
    if e_layout == "qkh":
        return (B, N, N, H)
    if e_layout == "compact":
        return (B, H, N, (N + 3) // 4 * 4)
    raise ValueError(f"e_layout must be one of {list(E_LAYOUTS)}, got {e_layout!r}")


def _flags(key_mask: bool, e_layout: str, generic: bool = False) -> int:
    if e_layout not in E_LAYOUTS:
        raise ValueError(f"e_layout must be one of {list(E_LAYOUTS)}, got {e_layout!r}")
    return (
        (_native.HZ_FLAG_KEY_MASK if key_mask else 0)
        | (_native.HZ_FLAG_E_QKH if e_layout == "qkh" else 0)
        | (_native.HZ_FLAG_E_COMPACT if e_layout == "compact" else 0)
        | (_native.HZ_FLAG_GENERIC if generic else 0)
    )


def compact_bias(e: Tensor, mask: Tensor, e_layout: str = "qhk") -> Tensor:
    """The compacted physical-pair layout of a bias given in ``e_layout`` (``"qhk"`` or
    ``"qkh"``), as ``hz_pair_bias`` writes it with ``HZ_FLAG_E_COMPACT``: ``[B, H, N, N4]``
    (N4 = N rounded up to a multiple of 4) whose block ``(b, h)`` holds, for walker b's n
    physical sites s_0 < ... < s_{n-1}, ``e[b, s_i, h, s_j]`` at flat position
    ``i * ceil4(n) + j``; the rest is zero and never read. Square-mask attention only. A
    layout conversion on the GPU (torch gather), for callers that hold a full bias."""
    if e_layout not in ("qhk", "qkh"):
        raise ValueError(f"e_layout must be 'qhk' or 'qkh', got {e_layout!r}")
    B, N = e.shape[0], e.shape[1]
    H = e.shape[2] if e_layout == "qhk" else e.shape[3]
    eh = e if e_layout == "qhk" else e.permute(0, 1, 3, 2)  # [B, N(query), H, N(key)]
    eh = eh.permute(0, 2, 1, 3)  # [B, H, Nq, Nk]
    m = (mask.to(device=e.device) != 0)
    # physical sites first, ascending (a stable sort of the inverted mask)
    order = torch.sort((~m).to(torch.int8), dim=1, stable=True).indices  # [B, N]
    g = torch.gather(eh, 2, order[:, None, :, None].expand(B, H, N, N))
    g = torch.gather(g, 3, order[:, None, None, :].expand(B, H, N, N))
    n = m.sum(dim=1)  # [B]
    n4 = (n + 3) // 4 * 4
    ar = torch.arange(N, device=e.device)
    size = N * ((N + 3) // 4 * 4)
    pos = ar[None, :, None] * n4[:, None, None] + ar[None, None, :]  # [B, i, j] -> i * ceil4(n) + j
    valid = (ar[None, :, None] < n[:, None, None]) & (ar[None, None, :] < n[:, None, None])
    pos = torch.where(valid, pos, torch.full_like(pos, size))  # invalid pairs land in a spare slot
    out = torch.zeros((B, H, size + 1), dtype=e.dtype, device=e.device)
    out.scatter_(2, pos.reshape(B, 1, N * N).expand(B, H, N * N), g.reshape(B, H, N * N))
    return out[:, :, :size].reshape(e_shape(B, N, H, "compact")).contiguous()


def _check_primals(q: Tensor, k: Tensor, v: Tensor, mask: Tensor, e: Optional[Tensor], e_layout: str):
    if q.dim() != 4:
        raise ValueError(f"q must have rank 4 [B, N, H, D], got shape {tuple(q.shape)}")
    B, N, H, D = q.shape
    if q.dtype not in _DTYPES:
        raise TypeError(f"q.dtype must be float32 or bfloat16, got {q.dtype}")
    if not q.is_cuda:
        raise ValueError("MHSEA kernels need GPU tensors (q is on %s)" % q.device)
    if D not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head dimension must be one of {list(SUPPORTED_HEAD_DIMS)}, got {D}")
    for name, t in (("k", k), ("v", v)):
        if tuple(t.shape) != (B, N, H, D):
            raise ValueError(f"{name}.shape must be {(B, N, H, D)}, got {tuple(t.shape)}")
        if t.dtype != q.dtype:
            raise TypeError(f"{name}.dtype must equal q.dtype ({q.dtype}), got {t.dtype}")
        if t.device != q.device:
            raise ValueError(f"{name} is on {t.device}, q on {q.device}")
    if tuple(mask.shape) != (B, N):
        raise ValueError(f"mask.shape must be {(B, N)}, got {tuple(mask.shape)}")
    if e is not None:
        want = e_shape(B, N, H, e_layout)
        if tuple(e.shape) != want:
            raise ValueError(f"e.shape must be {want}, got {tuple(e.shape)}")
        if e.dtype != q.dtype:
            raise TypeError(f"e.dtype must equal q.dtype ({q.dtype}), got {e.dtype}")
        _on_device(q.device, e=e)
    return B, N, H, D


def _c(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.contiguous()


def _on_device(device: torch.device, **tensors: Optional[Tensor]) -> None:
    """Every given tensor operand must live on ``device`` (the GPU of q): the kernels receive
    raw device pointers, so a host tensor here would be a memory fault, not an error."""
    for name, t in tensors.items():
        if t is not None and t.device != device:
            raise ValueError(f"{name} is on {t.device}, q on {device}: every tensor operand must be on q's GPU")


def _mask_u8(mask: Tensor, device: torch.device) -> Tensor:
    m = mask.to(device=device)
    if m.dtype == torch.bool:
        return m.contiguous().view(torch.uint8)
    return (m != 0).contiguous().view(torch.uint8)


def _tangent(t: Optional[Tensor], shape: tuple, dtype, name: str) -> Tuple[Optional[Tensor], int]:
    """Normalise one tangent operand to [T, *shape]; returns (tensor or None, T or 0)."""
    if t is None:
        return None, 0
    if tuple(t.shape) == shape:
        t = t.unsqueeze(0)
    if t.dim() != len(shape) + 1 or tuple(t.shape[1:]) != shape:
        raise ValueError(f"{name}.shape must be {shape} or [T, *{shape}], got {tuple(t.shape)}")
    if t.dtype != dtype:
        raise TypeError(f"{name}.dtype must be {dtype}, got {t.dtype}")
    return t.contiguous(), t.shape[0]


def _tangents(q, eshape, qt, kt, et, vt):
    shape = tuple(q.shape)
    qt, tq = _tangent(qt, shape, q.dtype, "qt")
    kt, tk = _tangent(kt, shape, q.dtype, "kt")
    vt, tv = _tangent(vt, shape, q.dtype, "vt")
    et, te = _tangent(et, eshape, q.dtype, "et")
    _on_device(q.device, qt=qt, kt=kt, vt=vt, et=et)
    counts = {x for x in (tq, tk, tv, te) if x}
    if len(counts) > 1:
        raise ValueError(f"tangent directions disagree: {sorted(counts)}")
    T = counts.pop() if counts else 1
    return qt, kt, et, vt, T


def mhsea_fwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Tensor,
    e: Optional[Tensor] = None,
    *,
    scale: float = 1.0,
    key_mask: bool = False,
    e_layout: str = "qhk",
    generic: bool = False,
    with_lse: bool = True,
) -> Tuple[Tensor, Optional[Tensor]]:
    """Forward: returns ``(out, lse)`` (lse is None when ``with_lse`` is False)."""
    B, N, H, D = _check_primals(q, k, v, mask, e, e_layout)
    q, k, v, e = _c(q), _c(k), _c(v), _c(e)
    m = _mask_u8(mask, q.device)
    out = torch.empty_like(q)
    lse = torch.empty((B, N, H), dtype=torch.float32, device=q.device) if with_lse else None
    _native.check(
        _native.lib().hz_mhsea_fwd(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(e), _ptr(v), _ptr(m), _ptr(out), _ptr(lse),
            B, N, H, D, _DTYPES[q.dtype], float(scale), _flags(key_mask, e_layout, generic),
        )
    )
    return out, lse


def mhsea_jvp(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Tensor,
    out: Tensor,
    lse: Tensor,
    qt: Optional[Tensor] = None,
    kt: Optional[Tensor] = None,
    vt: Optional[Tensor] = None,
    e: Optional[Tensor] = None,
    et: Optional[Tensor] = None,
    *,
    scale: float = 1.0,
    key_mask: bool = False,
    e_layout: str = "qhk",
    generic: bool = False,
) -> Tensor:
    """Tangent of the forward given its primal ``(out, lse)`` (the reference's lin primitive).

    Tangents are ``[B, N, H, D]`` (one direction) or ``[T, B, N, H, D]``; ``None`` is a
    zero tangent. Returns ``tout`` shaped like the given tangents.
    """
    B, N, H, D = _check_primals(q, k, v, mask, e, e_layout)
    e_shape_ = e_shape(B, N, H, e_layout)
    batched = any(t is not None and t.dim() == 5 for t in (qt, kt, vt)) or (et is not None and et.dim() == 5)
    qt, kt, et, vt, T = _tangents(q, e_shape_, qt, kt, et, vt)
    if tuple(out.shape) != (B, N, H, D) or out.dtype != q.dtype:
        raise ValueError("out must match q in shape and dtype")
    if tuple(lse.shape) != (B, N, H) or lse.dtype != torch.float32:
        raise ValueError(f"lse must be float32 of shape {(B, N, H)}")
    _on_device(q.device, out=out, lse=lse)
    q, k, v, e, out, lse = _c(q), _c(k), _c(v), _c(e), _c(out), _c(lse)
    m = _mask_u8(mask, q.device)
    tout = torch.empty((T, B, N, H, D), dtype=q.dtype, device=q.device)
    _native.check(
        _native.lib().hz_mhsea_jvp(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(e), _ptr(v), _ptr(m), _ptr(out), _ptr(lse),
            _ptr(qt), _ptr(kt), _ptr(et), _ptr(vt), T, _ptr(tout),
            B, N, H, D, _DTYPES[q.dtype], float(scale), _flags(key_mask, e_layout, generic),
        )
    )
    return tout if batched else tout[0]


def mhsea_fwd_jvp(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Tensor,
    qt: Optional[Tensor] = None,
    kt: Optional[Tensor] = None,
    vt: Optional[Tensor] = None,
    e: Optional[Tensor] = None,
    et: Optional[Tensor] = None,
    *,
    scale: float = 1.0,
    key_mask: bool = False,
    e_layout: str = "qhk",
    generic: bool = False,
    with_lse: bool = True,
) -> Tuple[Tensor, Optional[Tensor], Tensor]:
    """Fused forward + tangents: returns ``(out, lse, tout)`` in one pass over K/V."""
    B, N, H, D = _check_primals(q, k, v, mask, e, e_layout)
    e_shape_ = e_shape(B, N, H, e_layout)
    batched = any(t is not None and t.dim() == 5 for t in (qt, kt, vt)) or (et is not None and et.dim() == 5)
    qt, kt, et, vt, T = _tangents(q, e_shape_, qt, kt, et, vt)
    q, k, v, e = _c(q), _c(k), _c(v), _c(e)
    m = _mask_u8(mask, q.device)
    out = torch.empty_like(q)
    lse = torch.empty((B, N, H), dtype=torch.float32, device=q.device) if with_lse else None
    tout = torch.empty((T, B, N, H, D), dtype=q.dtype, device=q.device)
    _native.check(
        _native.lib().hz_mhsea_fwd_jvp(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(e), _ptr(v), _ptr(m),
            _ptr(qt), _ptr(kt), _ptr(et), _ptr(vt), T, _ptr(out), _ptr(lse), _ptr(tout),
            B, N, H, D, _DTYPES[q.dtype], float(scale), _flags(key_mask, e_layout, generic),
        )
    )
    return out, lse, (tout if batched else tout[0])


def mhsea_fwd_jvp_gated(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Tensor,
    qt: Optional[Tensor] = None,
    kt: Optional[Tensor] = None,
    vt: Optional[Tensor] = None,
    e: Optional[Tensor] = None,
    et: Optional[Tensor] = None,
    *,
    scale: float = 1.0,
    key_mask: bool = False,
    e_layout: str = "qhk",
    generic: bool = False,
) -> Tuple[Tensor, Optional[Tensor]]:
    """Fused forward (+ tangents) with the trunk's sigmoid-gate head collapse in the epilogue
    (``trunk.py:134-137``): head h < H/2 gates head h + H/2. Returns ``(y, ty)`` with
    ``y = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:]`` of shape ``[B, N, H/2, D]`` and its
    forward-mode tangents (``[T, B, N, H/2, D]`` for batched tangents, ``[B, N, H/2, D]``
    for one, None when no tangent is given). Serves fp32, any N and head dimension, even H,
    at most two tangent directions (``generic`` forces the LDS-streaming kernel)."""
    B, N, H, D = _check_primals(q, k, v, mask, e, e_layout)
    if q.dtype != torch.float32:
        raise TypeError(f"the gated collapse computes in float32, got {q.dtype}")
    if H % 2:
        raise ValueError(f"the gated collapse pairs head h with h + H/2: H must be even, got {H}")
    e_shape_ = e_shape(B, N, H, e_layout)
    if all(t is None for t in (qt, kt, vt, et)):
        T, batched = 0, False
    else:
        batched = any(t is not None and t.dim() == 5 for t in (qt, kt, vt)) or (et is not None and et.dim() == 5)
        qt, kt, et, vt, T = _tangents(q, e_shape_, qt, kt, et, vt)
    q, k, v, e = _c(q), _c(k), _c(v), _c(e)
    m = _mask_u8(mask, q.device)
    y = torch.empty((B, N, H // 2, D), dtype=q.dtype, device=q.device)
    ty = torch.empty((T, B, N, H // 2, D), dtype=q.dtype, device=q.device) if T else None
    _native.check(
        _native.lib().hz_mhsea_fwd_jvp_gated(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(e), _ptr(v), _ptr(m),
            _ptr(qt), _ptr(kt), _ptr(et), _ptr(vt), T, _ptr(y), _ptr(ty),
            B, N, H, D, float(scale), _flags(key_mask, e_layout, generic),
        )
    )
    return y, (None if ty is None else (ty if batched else ty[0]))


def gated_out_proj(y: Tensor, w_o: Tensor, ty: Optional[Tensor] = None,
                   mask: Optional[Tensor] = None) -> Tuple[Tensor, Optional[Tensor]]:
    """The attention block's output projection after the gate collapse: ``delta = y_flat @
    w_o`` (the trunk's ``W_O``, ``trunk.py:138-144``), times the site mask when ``mask`` is
    given (the tree's ``mask_q * (out_flat @ w_o)``, ``tree.py:1479-1488``), and the same for
    each tangent row ``ty [T, ...]`` (or a single ``[...]`` direction). ``y`` is ``[B, N,
    H/2, D]`` (``mhsea_fwd_jvp_gated``'s output) or ``[B, N, d_attn]``; float32 CUDA tensors.
    With a mask, rows of masked sites are written as zeros without being read (equal to the
    product for finite ``y``), so only the physical rows cost matrix work."""
    if y.dim() not in (3, 4):
        raise ValueError(f"y must be [B, N, H/2, D] or [B, N, d_attn], got {tuple(y.shape)}")
    B, N = y.shape[0], y.shape[1]
    d_attn = y[0, 0].numel()
    if y.dtype != torch.float32 or w_o.dtype != torch.float32:
        raise TypeError("y and w_o must be float32")
    if not y.is_cuda:
        raise ValueError(f"y is on {y.device}: the projection needs GPU tensors")
    if w_o.dim() != 2 or w_o.shape[0] != d_attn:
        raise ValueError(f"w_o must be [{d_attn}, d_e], got {tuple(w_o.shape)}")
    _on_device(y.device, w_o=w_o, ty=ty, mask=mask)
    d_e = w_o.shape[1]
    y2, w = y.reshape(B, N, d_attn).contiguous(), w_o.contiguous()
    batched = ty is not None and ty.dim() == y.dim() + 1
    t = None if ty is None else (ty if batched else ty.unsqueeze(0))
    T = 0 if t is None else t.shape[0]
    if t is not None:
        if tuple(t.shape[1:]) != tuple(y.shape) or t.dtype != torch.float32:
            raise ValueError(f"ty must be [T, *{tuple(y.shape)}] float32, got {tuple(ty.shape)} {ty.dtype}")
        t = t.reshape(T, B, N, d_attn).contiguous()
    m = None
    if mask is not None:
        if tuple(mask.shape) != (B, N):
            raise ValueError(f"mask must be [B, N] = {(B, N)}, got {tuple(mask.shape)}")
        m = _mask_u8(mask, y.device)
    delta = torch.empty((B, N, d_e), dtype=torch.float32, device=y.device)
    delta_t = torch.empty((T, B, N, d_e), dtype=torch.float32, device=y.device) if T else None
    _native.check(_native.lib().hz_gated_out_proj(_stream(y.device), _ptr(y2), _ptr(t), _ptr(w), _ptr(m),
                                                  _ptr(delta), _ptr(delta_t), B, N, d_attn, d_e, T))
    return delta, (None if delta_t is None else (delta_t if batched else delta_t[0]))


def mhsea_bwd_gated(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Tensor,
    lse: Tensor,
    out: Tensor,
    dy: Tensor,
    e: Optional[Tensor] = None,
    *,
    want_de: bool = True,
    scale: float = 1.0,
    key_mask: bool = False,
    e_layout: str = "qhk",
) -> Tuple[Tensor, Tensor, Optional[Tensor], Tensor]:
    """Reverse mode of the gated head collapse: ``(dq, dk, de, dv)`` for the cotangent
    ``dy [B, N, H/2, D]`` of ``y = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:]``, given the
    attention's ``(out, lse)`` (``hz_mhsea_bwd_gated``: the collapse's cotangent formed on
    the GPU, then the attention backward). float32."""
    B, N, H, D = _check_primals(q, k, v, mask, e, e_layout)
    if q.dtype != torch.float32:
        raise TypeError(f"the gated collapse computes in float32, got {q.dtype}")
    if H % 2:
        raise ValueError(f"the gated collapse pairs head h with h + H/2: H must be even, got {H}")
    if tuple(out.shape) != (B, N, H, D) or tuple(dy.shape) != (B, N, H // 2, D) or tuple(lse.shape) != (B, N, H):
        raise ValueError("out must be [B, N, H, D], dy [B, N, H/2, D] and lse [B, N, H]")
    _on_device(q.device, lse=lse, out=out, dy=dy)
    q, k, v, e, lse, out, dy = _c(q), _c(k), _c(v), _c(e), _c(lse), _c(out), _c(dy)
    m = _mask_u8(mask, q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    de = torch.empty_like(e) if (want_de and e is not None) else None
    work = torch.empty_like(out)
    _native.check(
        _native.lib().hz_mhsea_bwd_gated(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(e), _ptr(v), _ptr(m), _ptr(lse), _ptr(out), _ptr(dy),
            _ptr(dq), _ptr(dk), _ptr(de), _ptr(dv), _ptr(work), B, N, H, D, float(scale),
            _flags(key_mask, e_layout, False),
        )
    )
    return dq, dk, de, dv


def mhsea_bwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    mask: Tensor,
    lse: Tensor,
    out: Tensor,
    dout: Tensor,
    e: Optional[Tensor] = None,
    *,
    want_de: bool = True,
    scale: float = 1.0,
    key_mask: bool = False,
    e_layout: str = "qhk",
    generic: bool = False,
) -> Tuple[Tensor, Tensor, Optional[Tensor], Tensor]:
    """Reverse mode: returns ``(dq, dk, de, dv)`` (de is None when not requested)."""
    B, N, H, D = _check_primals(q, k, v, mask, e, e_layout)
    for name, t in (("out", out), ("dout", dout)):
        if tuple(t.shape) != (B, N, H, D) or t.dtype != q.dtype:
            raise ValueError(f"{name} must match q in shape and dtype")
    if tuple(lse.shape) != (B, N, H) or lse.dtype != torch.float32:
        raise ValueError(f"lse must be float32 of shape {(B, N, H)}")
    _on_device(q.device, lse=lse, out=out, dout=dout)
    q, k, v, e, lse, out, dout = map(_c, (q, k, v, e, lse, out, dout))
    m = _mask_u8(mask, q.device)
    dq = torch.empty_like(q)
    dk = torch.empty_like(q)
    dv = torch.empty_like(q)
    e_shape_ = e_shape(B, N, H, e_layout)
    de = torch.empty(e_shape_, dtype=q.dtype, device=q.device) if want_de else None
    _native.check(
        _native.lib().hz_mhsea_bwd(
            _stream(q.device), _ptr(q), _ptr(k), _ptr(e), _ptr(v), _ptr(m), _ptr(lse), _ptr(out),
            _ptr(dout), _ptr(dq), _ptr(dk), _ptr(de), _ptr(dv),
            B, N, H, D, _DTYPES[q.dtype], float(scale), _flags(key_mask, e_layout, generic),
        )
    )
    return dq, dk, de, dv


def rect_attention_fwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    bias: Optional[Tensor] = None,
    key_mask: Optional[Tensor] = None,
    scale: float = 1.0,
    gated: bool = False,
) -> Tensor:
    """Rectangular attention with a dense pair bias (``hz_rect_attention_fwd``).

    ``q [B, Nq, H, D]``, ``k, v [B, Nk, H, D]``, ``bias [B, Nq, Nk, H]`` (None: zero),
    ``key_mask [B, Nk]`` (None: every key); float32. Returns ``out [B, Nq, H, D]`` of
    ``softmax_j(scale q.k + where(key_mask, bias, -1e30)) v``, or with ``gated`` only the
    head collapse ``y [B, Nq, H/2, D] = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:]``
    (``hz_rect_attention_fwd_gated``).
    """
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k and v must have rank 4 [B, N, H, D]")
    B, Nq, H, D = q.shape
    Nk = k.shape[1]
    for name, t in (("q", q), ("k", k), ("v", v), ("bias", bias)):
        if t is not None and t.dtype != torch.float32:
            raise TypeError(f"{name}.dtype must be float32, got {t.dtype}")
    if not q.is_cuda:
        raise ValueError("rectangular attention needs GPU tensors (q is on %s)" % q.device)
    if D not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head dimension must be one of {list(SUPPORTED_HEAD_DIMS)}, got {D}")
    if tuple(k.shape) != (B, Nk, H, D) or tuple(v.shape) != (B, Nk, H, D):
        raise ValueError(f"k and v must have shape {(B, Nk, H, D)}, got {tuple(k.shape)} and {tuple(v.shape)}")
    if bias is not None and tuple(bias.shape) != (B, Nq, Nk, H):
        raise ValueError(f"bias must have shape {(B, Nq, Nk, H)}, got {tuple(bias.shape)}")
    if key_mask is not None and tuple(key_mask.shape) != (B, Nk):
        raise ValueError(f"key_mask must have shape {(B, Nk)}, got {tuple(key_mask.shape)}")
    _on_device(q.device, k=k, v=v, bias=bias)
    q, k, v, bias = map(_c, (q, k, v, bias))
    if gated and H % 2 != 0:
        raise ValueError(f"the gated collapse pairs head h with h + H/2: H must be even, got {H}")
    m = None if key_mask is None else _mask_u8(key_mask, q.device)
    out = torch.empty((B, Nq, H // 2, D) if gated else (B, Nq, H, D), dtype=q.dtype, device=q.device)
    fn = _native.lib().hz_rect_attention_fwd_gated if gated else _native.lib().hz_rect_attention_fwd
    _native.check(
        fn(_stream(q.device), _ptr(q), _ptr(k), _ptr(v), _ptr(bias), _ptr(m), _ptr(out), B, Nq, Nk, H, D,
           float(scale))
    )
    return out
