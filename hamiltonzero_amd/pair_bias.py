"""The attention coupling-bias producers on the gfx950 library (torch mirror): the trunk's
(``coupling_bias``) and the MLP-class one of the tree, readout and large-N callers
(``mlp_bias``, with the LCA-ALiBi term).

Reference: ``MultiHeadEvenAttention.__call__`` (``src/hamiltonzero/model/trunk.py:89-105``)::

    edge_pre  = self.ln_edge(edge)                       # _RMS, odd_ops.py:183-215
    coup_bias = self.bias_mlp(edge_pre)                  # UnnormalizedMLP, odd_ops.py:279-316
    coup_bias = coup_bias / sqrt(d_head)

``coupling_bias`` runs all three in one launch of ``hz_pair_bias`` (``include/hz_pair_bias.h``)
and writes the result straight into the attention's bias layout (``[B, N, H, N]``, the
reference's ``[B, N, N, H]`` with ``e_layout="qkh"``, or the compacted physical-pair layout
that the N <= 64 attention kernel reads most cheaply, ``e_layout="compact"``:
``kernels.compact_bias``), with the forward-mode tangent along ``edge_t`` when given. There is no CPU fallback: the HIP library is required and every
operand must be a float32 CUDA tensor on one device.

Parameters use the reference's names, flattened: ``ln_w`` (``ln_edge.weight``), ``w_in`` /
``b_in`` (``bias_mlp.in_proj``), ``w_1`` / ``b_1`` and ``w_2`` / ``b_2``
(``bias_mlp.block_l1s[0]`` / ``block_l2s[0]``), ``w_out`` / ``b_out``
(``bias_mlp.out_proj``); weights are ``[in, out]`` as in ``Linear`` (``odd_ops.py:78-87``).
"""

from __future__ import annotations

from typing import Mapping, Optional, Tuple, Union

import torch

from . import _native, kernels

Tensor = torch.Tensor

PARAM_NAMES = ("ln_w", "w_in", "b_in", "w_1", "b_1", "w_2", "b_2", "w_out", "b_out")
EDGE_CHANNELS = (32, 64, 96, 128)
HIDDEN = 64
HEADS = (16, 32, 64)


def _check(name: str, t: Tensor, device: torch.device, shape) -> Tensor:
    if t.dtype != torch.float32:
        raise TypeError(f"{name}.dtype must be float32, got {t.dtype}")
    if not t.is_cuda or t.device != device:
        raise ValueError(f"{name} is on {t.device}: every operand must be on {device}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t.contiguous()


def coupling_bias(
    edge: Tensor,
    params: Mapping[str, Tensor],
    *,
    d_head: int,
    inner_gain: float,
    mask: Optional[Tensor] = None,
    key_mask: bool = False,
    e_layout: str = "qhk",
    eps: float = 1e-5,
    edge_t: Optional[Tensor] = None,
) -> Union[Tensor, Tuple[Tensor, Tensor]]:
    """``bias_mlp(ln_edge(edge)) / sqrt(d_head)`` for ``edge [B, N, N, C]``.

    Returns ``e`` in the attention layout, or ``(e, e_t)`` when ``edge_t`` (``[B, N, N, C]``
    or ``[T, B, N, N, C]``) is given, ``e_t`` then ``[T, <layout of e>]`` (or without the T
    axis for a single direction). ``inner_gain`` is the MLP's ``n_layers ** -0.5``
    (``trunk.py:61``). With ``mask [B, N]`` only the pairs the attention reads are computed
    (see ``include/hz_pair_bias.h``; ``key_mask`` as in the attention call) and the others
    are zero. ``e_layout="compact"`` (square mask only) writes the layout of
    ``kernels.compact_bias``.
    """
    if edge.dim() != 4 or edge.shape[1] != edge.shape[2]:
        raise ValueError(f"edge must be [B, N, N, C], got {tuple(edge.shape)}")
    if e_layout not in kernels.E_LAYOUTS:
        raise ValueError(f"e_layout must be one of {list(kernels.E_LAYOUTS)}, got {e_layout!r}")
    if e_layout == "compact" and key_mask:
        raise ValueError("e_layout='compact' serves the square mask only (key_mask=False)")
    B, N, _, C = edge.shape
    if C not in EDGE_CHANNELS:
        raise ValueError(f"edge channels must be one of {list(EDGE_CHANNELS)}, got {C}")
    dev = edge.device
    edge = _check("edge", edge, dev, edge.shape)
    H = params["w_out"].shape[-1]
    if H not in HEADS:
        raise ValueError(f"heads (w_out's output width) must be one of {list(HEADS)}, got {H}")
    shapes = {"ln_w": (C,), "w_in": (C, HIDDEN), "b_in": (HIDDEN,), "w_1": (HIDDEN, HIDDEN), "b_1": (HIDDEN,),
              "w_2": (HIDDEN, HIDDEN), "b_2": (HIDDEN,), "w_out": (HIDDEN, H), "b_out": (H,)}
    p = {n: _check(n, params[n], dev, shapes[n]) for n in PARAM_NAMES}
    m = None
    if mask is not None:
        if tuple(mask.shape) != (B, N):
            raise ValueError(f"mask must be [B, N] = {(B, N)}, got {tuple(mask.shape)}")
        if not mask.is_cuda or mask.device != dev:
            raise ValueError(f"mask is on {mask.device}: every operand must be on {dev}")
        m = (mask != 0).to(torch.uint8).contiguous()
    tangents = None
    single = False
    if edge_t is not None:
        single = edge_t.dim() == 4
        tangents = edge_t.unsqueeze(0) if single else edge_t
        tangents = _check("edge_t", tangents, dev, (tangents.shape[0], B, N, N, C))
    eshape = kernels.e_shape(B, N, H, e_layout)
    alloc = torch.zeros if m is not None else torch.empty
    e = alloc(eshape, dtype=torch.float32, device=dev)
    T = 0 if tangents is None else tangents.shape[0]
    e_t = alloc((T, *eshape), dtype=torch.float32, device=dev) if T else None
    flags = kernels._flags(key_mask, e_layout)
    lib = _native.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    div = float(torch.sqrt(torch.tensor(float(d_head), dtype=torch.float32)))  # jnp.sqrt in float32
    for t in range(max(T, 1)):
        _native.check(lib.hz_pair_bias(
            stream, edge.data_ptr(), None if T == 0 else tangents[t].data_ptr(), None if m is None else m.data_ptr(),
            *(p[n].data_ptr() for n in PARAM_NAMES), e.data_ptr(), None if T == 0 else e_t[t].data_ptr(),
            B, N, C, HIDDEN, H, 1 if T else 0, float(inner_gain), float(eps), div, flags))
    if T == 0:
        return e
    return e, (e_t[0] if single else e_t)


MLP_PARAM_NAMES = ("w_in", "b_in", "norm_w", "w_1", "b_1", "w_2", "b_2", "out_norm_w", "w_out", "b_out")
MLP_HIDDEN = (32, 64, 128)
MLP_HEADS = (16, 32)


def lca_fixed_slopes(n_heads: int, device=None) -> Tensor:
    """``lca_fixed_slopes`` (``src/hamiltonzero/model/readout_leaf_context.py:166-169``):
    ``1.5 * 2^(-4 h / max(H - 1, 1))`` in float32."""
    head = torch.arange(n_heads, dtype=torch.float32, device=device)
    den = torch.clamp(torch.tensor(float(n_heads - 1), dtype=torch.float32, device=device), min=1.0)
    return 1.5 * torch.exp2(-(head * 4.0 / den))


def mlp_bias(
    edge: Tensor,
    params: Mapping[str, Tensor],
    *,
    d_head: int,
    inner_gain: float = 1.0,
    extra: Optional[Tensor] = None,
    alibi_slopes: Optional[Tensor] = None,
    row_offset: int = 0,
    mask: Optional[Tensor] = None,
    key_mask: bool = False,
    e_layout: str = "qkh",
    eps: float = 1e-5,
    edge_t: Optional[Tensor] = None,
    extra_t: Optional[Tensor] = None,
) -> Union[Tensor, Tuple[Tensor, Tensor]]:
    """The MLP-class coupling bias with the LCA-ALiBi term (``hz_pair_mlp_bias``,
    ``include/hz_pair_bias.h``): ``bias_mlp(x) / sqrt(d_head) - slope_h * lca(row_offset + i,
    j)`` for ``edge [B, Nq, Nk, C]`` — the tree's LevelEdgeAttn (``model/tree.py:1392-1456``,
    ``alibi_slopes = lca_fixed_slopes(H)`` when it passes a level, else None), the readout
    context (``model/readout_leaf_context.py:694-712``: ``extra`` = the direction channel
    concatenated to ``edge_n``, ``w_in`` with C + 1 rows) and the large-N trunk
    (``evaluation/sequence_trunk.py:962-972``: ``row_offset`` = the first local row's global
    index). ``params`` follow the reference's ``MLP`` (``odd_ops.py:218-276``), per block
    stacked: ``norm_w [n_blocks, hidden]`` (``block_norms[k].weight``), ``w_1`` / ``w_2``
    ``[n_blocks, hidden, hidden]``, ``b_1`` / ``b_2`` ``[n_blocks, hidden]``; ``out_norm_w``
    (``out_norm.weight``); weights ``[in, out]``. Returns ``e`` in ``e_layout`` (``"qkh"``:
    ``[B, Nq, Nk, H]``, the reference's and the rectangular attention's; ``"qhk"``: ``[B, Nq,
    H, Nk]``), or ``(e, e_t)`` with ``edge_t`` (and ``extra_t``) given. With ``mask [B, Nk]``
    only the pairs the attention reads are computed, the others are zero."""
    if edge.dim() != 4:
        raise ValueError(f"edge must be [B, Nq, Nk, C], got {tuple(edge.shape)}")
    if e_layout not in ("qhk", "qkh"):
        raise ValueError(f"e_layout must be 'qhk' or 'qkh', got {e_layout!r}")
    B, Nq, Nk, C = edge.shape
    if C not in EDGE_CHANNELS:
        raise ValueError(f"edge channels must be one of {list(EDGE_CHANNELS)}, got {C}")
    dev = edge.device
    edge = _check("edge", edge, dev, edge.shape)
    hidden = params["w_in"].shape[-1]
    if hidden not in MLP_HIDDEN:
        raise ValueError(f"hidden width must be one of {list(MLP_HIDDEN)}, got {hidden}")
    H = params["w_out"].shape[-1]
    if H not in MLP_HEADS:
        raise ValueError(f"heads (w_out's output width) must be one of {list(MLP_HEADS)}, got {H}")
    nb = params["w_1"].shape[0]
    cin = C + (1 if extra is not None else 0)
    shapes = {"w_in": (cin, hidden), "b_in": (hidden,), "norm_w": (nb, hidden), "w_1": (nb, hidden, hidden),
              "b_1": (nb, hidden), "w_2": (nb, hidden, hidden), "b_2": (nb, hidden), "out_norm_w": (hidden,),
              "w_out": (hidden, H), "b_out": (H,)}
    p = {n: _check(n, params[n], dev, shapes[n]) for n in MLP_PARAM_NAMES}
    ex = None if extra is None else _check("extra", extra, dev, (B, Nq, Nk))
    sl = None if alibi_slopes is None else _check("alibi_slopes", alibi_slopes, dev, (H,))
    m = None
    if mask is not None:
        if tuple(mask.shape) != (B, Nk):
            raise ValueError(f"mask must be [B, Nk] = {(B, Nk)}, got {tuple(mask.shape)}")
        if not mask.is_cuda or mask.device != dev:
            raise ValueError(f"mask is on {mask.device}: every operand must be on {dev}")
        m = (mask != 0).to(torch.uint8).contiguous()
    T = 0
    if edge_t is not None:
        T = 1
        edge_t = _check("edge_t", edge_t, dev, edge.shape)
        if ex is not None:
            extra_t = torch.zeros_like(ex) if extra_t is None else _check("extra_t", extra_t, dev, (B, Nq, Nk))
    eshape = (B, Nq, H, Nk) if e_layout == "qhk" else (B, Nq, Nk, H)
    alloc = torch.zeros if m is not None else torch.empty
    e = alloc(eshape, dtype=torch.float32, device=dev)
    e_t = alloc(eshape, dtype=torch.float32, device=dev) if T else None
    flags = (_native.HZ_FLAG_KEY_MASK if key_mask else 0) | (_native.HZ_FLAG_E_QKH if e_layout == "qkh" else 0)
    div = float(torch.sqrt(torch.tensor(float(d_head), dtype=torch.float32)))  # jnp.sqrt in float32
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    _native.check(_native.lib().hz_pair_mlp_bias(
        torch.cuda.current_stream(dev).cuda_stream, edge.data_ptr(), ptr(edge_t), ptr(ex),
        ptr(extra_t) if T else None, ptr(m), *(p[n].data_ptr() for n in MLP_PARAM_NAMES), ptr(sl), e.data_ptr(),
        ptr(e_t), B, Nq, Nk, C, hidden, H, nb, T, int(row_offset), float(inner_gain), float(eps), div, flags))
    return e if T == 0 else (e, e_t)


def inner_gain_for(n_layers: int) -> float:
    """``float(n_layers) ** (-0.5)`` (``trunk.py:61``)."""
    return float(n_layers) ** (-0.5)


__all__ = ["coupling_bias", "inner_gain_for", "lca_fixed_slopes", "mlp_bias", "MLP_PARAM_NAMES", "PARAM_NAMES"]
