"""CPU oracle of the reference's rectangular large-N attention — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
use this module, and only as the checker / the timed CPU baseline. The product
(``hamiltonzero_amd``) never imports it.

A float64 numpy restatement of the reference's forward-only evaluation attention (paths
relative to ``src/hamiltonzero/evaluation/``):

* ``noncausal_bias_mha(q, k, v, bias)`` (``pallas_mha.py:92-161``, kernel ``:43-89``):
  ``softmax_j(q_i . k_j + bias[i, j, h]) v_j`` per batch element and head, computed there
  as an online softmax in base 2 over key blocks (``:64-89``), which is the same function.
  Layouts ``q [B, Nq, H, D]``, ``k, v [B, Nk, H, D]``, ``bias [B, Nq, Nk, H]`` (``:111``).
* ``pallas_rectangular_edge_attention(q, k, v, bias, key_mask)``
  (``sequence_parallel.py:59-90``): masked keys get the bias ``-1e30`` (``:79-83``) and q
  is pre-scaled by ``D**-0.5`` (``:72,85``); one system ``[n, h, d]`` at a time.

The -1e30 replacement is applied literally (not by dropping keys), so the all-masked case
follows from the arithmetic: every score equals -1e30 in float32, and the result is the
mean of all value rows. ``rect_fwd`` evaluates that case at that precision (float64 would
keep the differences of q.k under -1e30 that float32 rounds away).

How it is pinned (tests/test_rect_oracle.py): explicit loops on tiny inputs; Nk = 1
(out = v); a dominant bias (out = that key's value row); zero scores (mean of physical
values); the all-masked mean; equality with the already-pinned square oracle
(``mhsea_oracle.fwd`` with the additive key mask and the ``[n, n, h]`` bias) when Nq = Nk;
the sequence-parallel identity (a block of query rows of the square problem equals the
rectangular problem on that block); invariance under a permutation of the keys and under
any finite change of masked keys' k and v and any change (NaN included) of their bias. Planted mistakes (bias read
transposed, mask ignored, scale on k only) fail these checks. ``rect_gated`` and
``sequence_attention_output`` compose ``rect_fwd`` with ``mhsea_oracle.gate_collapse`` and
``mhsea_oracle.out_proj`` (pinned in tests/test_gated_oracle.py); tests/test_rect_oracle.py
checks the composition against element loops, including the head pairing.
"""

from __future__ import annotations

import numpy as np

MASKED_BIAS = -1.0e30  # sequence_parallel.py:82


def rect_fwd(q, k, v, bias=None, key_mask=None, *, scale=1.0):
    """out [B, Nq, H, D] of noncausal_bias_mha((q * scale), k, v, where(mask, bias, -1e30)).

    ``key_mask`` [B, Nk] (None: every key). ``bias`` None means zero.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Nq, H, _D = q.shape
    Nk = k.shape[1]
    e = np.zeros((B, Nq, Nk, H)) if bias is None else np.asarray(bias, dtype=np.float64)
    if key_mask is None:
        key_mask = np.ones((B, Nk), dtype=bool)
    key_mask = np.asarray(key_mask, dtype=bool)
    # where(mask, bias, -1e30), sequence_parallel.py:79-83 (NaN bias of masked keys drops out)
    e = np.where(key_mask[:, None, :, None], e, MASKED_BIAS)
    # logits [B, H, Nq, Nk] = (q * scale) k^T + bias, pallas_mha.py:68-70
    s = np.einsum("bihd,bjhd->bhij", q * scale, k) + e.transpose(0, 3, 1, 2)
    all_masked = ~key_mask.any(axis=1)
    if all_masked.any():
        # float32 rounds q.k - 1e30 to -1e30 exactly: every weight of the row is equal.
        s[all_masked] = MASKED_BIAS
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    p /= p.sum(axis=-1, keepdims=True)
    # masked keys have weight exp(-1e30 - m) = 0 (as in the reference, a non-finite k or v
    # of a masked key would still propagate through q.k and 0 * v)
    return np.einsum("bhij,bjhd->bihd", p, v)


def rect_gated(q, k, v, bias=None, key_mask=None, *, scale=1.0):
    """y [B, Nq, H/2, D]: the large-N caller's head collapse after the rectangular attention,
    ``sigmoid(out[:, :, :H/2]) * out[:, :, H/2:]`` (``sequence_trunk.py:973-981``; the
    kernel's H is twice the module's n_heads), with ``out`` from :func:`rect_fwd`."""
    from .mhsea_oracle import gate_collapse

    return gate_collapse(rect_fwd(q, k, v, bias, key_mask, scale=scale))


def sequence_attention_output(q, k, v, bias, key_mask, w_o, row_mask, *, scale=1.0):
    """``row_mask[:, None] * (y.reshape(r, -1) @ w_o)`` per system (``sequence_trunk.py:
    982-984``), y from :func:`rect_gated`. w_o [H/2 * D, d_c], row_mask [B, Nq]."""
    from .mhsea_oracle import out_proj

    return out_proj(rect_gated(q, k, v, bias, key_mask, scale=scale), w_o, row_mask)


def rect_fwd_loops(q, k, v, bias, key_mask, *, scale=1.0):
    """Element-by-element restatement of ``rect_fwd`` for tiny inputs (independent code)."""
    import math

    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Nq, H, D = q.shape
    Nk = k.shape[1]
    out = np.zeros((B, Nq, H, D))
    for b in range(B):
        any_key = any(bool(key_mask[b][j]) for j in range(Nk))
        for h in range(H):
            for i in range(Nq):
                logits = []
                for j in range(Nk):
                    if not any_key:
                        logits.append(0.0)
                    elif not key_mask[b][j]:
                        logits.append(-math.inf)
                    else:
                        dot = sum(q[b, i, h, d] * scale * k[b, j, h, d] for d in range(D))
                        logits.append(dot + (0.0 if bias is None else float(bias[b, i, j, h])))
                mx = max(logits)
                w = [math.exp(x - mx) for x in logits]
                tot = sum(w)
                for d in range(D):
                    out[b, i, h, d] = sum(w[j] * v[b, j, h, d] for j in range(Nk) if w[j] > 0.0) / tot
    return out
