"""MI355X (gfx950) implementation of HamiltonZero's MHSEA attention hot path.

Public surface, named after the reference modules it replaces:

* :mod:`hamiltonzero_amd.edge_attention` — ``mhsea_tuned_edge_attention`` and
  ``reference_edge_attention`` (``src/hamiltonzero/model/pallas_attention.py``).
* :mod:`hamiltonzero_amd.mhsea_tuned` — ``mhsea_with_tuned_ad`` and the primitive pair
  (``src/hamiltonzero/model/_pallas_attn/mhsea_tuned.py``), and ``gated_edge_attention``,
  the attention call with the trunk's sigmoid-gate head collapse fused
  (``src/hamiltonzero/model/trunk.py``).
* :mod:`hamiltonzero_amd.rect_attention` — ``noncausal_bias_mha`` and
  ``pallas_rectangular_edge_attention`` (``src/hamiltonzero/evaluation/pallas_mha.py``,
  ``src/hamiltonzero/evaluation/sequence_parallel.py``), the large-N evaluation forward, and
  the large-N caller's head collapse fused into it (``gated_rectangular_edge_attention``,
  ``sequence_attention_output``: ``src/hamiltonzero/evaluation/sequence_trunk.py``).
* :mod:`hamiltonzero_amd.kernels` — tensor-level calls of the C ABI
  (``include/hz_mhsea.h``): forward, tangent, fused forward+tangent, backward,
  gated forward+tangent, rectangular forward.
"""

from .edge_attention import mhsea_tuned_edge_attention, reference_edge_attention
from .mhsea_tuned import (
    gated_edge_attention,
    mhsea_ad,
    mhsea_tuned_ad,
    mhsea_tuned_ad_lin,
    mhsea_tuned_ad_lin_transpose,
    mhsea_tuned_jvp,
    mhsea_with_tuned_ad,
)
from .rect_attention import (
    BlockSizes,
    gated_rectangular_edge_attention,
    noncausal_bias_mha,
    pallas_rectangular_edge_attention,
    sequence_attention_output,
)

__all__ = [
    "BlockSizes",
    "gated_edge_attention",
    "gated_rectangular_edge_attention",
    "mhsea_ad",
    "mhsea_tuned_ad",
    "mhsea_tuned_ad_lin",
    "mhsea_tuned_ad_lin_transpose",
    "mhsea_tuned_edge_attention",
    "mhsea_tuned_jvp",
    "mhsea_with_tuned_ad",
    "noncausal_bias_mha",
    "pallas_rectangular_edge_attention",
    "reference_edge_attention",
    "sequence_attention_output",
]
