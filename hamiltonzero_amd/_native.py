"""ctypes binding of ``libhz_mhsea.so`` (the C ABI declared in ``include/hz_mhsea.h``,
``include/hz_executor.h`` and ``include/hz_pair_bias.h``).

The library is the only compute path of this package: there is no CPU fallback. A
missing library raises :class:`NativeLibraryMissing` on first use.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libhz_mhsea.so"

HZ_DTYPE_F32 = 0
HZ_DTYPE_BF16 = 1
HZ_FLAG_KEY_MASK = 1
HZ_FLAG_E_QKH = 2
HZ_FLAG_GENERIC = 4
HZ_FLAG_E_COMPACT = 8
HZ_MAX_N = 16384

HZ_OK = 0
HZ_EINVAL = 1
HZ_ENULL = 2
HZ_EALIGN = 3
HZ_ELAUNCH = 4

# Every symbol the headers in include/ declare.
EXPORTED_SYMBOLS = (
    "hz_version",
    "hz_last_error",
    "hz_mhsea_fwd",
    "hz_mhsea_jvp",
    "hz_mhsea_fwd_jvp",
    "hz_mhsea_fwd_jvp_gated",
    "hz_mhsea_bwd",
    "hz_gated_out_proj",
    "hz_mhsea_bwd_gated",
    "hz_rect_attention_fwd",
    "hz_rect_attention_fwd_gated",
    "hz_quadrilinear_merge",
    "hz_factorized_apply",
    "hz_factorized_apply_noalloc",
    "hz_compiled_wavefunction_workspace",
    "hz_compiled_wavefunction",
    "hz_pair_bias",
    "hz_pair_mlp_bias",
)


class NativeLibraryMissing(RuntimeError):
    """libhz_mhsea.so has not been built (run ``python -m hamiltonzero_amd.build``)."""


class HzError(RuntimeError):
    """A non-zero status from the C ABI; ``code`` is the HZ_E* value."""

    def __init__(self, code: int, message: str):
        super().__init__(f"hz_mhsea error {code}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F = ctypes.c_float

_SIGNATURES = {
    "hz_version": ([], _INT),
    "hz_last_error": ([], ctypes.c_char_p),
    # stream, q, k, e, v, mask, out, lse, B, N, H, D, dtype, scale, flags
    "hz_mhsea_fwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _F, _INT], _INT),
    # stream, q, k, e, v, mask, out, lse, qt, kt, et, vt, T, tout, B, N, H, D, dtype, scale, flags
    "hz_mhsea_jvp": (
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _INT, _F, _INT],
        _INT,
    ),
    # stream, q, k, e, v, mask, qt, kt, et, vt, T, out, lse, tout, B, N, H, D, dtype, scale, flags
    "hz_mhsea_fwd_jvp": (
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _F, _INT],
        _INT,
    ),
    # stream, q, k, e, v, mask, qt, kt, et, vt, T, y, ty, B, N, H, D, scale, flags
    "hz_mhsea_fwd_jvp_gated": (
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _F, _INT],
        _INT,
    ),
    # stream, q, k, e, v, mask, lse, out, dout, dq, dk, de, dv, B, N, H, D, dtype, scale, flags
    "hz_mhsea_bwd": (
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _F, _INT],
        _INT,
    ),
    # stream, q, k, v, bias, key_mask, out, B, Nq, Nk, H, D, scale
    "hz_rect_attention_fwd": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F], _INT),
    # stream, q, k, v, bias, key_mask, y, B, Nq, Nk, H, D, scale
    "hz_rect_attention_fwd_gated": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F], _INT),
    # stream, T, u_a, u_b, out, M, G, R
    "hz_quadrilinear_merge": ([_P, _P, _P, _P, _P, _I64, _I64, _I64], _INT),
    # stream, x, V, h, U, residual, y, workspace, M, d_in, R, d_out, h_rows
    "hz_factorized_apply": ([_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64], _INT),
    "hz_factorized_apply_noalloc": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64], _INT),
    # stream, y, ty, w_o, mask, delta, delta_t, B, N, d_attn, d_e, T
    "hz_gated_out_proj": ([_P] * 7 + [_I64] * 5, _INT),
    # stream, q, k, e, v, mask, lse, out, dy, dq, dk, de, dv, dout_work, B, N, H, D, scale, flags
    "hz_mhsea_bwd_gated": ([_P] * 14 + [_I64] * 4 + [_F, _INT], _INT),
    # B, n_sites, d_z, R_leaf, d_m, R_merge, R_out
    "hz_compiled_wavefunction_workspace": ([_I64] * 7, _I64),
    # stream, q, q_weight, leaf_V, leaf_U, leaf_h, merge_T, merge_V, merge_U, merge_h, opcodes,
    # readout_V, readout_U, readout_h, log_abs, phase, workspace, workspace_bytes,
    # B, n_sites, d_q, d_z, R_leaf, G, d_r, R_merge, R_out, merge_eps
    "hz_compiled_wavefunction": ([_P] * 17 + [_I64] * 10 + [_F], _INT),
    # stream, edge, edge_t, mask, ln_w, w_in, b_in, w_1, b_1, w_2, b_2, w_out, b_out, e, e_t,
    # B, N, C, hidden, H, T, inner_gain, eps, bias_div, flags
    "hz_pair_bias": ([_P] * 15 + [_I64] * 6 + [_F, _F, _F, _INT], _INT),
    # stream, edge, edge_t, extra, extra_t, mask, w_in, b_in, norm_w, w_1, b_1, w_2, b_2,
    # out_norm_w, w_out, b_out, alibi_slopes, e, e_t, B, Nq, Nk, C, hidden, H, n_blocks, T,
    # row_offset, inner_gain, eps, bias_div, flags
    "hz_pair_mlp_bias": ([_P] * 19 + [_I64] * 9 + [_F, _F, _F, _INT], _INT),
}


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library, with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryMissing(
                    f"{LIB_PATH} is missing: build it with `python -m hamiltonzero_amd.build`"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (argtypes, restype) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = handle
    return _lib


def check(status: int) -> None:
    """Raise :class:`HzError` for a non-zero status, with the library's message."""
    if status != HZ_OK:
        msg = lib().hz_last_error()
        raise HzError(status, msg.decode() if msg else "")


def version() -> int:
    return int(lib().hz_version())
