"""C-ABI checks that need no GPU: the library loads, exports every symbol the header
declares, and rejects invalid arguments on the host before any GPU work."""

import ctypes
import re
from pathlib import Path

import pytest

from hamiltonzero_amd import _native

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def header_functions():
    text = "\n".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(hz_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        pytest.skip("libhz_mhsea.so not built (run python -m hamiltonzero_amd.build)")
    return _native.lib()


def test_header_and_binding_agree():
    assert header_functions() == sorted(_native.EXPORTED_SYMBOLS)


def test_exports_every_declared_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name
    assert _native.version() == 100


# Fake, 256-byte aligned device addresses: every call below must fail validation on the
# host and return before touching them.
A = 0x10000


def _fwd(lib, **over):
    args = dict(stream=None, q=A, k=A, e=None, v=A, mask=A, out=A, lse=None, B=2, N=64, H=8, D=32,
                dtype=0, scale=1.0, flags=0)
    args.update(over)
    return lib.hz_mhsea_fwd(*args.values())


@pytest.mark.parametrize(
    "over,code,needle",
    [
        (dict(D=24), _native.HZ_EINVAL, "head dimension"),
        (dict(D=128), _native.HZ_EINVAL, "head dimension"),
        (dict(N=0), _native.HZ_EINVAL, "N must be"),
        (dict(N=_native.HZ_MAX_N + 1), _native.HZ_EINVAL, "N must be"),
        (dict(B=0), _native.HZ_EINVAL, "B and H"),
        (dict(dtype=7), _native.HZ_EINVAL, "dtype"),
        (dict(flags=16), _native.HZ_EINVAL, "flag"),
        (dict(q=None), _native.HZ_ENULL, "q must not be NULL"),
        (dict(mask=None), _native.HZ_ENULL, "mask"),
        (dict(out=None), _native.HZ_ENULL, "out"),
        (dict(v=A + 4), _native.HZ_EALIGN, "aligned"),
        (dict(scale=float("nan")), _native.HZ_EINVAL, "scale"),
        # the compacted bias layout: square mask, float32, the N <= 64 kernel's shapes
        (dict(flags=8 | 1), _native.HZ_EINVAL, "excludes HZ_FLAG_KEY_MASK"),
        (dict(flags=8 | 2), _native.HZ_EINVAL, "excludes"),
        (dict(flags=8 | 4), _native.HZ_EINVAL, "excludes"),
        (dict(flags=8, D=64), _native.HZ_EINVAL, "HZ_FLAG_E_COMPACT needs"),
        (dict(flags=8, N=65), _native.HZ_EINVAL, "HZ_FLAG_E_COMPACT needs"),
        (dict(flags=8, dtype=1), _native.HZ_EINVAL, "HZ_FLAG_E_COMPACT needs"),
    ],
)
def test_fwd_rejects_bad_arguments(lib, over, code, needle):
    assert _fwd(lib, **over) == code
    assert needle in lib.hz_last_error().decode()


def test_jvp_rejects_bad_tangent_count(lib):
    rc = lib.hz_mhsea_jvp(None, A, A, None, A, A, A, A, None, None, None, None, 0, A,
                          2, 64, 8, 32, 0, 1.0, 0)
    assert rc == _native.HZ_EINVAL
    assert "T must be" in lib.hz_last_error().decode()
    rc = lib.hz_mhsea_fwd_jvp(None, A, A, None, A, A, None, None, None, None, 1, A, None, None,
                              2, 64, 8, 32, 0, 1.0, 0)
    assert rc == _native.HZ_ENULL and "tout" in lib.hz_last_error().decode()


def test_jvp_requires_primal_outputs(lib):
    rc = lib.hz_mhsea_jvp(None, A, A, None, A, A, A, None, None, None, None, None, 1, A,
                          2, 64, 8, 32, 0, 1.0, 0)
    assert rc == _native.HZ_ENULL and "lse" in lib.hz_last_error().decode()


def test_bwd_rejects_missing_cotangent_outputs(lib):
    rc = lib.hz_mhsea_bwd(None, A, A, None, A, A, A, A, A, A, None, None, A, 2, 64, 8, 32, 0, 1.0, 0)
    assert rc == _native.HZ_ENULL and "dk" in lib.hz_last_error().decode()
    rc = lib.hz_mhsea_bwd(None, A, A, None, A, A, A, A, A, A, A, A + 8, A, 2, 64, 8, 32, 0, 1.0, 0)
    assert rc == _native.HZ_EALIGN and "de" in lib.hz_last_error().decode()


def test_compact_bias_layout_is_refused_outside_the_forward_family(lib):
    rc = lib.hz_mhsea_bwd(None, A, A, A, A, A, A, A, A, A, A, A, A, 2, 64, 8, 32, 0, 1.0, 8)
    assert rc == _native.HZ_EINVAL and "forward family" in lib.hz_last_error().decode()
    # stream, edge, edge_t, mask, ln_w, w_in, b_in, w_1, b_1, w_2, b_2, w_out, b_out, e, e_t,
    # B, N, C, hidden, H, T, inner_gain, eps, bias_div, flags
    pb = [None] + [A] * 14 + [2, 64, 96, 64, 32, 1, 0.5, 1e-5, 4.0]
    assert lib.hz_pair_bias(*pb, 8 | 1) == _native.HZ_EINVAL
    assert "excludes HZ_FLAG_KEY_MASK" in lib.hz_last_error().decode()
    pb_large = [None] + [A] * 14 + [2, 300, 96, 64, 32, 1, 0.5, 1e-5, 4.0]
    assert lib.hz_pair_bias(*pb_large, 8) == _native.HZ_EINVAL
    assert "N <= 256" in lib.hz_last_error().decode()


def test_error_string_is_thread_local(lib):
    import threading

    assert _fwd(lib, D=24) == _native.HZ_EINVAL
    seen = {}

    def other():
        seen["msg"] = lib.hz_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "head dimension" in lib.hz_last_error().decode()


def test_check_raises_hz_error(lib):
    assert _fwd(lib, D=24) == _native.HZ_EINVAL
    with pytest.raises(_native.HzError) as err:
        _native.check(_native.HZ_EINVAL)
    assert err.value.code == _native.HZ_EINVAL


def test_signatures_declared(lib):
    assert lib.hz_mhsea_fwd.restype is ctypes.c_int
    assert len(lib.hz_mhsea_jvp.argtypes) == 21
    assert len(lib.hz_mhsea_fwd_jvp.argtypes) == 21
    assert len(lib.hz_mhsea_bwd.argtypes) == 20


def test_rect_rejects_bad_arguments(lib):
    # stream, q, k, v, bias, key_mask, out, B, Nq, Nk, H, D, scale
    base = [None, A, A, A, None, None, A, 1, 256, 1024, 16, 64, 0.125]

    def call(**over):
        args = list(base)
        names = ["stream", "q", "k", "v", "bias", "key_mask", "out", "B", "Nq", "Nk", "H", "D", "scale"]
        for key, val in over.items():
            args[names.index(key)] = val
        return lib.hz_rect_attention_fwd(*args)

    cases = [
        (dict(D=24), _native.HZ_EINVAL, "head dimension"),
        (dict(Nq=0), _native.HZ_EINVAL, "positive"),
        (dict(Nk=0), _native.HZ_EINVAL, "positive"),
        (dict(Nk=_native.HZ_MAX_N + 1), _native.HZ_EINVAL, "Nk must be"),
        (dict(H=0), _native.HZ_EINVAL, "B and H"),
        (dict(q=None), _native.HZ_ENULL, "q must not be NULL"),
        (dict(out=None), _native.HZ_ENULL, "out"),
        (dict(bias=A + 4), _native.HZ_EALIGN, "bias"),
        (dict(scale=float("inf")), _native.HZ_EINVAL, "scale"),
    ]
    for over, code, needle in cases:
        assert call(**over) == code, over
        assert needle in lib.hz_last_error().decode(), over
    assert len(lib.hz_rect_attention_fwd.argtypes) == 13
    # the gated variant: the same checks, and an even head count
    gated = lib.hz_rect_attention_fwd_gated
    assert len(gated.argtypes) == 13
    for over, code, needle in cases + [(dict(H=15), _native.HZ_EINVAL, "H must be even")]:
        args = list(base)
        names = ["stream", "q", "k", "v", "bias", "key_mask", "out", "B", "Nq", "Nk", "H", "D", "scale"]
        for key, val in over.items():
            args[names.index(key)] = val
        assert gated(*args) == code, over
        assert needle in lib.hz_last_error().decode(), over


def test_gated_rejects_bad_arguments(lib):
    # stream, q, k, e, v, mask, qt, kt, et, vt, T, y, ty, B, N, H, D, scale, flags
    names = ["stream", "q", "k", "e", "v", "mask", "qt", "kt", "et", "vt", "T", "y", "ty",
             "B", "N", "H", "D", "scale", "flags"]
    base = [None, A, A, None, A, A, None, None, None, None, 1, A, A, 2, 64, 8, 32, 0.125, 0]

    def call(**over):
        args = list(base)
        for key, val in over.items():
            args[names.index(key)] = val
        return lib.hz_mhsea_fwd_jvp_gated(*args)

    cases = [
        (dict(H=7), _native.HZ_EINVAL, "H must be even"),
        (dict(T=3), _native.HZ_EINVAL, "T must be in [0, 2]"),
        (dict(N=0), _native.HZ_EINVAL, "N must be"),
        (dict(N=_native.HZ_MAX_N + 1), _native.HZ_EINVAL, "N must be"),
        (dict(D=24), _native.HZ_EINVAL, "head dimension"),
        (dict(flags=16), _native.HZ_EINVAL, "flag"),
        (dict(y=None), _native.HZ_ENULL, "y must not be NULL"),
        (dict(ty=None), _native.HZ_ENULL, "ty must not be NULL"),
        (dict(qt=A + 4), _native.HZ_EALIGN, "qt"),
        (dict(scale=float("nan")), _native.HZ_EINVAL, "scale"),
    ]
    for over, code, needle in cases:
        assert call(**over) == code, over
        assert needle in lib.hz_last_error().decode(), over
    assert len(lib.hz_mhsea_fwd_jvp_gated.argtypes) == 19


def test_executor_entries_reject_bad_arguments(lib):
    qm = lib.hz_quadrilinear_merge
    assert qm(None, A, A, A, A, 64, 48, 16) == _native.HZ_EINVAL and b"rank" in lib.hz_last_error()
    assert qm(None, A, A, A, A, 0, 48, 32) == _native.HZ_EINVAL
    assert qm(None, None, A, A, A, 64, 48, 32) == _native.HZ_ENULL
    assert qm(None, A, A + 4, A, A, 64, 48, 32) == _native.HZ_EALIGN
    fa = lib.hz_factorized_apply
    assert fa(None, A, A, A, A, None, A, A, 64, 0, 1024, 1536, 32) == _native.HZ_EINVAL
    assert fa(None, A, A, A, A, None, A, None, 64, 1536, 1024, 1536, 32) == _native.HZ_ENULL
    assert fa(None, A, A, A, A, A + 8, A, A, 64, 1536, 1024, 1536, 32) == _native.HZ_EALIGN
    assert fa(None, A, A, A, A, None, A, A, 64, 1536, 1024, 1536, 0) == _native.HZ_EINVAL


def test_noalloc_apply_rejects_bad_arguments(lib):
    na = lib.hz_factorized_apply_noalloc
    assert len(na.argtypes) == 12
    assert na(None, A, A, A, A, None, A, 64, 1536, 65537, 1536, 32) == _native.HZ_EINVAL
    msg = lib.hz_last_error().decode()
    assert "R <= 65536" in msg and "no-alloc workspace" in msg
    assert na(None, A, A, A, A, None, A, 0, 1536, 1024, 1536, 32) == _native.HZ_EINVAL
    assert na(None, A, A, A, A, None, None, 64, 1536, 1024, 1536, 32) == _native.HZ_ENULL
    assert na(None, A, A, A, A, A + 8, A, 64, 1536, 1024, 1536, 32) == _native.HZ_EALIGN


def test_compiled_wavefunction_rejects_bad_arguments(lib):
    ws = lib.hz_compiled_wavefunction_workspace
    need = ws(4, 8, 32, 64, 64, 32, 16)
    assert need > 0 and ws(0, 8, 32, 64, 64, 32, 16) == -1
    f = lib.hz_compiled_wavefunction
    assert len(f.argtypes) == 28
    names = ["stream", "q", "q_weight", "leaf_V", "leaf_U", "leaf_h", "merge_T", "merge_V", "merge_U", "merge_h",
             "opcodes", "readout_V", "readout_U", "readout_h", "log_abs", "phase", "workspace", "workspace_bytes",
             "B", "n_sites", "d_q", "d_z", "R_leaf", "G", "d_r", "R_merge", "R_out", "merge_eps"]
    base = [None] + [A] * 16 + [need, 4, 8, 4, 32, 64, 2, 32, 32, 16, 1e-6]

    def call(**over):
        args = list(base)
        for key, val in over.items():
            args[names.index(key)] = val
        return f(*args)

    cases = [
        (dict(n_sites=6), _native.HZ_EINVAL, "power of two"),
        (dict(d_r=16), _native.HZ_EINVAL, "rank must be 32"),
        (dict(G=65), _native.HZ_EINVAL, "exceeds 2048"),
        (dict(B=0), _native.HZ_EINVAL, ">= 1"),
        (dict(workspace_bytes=need - 4), _native.HZ_EINVAL, "workspace_bytes"),
        (dict(merge_eps=float("nan")), _native.HZ_EINVAL, "merge_eps"),
        (dict(q=None), _native.HZ_ENULL, "q must not be NULL"),
        (dict(opcodes=None), _native.HZ_ENULL, "opcodes"),
        (dict(merge_T=None), _native.HZ_ENULL, "merge_T"),
        (dict(leaf_h=A + 4), _native.HZ_EALIGN, "leaf_h"),
    ]
    for over, code, needle in cases:
        assert call(**over) == code, over
        assert needle in lib.hz_last_error().decode(), over
