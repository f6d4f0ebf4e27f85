"""Concurrent calls of the C ABI from several host threads (include/hz_mhsea.h promises
re-entrant calls on distinct output buffers): each thread runs the forward+JVP, backward and
rectangular entry points on its own stream and buffers; every result must equal, bit for bit,
the same calls made from one thread (the kernels are deterministic)."""

import threading

import pytest
import torch

from hamiltonzero_amd import _native

pytestmark = pytest.mark.gpu


def _inputs(seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    B, N, H, D = 64, 64, 4, 32
    mk = lambda *s: torch.randn(*s, device="cuda", generator=g) * 0.2  # noqa: E731
    q, k, v, dout = mk(B, N, H, D), mk(B, N, H, D), mk(B, N, H, D), mk(B, N, H, D)
    qt, kt, vt = mk(1, B, N, H, D), mk(1, B, N, H, D), mk(1, B, N, H, D)
    m = torch.zeros(B, N, dtype=torch.uint8, device="cuda")
    m[:, :40] = 1
    e = mk(2, 96, 80, 8)
    rq, rk, rv = mk(2, 96, 8, 16), mk(2, 80, 8, 16), mk(2, 80, 8, 16)
    return dict(shape=(B, N, H, D), q=q, k=k, v=v, dout=dout, qt=qt, kt=kt, vt=vt, m=m, e=e, rq=rq, rk=rk, rv=rv)


def _run(lib, a, stream):
    P = lambda t: t.data_ptr()  # noqa: E731
    B, N, H, D = a["shape"]
    s = stream.cuda_stream
    out, tout = torch.empty_like(a["q"]), torch.empty_like(a["qt"])
    lse = torch.empty(B, N, H, device="cuda")
    dq, dk, dv = torch.empty_like(a["q"]), torch.empty_like(a["q"]), torch.empty_like(a["q"])
    rout = torch.empty_like(a["rq"])
    _native.check(lib.hz_mhsea_fwd_jvp(s, P(a["q"]), P(a["k"]), None, P(a["v"]), P(a["m"]), P(a["qt"]), P(a["kt"]), None,
                                       P(a["vt"]), 1, P(out), P(lse), P(tout), B, N, H, D, 0, 0.5, 0))
    _native.check(lib.hz_mhsea_bwd(s, P(a["q"]), P(a["k"]), None, P(a["v"]), P(a["m"]), P(lse), P(out), P(a["dout"]),
                                   P(dq), P(dk), None, P(dv), B, N, H, D, 0, 0.5, 0))
    _native.check(lib.hz_rect_attention_fwd(s, P(a["rq"]), P(a["rk"]), P(a["rv"]), P(a["e"]), None, P(rout),
                                            2, 96, 80, 8, 16, 0.25))
    stream.synchronize()
    return [out, tout, dq, dk, dv, rout]


def test_concurrent_host_threads_match_single_thread():
    print("[case] concurrent host threads", flush=True)
    lib = _native.lib()
    inputs = [_inputs(100 + i) for i in range(4)]
    main = torch.cuda.Stream()
    want = [_run(lib, a, main) for a in inputs]
    got = [None] * 4
    errors = []

    def worker(i):
        try:
            st = torch.cuda.Stream()
            for _ in range(5):
                got[i] = _run(lib, inputs[i], st)
        except Exception as exc:  # pragma: no cover - reported below
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(4):
        for w, g in zip(want[i], got[i]):
            assert torch.equal(w, g)
