"""Timed CPU baseline of the reference jnp attention path — TEST/BENCH INFRASTRUCTURE ONLY.

Used by ``bench.py``'s ``cpu_baseline`` leg (and its tests) to time the reference
algorithm on the host cores; never part of the product path.

It is a torch-CPU float32 port of the reference's jnp computation
(``src/hamiltonzero/model/pallas_attention.py:22-37`` einsum/softmax formula, with the
primitive's square mask and zeroed masked rows, ``_pallas_attn/mhsea.py:18-25``,
``_pallas_attn/mhsea_tuned.py:91``). Forward-mode uses ``torch.func.jvp`` (as JAX's jvp
of the jnp path would), reverse mode ``torch.func.vjp``. The reference's own files are
not executed (JAX is not installed).
"""

from __future__ import annotations

import os
import time

import numpy as np
import torch


def attention(q, k, v, mask, e=None):
    """out [B,N,H,D] of the primitive semantics, float32, on CPU tensors."""
    valid = mask[:, None, :, None] & mask[:, None, None, :]
    mq = mask[:, :, None, None].to(q.dtype)
    s = torch.einsum("bihd,bjhd->bhij", q * mq, k * mq)
    if e is not None:
        s = s + e.permute(0, 2, 1, 3)
    s = torch.where(valid, s, torch.full((), -1e4, dtype=s.dtype))
    p = torch.softmax(s, dim=-1)
    out = torch.einsum("bhij,bjhd->bihd", p, v * mq)
    return out * mq


def fwd_jvp(q, k, v, mask, qt, kt, vt):
    """(out, tout) by forward-mode autodiff of :func:`attention`."""
    return torch.func.jvp(lambda a, b, c: attention(a, b, c, mask), (q, k, v), (qt, kt, vt))


def gated(q, k, v, mask):
    """y [B,N,H/2,D]: :func:`attention` followed by the trunk's sigmoid-gate head collapse
    (trunk.py:134-137), head h < H/2 gating head h + H/2."""
    out = attention(q, k, v, mask)
    hh = out.shape[2] // 2
    return torch.sigmoid(out[:, :, :hh]) * out[:, :, hh:]


def fwd_jvp_gated(q, k, v, mask, qt, kt, vt):
    """(y, ydot) by forward-mode autodiff of :func:`gated`."""
    return torch.func.jvp(lambda a, b, c: gated(a, b, c, mask), (q, k, v), (qt, kt, vt))


def fwd_vjp(q, k, v, mask, dout):
    """(out, (dq, dk, dv)) by reverse-mode autodiff of :func:`attention`."""
    out, pullback = torch.func.vjp(lambda a, b, c: attention(a, b, c, mask), q, k, v)
    return out, pullback(dout)


def host_cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_walkers_per_s(work: str, B: int, N: int, H: int, D: int, n_phys: int, seed: int,
                       T: int = 1, bf16_inputs: bool = False, budget_s: float = 15.0,
                       threads: int | None = None) -> dict:
    """Time ``work`` ('fwd', 'fwd_jvp', 'fwd_jvp_gated' or 'fwd_vjp') on B walkers; returns
    walkers/s.

    Inputs follow the measurement recipe of the bench (default_rng(seed), N(0,1)/sqrt(D)
    for q/k/v, N(0,1) tangents and cotangent, the first n_phys sites physical). bf16
    configurations run in float32 on bf16-rounded inputs.
    """
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    rng = np.random.default_rng(seed)
    shape = (B, N, H, D)

    def draw(scale):
        x = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))
        return x.to(torch.bfloat16).float() if bf16_inputs else x

    q, k, v = draw(D ** -0.5), draw(D ** -0.5), draw(D ** -0.5)
    mask = torch.zeros((B, N), dtype=torch.bool)
    mask[:, :n_phys] = True
    if work == "fwd":
        fn = lambda: attention(q, k, v, mask)  # noqa: E731
    elif work == "fwd_jvp":
        tans = [(draw(1.0), draw(1.0), draw(1.0)) for _ in range(T)]
        fn = lambda: [fwd_jvp(q, k, v, mask, *t) for t in tans]  # noqa: E731
    elif work == "fwd_jvp_gated":
        tans = [(draw(1.0), draw(1.0), draw(1.0)) for _ in range(T)]
        fn = lambda: [fwd_jvp_gated(q, k, v, mask, *t) for t in tans]  # noqa: E731
    elif work == "fwd_vjp":
        dout = draw(1.0)
        fn = lambda: fwd_vjp(q, k, v, mask, dout)  # noqa: E731
    else:
        raise ValueError(work)
    with torch.no_grad() if work == "fwd" else torch.enable_grad():
        fn()  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 100000:
                break
    return {
        "walkers_per_s": B * reps / el,
        "seconds": el,
        "reps": reps,
        "threads": threads,
        "cpu_model": host_cpu_model(),
    }


def rect_attention(q, k, v, bias, key_mask, scale):
    """noncausal_bias_mha(q * scale, k, v, where(key_mask, bias, -1e30)) in torch-CPU float32
    (src/hamiltonzero/evaluation/sequence_parallel.py:79-90, pallas_mha.py:43-89)."""
    e = torch.where(key_mask[:, None, :, None], bias, torch.full((), -1e30, dtype=bias.dtype))
    s = torch.einsum("bihd,bjhd->bhij", q * scale, k) + e.permute(0, 3, 1, 2)
    return torch.einsum("bhij,bjhd->bihd", torch.softmax(s, dim=-1), v)


def time_rect_queries_per_s(Nq_sample: int, Nk: int, H: int, D: int, n_phys: int, seed: int,
                            budget_s: float = 15.0, threads: int | None = None) -> dict:
    """Time the rectangular forward for ``Nq_sample`` query rows of one system against all
    ``Nk`` keys (a sequence-parallel rank's share); returns query rows per second."""
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    rng = np.random.default_rng(seed)

    def draw(shape, scale):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))

    q = draw((1, Nq_sample, H, D), 1.0)
    k = draw((1, Nk, H, D), 1.0)
    v = draw((1, Nk, H, D), 1.0)
    bias = draw((1, Nq_sample, Nk, H), D ** -0.5)
    mask = torch.zeros((1, Nk), dtype=torch.bool)
    mask[:, :n_phys] = True
    with torch.no_grad():
        rect_attention(q, k, v, bias, mask, D ** -0.5)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            rect_attention(q, k, v, bias, mask, D ** -0.5)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 100000:
                break
    return {
        "queries_per_s": Nq_sample * reps / el,
        "seconds": el,
        "reps": reps,
        "threads": threads,
        "cpu_model": host_cpu_model(),
    }
