"""Timed CPU baseline of the reference jnp attention path — TEST/BENCH INFRASTRUCTURE ONLY.

Used by ``bench.py``'s ``cpu_baseline`` leg (and its tests) to time the reference
algorithm on the host cores; never part of the product path.

It is a torch-CPU float32 port of the reference's jnp computation
(``src/hamiltonzero/model/pallas_attention.py:22-37`` einsum/softmax formula, with the
primitive's square mask and zeroed masked rows, ``_pallas_attn/mhsea.py:18-25``,
``_pallas_attn/mhsea_tuned.py:91``). Forward-mode uses ``torch.func.jvp`` (as JAX's jvp
of the jnp path would), reverse mode ``torch.func.vjp``. The reference's own files are
not executed (JAX is not installed).

``time_walkers_per_s`` runs on the bench's own inputs (a walker sample of the GPU batch)
and returns the outputs of its last repetition, so the bench can compare them with the
GPU's results for the same walkers.
"""

from __future__ import annotations

import os
import time

import torch


def attention(q, k, v, mask, e=None):
    """out [B,N,H,D] of the primitive semantics, float32, on CPU tensors; e [B,N,H,N]."""
    valid = mask[:, None, :, None] & mask[:, None, None, :]
    mq = mask[:, :, None, None].to(q.dtype)
    s = torch.einsum("bihd,bjhd->bhij", q * mq, k * mq)
    if e is not None:
        s = s + e.permute(0, 2, 1, 3)
    s = torch.where(valid, s, torch.full((), -1e4, dtype=s.dtype))
    p = torch.softmax(s, dim=-1)
    out = torch.einsum("bhij,bjhd->bihd", p, v * mq)
    return out * mq


def fwd_jvp(q, k, v, mask, qt, kt, vt, e=None, et=None):
    """(out, tout) by forward-mode autodiff of :func:`attention`."""
    if e is None:
        return torch.func.jvp(lambda a, b, c: attention(a, b, c, mask), (q, k, v), (qt, kt, vt))
    return torch.func.jvp(lambda a, b, c, d: attention(a, b, c, mask, d), (q, k, v, e), (qt, kt, vt, et))


def gated(q, k, v, mask, e=None):
    """y [B,N,H/2,D]: :func:`attention` followed by the trunk's sigmoid-gate head collapse
    (trunk.py:134-137), head h < H/2 gating head h + H/2."""
    out = attention(q, k, v, mask, e)
    hh = out.shape[2] // 2
    return torch.sigmoid(out[:, :, :hh]) * out[:, :, hh:]


def fwd_jvp_gated(q, k, v, mask, qt, kt, vt, e=None, et=None):
    """(y, ydot) by forward-mode autodiff of :func:`gated`."""
    if e is None:
        return torch.func.jvp(lambda a, b, c: gated(a, b, c, mask), (q, k, v), (qt, kt, vt))
    return torch.func.jvp(lambda a, b, c, d: gated(a, b, c, mask, d), (q, k, v, e), (qt, kt, vt, et))


def fwd_vjp(q, k, v, mask, dout, e=None):
    """(out, (dq, dk, dv[, de])) by reverse-mode autodiff of :func:`attention` (the bias a
    differentiated input when given)."""
    if e is None:
        out, pullback = torch.func.vjp(lambda a, b, c: attention(a, b, c, mask), q, k, v)
    else:
        out, pullback = torch.func.vjp(lambda a, b, c, d: attention(a, b, c, mask, d), q, k, v, e)
    return out, pullback(dout)


def fwd_vjp_gated(q, k, v, mask, dy, e=None):
    """(y, (dq, dk, dv[, de])) by reverse-mode autodiff of :func:`gated` (the bias is a
    differentiated input when given)."""
    if e is None:
        y, pullback = torch.func.vjp(lambda a, b, c: gated(a, b, c, mask), q, k, v)
    else:
        y, pullback = torch.func.vjp(lambda a, b, c, d: gated(a, b, c, mask, d), q, k, v, e)
    return y, pullback(dy)


def host_cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_cpus() -> dict:
    """What the host offers this process: os.cpu_count(), the CPUs of its affinity mask and
    the cgroup CPU quota (cpu.max), if any."""
    info = {"os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)), "cgroup_cpu_quota": None}
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            quota, period = fh.read().split()[:2]
            if quota != "max":
                info["cgroup_cpu_quota"] = int(quota) / int(period)
    except (OSError, ValueError):
        pass
    return info


def default_threads() -> int:
    """Every host core this process may use: the affinity mask, capped by a cgroup quota."""
    info = host_cpus()
    n = info["affinity_cpus"] or info["os_cpu_count"] or 1
    if info["cgroup_cpu_quota"]:
        n = min(n, max(1, int(info["cgroup_cpu_quota"])))
    return n


def time_walkers_per_s(work: str, inputs: dict, budget_s: float = 15.0, threads: int | None = None) -> dict:
    """Time ``work`` ('fwd', 'fwd_jvp', 'fwd_jvp_gated', 'fwd_vjp' or 'fwd_vjp_gated') on the
    walkers of ``inputs`` (CPU float32 tensors: q, k, v, mask, optional e; tangents qt, kt,
    vt, et as [T, ...] for the forward-mode works; dout for 'fwd_vjp', dy for
    'fwd_vjp_gated'). Returns walkers/s and the outputs of the last repetition ('out', 'tout'
    [T, ...], 'y', 'ty', 'dq', 'dk', 'dv', 'de')."""
    threads = threads or default_threads()
    torch.set_num_threads(threads)
    q, k, v, mask, e = (inputs.get(n) for n in ("q", "k", "v", "mask", "e"))
    B = q.shape[0]
    if work in ("fwd_jvp", "fwd_jvp_gated"):
        T = inputs["qt"].shape[0]
        et = inputs.get("et")
        f = fwd_jvp if work == "fwd_jvp" else fwd_jvp_gated

        def fn():
            res = [f(q, k, v, mask, inputs["qt"][t], inputs["kt"][t], inputs["vt"][t], e,
                     None if et is None else et[t]) for t in range(T)]
            prim = res[0][0]
            tans = torch.stack([r[1] for r in res])
            return {"out": prim, "tout": tans} if work == "fwd_jvp" else {"y": prim, "ty": tans}
    elif work == "fwd":
        def fn():
            return {"out": attention(q, k, v, mask, e)}
    elif work == "fwd_vjp":
        def fn():
            out, grads = fwd_vjp(q, k, v, mask, inputs["dout"], e)
            res = {"out": out, "dq": grads[0], "dk": grads[1], "dv": grads[2]}
            if e is not None:
                res["de"] = grads[3]
            return res
    elif work == "fwd_vjp_gated":
        def fn():
            _, grads = fwd_vjp_gated(q, k, v, mask, inputs["dy"], e)
            res = dict(zip(("dq", "dk", "dv"), grads[:3]))
            if e is not None:
                res["de"] = grads[3]
            return res
    else:
        raise ValueError(work)
    with torch.no_grad() if work == "fwd" else torch.enable_grad():
        res = fn()  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            res = fn()
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
        "host_cpus": host_cpus(),
        "outputs": {n: t.detach() for n, t in res.items()},
    }


def rect_attention(q, k, v, bias, key_mask, scale):
    """noncausal_bias_mha(q * scale, k, v, where(key_mask, bias, -1e30)) in torch-CPU float32
    (src/hamiltonzero/evaluation/sequence_parallel.py:79-90, pallas_mha.py:43-89)."""
    e = torch.where(key_mask[:, None, :, None], bias, torch.full((), -1e30, dtype=bias.dtype))
    s = torch.einsum("bihd,bjhd->bhij", q * scale, k) + e.permute(0, 3, 1, 2)
    return torch.einsum("bhij,bjhd->bihd", torch.softmax(s, dim=-1), v)


def time_rect_queries_per_s(q, k, v, bias, key_mask, scale, budget_s: float = 15.0,
                            threads: int | None = None) -> dict:
    """Time the rectangular forward for the query rows of ``q [1, Nq_sample, H, D]`` against
    all keys (a sequence-parallel rank's share); returns query rows per second and the
    output of the last repetition."""
    threads = threads or default_threads()
    torch.set_num_threads(threads)
    with torch.no_grad():
        out = rect_attention(q, k, v, bias, key_mask, scale)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            out = rect_attention(q, k, v, bias, key_mask, scale)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 100000:
                break
    return {
        "queries_per_s": q.shape[1] * reps / el,
        "seconds": el,
        "reps": reps,
        "threads": threads,
        "cpu_model": host_cpu_model(),
        "host_cpus": host_cpus(),
        "out": out,
    }


def mlp_pair_bias(edge, params, gain, div, slopes=None, eps=1e-5):
    """The MLP-class coupling bias in torch-CPU float32 (odd_ops.py:256-276 MLP, / sqrt(d),
    + the LCA-ALiBi term on positions 0..n-1, tree.py:1436-1451): edge [B, N, N, C] ->
    [B, N, N, H]."""
    h = edge @ params["w_in"] + params["b_in"]
    for k in range(params["w_1"].shape[0]):
        n = h * (params["norm_w"][k] * torch.rsqrt(torch.mean(h * h, dim=-1, keepdim=True) + eps))
        u = n @ params["w_1"][k] + params["b_1"][k]
        h = h + gain * ((u * torch.sigmoid(u)) @ params["w_2"][k] + params["b_2"][k])
    n = h * (params["out_norm_w"] * torch.rsqrt(torch.mean(h * h, dim=-1, keepdim=True) + eps))
    e = (n @ params["w_out"] + params["b_out"]) / div
    if slopes is not None:
        idx = torch.arange(edge.shape[1])
        x = idx[:, None] ^ idx[None, :]
        lvl = (x[..., None] >= (2 ** torch.arange(13))).sum(-1).to(e.dtype)
        e = e - lvl[:, :, None] * slopes
    return e


def time_mlp_pair_bias_walkers_per_s(edge, edge_t, params, gain, div, slopes, budget_s: float = 15.0,
                                     threads: int | None = None) -> dict:
    """Time the bias and its forward-mode tangent (torch.func.jvp) on every pair of the
    walkers of ``edge [B_sample, N, N, C]``; returns walkers/s and (e, e_t) of the last
    repetition."""
    threads = threads or default_threads()
    torch.set_num_threads(threads)

    def fn():
        return torch.func.jvp(lambda x: mlp_pair_bias(x, params, gain, div, slopes), (edge,), (edge_t,))

    with torch.no_grad():
        res = fn()
        reps, t0 = 0, time.perf_counter()
        while True:
            res = fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 100000:
                break
    return {"walkers_per_s": edge.shape[0] * reps / el, "seconds": el, "reps": reps, "threads": threads,
            "cpu_model": host_cpu_model(), "host_cpus": host_cpus(), "e": res[0], "e_t": res[1]}


def rect_block(q, k, v, bias, key_mask, scale, w_o, row_mask):
    """The large-N attention tail in torch-CPU float32 (sequence_trunk.py:973-984): the
    rectangular attention, the head collapse sigmoid(out[:, :, :H/2]) * out[:, :, H/2:] and
    row_mask * (y_flat @ w_o). Returns (y, proj)."""
    out = rect_attention(q, k, v, bias, key_mask, scale)
    hh = out.shape[2] // 2
    y = torch.sigmoid(out[:, :, :hh]) * out[:, :, hh:]
    proj = (y.reshape(y.shape[0], y.shape[1], -1) @ w_o) * row_mask[:, :, None].to(y.dtype)
    return y, proj


def time_rect_block_queries_per_s(q, k, v, bias, key_mask, scale, w_o, row_mask, budget_s: float = 15.0,
                                  threads: int | None = None) -> dict:
    """Time :func:`rect_block` for the query rows of ``q [1, Nq_sample, H, D]`` against all
    keys; returns query rows per second and (y, proj) of the last repetition."""
    threads = threads or default_threads()
    torch.set_num_threads(threads)
    with torch.no_grad():
        res = rect_block(q, k, v, bias, key_mask, scale, w_o, row_mask)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            res = rect_block(q, k, v, bias, key_mask, scale, w_o, row_mask)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 100000:
                break
    return {
        "queries_per_s": q.shape[1] * reps / el,
        "seconds": el,
        "reps": reps,
        "threads": threads,
        "cpu_model": host_cpu_model(),
        "host_cpus": host_cpus(),
        "y": res[0],
        "proj": res[1],
    }


def executor_level(T, ul, ur, V, U, h):
    """One compiled-executor level's products in torch-CPU float32: the quadrilinear merge
    (einsum, _custom_lap_primitives.py:45-50) and the residual factorized apply
    (execute.py:24-31,104); rows are walkers x nodes, nodes innermost."""
    G, R = T.shape[0], T.shape[1]
    a = ul.reshape(-1, G, R)
    b = ur.reshape(-1, G, R)
    raw = torch.einsum("ijkl,Bik,Bil->Bij", T, a, b).reshape(ul.shape)
    W = h.shape[0]
    mixed = (raw @ V).reshape(-1, W, V.shape[1]) * h
    return raw + (mixed.reshape(raw.shape[0], -1) @ U)


def time_executor_level(T, ul, ur, V, U, h, budget_s: float = 15.0, threads: int | None = None) -> dict:
    """Time ``executor_level`` on the given rows; returns reps / seconds and the output."""
    threads = threads or default_threads()
    torch.set_num_threads(threads)
    with torch.no_grad():
        out = executor_level(T, ul, ur, V, U, h)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            out = executor_level(T, ul, ur, V, U, h)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 100000:
                break
    return {"reps": reps, "seconds": el, "threads": threads, "cpu_model": host_cpu_model(), "host_cpus": host_cpus(),
            "out": out}


def coupling_bias(edge, p, gain, d_head, eps=1e-5):
    """ln_edge + bias_mlp + 1/sqrt(d_head) over every pair (trunk.py:89-105), float32;
    edge [B, N, N, C] -> e [B, N, H, N] (the primitive's layout)."""
    y = edge * (p["ln_w"] * torch.rsqrt(torch.mean(edge * edge, dim=-1, keepdim=True) + eps))
    h0 = y @ p["w_in"] + p["b_in"]
    u = h0 @ p["w_1"] + p["b_1"]
    h1 = h0 + gain * ((u * torch.sigmoid(u)) @ p["w_2"] + p["b_2"])
    bias = (h1 @ p["w_out"] + p["b_out"]) / torch.sqrt(torch.tensor(float(d_head)))
    return bias.permute(0, 1, 3, 2)


def trunk_attention(q, k, v, edge, mask, p, gain, d_head, w_o=None):
    """The trunk's attention call with its produced bias and the gate collapse (q pre-scaled),
    then W_O on the flattened heads when given (trunk.py:134-144)."""
    y = gated(q, k, v, mask, coupling_bias(edge, p, gain, d_head))
    return y if w_o is None else y.reshape(y.shape[0], y.shape[1], -1) @ w_o


def time_trunk_walkers_per_s(inputs: dict, mask, params: dict, gain: float, d_head: int, budget_s: float = 15.0,
                             threads: int | None = None, w_o=None) -> dict:
    """Time the forward + JVP of :func:`trunk_attention` (tangents on q, k, v and edge) on
    the walkers of ``inputs``; returns walkers/s and the last repetition's y, ydot."""
    threads = threads or default_threads()
    torch.set_num_threads(threads)
    prim = tuple(inputs[n] for n in ("q", "k", "v", "edge"))
    tans = tuple(inputs[n] for n in ("qt", "kt", "vt", "edge_t"))

    def fn():
        return torch.func.jvp(lambda a, b, c, x: trunk_attention(a, b, c, x, mask, params, gain, d_head, w_o), prim,
                              tans)

    y, ty = fn()  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        y, ty = fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 100000:
            break
    return {"walkers_per_s": prim[0].shape[0] * reps / el, "seconds": el, "reps": reps, "threads": threads,
            "cpu_model": host_cpu_model(), "host_cpus": host_cpus(), "y": y.detach(), "ty": ty.detach()}


def compiled_wavefunction(p: dict, merge_eps: float):
    """CompiledFinetuneWaveFunction._forward_plain (compiled/model.py:143-180) in torch-CPU
    float32 on a dict of packed parameters (merge_h [L, n/2, R], opcodes [L, n/2])."""
    q = p["q"]
    B, n = q.shape[0], q.shape[1]
    z = q @ p["q_weight"]
    u = ((z @ p["leaf_V"]) * p["leaf_h"]) @ p["leaf_U"]
    rms = torch.sqrt(torch.mean(u * u, dim=-1, keepdim=True) + 1e-30)
    u, s = u / rms, torch.log(rms)[..., 0]
    level, width = 0, n // 2
    G, R = p["merge_T"].shape[0], p["merge_T"].shape[1]
    while width >= 1:
        ul, ur, sl, sr = u[:, 0::2], u[:, 1::2], s[:, 0::2], s[:, 1::2]
        raw = torch.einsum("ijkl,Bik,Bil->Bij", p["merge_T"], ul.reshape(-1, G, R), ur.reshape(-1, G, R))
        raw = raw.reshape(B, width, G * R)
        out = raw + ((raw @ p["merge_V"]) * p["merge_h"][level, :width]) @ p["merge_U"]
        scale = torch.sqrt(torch.mean(out * out, dim=-1) + merge_eps)
        ops = p["opcodes"][level, :width]
        both, left, right = ((ops == c).to(u.dtype) for c in (0, 1, 2))
        u = both[:, None] * (out / scale[..., None]) + left[:, None] * ul + right[:, None] * ur
        s = both * (sl + sr + torch.log(scale)) + left * sl + right * sr
        level, width = level + 1, width // 2
    psi = ((u[:, 0] @ p["readout_V"]) * p["readout_h"]) @ p["readout_U"]
    return 0.5 * torch.log(psi[:, 0] ** 2 + psi[:, 1] ** 2) + s[:, 0], torch.atan2(psi[:, 1], psi[:, 0])


def time_wavefunction_walkers_per_s(p: dict, merge_eps: float, budget_s: float = 15.0,
                                    threads: int | None = None) -> dict:
    """Time :func:`compiled_wavefunction` on the walkers of ``p['q']``."""
    threads = threads or default_threads()
    torch.set_num_threads(threads)
    with torch.no_grad():
        la, ph = compiled_wavefunction(p, merge_eps)
        reps, t0 = 0, time.perf_counter()
        while True:
            la, ph = compiled_wavefunction(p, merge_eps)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 100000:
                break
    return {"walkers_per_s": p["q"].shape[0] * reps / el, "seconds": el, "reps": reps, "threads": threads,
            "cpu_model": host_cpu_model(), "host_cpus": host_cpus(), "log_abs": la, "phase": ph}
