"""Throughput of the gfx950 MHSEA kernels on the path's synthetic benchmark configurations c1-c5.

Default (the driver's run): configuration c2 — fused forward + JVP, float32,
q/k/v [B=1024, N=64, H=8, D=32], one tangent per input, 36 physical sites of 64, seed 1.
One "step" is one fwd+JVP of the whole batch (one kernel launch, inputs resident in HBM).

Prints ONE JSON line with walkers/s, the roofline of the dominant kernel (live HIP-event
timing on the launch stream) and a CPU baseline (the jnp path's torch-CPU port, timed on
a bounded walker sample on this host; see oracle/cpu_baseline.py).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c1..c5|rect]
                       [--cpu-budget SECONDS] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+JVP attention walkers/sec at B=1024,L=64; % of MFMA/HBM roofline"
GATE_METRIC = ("fwd+JVP attention with the sigmoid-gate head collapse fused, walkers/sec at B=1024,L=64; "
               "% of MFMA/HBM roofline")
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2516.6

# name: (work, B, N, H, D, n_phys, T, dtype, seed, description)
CONFIGS = {
    "c1": ("fwd", 256, 8, 4, 32, 8, 0, "f32", 0, "attention forward, fp32, [256,8,4,32], no padding"),
    "c2": ("fwd_jvp", 1024, 64, 8, 32, 36, 1, "f32", 1,
           "forward + JVP, fp32, [1024,64,8,32], 36/64 physical sites (6x6 lattice)"),
    "c3": ("fwd_vjp", 4096, 64, 8, 64, 48, 0, "bf16", 2,
           "forward + VJP, bf16 I/O fp32 accumulate, [4096,64,8,64], 48/64 physical sites"),
    "c4": ("fwd_jvp", 512, 256, 8, 64, 225, 1, "f32", 3,
           "large-N forward + JVP, fp32, [512,256,8,64], 225/256 physical sites (15x15)"),
    "c5": ("fwd_jvp", 128, 1024, 16, 64, 1000, 2, "bf16", 4,
           "large-N stress forward + 2 JVP directions, bf16 I/O, [128,1024,16,64], 1000/1024 sites"),
    # The caller-side epilogue of the trunk (trunk.py:134-137) fused into c2's kernel: head h
    # gates head h + H/2, and only y = sigmoid(gate) * value and its tangent are written.
    # Reported beside the hot path, never as the default line.
    "gate": ("fwd_jvp_gated", 1024, 64, 8, 32, 36, 1, "f32", 1,
             "c2's forward + JVP with the sigmoid-gate head collapse fused, fp32, [1024,64,8,32] -> "
             "y, ydot [1024,64,4,32], 36/64 physical sites"),
    # The large-N evaluation forward (noncausal_bias_mha via pallas_rectangular_edge_attention):
    # one system, all queries against all keys, dense [Nq, Nk, H] bias. Not one of c1-c5:
    # reported beside the hot path, never as the default line.
    "rect": ("rect", 1, 4096, 16, 64, 4000, 0, "f32", 5,
             "rectangular forward with dense bias, fp32, one system, Nq=Nk=4096, H=16, D=64, "
             "4000/4096 physical keys"),
}
RECT_METRIC = "rectangular large-N forward (noncausal_bias_mha) query rows/sec; % of MFMA/HBM roofline"


def rect_algorithmic(B, Nq, Nk, H, D, n_phys):
    """Bytes and flops of one rectangular forward. padded: q, k, v, out and the bias
    [Nq, Nk, H] moved once, the key mask as uint8, 4 Nq Nk D flops per (system, head);
    effective: only physical keys' k, v and bias columns, and their flops."""
    row = H * D * 4
    padded_bytes = B * (2 * Nq * row + 2 * Nk * row + Nq * Nk * H * 4 + Nk)
    eff_bytes = B * (2 * Nq * row + 2 * n_phys * row + Nq * n_phys * H * 4 + Nk)
    return dict(padded_bytes=padded_bytes, eff_bytes=eff_bytes,
                padded_flops=B * H * 4 * Nq * Nk * D, eff_flops=B * H * 4 * Nq * n_phys * D)


def run_rect(args, desc, B, N, H, D, n_phys, seed):
    """Bench leg of the rectangular forward (hz_rect_attention_fwd)."""
    import torch

    from hamiltonzero_amd import _native

    lib = _native.lib()
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)

    def draw(shape, scale):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).to(dev)

    q = draw((B, N, H, D), 1.0)
    k = draw((B, N, H, D), 1.0)
    v = draw((B, N, H, D), 1.0)
    bias = draw((B, N, N, H), D ** -0.5)
    mask = torch.zeros((B, N), dtype=torch.uint8, device=dev)
    mask[:, :n_phys] = 1
    out = torch.empty_like(q)
    s = torch.cuda.current_stream(dev).cuda_stream
    scale = D ** -0.5

    def step():
        _native.check(lib.hz_rect_attention_fwd(s, q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
                                                mask.data_ptr(), out.data_ptr(), B, N, N, H, D, scale))

    ms = timed(step, args.steps, args.warmup, torch.cuda.current_stream(dev))
    t_s = ms / 1e3
    alg = rect_algorithmic(B, N, N, H, D, n_phys)
    roof = roofline(alg["padded_bytes"], alg["padded_flops"], t_s, "f32")
    roof["traffic"] = traffic_from_profile(args.config)
    roof["basis"] = "padded algorithmic bytes/flops (every q, k, v, out row and the full bias once)"
    roof["bytes_per_step"] = alg["padded_bytes"]
    roof["flops_per_step"] = alg["padded_flops"]
    roof_mask = roofline(alg["eff_bytes"], alg["eff_flops"], t_s, "f32")
    roof_mask["basis"] = "mask-aware algorithmic bytes/flops (physical keys only)"
    roof_mask["bytes_per_step"] = alg["eff_bytes"]
    roof_mask["flops_per_step"] = alg["eff_flops"]
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        sample = 64
        r = cpu_baseline.time_rect_queries_per_s(sample, N, H, D, n_phys, seed, budget_s=args.cpu_budget,
                                                 threads=threads)
        cpu = {"value": r["queries_per_s"], "unit": "queries/s", "cores": r["threads"], "kind": "port",
               "sample": f"{sample} query rows of one system against all {N} keys, {r['reps']} reps in "
                         f"{r['seconds']:.1f} s, torch-CPU fp32 port of the jnp formula ({r['cpu_model']})"}
    line = {
        "metric": RECT_METRIC, "value": B * N / t_s, "unit": "queries/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (numpy default_rng, N(0,1) q/k/v, N(0,1)/sqrt(D) bias)",
        "config": {"workload": f"rect: {desc}", "B": B, "Nq": N, "Nk": N, "H": H, "D": D, "n_phys": n_phys},
        "roofline": roof, "roofline_mask_aware": roof_mask, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def timed(step, steps, warmup, stream):
    """Average milliseconds of ``step`` over ``steps`` launches after ``warmup``, with HIP
    events recorded on the launch stream."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def algorithmic(work, B, N, H, D, n_phys, T, esize):
    """Algorithmic bytes and flops of one step.

    padded: every [B,N,H,D] tensor read or written once at the padded shape, plus the mask
            (uint8); flops (2 + 4T) G for fwd+JVP, 2G fwd, 6G fwd+VJP, G = 2 N^2 D per
            (walker, head), recompute not counted.
    effective: the same with the mask taken into account — inputs are needed only on
            physical rows (a masked row never influences a result), outputs are written on
            every row (zeros included), and only physical x physical pairs carry flops.
    """
    rowb = H * D * esize  # bytes of one site row of one [B,N,H,D] tensor
    if work == "fwd":
        n_in, n_out, g_mult, lse_b = 3, 1, 2, 0
    elif work == "fwd_jvp":
        n_in, n_out, g_mult, lse_b = 3 + 3 * T, 1 + T, 2 + 4 * T, 0
    elif work == "fwd_jvp_gated":  # outputs are y and its T tangents, each half a [B,N,H,D] tensor
        n_in, n_out, g_mult, lse_b = 3 + 3 * T, (1 + T) / 2, 2 + 4 * T, 0
    elif work == "fwd_vjp":
        # fwd: q,k,v in, out + lse out; bwd: q,k,v,out,dout + lse in, dq,dk,dv out
        n_in, n_out, g_mult, lse_b = 3 + 5, 1 + 3, 6, 2 * N * H * 4
    else:
        raise ValueError(work)
    padded_bytes = int(B * (N * rowb * (n_in + n_out) + N + lse_b))
    eff_bytes = int(B * (n_phys * rowb * n_in + N * rowb * n_out + N + lse_b))
    padded_flops = B * H * g_mult * 2 * N * N * D
    eff_flops = B * H * g_mult * 2 * n_phys * n_phys * D
    return dict(padded_bytes=padded_bytes, eff_bytes=eff_bytes, padded_flops=padded_flops,
                eff_flops=eff_flops)


def roofline(bytes_, flops, t_s, dtype):
    peak_c = BF16_PEAK_TFLOPS if dtype == "bf16" else FP32_PEAK_TFLOPS
    t_hbm = bytes_ / (HBM_PEAK_GBS * 1e9)
    t_cmp = flops / (peak_c * 1e12)
    if t_hbm >= t_cmp:
        ach = bytes_ / t_s / 1e9
        return {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ach / HBM_PEAK_GBS}
    ach = flops / t_s / 1e12
    return {"bound": "mfma", "achieved": ach, "peak": peak_c, "unit": "TFLOP/s", "frac": ach / peak_c}


def traffic_from_profile(config):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE), scaled by
    the copy-kernel calibration, if a summary for this configuration is committed."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        rec = json.load(fh)
    return rec.get("traffic_bytes_per_launch")


def copy_probe(mib, steps, warmup):
    """Device-to-device copies of a known size (hipMemcpyAsync -> the runtime's copyBuffer
    kernel): reads and writes exactly ``mib`` MiB per launch. Profiled under rocprofv3
    --pmc it gives the factor between FETCH_SIZE / WRITE_SIZE and real bytes."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    nbytes = n * 4
    print(json.dumps({"copy_probe_bytes": nbytes, "ms_per_copy": ms,
                      "gbs_read_plus_write": 2 * nbytes / ms / 1e6}), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--generic", action="store_true",
                    help="force the LDS-streaming kernels (HZ_FLAG_GENERIC) for comparison")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="instead of a configuration, time device-to-device copies of MIB MiB "
                         "(the calibration kernel for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    import torch

    from hamiltonzero_amd import _native

    if args.copy_probe:
        return copy_probe(args.copy_probe, args.steps, args.warmup)

    lib = _native.lib()
    work, B, N, H, D, n_phys, T, dtype, seed, desc = CONFIGS[args.config]
    if work == "rect":
        return run_rect(args, desc, B, N, H, D, n_phys, seed)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    hz_dtype = _native.HZ_DTYPE_BF16 if dtype == "bf16" else _native.HZ_DTYPE_F32
    esize = 2 if dtype == "bf16" else 4
    dev = torch.device("cuda:0")

    # Synthetic inputs: default_rng(seed); draw order q, k, v, tangents (per direction
    # qt, kt, vt), cotangent; q/k/v scaled by 1/sqrt(D).
    rng = np.random.default_rng(seed)
    shape = (B, N, H, D)

    def draw(scale):
        x = rng.standard_normal(shape, dtype=np.float32)
        if scale != 1.0:
            x *= np.float32(scale)
        return torch.from_numpy(x).to(device=dev, dtype=tdt)

    q, k, v = draw(D ** -0.5), draw(D ** -0.5), draw(D ** -0.5)
    tans = []
    for _ in range(T):
        tans.append([draw(1.0), draw(1.0), draw(1.0)])
    dout = draw(1.0) if work == "fwd_vjp" else None
    mask = torch.zeros((B, N), dtype=torch.uint8, device=dev)
    mask[:, :n_phys] = 1
    stream = torch.cuda.current_stream(dev)
    s = stream.cuda_stream
    out = torch.empty(shape, dtype=tdt, device=dev)
    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    fl = _native.HZ_FLAG_GENERIC if args.generic else 0

    if work == "fwd":
        def step():
            _native.check(lib.hz_mhsea_fwd(s, P(q), P(k), None, P(v), P(mask), P(out), None,
                                           B, N, H, D, hz_dtype, 1.0, fl))
    elif work in ("fwd_jvp", "fwd_jvp_gated"):
        qt = torch.stack([t[0] for t in tans]).contiguous()
        kt = torch.stack([t[1] for t in tans]).contiguous()
        vt = torch.stack([t[2] for t in tans]).contiguous()
        del tans
        tout = torch.empty((T, *shape), dtype=tdt, device=dev)

        def step():
            _native.check(lib.hz_mhsea_fwd_jvp(s, P(q), P(k), None, P(v), P(mask), P(qt), P(kt), None, P(vt), T,
                                               P(out), None, P(tout), B, N, H, D, hz_dtype, 1.0, fl))

        if work == "fwd_jvp_gated":
            y = torch.empty((B, N, H // 2, D), dtype=tdt, device=dev)
            ty = torch.empty((T, B, N, H // 2, D), dtype=tdt, device=dev)
            del out, tout

            def step():
                _native.check(lib.hz_mhsea_fwd_jvp_gated(s, P(q), P(k), None, P(v), P(mask), P(qt), P(kt), None,
                                                         P(vt), T, P(y), P(ty), B, N, H, D, 1.0, 0))
    else:
        lse = torch.empty((B, N, H), dtype=torch.float32, device=dev)
        dq, dk, dv = (torch.empty(shape, dtype=tdt, device=dev) for _ in range(3))

        def step():
            _native.check(lib.hz_mhsea_fwd(s, P(q), P(k), None, P(v), P(mask), P(out), P(lse),
                                           B, N, H, D, hz_dtype, 1.0, fl))
            _native.check(lib.hz_mhsea_bwd(s, P(q), P(k), None, P(v), P(mask), P(lse), P(out), P(dout),
                                           P(dq), P(dk), None, P(dv), B, N, H, D, hz_dtype, 1.0, fl))

    ms = timed(step, args.steps, args.warmup, stream)
    t_s = ms / 1e3
    walkers_s = B / t_s

    alg = algorithmic(work, B, N, H, D, n_phys, T, esize)
    # roofline: the per-walker algorithmic bytes / flops of the padded problem (every
    # [B,N,H,D] tensor moved once, (2+4T)G / 6G / 2G flops), the figure the reference's
    # own kernels are sized by. roofline_mask_aware: the stricter figure that counts only
    # physical input rows and physical x physical pairs (what this kernel must do).
    roof = roofline(alg["padded_bytes"], alg["padded_flops"], t_s, dtype)
    roof["traffic"] = traffic_from_profile(args.config)
    roof["basis"] = "padded algorithmic bytes/flops per walker x B (every row of every tensor once)"
    roof["bytes_per_step"] = alg["padded_bytes"]
    roof["flops_per_step"] = alg["padded_flops"]
    roof_mask = roofline(alg["eff_bytes"], alg["eff_flops"], t_s, dtype)
    roof_mask["basis"] = "mask-aware algorithmic bytes/flops (physical rows in, all rows out)"
    roof_mask["bytes_per_step"] = alg["eff_bytes"]
    roof_mask["flops_per_step"] = alg["eff_flops"]

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        sample = {"c1": 256, "c2": 64, "c3": 32, "c4": 4, "c5": 1, "gate": 64}[args.config]
        r = cpu_baseline.time_walkers_per_s(work, sample, N, H, D, n_phys, seed, T=max(T, 1),
                                            bf16_inputs=(dtype == "bf16"), budget_s=args.cpu_budget,
                                            threads=threads)
        cpu = {
            "value": r["walkers_per_s"],
            "unit": "walkers/s",
            "cores": r["threads"],
            "kind": "port",
            "sample": f"{sample} walkers of the same shape/mask/seed recipe, {r['reps']} reps in "
                      f"{r['seconds']:.1f} s, torch-CPU fp32 jnp-path port ({r['cpu_model']})",
        }

    line = {
        "metric": GATE_METRIC if work == "fwd_jvp_gated" else METRIC,
        "value": walkers_s,
        "unit": "walkers/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == "bf16" else "f32",
        "data": "synthetic (numpy default_rng, N(0,1)/sqrt(D) q/k/v, N(0,1) tangents)",
        "config": {"workload": f"{args.config}: {desc}", "B": B, "N": N, "H": H, "D": D,
                   "n_phys": n_phys, "T": T, "work": work,
                   "kernels": "generic" if args.generic else "auto"},
        "roofline": roof,
        "roofline_mask_aware": roof_mask,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
