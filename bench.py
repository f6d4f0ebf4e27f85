"""Throughput of the gfx950 MHSEA kernels on the path's synthetic benchmark configurations c1-c5.

Default (the driver's run): configuration c2 — fused forward + JVP, float32,
q/k/v [B=1024, N=64, H=8, D=32], one tangent per input, 36 physical sites of 64, seed 1.
One "step" is one fwd+JVP of the whole batch (one kernel launch, inputs resident in HBM).

Prints ONE JSON line with walkers/s, the roofline of the step (live HIP-event timing on the
launch stream) and a CPU baseline: the jnp path's torch-CPU port (oracle/cpu_baseline.py)
timed on a bounded walker sample of the same inputs on this host's cores; its outputs for
those walkers are compared with the GPU's (``cpu_baseline.check``), outside the timed region.

Beside the hot path (never the default line): ``c2split`` (the reference's two-launch
drop-in, forward then tangent from (out, lse)), ``c2e`` (c2 with the pair bias e and its
tangent), ``gate`` / ``gate_trunk`` (the trunk's sigmoid-gate head collapse fused), ``rect``
(the large-N rectangular forward), ``merge`` (one tree level of the compiled per-walker
executor: quadrilinear merge + residual factorized apply), ``wavefn`` (the whole compiled
per-walker wavefunction: leaf, every merge level, readout), ``trunk`` (the trunk's attention with
its bias produced from the edge features by ln_edge + bias_mlp, then the gated fwd+JVP).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]
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
RECT_METRIC = "rectangular large-N forward (noncausal_bias_mha) query rows/sec; % of MFMA/HBM roofline"
RECT_GATE_METRIC = ("large-N attention tail (rectangular attention + gate collapse fused, W_O) query rows/sec; "
                    "% of MFMA roofline")
EXECUTOR_METRIC = "compiled-executor merge level (quadrilinear merge + factorized apply) walkers/sec; % of MFMA roofline"
WAVEFN_METRIC = ("compiled per-walker wavefunction (leaf, 6 merge levels, readout -> log|psi|, phase) walkers/sec at "
                 "B=1024, 64 sites, fine-tune ranks; % of MFMA roofline")
TRUNK_METRIC = ("trunk attention block after W_QKV (ln_edge + bias_mlp producer, fwd+JVP with the gate collapse, "
                "W_O), walkers/sec at B=1024,L=64; % of MFMA roofline")
VJP_METRIC = "fwd+VJP attention walkers/sec at B=1024,L=64 (fp32 training path); % of MFMA/HBM roofline"
GATE_VJP_METRIC = ("fwd+VJP attention with the sigmoid-gate head collapse and the bias cotangent, walkers/sec at "
                   "B=1024,L=64; % of MFMA/HBM roofline")
TREE_BIAS_METRIC = ("tree coupling-bias producer (normalised pair MLP + LCA-ALiBi, with tangent) walkers/sec at "
                    "B=1024,L=64; % of MFMA roofline")
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2516.6
INFINITY_CACHE_BYTES = 256 << 20


class Config:
    """One benchmark configuration.

    work: fwd | fwd_jvp | fwd_jvp_split | fwd_jvp_gated | fwd_vjp | rect. chunk: walkers
    per launch (the step walks the batch in chunks). with_e: pair bias e [B,N,H,N] (and its
    tangents) present; e_layout "compact": handed to the kernels in the compacted physical-pair
    layout (HZ_FLAG_E_COMPACT, as hz_pair_bias writes it for the trunk). cpu_sample: walkers of
    the CPU baseline's sample."""

    def __init__(self, work, B, N, H, D, n_phys, T, dtype, seed, desc, *, chunk=None, with_e=False,
                 cpu_sample=64, metric=METRIC, d_c=0, e_layout="qhk"):
        self.work, self.B, self.N, self.H, self.D = work, B, N, H, D
        self.n_phys, self.T, self.dtype, self.seed, self.desc = n_phys, T, dtype, seed, desc
        self.chunk = chunk or B
        self.with_e = with_e
        self.cpu_sample = cpu_sample
        self.metric = metric
        self.d_c = d_c
        self.e_layout = e_layout


CONFIGS = {
    "c1": Config("fwd", 256, 8, 4, 32, 8, 0, "f32", 0, "attention forward, fp32, [256,8,4,32], no padding",
                 cpu_sample=256),
    "c2": Config("fwd_jvp", 1024, 64, 8, 32, 36, 1, "f32", 1,
                 "forward + JVP, fp32, [1024,64,8,32], 36/64 physical sites (6x6 lattice)"),
    "c3": Config("fwd_vjp", 4096, 64, 8, 64, 48, 0, "bf16", 2,
                 "forward + VJP, bf16 I/O fp32 accumulate, [4096,64,8,64], 48/64 physical sites", cpu_sample=32),
    "c4": Config("fwd_jvp", 512, 256, 8, 64, 225, 1, "f32", 3,
                 "large-N forward + JVP, fp32, [512,256,8,64], 225/256 physical sites (15x15), "
                 "processed in 32 walker chunks of 16", chunk=16, cpu_sample=4),
    "c5": Config("fwd_jvp", 128, 1024, 16, 64, 1000, 2, "bf16", 4,
                 "large-N stress forward + 2 JVP directions, bf16 I/O, [128,1024,16,64], 1000/1024 sites",
                 cpu_sample=1),
    # The reference's own drop-in route for c2: _outer_jvp binds the primal primitive, then
    # the lin primitive reads (out, lse) back (mhsea_tuned.py:104-118): two launches.
    "c2split": Config("fwd_jvp_split", 1024, 64, 8, 32, 36, 1, "f32", 1,
                      "c2 as the reference's two-launch route: forward (out, lse), then the tangent from "
                      "(out, lse)"),
    # c2 with the pair bias every model call passes (e [B,N,H,N] and its tangent).
    "c2e": Config("fwd_jvp", 1024, 64, 8, 32, 36, 1, "f32", 1,
                  "c2 with the pair bias: e [1024,64,8,64] and its tangent, fp32", with_e=True),
    # The caller-side epilogue of the trunk (trunk.py:134-137) fused into c2's kernel: head h
    # gates head h + H/2, and only y = sigmoid(gate) * value and its tangent are written.
    "gate": Config("fwd_jvp_gated", 1024, 64, 8, 32, 36, 1, "f32", 1,
                   "c2's forward + JVP with the sigmoid-gate head collapse fused, fp32, [1024,64,8,32] -> "
                   "y, ydot [1024,64,4,32], 36/64 physical sites", metric=GATE_METRIC),
    # The trunk's own attention call (config.py:20,26: 16 heads of 16 dims, doubled for the
    # gate) with its pair bias, through the fused collapse.
    "gate_trunk": Config("fwd_jvp_gated", 1024, 64, 32, 16, 36, 1, "f32", 1,
                         "the trunk's attention call: [1024,64,32,16] with pair bias e and its tangent in the "
                         "compacted physical-pair layout (as hz_pair_bias writes it), gate collapse fused -> y, "
                         "ydot [1024,64,16,16], 36/64 physical sites",
                         with_e=True, metric=GATE_METRIC, e_layout="compact"),
    # One tree level of the compiled per-walker executor at the fine-tune ranks: the
    # quadrilinear merge of node pairs and the residual factorized apply
    # (compiled/execute.py:103-104; merge_dim 1536 = 48 groups of rank 32, merge_rank 1024).
    "merge": Config("executor", 1024, 32, 48, 32, 1024, 0, "f32", 6,
                    "compiled-executor merge level: 1024 walkers x 32 node pairs, merge_dim 1536 (48 x 32), "
                    "merge_rank 1024: quadrilinear merge + residual factorized apply", cpu_sample=8,
                    metric=EXECUTOR_METRIC),
    # The whole compiled per-walker wavefunction at the fine-tune sizes (q_to_odd 4 -> 32,
    # leaf rank 1536, merge_dim 1536 = 48 x 32, merge rank 1024, readout rank 64; 64 sites ->
    # 6 merge levels): CompiledFinetuneWaveFunction._forward_plain (compiled/model.py:143-180).
    "wavefn": Config("wavefn", 1024, 64, 48, 32, 1024, 0, "f32", 8,
                     "compiled wavefunction: 1024 walkers x 64 sites, q [1024,64,4] -> leaf (rank 1536) -> 6 merge "
                     "levels (merge_dim 1536, rank 1024) -> readout (rank 64) -> log|psi|, phase", cpu_sample=2,
                     metric=WAVEFN_METRIC),
    # The trunk's attention call with the bias it really receives: the coupling bias produced
    # from the edge features (ln_edge + bias_mlp, trunk.py:89-105; edge_channels 96,
    # bias hidden 64, config.py:28,31) and its tangent, then the gated fwd + JVP.
    "trunk": Config("trunk", 1024, 64, 32, 16, 36, 1, "f32", 7,
                    "the trunk's attention block after W_QKV: edge [1024,64,64,96] and its tangent -> "
                    "ln_edge + bias_mlp -> e, e_t [1024,64,32,64] -> gated fwd+JVP [1024,64,32,16] -> y, ydot "
                    "[1024,64,256] -> W_O [256,512] -> delta, delta_t [1024,64,512], 36/64 physical sites", cpu_sample=4, metric=TRUNK_METRIC),
    # The reference's production gradient path in float32 (jax.value_and_grad through the
    # primitive's transpose rule, optim/production.py:238 -> mhsea_tuned.py:206-221 ->
    # custom_gradients.py:78-347) at c2's shape: forward (out, lse), then the VJP.
    "c2vjp": Config("fwd_vjp", 1024, 64, 8, 32, 36, 0, "f32", 1,
                    "forward + VJP (training), fp32, [1024,64,8,32], 36/64 physical sites: forward (out, lse), "
                    "then dq, dk, dv", metric=VJP_METRIC),
    # The training path with the pair bias every model call passes: its cotangent de is an
    # output too (the bias comes from the trainable pair MLP).
    "c2e_vjp": Config("fwd_vjp", 1024, 64, 8, 32, 36, 0, "f32", 1,
                      "forward + VJP (training) with the pair bias, fp32, [1024,64,8,32], e [1024,64,8,64], "
                      "36/64 physical sites: forward (out, lse), then dq, dk, dv and de", with_e=True,
                      metric=VJP_METRIC),
    # The same training path at c3's shape in float32, the precision the reference trains in
    # (pallas_attention.py:16-19 admits float32 only).
    "c3f32": Config("fwd_vjp", 4096, 64, 8, 64, 48, 0, "f32", 2,
                    "forward + VJP (training), fp32, [4096,64,8,64], 48/64 physical sites: forward (out, lse), "
                    "then dq, dk, dv", cpu_sample=16, metric=VJP_METRIC.replace("B=1024", "B=4096")),
    # The trunk's reverse mode: forward (out, lse) of its attention call, then the gate
    # collapse's cotangent and the attention backward with the bias cotangent de
    # (hz_mhsea_bwd_gated), at [1024,64,32,16] with pair bias.
    "gate_trunk_vjp": Config("fwd_vjp_gated", 1024, 64, 32, 16, 36, 0, "f32", 1,
                             "the trunk's attention call in reverse mode: forward (out, lse) of [1024,64,32,16] "
                             "with pair bias e [1024,64,32,64], then dy [1024,64,16,16] -> collapse cotangent -> "
                             "dq, dk, dv, de, 36/64 physical sites", with_e=True, cpu_sample=16,
                             metric=GATE_VJP_METRIC),
    # The large-N caller's attention tail (sequence_trunk.py:973-984): the rectangular
    # attention with the head collapse fused, then W_O [n_heads * d_head, d_c] (d_c = 512,
    # config.py:19) with the row mask.
    "rect_gate": Config("rect_gate", 1, 4096, 16, 64, 4000, 0, "f32", 5,
                        "large-N attention tail: rectangular attention with the gate collapse fused (one system, "
                        "Nq=Nk=4096, H=16 -> 8 gated heads, D=64, dense bias, 4000/4096 physical sites) -> y "
                        "[4096,8,64] -> W_O [512,512] on the physical rows", metric=RECT_GATE_METRIC, d_c=512),
    # The tree's LevelEdgeAttn coupling bias (tree.py:1392-1456): the normalised MLP over the
    # edge features (edge_channels 96 -> hidden 128 (level_edge_bias_mlp_dim) -> 16 heads, one
    # block, config.py:25,82-83), / sqrt(d_head), + LCA-ALiBi, with its forward-mode tangent;
    # D holds the hidden width and d_c the edge channels.
    "tree_bias": Config("pair_mlp", 1024, 64, 16, 128, 36, 1, "f32", 9,
                        "the tree's coupling-bias producer: edge [1024,64,64,96] and its tangent -> normalised MLP "
                        "(96 -> 128, one block, -> 16 heads) / sqrt(16) + LCA-ALiBi -> e, e_t [1024,64,64,16], "
                        "36/64 physical sites (square mask: the 36 x 36 pairs the attention reads)", cpu_sample=8,
                        metric=TREE_BIAS_METRIC, d_c=96),
    # The large-N evaluation forward (noncausal_bias_mha via pallas_rectangular_edge_attention):
    # one system, all queries against all keys, dense [Nq, Nk, H] bias.
    "rect": Config("rect", 1, 4096, 16, 64, 4000, 0, "f32", 5,
                   "rectangular forward with dense bias, fp32, one system, Nq=Nk=4096, H=16, D=64, "
                   "4000/4096 physical keys", metric=RECT_METRIC),
}


# Untimed run of the step before its warmup steps, in milliseconds of wall time. MI355X
# boosts its clock for the first milliseconds of a heavy load and then throttles below the
# level it settles at (c2: ~103 us per step over the first 2 ms, ~108 us over the next 5 ms,
# ~100 us once settled), so K steps timed straight after a short warmup measure that
# transient instead of the sustained rate a long walker run sees. Set by --settle-ms.
SETTLE_MS = 100.0


def timed(step, steps, warmup, stream):
    """Average milliseconds of ``step`` over ``steps`` steps after ``warmup``, with HIP
    events recorded on the launch stream, bracketed by device synchronisation. Before the
    warmup steps the step runs untimed for ``SETTLE_MS`` of wall time."""
    import time

    import torch

    torch.cuda.synchronize()
    t_end = time.perf_counter() + SETTLE_MS / 1e3
    while time.perf_counter() < t_end:
        for _ in range(8):
            step(0)
        torch.cuda.synchronize()
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def algorithmic(work, B, N, H, D, n_phys, T, esize, with_e=False, e_compact=False):
    """Algorithmic bytes and flops of one step.

    padded: every [B,N,H,D] tensor read or written once at the padded shape, plus the mask
            (uint8) and, with a bias, e and its T tangents [B,N,H,N] read once (e_compact:
            the compacted physical-pair layout holds only the physical pairs, so its bias
            counts n_phys^2 entries per (walker, head) in both figures); flops
            (2 + 4T) G for fwd+JVP, 2G fwd, 6G fwd+VJP, G = 2 N^2 D per (walker, head),
            recompute not counted.
    effective: the same with the mask taken into account — inputs are needed only on
            physical rows (a masked row never influences a result), bias entries only on
            physical pairs, outputs are written on every row (zeros included), and only
            physical x physical pairs carry flops.
    The two-launch route (fwd_jvp_split) is charged the fused figure: out and lse are its
    own intermediates.
    """
    rowb = H * D * esize  # bytes of one site row of one [B,N,H,D] tensor
    if work == "fwd":
        n_in, n_out, g_mult, lse_b, n_e = 3, 1, 2, 0, 1
    elif work in ("fwd_jvp", "fwd_jvp_split"):
        n_in, n_out, g_mult, lse_b, n_e = 3 + 3 * T, 1 + T, 2 + 4 * T, 0, 1 + T
    elif work == "fwd_jvp_gated":  # outputs are y and its T tangents, each half a [B,N,H,D] tensor
        n_in, n_out, g_mult, lse_b, n_e = 3 + 3 * T, (1 + T) / 2, 2 + 4 * T, 0, 1 + T
    elif work == "fwd_vjp":
        # fwd: q,k,v in, out + lse out; bwd: q,k,v,out,dout + lse in, dq,dk,dv out
        n_in, n_out, g_mult, lse_b, n_e = 3 + 5, 1 + 3, 6, 2 * N * H * 4, 2
    elif work == "fwd_vjp_gated":
        # fwd: q,k,v,e in, out + lse out; bwd: q,k,v,e,out + lse and dy (half a tensor) in,
        # dq,dk,dv and de out (de written on every pair, zeros included)
        n_in, n_out, g_mult, lse_b, n_e = 3 + 4.5, 1 + 3, 6, 2 * N * H * 4, 2
    else:
        raise ValueError(work)
    n_e_out = 1 if work in ("fwd_vjp", "fwd_vjp_gated") else 0  # de (every pair) when the bias is an input
    e_eff = (n_e * n_phys * n_phys + n_e_out * N * N) * H * esize if with_e else 0
    e_pad = e_eff if e_compact else ((n_e + n_e_out) * N * H * N * esize if with_e else 0)
    padded_bytes = int(B * (N * rowb * (n_in + n_out) + N + lse_b + e_pad))
    eff_bytes = int(B * (n_phys * rowb * n_in + N * rowb * n_out + N + lse_b + e_eff))
    padded_flops = B * H * g_mult * 2 * N * N * D
    eff_flops = B * H * g_mult * 2 * n_phys * n_phys * D
    return dict(padded_bytes=padded_bytes, eff_bytes=eff_bytes, padded_flops=padded_flops,
                eff_flops=eff_flops)


def rect_algorithmic(B, Nq, Nk, H, D, n_phys):
    """Bytes and flops of one rectangular forward. padded: q, k, v, out and the bias
    [Nq, Nk, H] moved once, the key mask as uint8, 4 Nq Nk D flops per (system, head);
    effective: only physical keys' k, v and bias columns, and their flops."""
    row = H * D * 4
    padded_bytes = B * (2 * Nq * row + 2 * Nk * row + Nq * Nk * H * 4 + Nk)
    eff_bytes = B * (2 * Nq * row + 2 * n_phys * row + Nq * n_phys * H * 4 + Nk)
    return dict(padded_bytes=padded_bytes, eff_bytes=eff_bytes,
                padded_flops=B * H * 4 * Nq * Nk * D, eff_flops=B * H * 4 * Nq * n_phys * D)


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
    """HBM bytes per step measured by rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE), scaled by
    the copy-kernel calibration, if a summary for this configuration is committed."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        rec = json.load(fh)
    return rec.get("traffic_bytes_per_launch")


def issued_flops_from_profile(config):
    """Matrix flops the kernels of one step issue (rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_*
    x 512, summed over the step's launches), if the committed profile summary records them.
    Differs from the algorithmic flops where MFMA tiles carry padding rows."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        return json.load(fh).get("mfma_flops_issued_per_step")


def copy_probe(mib, steps, warmup):
    """Device-to-device copies of a known size (hipMemcpyAsync -> the runtime's copyBuffer
    kernel): reads and writes exactly ``mib`` MiB per launch. Profiled under rocprofv3
    --pmc it gives the factor between FETCH_SIZE / WRITE_SIZE and real bytes."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    ms = timed(lambda i: dst.copy_(src), steps, warmup, torch.cuda.current_stream())
    nbytes = n * 4
    print(json.dumps({"copy_probe_bytes": nbytes, "ms_per_copy": ms,
                      "gbs_read_plus_write": 2 * nbytes / ms / 1e6}), flush=True)
    return 0


def rel_err(got, want):
    """max |got - want| / max |want| (float64)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def draw_inputs(cfg):
    """Synthetic inputs: default_rng(seed); draw order q, k, v, tangents (per direction
    qt, kt, vt), the cotangent (fwd+VJP), then the bias e and its tangents (bias configs);
    q/k/v scaled by 1/sqrt(D), tangents, cotangent and bias N(0,1) (the bias x 1/2).
    bf16 configurations round the float32 draws to bf16 (nearest even)."""
    import torch

    rng = np.random.default_rng(cfg.seed)
    shape = (cfg.B, cfg.N, cfg.H, cfg.D)
    eshape = (cfg.B, cfg.N, cfg.H, cfg.N)

    def draw(sh, scale):
        x = rng.standard_normal(sh, dtype=np.float32)
        if scale != 1.0:
            x *= np.float32(scale)
        if cfg.dtype == "bf16":
            x = torch.from_numpy(x).bfloat16().float().numpy()
        return x

    a = {"q": draw(shape, cfg.D ** -0.5), "k": draw(shape, cfg.D ** -0.5), "v": draw(shape, cfg.D ** -0.5)}
    if cfg.T:
        tans = [[draw(shape, 1.0) for _ in range(3)] for _ in range(cfg.T)]
        for i, nm in enumerate(("qt", "kt", "vt")):
            a[nm] = np.stack([t[i] for t in tans])
    if cfg.work == "fwd_vjp":
        a["dout"] = draw(shape, 1.0)
    if cfg.work == "fwd_vjp_gated":
        a["dy"] = draw((cfg.B, cfg.N, cfg.H // 2, cfg.D), 1.0)
    if cfg.with_e:
        a["e"] = draw(eshape, 0.5)
        if cfg.T:
            a["et"] = np.stack([draw(eshape, 1.0) for _ in range(cfg.T)])
    mask = np.zeros((cfg.B, cfg.N), dtype=bool)
    mask[:, :cfg.n_phys] = True
    a["mask"] = mask
    return a


def run_attention(args, cfg):
    import torch

    from hamiltonzero_amd import _native, kernels

    lib = _native.lib()
    tdt = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    hz_dtype = _native.HZ_DTYPE_BF16 if cfg.dtype == "bf16" else _native.HZ_DTYPE_F32
    esize = 2 if cfg.dtype == "bf16" else 4
    dev = torch.device("cuda:0")
    B, N, H, D, T = cfg.B, cfg.N, cfg.H, cfg.D, cfg.T
    shape = (B, N, H, D)
    host = draw_inputs(cfg)

    # Configurations whose touched bytes per step (the mask-aware figure: the kernels read
    # physical rows only) are below twice the 256 MB Infinity Cache run on enough copies of
    # their buffers, used in turn, that no step finds its inputs left in the cache by the
    # previous steps. --buffer-sets overrides the count (1: every step on the same buffers).
    alg = algorithmic(cfg.work, B, N, H, D, cfg.n_phys, T, esize, cfg.with_e,
                      e_compact=cfg.with_e and cfg.e_layout == "compact")
    copies = max(1, -(-2 * INFINITY_CACHE_BYTES // alg["eff_bytes"]))
    if args.buffer_sets:
        copies = args.buffer_sets

    compact = cfg.with_e and cfg.e_layout == "compact"

    def dev_set():
        d = {}
        for nm, x in host.items():
            if nm == "mask":
                d[nm] = torch.from_numpy(x.astype(np.uint8)).to(dev)
            else:
                d[nm] = torch.from_numpy(x).to(device=dev, dtype=tdt).contiguous()
        if compact:  # the layout conversion happens once, outside the timed steps
            m = d["mask"]
            d["e"] = kernels.compact_bias(d["e"], m)
            if "et" in d:
                d["et"] = torch.stack([kernels.compact_bias(x, m) for x in d["et"]])
        d["out"] = torch.empty(shape, dtype=tdt, device=dev)
        d["lse"] = torch.empty((B, N, H), dtype=torch.float32, device=dev)
        if cfg.work in ("fwd_jvp", "fwd_jvp_split"):
            d["tout"] = torch.empty((T, *shape), dtype=tdt, device=dev)
        if cfg.work == "fwd_jvp_gated":
            del d["out"]
            d["y"] = torch.empty((B, N, H // 2, D), dtype=tdt, device=dev)
            d["ty"] = torch.empty((T, B, N, H // 2, D), dtype=tdt, device=dev)
        if cfg.work in ("fwd_vjp", "fwd_vjp_gated"):
            for nm in ("dq", "dk", "dv"):
                d[nm] = torch.empty(shape, dtype=tdt, device=dev)
        if cfg.work == "fwd_vjp_gated":
            d["dout_work"] = torch.empty(shape, dtype=torch.float32, device=dev)
        if cfg.work in ("fwd_vjp", "fwd_vjp_gated") and cfg.with_e:
            d["de"] = torch.empty((B, N, H, N), dtype=tdt, device=dev)
        return d

    sets = [dev_set() for _ in range(copies)]
    stream = torch.cuda.current_stream(dev)
    s = stream.cuda_stream
    fl = _native.HZ_FLAG_GENERIC if args.generic else 0
    fl_e = _native.HZ_FLAG_E_COMPACT if compact else 0
    row = N * H * D * esize  # bytes of one walker of a [B,N,H,D] tensor
    erow = int(np.prod(kernels.e_shape(1, N, H, cfg.e_layout if cfg.with_e else "qhk"))) * esize  # one walker of e

    def P(d, nm, b0=0, per=row):
        t = d.get(nm)
        return None if t is None else t.data_ptr() + b0 * per

    def launch(d, b0, nb):
        """One launch of the step's entry point(s) on walkers [b0, b0 + nb) of buffer set d.
        Tangent operands keep their stride B*N*H*D between directions only when nb == B."""
        assert T <= 1 or nb == B, "chunked launches assume one tangent direction"
        q, k, v, m = P(d, "q", b0), P(d, "k", b0), P(d, "v", b0), P(d, "mask", b0, N)
        e, et = P(d, "e", b0, erow), P(d, "et", b0, erow)
        if cfg.work == "fwd":
            _native.check(lib.hz_mhsea_fwd(s, q, k, e, v, m, P(d, "out", b0), None, nb, N, H, D, hz_dtype, 1.0, fl))
        elif cfg.work == "fwd_jvp":
            _native.check(lib.hz_mhsea_fwd_jvp(s, q, k, e, v, m, P(d, "qt", b0), P(d, "kt", b0), et, P(d, "vt", b0),
                                               T, P(d, "out", b0), None, P(d, "tout", b0), nb, N, H, D, hz_dtype,
                                               1.0, fl))
        elif cfg.work == "fwd_jvp_split":
            lse = P(d, "lse", b0, N * H * 4)
            _native.check(lib.hz_mhsea_fwd(s, q, k, e, v, m, P(d, "out", b0), lse, nb, N, H, D, hz_dtype, 1.0, fl))
            _native.check(lib.hz_mhsea_jvp(s, q, k, e, v, m, P(d, "out", b0), lse, P(d, "qt", b0), P(d, "kt", b0),
                                           et, P(d, "vt", b0), T, P(d, "tout", b0), nb, N, H, D, hz_dtype, 1.0, fl))
        elif cfg.work == "fwd_jvp_gated":
            _native.check(lib.hz_mhsea_fwd_jvp_gated(s, q, k, e, v, m, P(d, "qt", b0), P(d, "kt", b0), et,
                                                     P(d, "vt", b0), T, P(d, "y", b0, row // 2),
                                                     P(d, "ty", b0, row // 2), nb, N, H, D, 1.0, fl | fl_e))
        elif cfg.work == "fwd_vjp_gated":
            lse = P(d, "lse", b0, N * H * 4)
            _native.check(lib.hz_mhsea_fwd(s, q, k, e, v, m, P(d, "out", b0), lse, nb, N, H, D, hz_dtype, 1.0, fl))
            _native.check(lib.hz_mhsea_bwd_gated(s, q, k, e, v, m, lse, P(d, "out", b0), P(d, "dy", b0, row // 2),
                                                 P(d, "dq", b0), P(d, "dk", b0), P(d, "de", b0, erow),
                                                 P(d, "dv", b0), P(d, "dout_work", b0), nb, N, H, D, 1.0, fl))
        else:
            lse = P(d, "lse", b0, N * H * 4)
            _native.check(lib.hz_mhsea_fwd(s, q, k, e, v, m, P(d, "out", b0), lse, nb, N, H, D, hz_dtype, 1.0, fl))
            _native.check(lib.hz_mhsea_bwd(s, q, k, e, v, m, lse, P(d, "out", b0), P(d, "dout", b0), P(d, "dq", b0),
                                           P(d, "dk", b0), P(d, "de", b0, erow), P(d, "dv", b0), nb, N, H, D,
                                           hz_dtype, 1.0, fl))

    def step(i):
        d = sets[i % copies]
        for b0 in range(0, B, cfg.chunk):
            launch(d, b0, min(cfg.chunk, B - b0))

    ms = timed(step, args.steps, args.warmup, stream)
    t_s = ms / 1e3

    roof = roofline(alg["padded_bytes"], alg["padded_flops"], t_s, cfg.dtype)
    roof["traffic"] = traffic_from_profile(args.config)
    roof["basis"] = "padded algorithmic bytes/flops per walker x B (every row of every tensor once)"
    roof["bytes_per_step"] = alg["padded_bytes"]
    roof["flops_per_step"] = alg["padded_flops"]
    roof_mask = roofline(alg["eff_bytes"], alg["eff_flops"], t_s, cfg.dtype)
    roof_mask["basis"] = "mask-aware algorithmic bytes/flops (physical rows and pairs in, all rows out)"
    roof_mask["bytes_per_step"] = alg["eff_bytes"]
    roof_mask["flops_per_step"] = alg["eff_flops"]
    issued = issued_flops_from_profile(args.config)
    if issued:
        peak_c = BF16_PEAK_TFLOPS if cfg.dtype == "bf16" else FP32_PEAK_TFLOPS
        roof["issued"] = {"basis": "matrix flops the kernels issue (rocprofv3 MFMA MOPS x 512, profiles/)",
                          "flops_per_step": issued, "achieved": issued / t_s / 1e12, "unit": "TFLOP/s",
                          "peak": peak_c, "frac": issued / t_s / 1e12 / peak_c}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_leg(args, cfg, host, sets[0])

    line = {
        "metric": cfg.metric,
        "value": B / t_s,
        "unit": "walkers/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup, "settle_ms": args.settle_ms,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == "bf16" else "f32",
        "data": "synthetic (numpy default_rng, N(0,1)/sqrt(D) q/k/v, N(0,1) tangents)",
        "config": {"workload": f"{args.config}: {cfg.desc}", "B": B, "N": N, "H": H, "D": D,
                   "n_phys": cfg.n_phys, "T": T, "work": cfg.work, "walkers_per_launch": cfg.chunk,
                   "bias": cfg.with_e, "buffer_sets": copies, "touched_bytes_per_set": alg["eff_bytes"],
                   "kernels": "generic" if args.generic else "auto"},
        "roofline": roof,
        "roofline_mask_aware": roof_mask,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_leg(args, cfg, host, dset):
    """Time the torch-CPU port of the jnp path on the first walkers of the bench's own
    inputs and compare its outputs with the GPU's outputs of those walkers."""
    import torch

    from oracle import cpu_baseline

    n = min(cfg.cpu_sample, cfg.B)
    work = "fwd_jvp" if cfg.work == "fwd_jvp_split" else cfg.work
    inputs = {nm: torch.from_numpy(np.ascontiguousarray(x[:, :n] if nm in ("qt", "kt", "vt", "et") else x[:n]))
              for nm, x in host.items()}
    r = cpu_baseline.time_walkers_per_s(work, inputs, budget_s=args.cpu_budget)
    tol = 2e-2 if cfg.dtype == "bf16" else 1e-5
    errs = {}
    for nm, want in r["outputs"].items():
        got = dset[nm].float().cpu().numpy()
        got = got[:, :n] if nm in ("tout", "ty") else got[:n]
        errs[nm] = rel_err(got, want.numpy())
    bf16_note = " (fp32 on the bf16-rounded inputs)" if cfg.dtype == "bf16" else ""
    return {
        "value": r["walkers_per_s"],
        "unit": "walkers/s",
        "cores": r["threads"],
        "kind": "port",
        "sample": f"the first {n} walkers of the same inputs, {r['reps']} reps in {r['seconds']:.1f} s, torch-CPU "
                  f"fp32 port of the jnp path{bf16_note} ({r['cpu_model']})",
        "host_cpus": r["host_cpus"],
        "check": {"max_rel_err_vs_gpu": errs, "tol": tol, "ok": all(e <= tol for e in errs.values())},
    }


def run_rect(args, cfg):
    """Bench leg of the rectangular forward (hz_rect_attention_fwd)."""
    import torch

    from hamiltonzero_amd import _native

    lib = _native.lib()
    dev = torch.device("cuda:0")
    B, N, H, D, n_phys = cfg.B, cfg.N, cfg.H, cfg.D, cfg.n_phys
    rng = np.random.default_rng(cfg.seed)

    def draw(shape, scale):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))

    qh, kh, vh = draw((B, N, H, D), 1.0), draw((B, N, H, D), 1.0), draw((B, N, H, D), 1.0)
    biash = draw((B, N, N, H), D ** -0.5)
    maskh = torch.zeros((B, N), dtype=torch.bool)
    maskh[:, :n_phys] = True
    q, k, v, bias = (x.to(dev) for x in (qh, kh, vh, biash))
    mask = maskh.to(torch.uint8).to(dev)
    out = torch.empty_like(q)
    s = torch.cuda.current_stream(dev).cuda_stream
    scale = D ** -0.5

    def step(i):
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

        sample = 64
        r = cpu_baseline.time_rect_queries_per_s(qh[:, :sample], kh, vh, biash[:, :sample], maskh, scale,
                                                 budget_s=args.cpu_budget)
        err = rel_err(out[:, :sample].cpu().numpy(), r["out"].numpy())
        cpu = {"value": r["queries_per_s"], "unit": "queries/s", "cores": r["threads"], "kind": "port",
               "sample": f"the first {sample} query rows of the same system against all {N} keys, {r['reps']} reps "
                         f"in {r['seconds']:.1f} s, torch-CPU fp32 port of the jnp formula ({r['cpu_model']})",
               "host_cpus": r["host_cpus"],
               "check": {"max_rel_err_vs_gpu": {"out": err}, "tol": 1e-5, "ok": err <= 1e-5}}
    line = {
        "metric": cfg.metric, "value": B * N / t_s, "unit": "queries/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": args.settle_ms, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (numpy default_rng, N(0,1) q/k/v, N(0,1)/sqrt(D) bias)",
        "config": {"workload": f"rect: {cfg.desc}", "B": B, "Nq": N, "Nk": N, "H": H, "D": D, "n_phys": n_phys},
        "roofline": roof, "roofline_mask_aware": roof_mask, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_rect_gate(args, cfg):
    """Bench leg of the large-N attention tail (sequence_trunk.py:973-984): the rectangular
    attention with the head collapse fused (hz_rect_attention_fwd_gated), then W_O with the
    row mask (hz_gated_out_proj). The roofline is the gated attention kernel's, timed on its
    own over the same number of launches."""
    import torch

    from hamiltonzero_amd import _native

    lib = _native.lib()
    dev = torch.device("cuda:0")
    B, N, H, D, n_phys, d_c = cfg.B, cfg.N, cfg.H, cfg.D, cfg.n_phys, cfg.d_c
    hh = H // 2
    rng = np.random.default_rng(cfg.seed)

    def draw(shape, scale):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))

    qh, kh, vh = draw((B, N, H, D), 1.0), draw((B, N, H, D), 1.0), draw((B, N, H, D), 1.0)
    biash = draw((B, N, N, H), D ** -0.5)
    w_oh = draw((hh * D, d_c), (hh * D) ** -0.5)
    maskh = torch.zeros((B, N), dtype=torch.bool)
    maskh[:, :n_phys] = True
    q, k, v, bias, w_o = (x.to(dev) for x in (qh, kh, vh, biash, w_oh))
    mask = maskh.to(torch.uint8).to(dev)
    y = torch.empty((B, N, hh, D), dtype=torch.float32, device=dev)
    proj = torch.empty((B, N, d_c), dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    scale = D ** -0.5

    def attend(i):
        _native.check(lib.hz_rect_attention_fwd_gated(s, q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
                                                      mask.data_ptr(), y.data_ptr(), B, N, N, H, D, scale))

    def project(i):
        _native.check(lib.hz_gated_out_proj(s, y.data_ptr(), None, w_o.data_ptr(), mask.data_ptr(), proj.data_ptr(),
                                            None, B, N, hh * D, d_c, 0))

    def step(i):
        attend(i)
        project(i)

    stream = torch.cuda.current_stream(dev)
    ms = timed(step, args.steps, args.warmup, stream)
    ms_att = timed(attend, args.steps, args.warmup, stream)
    ms_proj = timed(project, args.steps, args.warmup, stream)
    t_s = ms / 1e3
    # the gated kernel: q, k, v, the bias and y once; 4 Nq Nk D flops per (system, head)
    att_pad = dict(bytes=B * (N * H * D * 4 * 3 + N * N * H * 4 + N * hh * D * 4 + N), flops=B * H * 4 * N * N * D)
    att_eff = dict(bytes=B * (N * H * D * 4 + 2 * n_phys * H * D * 4 + N * n_phys * H * 4 + N * hh * D * 4 + N),
                   flops=B * H * 4 * N * n_phys * D)
    roof = roofline(att_pad["bytes"], att_pad["flops"], ms_att / 1e3, "f32")
    roof.update({"kernel": "rect_attention_fwd_kernel (gated)", "traffic": traffic_from_profile(args.config),
                 "basis": "padded algorithmic bytes/flops of the gated attention kernel (q, k, v, bias, y once)",
                 "bytes_per_launch": att_pad["bytes"], "flops_per_launch": att_pad["flops"],
                 "step": {"attention_ms": ms_att, "out_proj_ms": ms_proj,
                          "out_proj_flops": 2 * B * n_phys * hh * D * d_c}})
    roof_mask = roofline(att_eff["bytes"], att_eff["flops"], ms_att / 1e3, "f32")
    roof_mask["basis"] = "mask-aware (physical keys' k, v, bias columns and flops only)"
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        sample = 64
        r = cpu_baseline.time_rect_block_queries_per_s(qh[:, :sample], kh, vh, biash[:, :sample], maskh, scale,
                                                       w_oh, maskh[:, :sample], budget_s=args.cpu_budget)
        err_y = rel_err(y[:, :sample].cpu().numpy(), r["y"].numpy())
        err_p = rel_err(proj[:, :sample].cpu().numpy(), r["proj"].numpy())
        cpu = {"value": r["queries_per_s"], "unit": "queries/s", "cores": r["threads"], "kind": "port",
               "sample": f"the first {sample} query rows of the same system against all {N} keys, {r['reps']} reps "
                         f"in {r['seconds']:.1f} s, torch-CPU fp32 port (attention, collapse, W_O) ({r['cpu_model']})",
               "host_cpus": r["host_cpus"],
               "check": {"max_rel_err_vs_gpu": {"y": err_y, "proj": err_p}, "tol": 1e-5,
                         "ok": err_y <= 1e-5 and err_p <= 1e-5}}
    line = {
        "metric": cfg.metric, "value": B * N / t_s, "unit": "queries/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": args.settle_ms, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (numpy default_rng, N(0,1) q/k/v, N(0,1)/sqrt(D) bias, N(0,1)/sqrt(fan_in) W_O)",
        "config": {"workload": f"{args.config}: {cfg.desc}", "B": B, "Nq": N, "Nk": N, "H": H, "D": D,
                   "n_phys": n_phys, "d_c": d_c},
        "roofline": roof, "roofline_mask_aware": roof_mask, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_pair_mlp(args, cfg):
    """Bench leg of the MLP-class bias producer (hz_pair_mlp_bias) at the tree's shape: edge
    [B, N, N, C] and its tangent -> bias and tangent [B, N, N, H] (the reference's layout) on
    the pairs the square-mask attention reads, with the LCA-ALiBi term."""
    import torch

    from hamiltonzero_amd import _native

    lib = _native.lib()
    dev = torch.device("cuda:0")
    B, N, H, n_phys, C, Hd, nb = cfg.B, cfg.N, cfg.H, cfg.n_phys, cfg.d_c, cfg.D, 1
    d_head = 16
    rng = np.random.default_rng(cfg.seed)

    def w(*shape):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(shape[-2] ** -0.5))

    def small(*shape):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(0.1))

    ph = {"w_in": w(C, Hd), "b_in": small(Hd), "norm_w": 1.0 + small(nb, Hd), "w_1": w(nb, Hd, Hd),
          "b_1": small(nb, Hd), "w_2": w(nb, Hd, Hd), "b_2": small(nb, Hd), "out_norm_w": 1.0 + small(Hd),
          "w_out": w(Hd, H), "b_out": small(H)}
    names = ("w_in", "b_in", "norm_w", "w_1", "b_1", "w_2", "b_2", "out_norm_w", "w_out", "b_out")
    p = {k: v.to(dev) for k, v in ph.items()}
    edge = torch.randn((B, N, N, C), device=dev, generator=torch.Generator(device=dev).manual_seed(cfg.seed))
    edge_t = torch.randn((B, N, N, C), device=dev, generator=torch.Generator(device=dev).manual_seed(cfg.seed + 1))
    maskh = torch.zeros((B, N), dtype=torch.bool)
    maskh[:, :n_phys] = True
    mask = maskh.to(torch.uint8).to(dev)
    slopes_h = 1.5 * torch.exp2(-(torch.arange(H, dtype=torch.float32) * 4.0 / max(H - 1, 1)))
    slopes = slopes_h.to(dev)
    e = torch.zeros((B, N, N, H), dtype=torch.float32, device=dev)
    e_t = torch.zeros_like(e)
    div = float(np.sqrt(np.float32(d_head)))
    s = torch.cuda.current_stream(dev).cuda_stream

    def step(i):
        _native.check(lib.hz_pair_mlp_bias(s, edge.data_ptr(), edge_t.data_ptr(), None, None, mask.data_ptr(),
                                           *(p[k].data_ptr() for k in names), slopes.data_ptr(), e.data_ptr(),
                                           e_t.data_ptr(), B, N, N, C, Hd, H, nb, 1, 0, 1.0, 1e-5, div,
                                           _native.HZ_FLAG_E_QKH))

    ms = timed(step, args.steps, args.warmup, torch.cuda.current_stream(dev))
    t_s = ms / 1e3
    pairs = B * n_phys * n_phys
    flops_pair = 2 * 2 * (C * Hd + 2 * nb * Hd * Hd + Hd * H)  # primal and tangent
    bytes_pair = 4 * (2 * C + 2 * H)
    roof = roofline(pairs * bytes_pair, pairs * flops_pair, t_s, "f32")
    roof.update({"kernel": "pair_mlp_bias_kernel", "traffic": traffic_from_profile(args.config),
                 "basis": f"computed pairs ({pairs}: the {n_phys} x {n_phys} physical pairs of each walker) x "
                          f"{flops_pair} flops / {bytes_pair} bytes (edge, edge_t in; e, e_t out)",
                 "bytes_per_step": pairs * bytes_pair, "flops_per_step": pairs * flops_pair,
                 "reference_equivalent": {"pairs": B * N * N, "flops_per_step": B * N * N * flops_pair}})
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        n = cfg.cpu_sample
        eh, eth = edge[:n, :n_phys, :n_phys].cpu().contiguous(), edge_t[:n, :n_phys, :n_phys].cpu().contiguous()
        r = cpu_baseline.time_mlp_pair_bias_walkers_per_s(eh, eth, ph, 1.0, div, slopes_h, budget_s=args.cpu_budget)
        got, got_t = e[:n, :n_phys, :n_phys].cpu().numpy(), e_t[:n, :n_phys, :n_phys].cpu().numpy()
        errs = {"e": rel_err(got, r["e"].numpy()), "e_t": rel_err(got_t, r["e_t"].numpy())}
        cpu = {"value": r["walkers_per_s"], "unit": "walkers/s", "cores": r["threads"], "kind": "port",
               "sample": f"the physical {n_phys} x {n_phys} pairs of the first {n} walkers, {r['reps']} reps in "
                         f"{r['seconds']:.1f} s, torch-CPU fp32 port of the MLP, ALiBi and torch.func.jvp "
                         f"({r['cpu_model']})",
               "host_cpus": r["host_cpus"], "check": {"max_rel_err_vs_gpu": errs, "tol": 1e-5,
                                                      "ok": all(v <= 1e-5 for v in errs.values())}}
    line = {
        "metric": cfg.metric, "value": B / t_s, "unit": "walkers/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": args.settle_ms, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (torch N(0,1) edge and tangent; numpy default_rng weights N(0,1)/sqrt(fan_in))",
        "config": {"workload": f"{args.config}: {cfg.desc}", "B": B, "N": N, "C": C, "hidden": Hd, "H": H,
                   "n_blocks": nb, "n_phys": n_phys, "T": 1},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_executor(args, cfg):
    """Bench leg of one compiled-executor tree level (hz_quadrilinear_merge, hz_factorized_apply).
    Config fields: B walkers, N node pairs (width), H groups, D rank d_r, n_phys merge_rank."""
    import torch

    from hamiltonzero_amd import _native

    lib = _native.lib()
    dev = torch.device("cuda:0")
    B, W, G, R, Rm = cfg.B, cfg.N, cfg.H, cfg.D, cfg.n_phys
    dm = G * R
    M = B * W
    rng = np.random.default_rng(cfg.seed)

    def draw(shape, scale):
        return rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)

    host = {"T": draw((G, R, R, R), 1.0 / R), "ul": draw((M, dm), 1.0), "ur": draw((M, dm), 1.0),
            "V": draw((dm, Rm), dm ** -0.5), "U": draw((Rm, dm), Rm ** -0.5), "h": draw((W, Rm), 1.0)}
    d = {k: torch.from_numpy(v).to(dev) for k, v in host.items()}
    raw = torch.empty((M, dm), dtype=torch.float32, device=dev)
    out = torch.empty_like(raw)
    work = torch.empty((M, Rm), dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def merge(i):
        _native.check(lib.hz_quadrilinear_merge(s, P(d["T"]), P(d["ul"]), P(d["ur"]), P(raw), M, G, R))

    def apply(i):
        _native.check(lib.hz_factorized_apply(s, P(raw), P(d["V"]), P(d["h"]), P(d["U"]), P(raw), P(out), P(work),
                                              M, dm, Rm, dm, W))

    def step(i):
        merge(i)
        apply(i)

    stream = torch.cuda.current_stream(dev)
    ms = timed(step, args.steps, args.warmup, stream)
    t_s = ms / 1e3
    merge_flops = 2 * M * G * R ** 3
    apply_flops = 2 * M * (dm * Rm + Rm * dm)
    flops = merge_flops + apply_flops
    bytes_ = 4 * (3 * M * dm + G * R ** 3 + 2 * dm * Rm + W * Rm)  # u_left, u_right, out; T, V, U, h
    # The dominant kernel, the merge, timed on its own over the same number of launches.
    ms_merge = timed(merge, args.steps, args.warmup, stream)
    ms_apply = timed(apply, args.steps, args.warmup, stream)
    roof = roofline(4 * (3 * M * dm + G * R ** 3), merge_flops, ms_merge / 1e3, "f32")
    roof["traffic"] = traffic_from_profile(args.config)
    roof["kernel"] = "hz::quadrilinear_merge_kernel"
    roof["basis"] = ("algorithmic flops of the merge launch, 2 M G d_r^3 (d_r outputs per group, each a "
                     "contraction over the d_r^2 pairs k, l), per average launch duration")
    roof["step"] = {"ms": ms, "flops": flops, "bytes": bytes_, "tflops": flops / t_s / 1e12,
                    "merge_ms": ms_merge, "apply_ms": ms_apply,
                    "apply_tflops": apply_flops / (ms_apply / 1e3) / 1e12}
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        n = cfg.cpu_sample
        rows = n * W
        r = cpu_baseline.time_executor_level(torch.from_numpy(host["T"]), torch.from_numpy(host["ul"][:rows]),
                                             torch.from_numpy(host["ur"][:rows]), torch.from_numpy(host["V"]),
                                             torch.from_numpy(host["U"]), torch.from_numpy(host["h"]),
                                             budget_s=args.cpu_budget)
        err = rel_err(out[:rows].cpu().numpy(), r["out"].numpy())
        cpu = {"value": n * r["reps"] / r["seconds"],
               "unit": "walkers/s", "cores": r["threads"], "kind": "port",
               "sample": f"the first {n} walkers ({rows} node pairs) of the same inputs, {r['reps']} reps in "
                         f"{r['seconds']:.1f} s, torch-CPU fp32 einsum + matmul ({r['cpu_model']})",
               "host_cpus": r["host_cpus"],
               "check": {"max_rel_err_vs_gpu": {"out": err}, "tol": 1e-5, "ok": err <= 1e-5}}
    line = {
        "metric": cfg.metric, "value": B / t_s, "unit": "walkers/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": args.settle_ms, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (numpy default_rng; T ~ N(0,1)/d_r, unit carriers)",
        "config": {"workload": f"{args.config}: {cfg.desc}", "walkers": B, "node_pairs": W, "groups": G, "d_r": R,
                   "merge_rank": Rm},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_trunk(args, cfg):
    """Bench leg of the trunk attention with its produced bias: hz_pair_bias (edge, edge_t ->
    e, e_t in the compacted physical-pair layout), hz_mhsea_fwd_jvp_gated, then W_O
    (hz_gated_out_proj).
    Config: B, N, H (kernel heads), D (d_head), n_phys, T = 1; edge channels 96, bias hidden
    64. W_O receives the site mask: the gated attention writes the masked sites' rows of y as
    exact zeros and W_O has no bias (trunk.py:54), so the masked product, which skips those
    rows, equals the reference's unmasked W_O."""
    import torch

    from hamiltonzero_amd import _native, kernels

    lib = _native.lib()
    dev = torch.device("cuda:0")
    B, N, H, D, n_phys, C, HID = cfg.B, cfg.N, cfg.H, cfg.D, cfg.n_phys, 96, 64
    gain = 8 ** -0.5  # n_layers = 8 (config.py:23)
    gen = torch.Generator(device=dev).manual_seed(cfg.seed)

    def rnd(shape, scale=1.0):
        return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * scale

    shape = (B, N, H, D)
    d = {"q": rnd(shape, D ** -0.5), "k": rnd(shape, D ** -0.5), "v": rnd(shape),
         "qt": rnd((1, *shape)), "kt": rnd((1, *shape)), "vt": rnd((1, *shape)),
         "edge": rnd((B, N, N, C)), "edge_t": rnd((B, N, N, C))}
    d_attn, d_e = H // 2 * D, 512  # W_O: attn_dim 256 -> d_e 512 (config.py:17,26; trunk.py:54)
    w_o = rnd((d_attn, d_e), d_attn ** -0.5)
    d["delta"] = torch.empty((B, N, d_e), dtype=torch.float32, device=dev)
    d["delta_t"] = torch.empty((1, B, N, d_e), dtype=torch.float32, device=dev)
    params = {"ln_w": 1.0 + 0.1 * rnd((C,)), "w_in": rnd((C, HID), C ** -0.5), "b_in": rnd((HID,), 0.1),
              "w_1": rnd((HID, HID), HID ** -0.5), "b_1": rnd((HID,), 0.1), "w_2": rnd((HID, HID), HID ** -0.5),
              "b_2": rnd((HID,), 0.1), "w_out": rnd((HID, H), HID ** -0.5), "b_out": rnd((H,), 0.1)}
    mask = torch.zeros((B, N), dtype=torch.uint8, device=dev)
    mask[:, :n_phys] = 1
    eshape = kernels.e_shape(B, N, H, "compact")  # the layout the N <= 64 kernel reads cheapest
    d["e"] = torch.zeros(eshape, dtype=torch.float32, device=dev)
    d["et"] = torch.zeros((1, *eshape), dtype=torch.float32, device=dev)
    fl_e = _native.HZ_FLAG_E_COMPACT
    d["y"] = torch.empty((B, N, H // 2, D), dtype=torch.float32, device=dev)
    d["ty"] = torch.empty((1, B, N, H // 2, D), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    s = stream.cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731
    div = float(np.sqrt(np.float32(D)))
    names = ("ln_w", "w_in", "b_in", "w_1", "b_1", "w_2", "b_2", "w_out", "b_out")

    def produce(i):
        _native.check(lib.hz_pair_bias(s, P(d["edge"]), P(d["edge_t"]), P(mask), *(P(params[n]) for n in names),
                                       P(d["e"]), P(d["et"]), B, N, C, HID, H, 1, gain, 1e-5, div, fl_e))

    def attend(i):
        _native.check(lib.hz_mhsea_fwd_jvp_gated(s, P(d["q"]), P(d["k"]), P(d["e"]), P(d["v"]), P(mask), P(d["qt"]),
                                                 P(d["kt"]), P(d["et"]), P(d["vt"]), 1, P(d["y"]), P(d["ty"]), B, N,
                                                 H, D, 1.0, fl_e))

    def project(i):
        _native.check(lib.hz_gated_out_proj(s, P(d["y"]), P(d["ty"]), P(w_o), P(mask), P(d["delta"]),
                                            P(d["delta_t"]), B, N, d_attn, d_e, 1))

    def step(i):
        produce(i)
        attend(i)
        project(i)

    ms = timed(step, args.steps, args.warmup, stream)
    ms_prod = timed(produce, args.steps, args.warmup, stream)
    ms_att = timed(attend, args.steps, args.warmup, stream)
    ms_proj = timed(project, args.steps, args.warmup, stream)
    # The producer's algorithmic work on the pairs it computes (both sites physical): the
    # MLP's products for the primal and the tangent, edge and edge_t rows in, e and e_t out.
    pairs_eff = B * n_phys * n_phys
    pairs_all = B * N * N
    fl_pair = 2 * (C * HID + 2 * HID * HID + HID * H)
    flops_eff, flops_all = 2 * fl_pair * pairs_eff, 2 * fl_pair * pairs_all
    bytes_eff = pairs_eff * 4 * (2 * C + 2 * H)
    roof = roofline(bytes_eff, flops_eff, ms_prod / 1e3, "f32")
    roof["traffic"] = traffic_from_profile(args.config)
    roof["kernel"] = "hz::pair_bias_kernel<96,2,true>"
    roof["basis"] = ("the producer launch: 2 x (C d_h + 2 d_h^2 + d_h H) x 2 flops per computed pair (primal and "
                     "tangent), computed pairs = B n_phys^2 (the pairs the attention reads); bytes: edge and edge_t "
                     "rows of those pairs in, e and e_t out")
    roof["bytes_per_launch"] = bytes_eff
    roof["flops_per_launch"] = flops_eff
    roof["reference_equivalent"] = {
        "basis": "every pair computed, as the reference's bias_mlp over the full [N, N] edge tensor does",
        "flops": flops_all, "tflops": flops_all / (ms_prod / 1e3) / 1e12}
    roof["step"] = {"ms": ms, "producer_ms": ms_prod, "attention_ms": ms_att, "out_proj_ms": ms_proj}

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        n = min(cfg.cpu_sample, B)
        host = {nm: t[:n].cpu() if nm not in ("qt", "kt", "vt") else t[0, :n].cpu()
                for nm, t in d.items() if nm in ("q", "k", "v", "qt", "kt", "vt", "edge", "edge_t")}
        hp = {nm: t.cpu() for nm, t in params.items()}
        r = cpu_baseline.time_trunk_walkers_per_s(host, mask[:n].bool().cpu(), hp, gain, D,
                                                  budget_s=args.cpu_budget, w_o=w_o.cpu())
        errs = {"delta": rel_err(d["delta"][:n].cpu().numpy(), r["y"].numpy()),
                "delta_t": rel_err(d["delta_t"][0, :n].cpu().numpy(), r["ty"].numpy())}
        tol = 2e-5
        cpu = {"value": r["walkers_per_s"], "unit": "walkers/s", "cores": r["threads"], "kind": "port",
               "sample": f"the first {n} walkers of the same inputs, {r['reps']} reps in {r['seconds']:.1f} s, "
                         f"torch-CPU fp32 port of the jnp path (ln_edge + bias_mlp over every pair, then the "
                         f"attention, gate collapse and W_O, forward mode by torch.func.jvp) ({r['cpu_model']})",
               "host_cpus": r["host_cpus"],
               "check": {"max_rel_err_vs_gpu": errs, "tol": tol, "ok": all(v <= tol for v in errs.values())}}
    line = {
        "metric": cfg.metric, "value": B / (ms / 1e3), "unit": "walkers/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": args.settle_ms, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (torch.randn on the GPU, seeded; weights N(0, fan_in^-1/2), small random biases)",
        "config": {"workload": f"{args.config}: {cfg.desc}", "B": B, "N": N, "H": H, "D": D, "n_phys": n_phys,
                   "T": 1, "edge_channels": C, "bias_hidden": HID},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_wavefn(args, cfg):
    """Bench leg of the whole compiled wavefunction (hz_compiled_wavefunction, one call per
    step). Config: B walkers, N sites, H groups G (d_m = 32 G), n_phys = merge rank."""
    import torch

    from hamiltonzero_amd import _native

    lib = _native.lib()
    dev = torch.device("cuda:0")
    B, n, G, R_merge = cfg.B, cfg.N, cfg.H, cfg.n_phys
    d_q, d_z, R_leaf, R_out, d_r = 4, 32, 1536, 64, 32
    dm = G * d_r
    gen = torch.Generator(device=dev).manual_seed(cfg.seed)

    def w(i, o):
        return torch.randn((i, o), generator=gen, device=dev) * i ** -0.5

    L = n.bit_length() - 1
    prm = {"q": torch.randn((B, n, d_q), generator=gen, device=dev), "q_weight": w(d_q, d_z),
           "leaf_V": w(d_z, R_leaf), "leaf_U": w(R_leaf, dm),
           "leaf_h": torch.randn((n, R_leaf), generator=gen, device=dev),
           "merge_T": torch.randn((G, d_r, d_r, d_r), generator=gen, device=dev) / d_r,
           "merge_V": w(dm, R_merge), "merge_U": w(R_merge, dm),
           "merge_h": torch.randn((L, n // 2, R_merge), generator=gen, device=dev),
           "opcodes": torch.zeros((L, n // 2), dtype=torch.uint8, device=dev),  # every node merges
           "readout_V": w(dm, R_out), "readout_U": w(R_out, 2),
           "readout_h": torch.randn((R_out,), generator=gen, device=dev)}
    log_abs = torch.empty(B, device=dev)
    phase = torch.empty(B, device=dev)
    nbytes = lib.hz_compiled_wavefunction_workspace(B, n, d_z, R_leaf, dm, R_merge, R_out)
    work = torch.empty(nbytes // 4 + 64, device=dev)
    stream = torch.cuda.current_stream(dev)
    names = ("q", "q_weight", "leaf_V", "leaf_U", "leaf_h", "merge_T", "merge_V", "merge_U", "merge_h", "opcodes",
             "readout_V", "readout_U", "readout_h")

    def step(i):
        _native.check(lib.hz_compiled_wavefunction(stream.cuda_stream, *(prm[k].data_ptr() for k in names),
                                                   log_abs.data_ptr(), phase.data_ptr(), work.data_ptr(), nbytes, B,
                                                   n, d_q, d_z, R_leaf, G, d_r, R_merge, R_out, 1e-6))

    ms = timed(step, args.steps, args.warmup, stream)
    rows = B * n
    merge_rows = B * (n - 1)  # every level's nodes: n/2 + n/4 + ... + 1 per walker
    flops = (2 * rows * (d_q * d_z + d_z * R_leaf + R_leaf * dm)
             + merge_rows * (2 * G * d_r ** 3 + 2 * (dm * R_merge + R_merge * dm))
             + 2 * B * (dm * R_out + R_out * 2))
    roof = roofline(4 * (rows * d_q + B * 2), flops, ms / 1e3, "f32")
    roof["traffic"] = traffic_from_profile(args.config)
    roof["kernel"] = "hz_compiled_wavefunction (every launch of the step)"
    roof["basis"] = ("algorithmic flops of the step: the leaf GEMMs 2 B n (d_q d_z + d_z R_leaf + R_leaf d_m), per "
                     "merged node 2 G d_r^3 + 4 d_m R_merge, the readout; per average step duration")
    roof["flops_per_step"] = flops
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        k = min(cfg.cpu_sample, B)
        host = {nm: t.cpu() for nm, t in prm.items()}
        host["q"] = host["q"][:k]
        r = cpu_baseline.time_wavefunction_walkers_per_s(host, 1e-6, budget_s=args.cpu_budget)
        got_la, got_ph = log_abs[:k].cpu().double().numpy(), phase[:k].cpu().double().numpy()
        d_la = float(np.max(np.abs(got_la - r["log_abs"].double().numpy())))
        d_ph = float(np.max(np.abs(np.angle(np.exp(1j * (got_ph - r["phase"].double().numpy()))))))
        tol = 1e-4
        cpu = {"value": r["walkers_per_s"], "unit": "walkers/s", "cores": r["threads"], "kind": "port",
               "sample": f"the first {k} walkers of the same inputs, {r['reps']} reps in {r['seconds']:.1f} s, "
                         f"torch-CPU fp32 port of _forward_plain ({r['cpu_model']})",
               "host_cpus": r["host_cpus"],
               "check": {"max_abs_diff_vs_gpu": {"log_abs": d_la, "phase": d_ph}, "tol": tol,
                         "ok": d_la <= tol * max(1.0, float(np.max(np.abs(got_la)))) and d_ph <= tol}}
    line = {
        "metric": cfg.metric, "value": B / (ms / 1e3), "unit": "walkers/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": args.settle_ms, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (torch.randn on the GPU, seeded; weights N(0, fan_in^-1/2); every node merges)",
        "config": {"workload": f"{args.config}: {cfg.desc}", "walkers": B, "n_sites": n, "d_q": d_q, "d_z": d_z,
                   "leaf_rank": R_leaf, "merge_dim": dm, "merge_rank": R_merge, "readout_rank": R_out},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def main(argv=None):
    global SETTLE_MS
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed run of the step before the warmup steps (wall-time ms)")
    ap.add_argument("--generic", action="store_true",
                    help="force the LDS-streaming kernels (HZ_FLAG_GENERIC) for comparison")
    ap.add_argument("--buffer-sets", type=int, default=0, metavar="N",
                    help="run the attention step over N copies of its buffers in turn (default: enough that the "
                         "touched bytes of the copies exceed twice the 256 MB Infinity Cache)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="instead of a configuration, time device-to-device copies of MIB MiB "
                         "(the calibration kernel for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args(argv)
    SETTLE_MS = args.settle_ms

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build runs the path on a single GPU (walkers shard "
              f"across GPUs with no communication, so the per-GPU figure is the N=1 figure); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    if args.copy_probe:
        return copy_probe(args.copy_probe, args.steps, args.warmup)
    cfg = CONFIGS[args.config]
    if cfg.work == "rect":
        return run_rect(args, cfg)
    if cfg.work == "rect_gate":
        return run_rect_gate(args, cfg)
    if cfg.work == "pair_mlp":
        return run_pair_mlp(args, cfg)
    if cfg.work == "executor":
        return run_executor(args, cfg)
    if cfg.work == "trunk":
        return run_trunk(args, cfg)
    if cfg.work == "wavefn":
        return run_wavefn(args, cfg)
    return run_attention(args, cfg)


if __name__ == "__main__":
    sys.exit(main())
