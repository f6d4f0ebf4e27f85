"""Host-side checks of bench.py: the algorithmic bytes / flops behind ``roofline`` equal the
per-configuration figures of the measurement definition (every [B, L, H, D] tensor moved
once, mask as uint8, (2 + 4T) G / 6G / 2G flops with G = 2 L^2 D per walker and head), and
the multi-GPU request is refused with a message."""

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


@pytest.mark.parametrize(
    "name,bytes_,flops",
    [
        ("c1", 4_196_352, 8_388_608),
        ("c2", 536_936_448, 12_884_901_888),
        ("c3", 3_238_264_832, 103_079_215_104),
        ("c4", 2_147_614_720, 206_158_430_208),
        ("c5", 3_221_356_544, 2_748_779_069_440),
    ],
)
def test_padded_figures(name, bytes_, flops):
    c = bench.CONFIGS[name]
    a = bench.algorithmic(c.work, c.B, c.N, c.H, c.D, c.n_phys, c.T, 2 if c.dtype == "bf16" else 4, c.with_e)
    assert a["padded_bytes"] == bytes_
    assert a["padded_flops"] == flops


def test_bias_adds_e_and_its_tangents():
    c = bench.CONFIGS["c2e"]
    plain = bench.algorithmic("fwd_jvp", c.B, c.N, c.H, c.D, c.n_phys, c.T, 4, False)
    with_e = bench.algorithmic("fwd_jvp", c.B, c.N, c.H, c.D, c.n_phys, c.T, 4, True)
    assert with_e["padded_bytes"] - plain["padded_bytes"] == 268_435_456  # e and et, fp32
    assert with_e["eff_bytes"] - plain["eff_bytes"] == 2 * 1024 * 36 * 8 * 36 * 4


def test_split_route_is_charged_the_fused_figure():
    c = bench.CONFIGS["c2split"]
    a = bench.algorithmic(c.work, c.B, c.N, c.H, c.D, c.n_phys, c.T, 4)
    assert a["padded_bytes"] == 536_936_448


def test_c4_runs_in_chunks_of_16():
    assert bench.CONFIGS["c4"].chunk == 16 and bench.CONFIGS["c4"].B == 512


def test_multi_gpu_request_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_merge_level_config_is_fine_tune_shaped():
    """The executor bench leg runs one tree level at the fine-tune ranks (config.py:21-29):
    48 groups of d_r = 32 (merge_dim 1536), merge_rank 1024, 1024 walkers x 32 node pairs."""
    cfg = bench.CONFIGS["merge"]
    assert (cfg.work, cfg.B, cfg.N, cfg.H, cfg.D, cfg.n_phys) == ("executor", 1024, 32, 48, 32, 1024)


def test_reverse_mode_configs():
    """c2vjp: the fp32 training path at c2's shape, charged 12 tensor passes + 2 lse passes
    and 6G; gate_trunk_vjp: the gated reverse mode at the trunk's shape, charged the
    forward's q, k, v, e, the backward's q, k, v, e, out and dy (half a tensor), the outputs
    out, dq, dk, dv and de (every pair), and 6G."""
    c = bench.CONFIGS["c2vjp"]
    a = bench.algorithmic(c.work, c.B, c.N, c.H, c.D, c.n_phys, c.T, 4, c.with_e)
    row = c.H * c.D * 4
    assert a["padded_bytes"] == c.B * (c.N * row * 12 + c.N + 2 * c.N * c.H * 4)
    assert a["padded_flops"] == c.B * c.H * 6 * 2 * c.N * c.N * c.D
    g = bench.CONFIGS["gate_trunk_vjp"]
    a = bench.algorithmic(g.work, g.B, g.N, g.H, g.D, g.n_phys, g.T, 4, g.with_e)
    row = g.H * g.D * 4
    e_all = g.N * g.H * g.N * 4
    assert a["padded_bytes"] == g.B * (g.N * row * 11.5 + g.N + 2 * g.N * g.H * 4 + 3 * e_all)
    e_phys = g.n_phys * g.H * g.n_phys * 4
    assert a["eff_bytes"] == int(g.B * (g.n_phys * row * 7.5 + g.N * row * 4 + g.N + 2 * g.N * g.H * 4
                                         + 2 * e_phys + e_all))
    assert a["padded_flops"] == g.B * g.H * 6 * 2 * g.N * g.N * g.D


def test_buffer_rotation_covers_twice_the_infinity_cache():
    """The default buffer-set count makes the touched (mask-aware) bytes of all sets exceed
    twice the 256 MB Infinity Cache: c2's 361 MB per set needs two."""
    c = bench.CONFIGS["c2"]
    a = bench.algorithmic(c.work, c.B, c.N, c.H, c.D, c.n_phys, c.T, 4, c.with_e)
    sets = max(1, -(-2 * bench.INFINITY_CACHE_BYTES // a["eff_bytes"]))
    assert sets == 2 and sets * a["eff_bytes"] >= 2 * bench.INFINITY_CACHE_BYTES
