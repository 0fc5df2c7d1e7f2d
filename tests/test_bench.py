"""bench.py contract pieces that need no GPU: the FLOP accounting of each workload (the
per-config totals of the op's FLOP formula F = 4 B Hq d (N bs_l + N K bs + nb^2) +
2 B Hq d nb^2) and the refusal of more than one GPU."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("name,gflop", [
    ("nside16", 5.051),          # cfg1
    ("nside64", 167.000),        # cfg2
    ("nside32_b24", 1319.70),    # cfg3
    ("nside32_sweep", 41.24),    # cfg5
    ("nside64_sweep", 167.00),
    ("nside128", 700.62),
])
def test_flop_totals(name, gflop):
    fl = bench.flop_counts(bench.WORKLOADS[name])
    assert fl["total"] == fl["attn"] + fl["cmp_scores"]
    assert fl["total"] / 1e9 == pytest.approx(gflop, abs=0.006 * max(1.0, gflop / 100))


def test_attention_flops_are_tiles_times_tile_flops():
    wl = bench.WORKLOADS["nside64"]
    tiles = wl.batch * wl.q_heads * (wl.seq_len // 64) * (wl.block_attn_size // 64 + wl.sparse_block_count * wl.sparse_block_size // 64)
    assert tiles == 156672
    assert bench.flop_counts(wl)["attn"] == tiles * 4 * 64 * 64 * 64


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""
