"""Workload arithmetic matches the measurement plan's figures (no GPU)."""

import pytest
import torch

from dexter_amd.bench.workloads import CONFIGS, make_inputs

# (GFLOP per call, algorithmic bytes per call) for C0..C4.
EXPECTED = {
    "C0": (0.001572864, 196_608),
    "C1": (1.354432512, 17_338_368),
    "C2": (463.856467968, 201_326_592),
    "C3": (153.64343808, 186_982_400),
    "C4": (6.272753664, 68_886_528),
}


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_flops_and_bytes(name):
    cfg = CONFIGS[name]
    gflop, nbytes = EXPECTED[name]
    assert cfg.flops() / 1e9 == pytest.approx(gflop, rel=1e-12)
    assert cfg.bytes() == nbytes


def test_c2_is_56_percent_dense():
    cfg = CONFIGS["C2"]
    assert cfg.visible_pairs() / (8192 * 8192) == pytest.approx(0.5625)


def test_inputs_are_seeded_and_shaped():
    a = make_inputs(CONFIGS["C0"])
    b = make_inputs(CONFIGS["C0"])
    assert torch.equal(a.q, b.q) and a.q.shape == (1, 48, 4, 64) and a.q.dtype == torch.float32
    c4 = make_inputs(CONFIGS["C4"])
    assert c4.q.shape == (4, 99, 24, 128) and c4.k.shape == (4, 3336, 24, 128)
    big = (c4.q.float().abs() > 8).float().mean().item()
    assert 0.0005 < big < 0.02  # ~1% of entries scaled x20 (minus those landing small)


@pytest.mark.parametrize("argv, env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                       ([], {"WORLD_SIZE": "4"})])
def test_bench_refuses_more_than_one_gpu(argv, env):
    """bench.py measures one GPU: asked for more, it exits with code 2 and says so, before
    importing torch or touching a device."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    proc = subprocess.run([sys.executable, str(root / "bench.py"), *argv],
                          env={**os.environ, **env}, capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""
