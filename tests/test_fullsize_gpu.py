"""Bit-exact parity at BASELINE's own sizes (C2, C5).

C1 (1,024 generated levels x 1,000 steps) and C2 (16,384 x 512) are replayed in full by
the CPU restatement on the host cores and compared every step: state hash and out[] for
every world, the uint8 observation every step (C1) or every 8th step (C2). C5 runs at its
full 262,144 worlds with 40 monsters on the GPU; worlds are independent and keyed by
their index, so the first 2,048 of them are replayed on the host and compared (hash and
out every step, observations every 16th). Actions: uniform over the 16 semantic actions
from a seeded stream, as the configs specify."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def run(pkg, cfg, n_gpu, n_cpu, steps, obs_every, seed=2026):
    gpu = pkg.Env(n_gpu, cfg, seed=seed)
    cpu = O.OracleEnv(n_cpu, cfg, seed=seed, threads=16)
    rng = np.random.default_rng(seed)
    dones = 0
    for k in range(-1, steps):
        if k >= 0:
            a = rng.integers(0, 16, n_gpu).astype(np.int64)
            gpu.step(torch.from_numpy(a).cuda())
            cpu.step(a[:n_cpu])
            dones += int(cpu.out[:, 1].sum())
        if k % 64 == 0:
            print(f'[fullsize] n={n_gpu} step {k}', flush=True)
        torch.cuda.synchronize()
        gh = gpu.hash[:n_cpu].cpu().numpy().view(np.uint32)
        assert np.array_equal(gh, cpu.hash), f'hash differs at step {k}: {np.flatnonzero(gh != cpu.hash)[:8]}'
        if k >= 0:
            go = gpu.out[:n_cpu].cpu().numpy()
            assert np.array_equal(go.view(np.uint32), cpu.out.view(np.uint32)), f'out differs at step {k}'
        if k % obs_every == 0 or k == steps - 1:
            assert np.array_equal(gpu.obs[:n_cpu].cpu().numpy(), cpu.obs), f'observation differs at step {k}'
    return dones


def test_c1_full(pkg):
    """C1: 1,024 worlds x 1,000 steps, 8 monsters, HP U[5,30], counter RNG."""
    assert run(pkg, pkg.baseline_config(8), 1024, 1024, 1000, 1) > 0


def test_c2_full(pkg):
    """C2: 16,384 worlds x 512 steps with the 15x15x8 observation."""
    assert run(pkg, pkg.baseline_config(8), 16384, 16384, 512, 8) > 0


def test_c5_full_size_slice(pkg):
    """C5: 262,144 worlds x 256 steps, 40 monsters, HP U[40,60], half awake at spawn;
    the first 2,048 worlds replayed on the host."""
    assert run(pkg, pkg.stress_config(), 262144, 2048, 256, 16) > 0
