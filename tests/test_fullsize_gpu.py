"""Bit-exact parity at BASELINE's own sizes (C2, C3, C5).

C1 (1,024 generated levels x 1,000 steps) and C2 (16,384 x 512) are replayed in full by
the CPU restatement on the host cores and compared every step: state hash and out[] for
every world, the uint8 observation every step (C1) or every 8th step (C2). C3 and C5 run
at their full sizes on the GPU (65,536 worlds x 128 steps with the bf16 policy choosing
the actions; 262,144 worlds x 256 steps with 40 monsters); worlds are independent and keyed
by their index, so the first 2,048 of them are replayed on the host and compared (hash and
out every step, observations every 8th / 16th). Every 8th step the decoded state rows of the
compared worlds (the first 2,048 in C2) are checked field by field as well
(tests/envstate.py). Actions: uniform over the 16 semantic actions from a seeded stream (C1,
C2, C5), or the fused policy's samples (C3)."""
import importlib

import numpy as np
import pytest
import torch

from envstate import assert_same_worlds
from oracle import oracle as O

STATE_EVERY = 8
STATE_WORLDS = 2048

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
        if k % STATE_EVERY == 0 or k == steps - 1:
            m = min(n_cpu, STATE_WORLDS)
            assert_same_worlds(gpu.fields(slice(0, m)), cpu.fields(slice(0, m)), cfg,
                               obs=gpu.obs[:m].cpu().numpy(), label=f'step {k}')
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


def test_c5_ar_head_workload(pkg):
    """C5's bench workload (bench.py --mode stress): the stress layout driven by the
    autoregressive verb x target policy and its two-stage draw fused in one kernel
    (d1_policy_fwd_sample_ar), whose actions include waits, REST, stairs and unreachable
    targets (-1) besides moves and attacks. 8,192 worlds x 96 steps; the first 2,048 are
    replayed on the host with the same actions (hash and out every step, observations every
    16th)."""
    P = importlib.import_module('dcss-auto_amd.policy')
    cfg = pkg.stress_config()
    n, n_cpu, steps = 8192, 2048, 96
    gpu = pkg.Env(n, cfg, seed=3)
    cpu = O.OracleEnv(n_cpu, cfg, seed=3, threads=16)
    model = P.ARPolicy(seed=0).cuda().to(torch.bfloat16)
    a = torch.empty(n, dtype=torch.int64, device='cuda')
    logp, value = torch.empty(n, device='cuda'), torch.empty(n, device='cuda')
    seen, dones = set(), 0
    for k in range(steps):
        P.policy_fwd_sample_ar(gpu.obs, model.packed(), 11, k, a, logp, value)
        an = a.cpu().numpy()
        seen.update(np.unique(an[:n_cpu]).tolist())
        gpu.step(a)
        cpu.step(an[:n_cpu])
        dones += int(cpu.out[:, 1].sum())
        if k % 32 == 0:
            print(f'[c5 ar] step {k}', flush=True)
        torch.cuda.synchronize()
        gh = gpu.hash[:n_cpu].cpu().numpy().view(np.uint32)
        assert np.array_equal(gh, cpu.hash), f'hash differs at step {k}: {np.flatnonzero(gh != cpu.hash)[:8]}'
        go = gpu.out[:n_cpu].cpu().numpy()
        assert np.array_equal(go.view(np.uint32), cpu.out.view(np.uint32)), f'out differs at step {k}'
        if k % 16 == 0 or k == steps - 1:
            assert np.array_equal(gpu.obs[:n_cpu].cpu().numpy(), cpu.obs), f'observation differs at step {k}'
        if k % STATE_EVERY == 0 or k == steps - 1:
            assert_same_worlds(gpu.fields(slice(0, n_cpu)), cpu.fields(), cfg,
                               obs=gpu.obs[:n_cpu].cpu().numpy(), label=f'step {k}')
    assert {-1, 16, 17, 18} <= seen, sorted(seen)   # every non-move kind of action occurred
    assert dones > 0


def test_c3_full_size(pkg):
    """C3: 65,536 worlds x 128 steps of env step + observation + the fused bf16 policy forward
    with the counter-RNG sample, the sampled actions driving the env. The first 2,048 worlds
    are replayed on the host with the same actions (hash and out every step, observations
    every 8th). Every 32nd step, 512 rows spread over the whole batch check the kernel's
    logits and value against an fp32 restatement of the MLP (2e-2 of the output scale, the
    bf16 bar), its actions against the inverse CDF of the oracle's Philox uniforms and its
    log-probabilities against log-softmax of its own logits (1e-5, the fp32 bar)."""
    P = importlib.import_module('dcss-auto_amd.policy')
    cfg = pkg.baseline_config(8)
    n, n_cpu, steps, seed = 65536, 2048, 128, 77
    gpu = pkg.Env(n, cfg, seed=2026)
    cpu = O.OracleEnv(n_cpu, cfg, seed=2026, threads=16)
    model = P.Policy(seed=3).cuda().to(torch.bfloat16)
    wpk, b1, b2, b3 = model.packed()
    w = [m.weight.detach().float().cpu() for m in (model.l1, model.l2, model.head)]
    b = [m.bias.detach().float().cpu() for m in (model.l1, model.l2, model.head)]
    actions = torch.empty(n, dtype=torch.int64, device='cuda')
    logp = torch.empty(n, device='cuda')
    value = torch.empty(n, device='cuda')
    logits = torch.empty((n, P.N_ACTIONS), device='cuda')
    rows = np.arange(0, n, n // 512) + np.arange(512) % 7
    key = [seed & 0xFFFFFFFF, seed >> 32]
    dones = 0
    for k in range(steps):
        obs = gpu.obs.reshape(n, -1)
        P.policy_fwd_sample(obs, wpk, b1, b2, b3, seed, k, actions, logp, value, logits=logits)
        if k % 32 == 0 or k == steps - 1:
            print(f'[fullsize] C3 policy check at step {k}', flush=True)
            x = obs[torch.from_numpy(rows).cuda()].float().cpu()
            h = torch.relu(x @ w[0].T + b[0])
            h = torch.relu(h @ w[1].T + b[1])
            z = h @ w[2].T + b[2]
            got = torch.cat([logits[rows].cpu(), value[rows].cpu()[:, None]], 1)
            scale = float(z.abs().max()) + 1e-6
            assert float((got - z).abs().max()) <= 2e-2 * scale, f'policy outputs at step {k}'
            lz = logits[rows].cpu().double()
            lsm = torch.log_softmax(lz, 1)
            a = actions[rows].cpu()
            assert torch.allclose(logp[rows].cpu().double(), lsm.gather(1, a[:, None])[:, 0], rtol=1e-5, atol=1e-6)
            u = np.array([(int(O.philox([0, k, int(i), 3], key)[0]) >> 8) / 16777216.0 for i in rows])
            c = np.cumsum(torch.softmax(lz, 1).numpy(), 1)
            want = np.array([int(np.argmax(u[j] < c[j])) if (u[j] < c[j]).any() else P.N_ACTIONS - 1
                             for j in range(len(rows))])
            clear = np.abs(c - u[:, None]).min(1) > 1e-5
            assert clear.sum() > 500 and np.array_equal(a.numpy()[clear], want[clear]), f'samples at step {k}'
        gpu.step(actions)
        a_cpu = actions[:n_cpu].cpu().numpy()
        cpu.step(a_cpu)
        dones += int(cpu.out[:, 1].sum())
        torch.cuda.synchronize()
        gh = gpu.hash[:n_cpu].cpu().numpy().view(np.uint32)
        assert np.array_equal(gh, cpu.hash), f'hash differs at step {k}: {np.flatnonzero(gh != cpu.hash)[:8]}'
        go = gpu.out[:n_cpu].cpu().numpy()
        assert np.array_equal(go.view(np.uint32), cpu.out.view(np.uint32)), f'out differs at step {k}'
        if k % 8 == 0 or k == steps - 1:
            assert np.array_equal(gpu.obs[:n_cpu].cpu().numpy(), cpu.obs), f'observation differs at step {k}'
            assert_same_worlds(gpu.fields(slice(0, n_cpu)), cpu.fields(), cfg,
                               obs=gpu.obs[:n_cpu].cpu().numpy(), label=f'step {k}')
    assert dones > 0
