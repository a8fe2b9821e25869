#!/usr/bin/env python3
"""Benchmark of the D:1 rollout hot path on one MI355X, with C4, the
training loop, C5 and the CPU baseline beside it.

One step = one pass over 65,536 worlds: the HIP env step (transition + auto-reset +
15x15x8 uint8 observation) and the fused HIP policy kernel (bf16 MLP 1800->256->256 with a
16-logit head and a value head on MFMA, then the counter-RNG categorical sample of the next
actions). The worlds run as two row ranges of 32,768, each a step -> policy pipeline on its
own stream (`--streams 1`: one range, one stream). Inputs stay resident in HBM; the timed
region is bracketed by synchronisations.
Prints one JSON line: C3 decisions/s as `value`, then `ppo` (C4 samples/s, median of three
updates after a warm one), `train` (rollout + update iterations), `stress` (C5 at 262,144
worlds with 40 monsters) and `cpu_baseline` (C1 on the CPU restatement at 1 thread and at
this job's CPU share).

  python bench.py [--steps K] [--warmup W] [--envs N] [--gpus 1] [--mode ...]
"""
import argparse
import importlib
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# Algorithmic bytes per env step at 8 monsters (what one step must read or write): obs 1800 +
# action 1 + reward/done/hash 9 + 2 x (24 + 7 x 8) dynamic state + 600 seen/viewed band
# + 700 level bitmap.
STEP_BYTES = {8: 3270, 40: 3718}
TRUNK_FLOPS = 2 * (1800 * 256 + 256 * 256 + 256 * 17)
# The autoregressive policy per sample: trunk, verb logits + value (9 outputs), the target
# MLP's trunk part (64), and its output layer (25 x 64) for the drawn verb only
AR_FLOPS = 2 * (1800 * 256 + 256 * 256 + 256 * 9 + 256 * 64 + 64 * 25)


def measured_traffic(path=ROOT / 'profiles' / 'k_step_hbm_traffic.md'):
    """HBM bytes per k_step launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (calibrated against a copy kernel), or None when absent."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith('traffic_bytes_per_launch:'):
                return float(line.split(':')[1])
    except OSError:
        pass
    return None


def host_cpus():
    """(threads this job may use, nproc, CPU model): the affinity mask is what `nproc`
    reports; a GPU box shares its host with other jobs, one CPU share of 16 per GPU."""
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, 'sched_getaffinity') else (os.cpu_count() or 1)
    model = 'unknown'
    try:
        for line in pathlib.Path('/proc/cpuinfo').read_text().splitlines():
            if line.startswith('model name'):
                model = line.split(':', 1)[1].strip()
                break
    except OSError:
        pass
    return min(16, nproc), nproc, model


def cpu_c1(threads, envs=1024, steps=1000, runs=1):
    """C1 on the CPU restatement (oracle/, OpenMP over worlds, schedule(static) as
    gpu-d1/src/bench.cu:167-184): `runs` runs of 1,024 generated levels x 1,000 steps,
    8 monsters, uniform random actions over 16; returns (decisions/s, seconds)."""
    import numpy as np
    from oracle import oracle as O
    pkg = importlib.import_module('dcss-auto_amd')
    dt = 0.0
    for r in range(runs):
        env = O.OracleEnv(envs, pkg.baseline_config(), seed=1 + r, threads=threads)
        actions = np.random.default_rng(2 + r).integers(0, 16, (steps, envs)).astype(np.int64)
        t0 = time.perf_counter()
        for k in range(steps):
            env.step(actions[k])
        dt += time.perf_counter() - t0
    return runs * envs * steps / dt, dt


def cpu_baseline():
    """The CPU path timed beside the GPU: C1 at every thread of this job's CPU share (three
    runs) and at one thread (one run), about 20 s of CPU work in all."""
    threads, nproc, model = host_cpus()
    rate, dt = cpu_c1(threads, runs=3)
    one, dt1 = cpu_c1(1, runs=1)
    return {'value': rate, 'unit': 'env decisions/s', 'cores': threads, 'kind': 'port',
            'sample': f'C1 full (1024 generated levels x 1000 steps, 8 monsters, random actions, step+obs+hash): '
                      f'3 runs on {threads} threads ({dt:.2f} s wall), 1 run on 1 thread ({dt1:.2f} s)',
            'single_thread': {'value': one, 'cores': 1},
            'nproc': nproc, 'cpu_model': model}


def ppo_bench(args, env, rollout_model, policy_mod, dev):
    """C4: a real T x N rollout fills the buffer (obs written in place by the env), then
    rewards/dones/values are replaced by C4's synthetic draws (r = 0 w.p. 0.97 else
    U(-1,1), done ~ Bernoulli(0.01), v ~ N(0,1)); the timed region is GAE + advantage
    normalisation + 4 epochs of 8,192-sample minibatch updates (fwd+bwd+clip+Adam)."""
    import torch
    ppo_mod = importlib.import_module('dcss-auto_amd.ppo')
    T, n = args.horizon, args.envs
    buf = ppo_mod.RolloutBuffer(T, n, device=dev)
    actions = torch.zeros(n, dtype=torch.int64, device=dev)
    with torch.no_grad():
        obs = env.obs
        for t in range(T):
            buf.obs[t].copy_(obs.view(n, -1))
            logits, value = rollout_model(obs)
            policy_mod.sample(logits, 7, t, actions, buf.logp[t])
            buf.actions[t].copy_(actions)
            obs, _ = env.step(actions)
    g = torch.Generator(device=dev).manual_seed(4)
    buf.rewards.copy_(torch.where(torch.rand(T, n, device=dev, generator=g) < 0.97, 0.0,
                                  torch.rand(T, n, device=dev, generator=g) * 2 - 1))
    buf.dones.copy_((torch.rand(T, n, device=dev, generator=g) < 0.01).to(torch.uint8))
    buf.values.copy_(torch.randn(T, n, device=dev, generator=g))
    buf.bootstrap.copy_(torch.randn(n, device=dev, generator=g))
    model = policy_mod.Policy(seed=0).to(dev)           # fp32 master weights
    if args.eager_ppo:
        trainer = ppo_mod.PPO(model)                     # torch autograd + fused Adam, eager
        trainer.update(ppo_mod.RolloutBuffer(2, 8192, device=dev))   # warm the eager path
    else:
        trainer = ppo_mod.FastPPO(model, graph=True)     # explicit fwd/bwd, HIP-graph minibatch step
        trainer._capture(buf)                            # capture once per buffer, outside the timing
    gen = torch.Generator(device=dev).manual_seed(5)
    trainer.update(buf, generator=gen)                  # warm: first replays, allocator, caches
    times = []
    for _ in range(args.ppo_updates):                   # the reference warms twice and times 12
        torch.cuda.synchronize()                        # (gpu-d1/PERFORMANCE.md:7); the median is reported
        t0 = time.perf_counter()
        loss = trainer.update(buf, generator=gen)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    samples = T * n
    flops = samples * trainer.epochs * (TRUNK_FLOPS + 2 * (1800 * 256 + 2 * 256 * 256 + 2 * 256 * 17))
    return {'metric': 'PPO samples/sec (C4: GAE + 4 epochs x 8,192-sample minibatches)', 'value': samples / dt,
            'unit': 'samples/s', 'sample_epochs_per_s': samples * trainer.epochs / dt, 'update_s': dt,
            'update_s_all': times, 'timing': f'median of {len(times)} updates after one warm update',
            'n_gpus': 1, 'higher_is_better': True, 'dtype': 'bf16 trunk, fp32 master',
            'loss_terms': [float(v) for v in torch.as_tensor(loss).flatten()[:3]], 'graph': trainer.graph,
            'path': 'autograd eager' if args.eager_ppo else 'explicit fwd/bwd, HIP graph',
            'config': {'workload': 'C4', 'T': T, 'envs': n, 'epochs': trainer.epochs, 'minibatch': trainer.minibatch,
                       'gamma': 0.99, 'lambda': 0.95, 'clip': 0.2, 'vcoef': 0.5, 'ecoef': 0.01},
            'mfma': {'achieved': flops / dt / 1e12, 'peak': BF16_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': flops / dt / 1e12 / BF16_PEAK_TFLOPS}}


def train_bench(args, dev, updates=2):
    """End-to-end PPO training at C3/C4's shapes: every update is a T=128 rollout over
    65,536 worlds (one HIP-graph replay of T x (forward, sample, env step)) and the C4
    update (GAE + 4 epochs of 8,192-sample minibatches); one warm-up update (graph
    captures), then `updates` timed."""
    import torch
    pkg = importlib.import_module('dcss-auto_amd')
    P = importlib.import_module('dcss-auto_amd.policy')
    train = importlib.import_module('dcss-auto_amd.train')
    env = pkg.Env(args.envs, pkg.baseline_config(args.monsters), seed=1, hash=False)
    tr = train.Trainer(env, P.Policy(seed=0).to(dev), horizon=args.horizon)
    tr.train(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tr.train(updates)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    decisions = updates * args.horizon * args.envs
    return {'metric': 'PPO training decisions/s (T=128 rollout + 4-epoch update per iteration)', 'value': decisions / dt,
            'unit': 'decisions/s', 's_per_update': dt / updates, 'updates': updates, 'path': 'graph rollout + graph PPO',
            'config': {'workload': 'C3 rollout + C4 update', 'envs': args.envs, 'T': args.horizon, 'epochs': tr.ppo.epochs,
                       'minibatch': tr.ppo.minibatch}}


REFERENCE_PANEL_S = 2.312   # gpu-d1/PERFORMANCE.md:29: fixed panel with frozen worlds, median of three


def panel_bench(args):
    """The reference's fixed-panel evaluation harness (gpu-d1/scripts/benchmark_evaluation.py):
    1,024 learning-task worlds on 32 maps (map_filter -2: 32 episodes per map), 1,024
    decisions with finished worlds frozen, median of three after a warm-up. The reference's
    32 validation maps and trained checkpoint are not in its repository: the maps here are
    32 generated levels and the policies are the task's heuristic controller and a
    random-init policy of the reference's shape, so outcome rates differ from its run."""
    import statistics
    import torch
    pkg = importlib.import_module('dcss-auto_amd')
    learn = importlib.import_module('dcss-auto_amd.learn')
    floors = pkg.Env(32, pkg.baseline_config(8), seed=21, hash=False).floors()
    env = learn.LearnEnv(1024, maps=learn.LearnMaps(floors), map_filter=-2, limit=2048, clump=1)
    policy = learn.MaskedPolicy().cuda()
    out = {}
    for name, pol in (('heuristic', 'heuristic'), ('policy', policy)):
        learn.evaluate_panel(env, pol, decisions=64)   # warm-up
        runs = [learn.evaluate_panel(env, pol, decisions=1024, active=True) for _ in range(3)]
        sec = statistics.median(r['seconds'] for r in runs)
        r = runs[0]
        out[name] = {'seconds': sec, 'clear_rate': r['clear_rate'], 'death_rate': r['death_rate'], 'kills': r['kills'],
                     'unfinished': r['unfinished']}
    return {'metric': 'fixed-panel evaluation seconds (1,024 worlds = 32 maps x 32 episodes, 1,024 decisions, frozen worlds)',
            'value': out['policy']['seconds'], 'unit': 's', 'higher_is_better': False, 'n_gpus': 1,
            'reference': {'value': REFERENCE_PANEL_S, 'source': 'gpu-d1/PERFORMANCE.md:29',
                          'note': 'trained policy on the 32 validation maps, its own GPU'},
            'runs': out, 'config': {'workload': 'panel', 'maps': 'generated', 'worlds': 1024, 'decisions': 1024,
                                    'limit': 2048}}


EVERY = 8   # timed steps per sampled set of per-kernel events
REFERENCE_WAITS_PER_S = 10.165e6   # gpu-d1/RESULTS.md:16, warp per world, RTX 5000 Max-Q


def wait_bench(args, worlds=8192, count=8, chunk=64, waits=4096):
    """The reference's sustained wait comparison (gpu-d1/RESULTS.md:5-16): 8,192 worlds,
    8 monsters, mixed approach/contact phases, 64 waits per kernel, 4,096 waits per world."""
    import torch
    wait = importlib.import_module('dcss-auto_amd.wait')
    w = wait.WaitWorlds(worlds, count, 'mixed', seed=42)
    w.run(chunk)                       # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(waits // chunk):
        w.run(chunk)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    rate = worlds * waits / dt
    return {'metric': 'monster waits/s (reference wait benchmark, 8,192 worlds, 8 monsters, mixed)',
            'value': rate, 'unit': 'waits/s', 'n_gpus': 1, 'higher_is_better': True,
            'vs_baseline': rate / REFERENCE_WAITS_PER_S,
            'baseline': {'value': REFERENCE_WAITS_PER_S, 'source': 'gpu-d1/RESULTS.md:16', 'hardware': 'Quadro RTX 5000 Max-Q'},
            'config': {'workload': 'wait', 'worlds': worlds, 'monsters': count, 'scenario': 'mixed',
                       'waits_per_kernel': chunk, 'waits_per_world': waits}, 'seconds': dt}


def row_ranges(n, k):
    """k contiguous row ranges covering 0..n-1."""
    return [(n * j // k, n * (j + 1) // k) for j in range(k)]


def event_stride(steps, launches_per_step=1):
    """Timed steps per sampled set of per-kernel HIP events: every 8th step of a long run
    (three event records per step cost the measured loop ~4%), and in a short one the widest
    stride whose sampled steps still give each kernel ten or more timed launches
    (`launches_per_step` launches of it per step)."""
    return max(1, min(EVERY, steps * launches_per_step // 10))


def roofline(kernel, achieved, launch_ms, step_bytes, traffic, launches):
    """The bench line's roofline object: algorithmic GB/s (bytes per world-step x worlds /
    mean launch time from HIP events in the timed region) against HBM peak, and beside it
    the counter-based rate: HBM bytes per launch read by rocprofv3 FETCH_SIZE + WRITE_SIZE
    (copy-kernel calibrated, committed under profiles/) over the same live launch time."""
    r = {'bound': 'hbm', 'kernel': kernel, 'achieved': achieved, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
         'frac': achieved / HBM_PEAK_GBS, 'traffic': traffic, 'bytes_per_env_step': step_bytes,
         'avg_launch_ms': launch_ms, 'timed_launches': launches}
    if traffic:
        counted = traffic / (launch_ms * 1e-3) / 1e9
        r['counter_gbs'] = counted
        r['counter_frac'] = counted / HBM_PEAK_GBS
    return r


def stress_counters(args, envs=262144, horizon=256, warmup=4):
    """The C5 stress workload of stress_bench (same worlds, policy, seeds and steps), after a
    256 MiB device copy that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE, untimed: the
    k_step_crowd dispatches warmup+1 .. warmup+horizon are the bench's timed launches."""
    import torch
    pkg = importlib.import_module('dcss-auto_amd')
    P = importlib.import_module('dcss-auto_amd.policy')
    dev = torch.device('cuda:0')
    src = torch.ones(64 << 20, dtype=torch.int32, device=dev)   # 256 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    env = pkg.Env(envs, pkg.stress_config(), seed=3, hash=False)
    model = P.ARPolicy(seed=0).to(dev).to(torch.bfloat16)
    packed = model.packed()
    actions = torch.zeros(envs, dtype=torch.int64, device=dev)
    logp, value = torch.empty(envs, device=dev), torch.empty(envs, device=dev)
    obs = env.obs.view(envs, -1)
    for t in range(warmup + horizon):
        env.step(actions)
        P.policy_fwd_sample_ar(obs, packed, 11, t, actions, logp, value)
    torch.cuda.synchronize()
    return {'mode': 'stress-counters', 'copy_bytes': src.numel() * 4, 'env_steps': warmup + horizon, 'envs': envs,
            'timed_dispatches': [warmup + 1, warmup + horizon]}


def stress_bench(args, envs=262144, horizon=256, warmup=4):
    """C5: 262,144 generated-level worlds with 40 monsters (HP U[40,60], half awake at
    spawn), the bf16 trunk with the autoregressive verb(8) x target(25) head and its
    two-stage counter-RNG draw fused into one kernel (d1_policy_fwd_sample_ar), 256 steps.
    Reports decisions/s and k_step's algorithmic HBM rate."""
    import torch
    pkg = importlib.import_module('dcss-auto_amd')
    P = importlib.import_module('dcss-auto_amd.policy')
    dev = torch.device('cuda:0')
    env = pkg.Env(envs, pkg.stress_config(), seed=3, hash=False)
    model = P.ARPolicy(seed=0).to(dev).to(torch.bfloat16)
    packed = model.packed()
    actions = torch.zeros(envs, dtype=torch.int64, device=dev)
    logp = torch.empty(envs, device=dev)
    value = torch.empty(envs, device=dev)
    obs = env.obs.view(envs, -1)

    def one(t, ev=None):
        if ev is not None:
            ev[0].record()
        env.step(actions)
        if ev is not None:
            ev[1].record()
        P.policy_fwd_sample_ar(obs, packed, 11, t, actions, logp, value)
        if ev is not None:
            ev[2].record()

    for t in range(warmup):
        one(t)
    torch.cuda.synchronize()
    every = event_stride(horizon)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(0, horizon, every)]
    t0 = time.perf_counter()
    for k in range(horizon):
        one(warmup + k, events[k // every] if k % every == 0 else None)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = sum(e[0].elapsed_time(e[1]) for e in events) / len(events)
    policy_ms = sum(e[1].elapsed_time(e[2]) for e in events) / len(events)
    achieved = STEP_BYTES[40] * envs / (step_ms * 1e-3) / 1e9
    traffic = measured_traffic(ROOT / 'profiles' / 'k_step_c5_counters.md')
    return {'metric': 'env decisions/sec at 262,144 envs, 40 monsters, AR 8x25 head (C5)',
            'value': envs * horizon / wall, 'unit': 'decisions/s', 'n_gpus': 1, 'higher_is_better': True,
            'ms_per_step': wall / horizon * 1e3,
            'config': {'workload': 'C5', 'envs': envs, 'monsters': 40, 'hp': [40, 60], 'awake_pct': 50,
                       'head': 'AR verb 8 x target 25', 'horizon': horizon},
            'policy': {'kernel': 'd1t::k_policy<2> (trunk + AR head + two-stage draw)', 'avg_launch_ms': policy_ms,
                       'mfma_tflops': AR_FLOPS * envs / (policy_ms * 1e-3) / 1e12},
            'roofline': roofline('d1::k_step', achieved, step_ms, STEP_BYTES[40], traffic, len(events))}


def controller_bench(args, warmup=8):
    """The v1 task (map 1057, 8 monsters, all awake) at --envs worlds driven by the v1 pursuit
    controller on the GPU (Env.heuristic -> d1_heuristic, gpu-d1/src/learn.cu:599-621) then
    the env step, --steps timed decisions; HIP events time each kernel."""
    import torch
    pkg = importlib.import_module('dcss-auto_amd')
    n = args.envs
    env = pkg.Env(n, pkg.v1_config(8, sleep=False), seed=1, hash=False)
    actions = torch.zeros(n, dtype=torch.int64, device='cuda')
    for _ in range(warmup):
        env.step(env.heuristic(out=actions))
    torch.cuda.synchronize()
    every = event_stride(args.steps)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(0, args.steps, every)]
    t0 = time.perf_counter()
    for k in range(args.steps):
        ev = events[k // every] if k % every == 0 else None
        if ev is not None:
            ev[0].record()
        env.heuristic(out=actions)
        if ev is not None:
            ev[1].record()
        env.step(actions)
        if ev is not None:
            ev[2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ctl_ms = sum(e[0].elapsed_time(e[1]) for e in events) / len(events)
    step_ms = sum(e[1].elapsed_time(e[2]) for e in events) / len(events)
    return {'metric': 'v1 controller + env step decisions/sec', 'value': n * args.steps / wall, 'unit': 'decisions/s',
            'envs': n, 'steps': args.steps, 'controller_ms': ctl_ms, 'step_ms': step_ms,
            'config': {'workload': 'v1 task, map 1057, 8 awake monsters', 'controller': 'd1_heuristic (joint actions)'}}


# Algorithmic bytes of one learning-task decision (k_learn_step): fp32 observation 4060 +
# mask 76 + outcome 180 + action 8 + 2 x (80 header + 192 enemies) + 2 x 840 memory
# bitmap + 840 floor bitmap; the frontier list (2 bytes per anchor read, changed
# entries written) is left out.
LEARN_STEP_BYTES = 4060 + 76 + 180 + 8 + 2 * 272 + 2 * 840 + 840


def learn_cpu_baseline(envs=4096, steps=500, threads=None):
    """The learning-task restatement (oracle/learn_oracle.c, OpenMP over worlds) on map
    1057 with the controller's actions."""
    from oracle import oracle as O
    pkg = importlib.import_module('dcss-auto_amd')
    threads = threads or host_cpus()[0]
    env = O.OracleLearn(envs, O.LearnTablesHost(pkg.data.map1057()['floor'][None]), seed=1, threads=threads)
    t0 = time.perf_counter()
    for _ in range(steps):
        env.step(env.heuristic())
    dt = time.perf_counter() - t0
    return {'value': envs * steps / dt, 'unit': 'decisions/s (step+obs+mask+heuristic)', 'cores': threads,
            'kind': 'port', 'sample': f'{envs} worlds x {steps} heuristic decisions on map 1057, {dt:.2f} s wall'}


def learn_bench(args, warmup=8):
    """The d1-stairs-v2 drop-in (learn_* ABI): N worlds on map 1057 driven by the library's
    own controller (learn_heuristic), each decision = one learn_step (joint action, REST
    repeats, monster turns, auto-reset, fp32 observation [1015], mask [19], outcome [45])."""
    import torch
    L = importlib.import_module('dcss-auto_amd.learn')
    n = args.envs
    env = L.LearnEnv(n, seed=1, clump=1)
    for _ in range(warmup):
        env.step(env.heuristic())
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(0, args.steps, EVERY)]
    t0 = time.perf_counter()
    for k in range(args.steps):   # per-kernel events on every EVERY-th decision, as in the rollout
        e = ev[k // EVERY] if k % EVERY == 0 else None
        if e is not None:
            e[0].record()
        a = env.heuristic()
        if e is not None:
            e[1].record()
        env.step(a)
        if e is not None:
            e[2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    heur_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / len(ev)
    step_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / len(ev)
    achieved = LEARN_STEP_BYTES * n / (step_ms * 1e-3) / 1e9
    result = {'metric': 'learning-task decisions/s (d1-stairs-v2 learn_* drop-in, controller actions)',
              'value': n * args.steps / wall, 'unit': 'decisions/s', 'n_gpus': 1, 'steps': args.steps,
              'warmup': warmup, 'ms_per_step': wall / args.steps * 1e3, 'higher_is_better': True,
              'scaling': 'weak', 'vs_baseline': None, 'dtype': 'int16/u8 state, fp32 obs',
              'data': 'synthetic: map 1057, 24 enemies, clump mode 1',
              'config': {'workload': 'learn', 'envs': n, 'obs': 'fp32 1015', 'clump': 1},
              'roofline': roofline('d1::learn::k_learn_step', achieved, step_ms, LEARN_STEP_BYTES,
                                   measured_traffic(ROOT / 'profiles' / 'k_learn_step_learn.md'), len(ev)),
              'heuristic_ms': heur_ms, 'step_ms': step_ms,
              'errors': int(env.errors().numel())}
    if not args.no_cpu_baseline:
        result['cpu_baseline'] = learn_cpu_baseline()
    return result


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=128)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--envs', type=int, default=65536)
    ap.add_argument('--monsters', type=int, default=8)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--mode', choices=['rollout', 'counters', 'ppo', 'train', 'panel', 'wait', 'stress',
                                       'stress-counters', 'learn', 'controller'],
                    default='rollout',
                    help='counters: a 256 MiB copy (counter calibration) then env steps only, for rocprofv3 --pmc; '
                         'stress-counters: the same calibration, then the C5 stress workload untimed; '
                         'ppo: C4, GAE + 4-epoch PPO update over a T x envs rollout buffer; '
                         'train: rollout + update iterations of the training loop')
    ap.add_argument('--horizon', type=int, default=128, help='T of the PPO rollout buffer')
    ap.add_argument('--eager-ppo', action='store_true', help='run the PPO update without HIP-graph capture')
    ap.add_argument('--no-ppo', action='store_true', help='rollout mode: skip the C4 PPO and training measurements that follow')
    ap.add_argument('--no-stress', action='store_true', help='rollout mode: skip the C5 stress measurement that follows')
    ap.add_argument('--ppo-updates', type=int, default=3, help='timed C4 updates (after one warm update); median reported')
    ap.add_argument('--streams', type=int, default=2, choices=(1, 2),
                    help='rollout and counters modes: the worlds as this many row ranges, each stepped and sampled '
                         'on its own stream (default 2)')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) > 1:
        print('bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)', file=sys.stderr)
        sys.exit(2)

    import torch
    if args.mode == 'wait':
        print(json.dumps(wait_bench(args)), flush=True)
        return
    if args.mode == 'stress':
        print(json.dumps(stress_bench(args)), flush=True)
        return
    if args.mode == 'stress-counters':
        print(json.dumps(stress_counters(args)), flush=True)
        return
    if args.mode == 'learn':
        print(json.dumps(learn_bench(args)), flush=True)
        return
    if args.mode == 'controller':
        print(json.dumps(controller_bench(args)), flush=True)
        return
    if args.mode == 'panel':
        print(json.dumps(panel_bench(args)), flush=True)
        return
    if args.mode == 'train':
        print(json.dumps(train_bench(args, torch.device('cuda:0'))), flush=True)
        return
    pkg = importlib.import_module('dcss-auto_amd')
    policy_mod = importlib.import_module('dcss-auto_amd.policy')
    dev = torch.device('cuda:0')
    cfg = pkg.baseline_config(args.monsters) if args.monsters <= 8 else pkg.stress_config()
    n = args.envs
    env = pkg.Env(n, cfg, seed=1, hash=False)
    model = policy_mod.Policy(seed=0).to(dev).to(torch.bfloat16)
    actions = torch.zeros(n, dtype=torch.int64, device=dev)
    logp = torch.zeros(n, dtype=torch.float32, device=dev)
    seed = 12345
    if args.mode == 'counters':
        src = torch.ones(64 << 20, dtype=torch.int32, device=dev)   # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        parts = row_ranges(n, args.streams)   # the rollout's launches: one per row range
        for t in range(args.steps):
            actions.random_(0, 16)
            for lo, hi in parts:
                env.step_rows(lo, hi, actions)
        torch.cuda.synchronize()
        print(json.dumps({'mode': 'counters', 'copy_bytes': src.numel() * 4, 'env_steps': args.steps, 'envs': n,
                          'worlds_per_launch': n // args.streams}))
        return

    if args.mode == 'ppo':
        print(json.dumps(ppo_bench(args, env, model, policy_mod, dev)), flush=True)
        return

    wpk, b1, b2, b3 = model.packed()
    value = torch.empty(n, dtype=torch.float32, device=dev)

    # The worlds as `streams` row ranges, each a pipeline of its own on its own stream (every
    # stream at the default priority): env step, then forward + counter-RNG sample in one
    # kernel. A range's next step depends only on its own actions, so the ranges' kernels
    # overlap and fill one another's launch tails. Each range samples with its own key.
    parts = row_ranges(n, args.streams)
    streams = [torch.cuda.current_stream()] if len(parts) == 1 else [torch.cuda.Stream() for _ in parts]
    obs = env.obs.view(n, -1)

    def one_step(t, ev=None):
        for j, ((lo, hi), st) in enumerate(zip(parts, streams)):
            with torch.cuda.stream(st):
                if ev is not None:
                    ev[j][0].record()
                env.step_rows(lo, hi, actions)
                if ev is not None:
                    ev[j][1].record()
                policy_mod.policy_fwd_sample(obs[lo:hi], wpk, b1, b2, b3, seed + 7919 * j, t, actions[lo:hi],
                                             logp[lo:hi], value[lo:hi])
                if ev is not None:
                    ev[j][2].record()

    torch.cuda.synchronize()   # the new streams start after the set-up on the default one
    for t in range(args.warmup):
        one_step(t)
    torch.cuda.synchronize()
    # per-kernel HIP events (on each range's own stream) on every EVERY-th step of the timed
    # region: an event record costs the stream a few microseconds, so events around every
    # launch would slow the throughput being measured (three per step: ~4%). With two
    # ranges the launches share the GPU with the other range's, and their durations say so.
    every = event_stride(args.steps, len(parts))
    events = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in parts]
              for _ in range(0, args.steps, every)]
    t0 = time.perf_counter()
    for k in range(args.steps):
        one_step(args.warmup + k, events[k // every] if k % every == 0 else None)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    flat = [e for per_step in events for e in per_step]
    step_ms = sum(e[0].elapsed_time(e[1]) for e in flat) / len(flat)
    trunk_ms = sum(e[1].elapsed_time(e[2]) for e in flat) / len(flat)
    decisions = n * args.steps / wall
    # The kernels alone (outside the timed region): whole-batch launches on one stream, with
    # nothing else on the GPU, for the per-kernel rooflines beside the pipeline's
    iso = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(8)]
    for k, e in enumerate(iso):
        e[0].record()
        env.step(actions)
        e[1].record()
        policy_mod.policy_fwd_sample(obs, wpk, b1, b2, b3, seed, args.warmup + args.steps + k, actions, logp, value)
        e[2].record()
    torch.cuda.synchronize()
    iso_step_ms = sum(e[0].elapsed_time(e[1]) for e in iso) / len(iso)
    iso_trunk_ms = sum(e[1].elapsed_time(e[2]) for e in iso) / len(iso)
    step_bytes = STEP_BYTES.get(args.monsters, 3270)
    per_launch = n // len(parts)
    achieved = step_bytes * per_launch / (step_ms * 1e-3) / 1e9
    trunk_tflops = TRUNK_FLOPS * per_launch / (trunk_ms * 1e-3) / 1e12
    result = {
        'metric': 'env decisions/sec at 65,536 envs (1 GPU): step+obs+policy+sample',
        'value': decisions,
        'unit': 'decisions/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': wall / args.steps * 1e3,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'int16/u8 env, bf16 trunk',
        'data': 'synthetic: generated 80x70 levels, random-init N(0,0.02) bf16 policy',
        'config': {'workload': 'C3', 'envs': n, 'monsters': args.monsters, 'obs': '15x15x8 uint8',
                   'policy': '1800-256-256 ReLU, 16 logits + value, bf16', 'sampler': 'Philox counter RNG',
                   'rollout_steps': args.steps,
                   'pipeline': f'{len(parts)} row ranges of {per_launch} worlds, one stream each'},
        'roofline': dict(roofline('d1::k_step', achieved, step_ms, step_bytes, measured_traffic(), len(flat)),
                         worlds_per_launch=per_launch,
                         isolated={'worlds_per_launch': n, 'avg_launch_ms': iso_step_ms,
                                   'achieved': step_bytes * n / (iso_step_ms * 1e-3) / 1e9,
                                   'frac': step_bytes * n / (iso_step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                   'launches': len(iso), 'note': 'one stream, after the timed region'}),
        'trunk': {'bound': 'mfma', 'achieved': trunk_tflops, 'peak': BF16_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                  'frac': trunk_tflops / BF16_PEAK_TFLOPS, 'avg_ms': trunk_ms, 'rows_per_launch': per_launch,
                  'isolated': {'rows_per_launch': n, 'avg_ms': iso_trunk_ms,
                               'achieved': TRUNK_FLOPS * n / (iso_trunk_ms * 1e-3) / 1e12,
                               'frac': TRUNK_FLOPS * n / (iso_trunk_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}},
    }
    if not args.no_ppo:   # the metric's second number: C4 PPO samples/s, measured after the rollout
        ppo = ppo_bench(args, env, model, policy_mod, dev)
        result['ppo'] = {k: ppo[k] for k in ('metric', 'value', 'unit', 'update_s', 'sample_epochs_per_s', 'dtype',
                                             'path', 'config', 'mfma')}
        del ppo
        result['train'] = train_bench(args, dev)
    if not args.no_stress:   # C5 at its own size: decisions/s and k_step's HBM rate against peak
        del env
        torch.cuda.empty_cache()
        stress = stress_bench(args)
        result['stress'] = {k: stress[k] for k in ('metric', 'value', 'unit', 'ms_per_step', 'config', 'roofline')}
    if not args.no_cpu_baseline:
        result['cpu_baseline'] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
