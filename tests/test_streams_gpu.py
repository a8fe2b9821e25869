"""Every entry point runs on the caller's stream (torch's current stream), as the reference
requires of its kernels: "Custom kernels must honor the stream that produces actions and
consumes observations" (gpu-d1/scripts/test_learning.py:62-69). Each call is made once under
the default stream and once inside `with torch.cuda.stream(side)` on tensors created there,
and the results must be identical bit for bit: Env.step (with a reset) and its v1 controller, LearnEnv.step and
its controller, the fused policy forward + sample (plain and autoregressive head), and the
PPO minibatch step."""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def on_side_stream(fn):
    """fn() under a fresh non-default stream (default priority); its results are read after
    that stream has finished."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = fn()
    side.synchronize()
    torch.cuda.synchronize()
    return out


def test_env_step_on_a_side_stream(pkg):
    print('[streams] env', flush=True)

    def run():
        env = pkg.Env(37, pkg.v1_config(6, sleep=False), seed=91)
        g = torch.Generator(device='cuda').manual_seed(5)
        outs = []
        for k in range(40):
            # odd steps: the v1 controller's actions, made on this stream
            a = env.heuristic() if k % 2 else torch.randint(0, 19, (37,), device='cuda', generator=g)
            env.step(a)
            outs.append((env.obs.clone(), env.out.clone(), env.state.clone(), env.hash.clone(), a.clone()))
        # the reference's own case: one WAIT on fresh worlds
        env.reset(91)
        env.step(torch.full((37,), 16, dtype=torch.int64, device='cuda'))
        outs.append((env.obs.clone(), env.out.clone(), env.state.clone(), env.hash.clone(), env.heuristic()))
        return outs

    want = run()
    torch.cuda.synchronize()
    got = on_side_stream(run)
    for k, (w, g) in enumerate(zip(want, got)):
        for a, b in zip(w, g):
            assert torch.equal(a, b), f'step {k}'


def test_env_row_ranges_on_two_streams(pkg):
    """Env.step_rows: two disjoint row ranges stepped on two concurrent streams (the C3
    bench's pipeline) give exactly the rows of whole-batch steps: each world's step reads
    only its own row and action."""
    print('[streams] row ranges', flush=True)
    n, h = 3000, 1234   # uneven ranges, several workgroups each
    cfg = pkg.baseline_config(8)
    whole = pkg.Env(n, cfg, seed=17, hash=False)
    split = pkg.Env(n, cfg, seed=17, hash=False)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    g = torch.Generator(device='cuda').manual_seed(9)
    torch.cuda.synchronize()
    for k in range(60):
        a = torch.randint(0, 19, (n,), device='cuda', generator=g)
        whole.step(a)
        torch.cuda.synchronize()
        with torch.cuda.stream(sa):
            split.step_rows(0, h, a)
        with torch.cuda.stream(sb):
            split.step_rows(h, n, a)
        torch.cuda.synchronize()
        assert torch.equal(whole.state, split.state), f'step {k}: state rows'
        assert torch.equal(whole.obs, split.obs), f'step {k}: observations'
        assert torch.equal(whole.out, split.out), f'step {k}: out rows'
    with pytest.raises(ValueError):
        split.step_rows(5, 5, a)
    with pytest.raises(ValueError):
        split.step_rows(0, n + 1, a)


def test_learn_step_on_a_side_stream():
    print('[streams] learn', flush=True)
    L = importlib.import_module('dcss-auto_amd.learn')
    maps = L.LearnMaps()

    def run():
        env = L.LearnEnv(48, seed=3, maps=maps)
        outs = []
        for k in range(30):
            a = env.heuristic().clone()
            env.step(a)
            outs.append((a, env.obs.clone(), env.mask.clone(), env.out.clone(), env.state.clone()))
        return outs

    want = run()
    torch.cuda.synchronize()
    got = on_side_stream(run)
    for k, (w, g) in enumerate(zip(want, got)):
        for a, b in zip(w, g):
            assert torch.equal(a, b), f'step {k}'


def test_policy_forward_sample_on_a_side_stream():
    print('[streams] policy', flush=True)
    P = importlib.import_module('dcss-auto_amd.policy')
    model = P.Policy(seed=4).cuda().to(torch.bfloat16)
    g = torch.Generator(device='cuda').manual_seed(1)
    obs = torch.randint(0, 30, (4133, 1800), dtype=torch.uint8, device='cuda', generator=g)

    def run():
        wpk, b1, b2, b3 = (t.clone() for t in model.packed())
        n = obs.shape[0]
        x = obs.clone()
        actions = torch.empty(n, dtype=torch.int64, device='cuda')
        logp = torch.empty(n, device='cuda')
        value = torch.empty(n, device='cuda')
        logits = torch.empty((n, P.N_ACTIONS), device='cuda')
        P.policy_fwd_sample(x, wpk, b1, b2, b3, 42, 9, actions, logp, value, logits=logits)
        return actions, logp, value, logits

    want = run()
    torch.cuda.synchronize()
    got = on_side_stream(run)
    for a, b in zip(want, got):
        assert torch.equal(a, b)


def test_ar_policy_forward_sample_on_a_side_stream():
    print('[streams] ar policy', flush=True)
    P = importlib.import_module('dcss-auto_amd.policy')
    model = P.ARPolicy(seed=6).cuda().to(torch.bfloat16)
    model.packed()
    g = torch.Generator(device='cuda').manual_seed(2)
    obs = torch.randint(0, 30, (3001, 1800), dtype=torch.uint8, device='cuda', generator=g)

    def run():
        n = obs.shape[0]
        x = obs.clone()
        action = torch.empty(n, dtype=torch.int64, device='cuda')
        logp, value = torch.empty(n, device='cuda'), torch.empty(n, device='cuda')
        verb_logits = torch.empty((n, P.N_VERBS), device='cuda')
        P.policy_fwd_sample_ar(x, model.packed(), 17, 5, action, logp, value, verb_logits=verb_logits)
        return action, logp, value, verb_logits

    want = run()
    torch.cuda.synchronize()
    got = on_side_stream(run)
    for a, b in zip(want, got):
        assert torch.equal(a, b)


def test_ppo_step_on_a_side_stream():
    print('[streams] ppo', flush=True)
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    T, N = 2, 4096
    g = torch.Generator(device='cuda').manual_seed(6)
    obs = torch.randint(0, 20, (T, N, 1800), dtype=torch.uint8, device='cuda', generator=g)
    act = torch.randint(0, 16, (T, N), device='cuda', generator=g)
    lp = -torch.rand(T, N, device='cuda', generator=g) * 3
    adv = torch.randn(T * N, device='cuda', generator=g)
    ret = torch.randn(T * N, device='cuda', generator=g)
    perm = torch.randperm(T * N, device='cuda', generator=g)

    def run():
        fast = ppo.FastPPO(P.Policy(seed=21).cuda(), minibatch=2048, graph=False)
        buf = ppo.RolloutBuffer(T, N)
        buf.obs.copy_(obs)
        buf.actions.copy_(act)
        buf.logp.copy_(lp)
        o, a, l = fast._views(buf)
        fast.set_order(perm)
        a2, r2 = adv.clone(), ret.clone()
        for _ in range(3):
            fast._step(o, a, l, a2, r2)
        F = fast.flat
        return F.p.clone(), F.pb.clone(), F.m.clone(), F.v.clone(), fast.step_t.clone(), fast.loss_parts.clone()

    want = run()
    torch.cuda.synchronize()
    got = on_side_stream(run)
    for a, b in zip(want, got):
        assert torch.equal(a, b)
