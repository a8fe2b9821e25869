"""REST is repeated WAITs (the property the reference's own semantic self-test asserts for
its macro, gpu-d1/branches/semantic-actions-v1/src/semantic_tests.cu:12-45, and that the
d1-stairs-v2 transition keeps, branches/d1-stairs-v2/src/learn.cu:853-875): one REST
decision leaves every world, RNG included, exactly where WAITs repeated as many turns
leave it, and its reward is their rewards summed in order. Checked on the HIP library
against itself with the reference's PCG stream (per-draw sequence), independent of the
oracle. Only the decision and counter-step fields differ (one decision vs k). Also: an
invalid decision is exactly one WAIT turn."""
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu

T_OFF, DEC_OFF, TICKS_OFF = 20, 44, 36   # header: u32 t, i32 decisions, i32 ticks


def i32(state, off):
    return state[:, off:off + 4].contiguous().view(torch.int32)[:, 0]


def test_rest_equals_repeated_waits(pkg):
    print('[rest] REST vs WAITs', flush=True)
    n = 2048
    env = pkg.Env(n, pkg.reference_config(24), seed=21, hash=False)
    g = torch.Generator().manual_seed(4)
    for _ in range(80):   # moves, attacks and waits: players get hurt, monsters wake
        env.step(torch.randint(0, 17, (n,), generator=g).cuda())
    before = env.state.clone()
    _, out = env.step(torch.full((n,), 17, dtype=torch.int64, device='cuda'))
    rest_state, rest_out = env.state.clone(), out.clone()
    done = rest_out[:, 1] > 0
    k = i32(rest_state, TICKS_OFF) - i32(before, TICKS_OFF)   # turns the decision took
    live = ~done
    assert bool((k[live] >= 1).all())
    assert int((k[live] > 1).sum()) >= 20, 'too few real rests to test'
    env.state.copy_(before)
    total = torch.zeros(n, device='cuda')
    wait = torch.full((n,), 16, dtype=torch.int64, device='cuda')
    for i in range(int(k[live].max())):
        act = live & (k > i)
        _, o = env.step(wait, active=act)
        total = torch.where(act, total + o[:, 0], total)   # fp32, in turn order, as the macro sums
    torch.cuda.synchronize()
    a, b = rest_state[live].clone(), env.state[live].clone()
    assert torch.equal(i32(b, DEC_OFF) - i32(a, DEC_OFF), k[live] - 1)
    for off in (T_OFF, DEC_OFF):   # the only fields allowed to differ
        a[:, off:off + 4] = 0
        b[:, off:off + 4] = 0
    assert torch.equal(a, b)
    assert torch.equal(total[live], rest_out[live, 0])


def test_learning_task_rest_equals_repeated_waits():
    """The same on the learn_* drop-in (d1-stairs-v2 task, map 1057, 24 enemies): state,
    frontier list, observation and mask equal; out[0] and out[40] (undiscounted in this
    task) are the summed rewards and out[26] the turn count."""
    L = importlib.import_module('dcss-auto_amd.learn')
    print('[rest] learning task', flush=True)
    n = 2048
    env = L.LearnEnv(n, seed=33, clump=0)
    g = torch.Generator().manual_seed(6)
    for _ in range(80):
        env.step(torch.randint(0, 17, (n,), generator=g).cuda())
    before = (env.state.clone(), env.obs.clone(), env.mask.clone())
    _, out = env.step(torch.full((n,), 17, dtype=torch.int64, device='cuda'))
    rest_state, rest_obs, rest_mask, rest_out = env.state.clone(), env.obs.clone(), env.mask.clone(), out.clone()
    done = rest_out[:, 1] > 0
    k = rest_out[:, 26].to(torch.int64)
    live = ~done
    assert bool((k[live] >= 1).all()) and int((k[live] > 1).sum()) >= 20, 'too few real rests to test'
    env.state.copy_(before[0]); env.obs.copy_(before[1]); env.mask.copy_(before[2])
    total = torch.zeros(n, device='cuda')
    wait = torch.full((n,), 16, dtype=torch.int64, device='cuda')
    for i in range(int(k[live].max())):
        act = live & (k > i)
        _, o = env.step(wait, active=act)
        total = torch.where(act, total + o[:, 0], total)
    torch.cuda.synchronize()
    a, b = rest_state[live].clone(), env.state[live].clone()
    DEC = 32   # learn header: i32 decisions
    assert torch.equal(i32(b, DEC) - i32(a, DEC), k[live].to(torch.int32) - 1)
    a[:, DEC:DEC + 4] = 0
    b[:, DEC:DEC + 4] = 0
    assert torch.equal(a, b)
    assert torch.equal(env.obs[live], rest_obs[live]) and torch.equal(env.mask[live], rest_mask[live])
    assert torch.equal(total[live], rest_out[live, 0]) and torch.equal(total[live], rest_out[live, 40])


def test_invalid_actions_are_one_wait(pkg):
    """An invalid decision degrades to one ordinary WAIT turn, not a zero-time transition
    (the reference's semantic self-test, semantic_tests.cu:44): out-of-range codes on the
    HIP env, and on the learning task every action its own mask marks invalid."""
    print('[rest] invalid actions', flush=True)
    n = 2048
    env = pkg.Env(n, pkg.reference_config(24), seed=5, hash=False)
    g = torch.Generator().manual_seed(8)
    for _ in range(40):
        env.step(torch.randint(0, 17, (n,), generator=g).cuda())
    before = env.state.clone()
    codes = torch.tensor([-1, 19, 50, 1000, 2000, -7], dtype=torch.int64)
    bad = codes[torch.randint(0, len(codes), (n,), generator=g)].cuda()
    _, o1 = env.step(bad)
    s1, out1, obs1 = env.state.clone(), o1.clone(), env.obs.clone()
    env.state.copy_(before)
    _, o2 = env.step(torch.full((n,), 16, dtype=torch.int64, device='cuda'))
    assert torch.equal(s1, env.state) and torch.equal(out1, o2) and torch.equal(obs1, env.obs)

    L = importlib.import_module('dcss-auto_amd.learn')
    lenv = L.LearnEnv(n, seed=9, clump=0)
    for _ in range(40):
        lenv.step(torch.randint(0, 17, (n,), generator=g).cuda())
    masked = (lenv.mask[:, :19] == 0)
    assert int(masked.any(1).sum()) > n // 2
    pick = torch.where(masked, torch.rand(n, 19, device='cuda'), torch.full((n, 19), -1.0, device='cuda')).argmax(1)
    acts = torch.where(masked.any(1), pick, torch.full_like(pick, 16)).contiguous()
    before = (lenv.state.clone(), lenv.obs.clone(), lenv.mask.clone())
    _, o1 = lenv.step(acts)
    s1, out1, obs1, m1 = lenv.state.clone(), o1.clone(), lenv.obs.clone(), lenv.mask.clone()
    lenv.state.copy_(before[0]); lenv.obs.copy_(before[1]); lenv.mask.copy_(before[2])
    _, o2 = lenv.step(torch.full((n,), 16, dtype=torch.int64, device='cuda'))
    assert torch.equal(s1, lenv.state) and torch.equal(obs1, lenv.obs) and torch.equal(m1, lenv.mask)
    # the outcome rows agree except the REST statistics of worlds that asked for an invalid REST
    keep = torch.ones(45, dtype=torch.bool, device='cuda')
    keep[34:40] = False
    assert torch.equal(out1[:, keep], o2[:, keep])
    assert bool((out1[acts == 17, 38] == 1).all())   # flagged as an invalid REST
