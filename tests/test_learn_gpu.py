"""GPU parity of the learn_* drop-in (libd1learn_clump{0,1}.so) against the CPU
restatement (oracle/learn_oracle.c): every step, bit for bit, the fp32 observation,
the mask, the 45 outcome fields, the controller's actions and the world state
(RNG, player, enemies, memory bitmap, frontier-list order)."""
import ctypes as C
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
W, N = 80, 5600


@pytest.fixture(scope='module')
def L():
    return importlib.import_module('dcss-auto_amd.learn')


@pytest.fixture(scope='module')
def O():
    from oracle import oracle
    oracle.learn_lib()
    return oracle


def gen_floors(O, k, seed=11):
    return [O.level(seed, e) for e in range(k)]


def compare_state(L, O, gpu_env, ref, step):
    g = L.decode_rows(gpu_env.state.cpu().numpy())
    r = ref.fields()
    names = {'player': 'player', 'hp': 'hp', 'regen': 'regen', 'blocks': 'blocks', 'ticks': 'ticks',
             'killed': 'killed', 'decisions': 'decisions', 'floor_seen': 'floor_seen', 'episode': 'episode',
             'first_stair_tick': 'first_stair_tick', 'map_id': 'map_id', 'next_slot': 'next_slot',
             'frontier_count': 'frontier_count', 'clumped': 'placement_clumped', 'error': 'error'}
    for gk, rk in names.items():
        np.testing.assert_array_equal(g[gk], ref.scalar(rk), err_msg=f'{gk} at step {step}')
    np.testing.assert_array_equal(g['stairs'], r['stairs'], err_msg=f'stairs at step {step}')
    np.testing.assert_array_equal(g['rng_state'], r['rng'][:, :8].copy().view(np.uint64)[:, 0],
                                  err_msg=f'rng at step {step}')
    for gk, rk in (('pos', 'pos'), ('hp', 'mhp'), ('energy', 'energy'), ('awake', 'awake'), ('slot', 'enemy_slot')):
        np.testing.assert_array_equal(g['mon'][gk], r[rk][:, :24], err_msg=f'enemy {gk} at step {step}')
    enc = (g['encountered'][:, None] >> np.arange(24, dtype=np.uint64)) & 1
    np.testing.assert_array_equal(enc, r['encountered'][:, :24], err_msg=f'encountered at step {step}')
    for i in range(len(g)):
        assert np.array_equal(L.bitmap_cells(g['viewed'][i]), r['viewed'][i].astype(bool)), f'viewed env {i} step {step}'
        n = int(g['frontier_count'][i])
        assert np.array_equal(g['frontier'][i][:n], r['frontier_cells'][i][:n].astype(np.uint16)), \
            f'frontier list env {i} step {step}'


def run_parity(L, O, floors, batch, steps, seed, clump, map_filter, check_state_every=1, limit=2048, rest_every=0):
    maps = L.LearnMaps(np.stack(floors))
    host = O.LearnTablesHost(np.stack(floors))
    assert np.array_equal(maps.los.cpu().numpy().view(np.uint32), host.los), 'LOS tables differ'
    env = L.LearnEnv(batch, seed=seed, maps=maps, map_filter=map_filter, clump=clump, limit=limit)
    ref = O.OracleLearn(batch, host, seed=seed, clump=clump, map_filter=map_filter, limit=limit, threads=8)
    ref.deadline_rests = 0
    rng = np.random.default_rng(seed)
    torch.cuda.synchronize()
    for step in range(steps):
        print(f'learn parity clump={clump} maps={len(floors)} step {step}', flush=True)
        assert np.array_equal(env.obs.cpu().numpy().view(np.uint32), ref.obs.view(np.uint32)), f'obs at step {step}'
        assert np.array_equal(env.mask.cpu().numpy(), ref.mask), f'mask at step {step}'
        if step % check_state_every == 0:
            compare_state(L, O, env, ref, step)
        h = ref.heuristic()
        assert np.array_equal(env.heuristic().cpu().numpy(), h), f'heuristic at step {step}'
        if rest_every and step % rest_every == 0:
            a = np.full(batch, 17, np.int64)
        elif step % 3 == 2:   # mix in random (also invalid) actions, some past 32 bits
            a = rng.integers(-1, 21, batch).astype(np.int64)
            wide = rng.random(batch) < 0.25   # low 32 bits an action, as the reference's int takes it
            a[wide] += rng.choice(np.array([2**32, -(2**32), 2**40, 5 * 2**33], np.int64), int(wide.sum()))
        else:
            a = h
        env.step(torch.from_numpy(a).cuda())
        assert ref.step(a) == 0
        assert np.array_equal(env.out.cpu().numpy().view(np.uint32), ref.out.view(np.uint32)), f'out at step {step}'
        o = ref.out   # REST decisions of several turns that ran into the deadline
        ref.deadline_rests += int(((o[:, 34] > 0) & (o[:, 35] > 1) & (o[:, 7] > 0)).sum())
    compare_state(L, O, env, ref, steps)
    return env, ref


def test_los_compiler_matches_fixture(L, golden):
    maps = L.LearnMaps()
    torch.cuda.synchronize()
    assert np.array_equal(maps.los[0].cpu().numpy().view(np.uint32), np.load(golden / 'map1057_los.npz')['los'])


def test_parity_map1057(L, O):
    env, ref = run_parity(L, O, [O.pkg.data.map1057()['floor']], batch=48, steps=300, seed=471, clump=0,
                          map_filter=-1)
    assert ref.scalar('episode').sum() > 0   # some episodes ended and reset inside the run


def test_parity_multimap_clumped(L, O):
    floors = [O.pkg.data.map1057()['floor']] + gen_floors(O, 3)
    env, ref = run_parity(L, O, floors, batch=48, steps=240, seed=5, clump=1, map_filter=-2, check_state_every=4)
    assert len(set(ref.scalar('map_id').tolist())) > 1
    assert ref.scalar('placement_clumped').any()


def test_parity_rests_into_the_deadline(L, O):
    """60-turn episodes with a REST decision every other step: many-turn rests end at full
    HP or run into the deadline (the turn that reaches it ends the episode and resets the
    world), on top of the controller's and random decisions; every step equals the CPU
    restatement's, observation, mask, outcome row and state."""
    env, ref = run_parity(L, O, [O.pkg.data.map1057()['floor']], batch=96, steps=300, seed=7, clump=0, map_filter=-1,
                          check_state_every=2, limit=60, rest_every=2)
    assert ref.deadline_rests > 20, ref.deadline_rests


@pytest.mark.parametrize('limit', [1, 2])
def test_parity_degenerate_deadlines(L, O, limit):
    """Deadlines of one and two turns (the first or second turn of every episode reaches
    it): each step times the episodes out and resets the worlds exactly as the CPU
    restatement does; a deadline below one turn is refused."""
    run_parity(L, O, [O.pkg.data.map1057()['floor']], batch=32, steps=24, seed=11, clump=0, map_filter=-1,
               check_state_every=1, limit=limit, rest_every=3)
    with pytest.raises(ValueError):
        L.LearnEnv(4, limit=0)


def test_active_mask_freezes_worlds(L, O):
    env = L.LearnEnv(32, seed=3)
    ref = O.OracleLearn(32, O.LearnTablesHost(O.pkg.data.map1057()['floor'][None]), seed=3)
    rng = np.random.default_rng(0)
    for step in range(40):
        active = rng.random(32) < 0.6
        a = ref.heuristic()
        before_state = env.state.clone()
        before_obs, before_out = env.obs.clone(), env.out.clone()
        env.step(torch.from_numpy(a).cuda(), torch.from_numpy(active).cuda())
        ref.step(a, active)
        frozen = torch.from_numpy(~active).cuda()
        assert torch.equal(env.state[frozen], before_state[frozen])
        assert torch.equal(env.obs[frozen], before_obs[frozen]) and torch.equal(env.out[frozen], before_out[frozen])
        assert np.array_equal(env.obs.cpu().numpy().view(np.uint32), ref.obs.view(np.uint32)), f'obs {step}'


def test_error_codes(L, pkg):
    env = L.LearnEnv(4, seed=1)
    lib = env.lib
    args = (env.state.data_ptr(), 4, C.byref(env.config), C.byref(env.tables), 1, env.obs.data_ptr(),
            env.mask.data_ptr(), env.stream)
    assert lib.learn_init(*args, 0) == -3            # no host path
    bad = pkg.config.learn_config(23)
    assert lib.learn_init(env.state.data_ptr(), 4, C.byref(bad), C.byref(env.tables), 1, env.obs.data_ptr(),
                          env.mask.data_ptr(), env.stream, 1) == -2
    assert lib.learn_turn_cost() == np.float32(1e-5) and lib.learn_return_gamma() == 1.0
    assert (lib.learn_obs_size(), lib.learn_action_size(), lib.learn_out_size(), lib.learn_config_bytes()) == \
        (1015, 19, 45, 140)


def test_parity_at_scale_slice(L, O):
    """8,192 worlds x 256 steps on four maps (map 1057 + three generated levels, first
    episodes balanced over the maps, clumped placement in a third of resets): worlds are
    independent and keyed by their index, so the first 512 are replayed by the restatement.
    Observation (bit patterns), mask and the 45 outcome fields every step, the controller's
    actions every 4th, the full world state every 16th (the reference's rows:
    gpu-d1/branches/d1-stairs-v2/src/learn.cu:891-946)."""
    floors = [O.pkg.data.map1057()['floor']] + gen_floors(O, 3, seed=23)
    maps = L.LearnMaps(np.stack(floors))
    host = O.LearnTablesHost(np.stack(floors))
    n, n_cpu, steps, seed = 8192, 512, 256, 1234
    env = L.LearnEnv(n, seed=seed, maps=maps, map_filter=-2, clump=1)
    ref = O.OracleLearn(n_cpu, host, seed=seed, clump=1, map_filter=-2, threads=16)
    rng = np.random.default_rng(seed)
    for step in range(steps):
        if step % 16 == 0:
            print(f'learn parity at scale: step {step}', flush=True)
            compare_state_slice(L, O, env, ref, step, n_cpu)
        h = env.heuristic()
        if step % 4 == 0:
            assert np.array_equal(h[:n_cpu].cpu().numpy(), ref.heuristic()), f'heuristic at step {step}'
        if step % 3 == 2:
            a = torch.from_numpy(rng.integers(-1, 21, n).astype(np.int64)).cuda()
        else:
            a = h
        env.step(a)
        assert ref.step(a[:n_cpu].cpu().numpy()) == 0
        assert np.array_equal(env.obs[:n_cpu].cpu().numpy().view(np.uint32), ref.obs.view(np.uint32)), f'obs {step}'
        assert np.array_equal(env.mask[:n_cpu].cpu().numpy(), ref.mask), f'mask at step {step}'
        assert np.array_equal(env.out[:n_cpu].cpu().numpy().view(np.uint32), ref.out.view(np.uint32)), f'out {step}'
    compare_state_slice(L, O, env, ref, steps, n_cpu)
    assert ref.scalar('episode').sum() > 0 and ref.scalar('placement_clumped').any()


def compare_state_slice(L, O, env, ref, step, n_cpu):
    class Rows:   # the first n_cpu state rows of the GPU batch, as compare_state reads them
        state = env.state[:n_cpu]
    compare_state(L, O, Rows, ref, step)
