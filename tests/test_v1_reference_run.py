"""The reference's own recorded parity run, replayed on the CPU restatement.

gpu-d1/scripts/test_learning.py:39-61 steps the default v1 build (gpu-d1/Makefile:14-16: no
SLEEP_ON, so every monster is awake from the start) on map 1057: 37 worlds, seed 91, with 1, 6
and 8 enemies, 300 steps each. Even steps take the v1 pursuit controller's actions
(gpu-d1/src/learn.cu:599-621), odd steps torch.randint(0, 9, (37,)) after one
torch.manual_seed(137) (tests/golden/v1_random_actions.npz, written by make_v1_actions.py).
Its log records the episodes that ended in each run (gpu-d1/results/learning-v1-tests.log:1-3):
352, 136 and 133. Those counts compose the reset's draw order, the transition, the monster
rules and the controller over 11,100 world-steps per run, so they pin all four together.

v1's actions are a direction 0-7 (move, or melee when the cell holds a monster: the "bump")
or 8 (wait); this build's joint actions split the bump into MOVE d (0-7) and ATTACK d (8-15),
so each v1 action is mapped on the world it is applied to: a direction whose cell holds a
monster -> ATTACK, any other direction -> MOVE (a wall then leaves the player in place, as in
v1), 8 -> WAIT (16).
"""
import importlib
import pathlib

import numpy as np
import pytest

from oracle import oracle as O

pkg = importlib.import_module('dcss-auto_amd')
GOLDEN = pathlib.Path(__file__).resolve().parent / 'golden'
TERMINATIONS = {1: 352, 6: 136, 8: 133}   # gpu-d1/results/learning-v1-tests.log:1-3
RUNS = (1, 6, 8)
DX = (0, 1, 0, -1, 1, 1, -1, -1)          # N, E, S, W, NE, SE, SW, NW (gpu-d1/src/sim.h:201-206)
DY = (-1, 0, 1, 0, -1, 1, 1, -1)


def random_stream():
    return np.load(GOLDEN / 'v1_random_actions.npz')['actions'].astype(np.int64)


def joint_actions(player, occupied, v1):
    """v1 actions -> joint actions for worlds whose player cells are `player` and whose
    occupancy test is `occupied(i, cell)`."""
    out = np.empty(len(v1), np.int64)
    for i, a in enumerate(v1):
        a = int(a)
        if a == 8:
            out[i] = 16
            continue
        x, y = int(player[i]) % 80 + DX[a], int(player[i]) // 80 + DY[a]
        bump = 0 <= x < 80 and 0 <= y < 70 and occupied(i, y * 80 + x)
        out[i] = 8 + a if bump else a
    return out


def replay(enemies, stream, on_step=None):
    """The run of test_learning.py:41-59 on the oracle; returns the number of episodes ended."""
    cfg = pkg.v1_config(enemies, sleep=False)
    env = O.OracleEnv(37, cfg, seed=91)
    ended = 0
    for k in range(300):
        v1 = stream[k // 2] if k % 2 else env.heuristic_v1()
        f = env.fields()
        actions = joint_actions(f['player'], lambda i, p: f['occ'][i][p] >= 0, v1)
        env.step(actions)
        o = env.out
        # the reference run's own per-step checks (test_learning.py:54-57)
        assert np.array_equal(o[:, 1], o[:, 2] + o[:, 6] + o[:, 7])
        assert ((o[:, 3] >= 0) & (o[:, 3] <= enemies)).all() and ((o[:, 4] >= 0) & (o[:, 4] <= 18)).all()
        ended += int(o[:, 1].sum())
        if on_step is not None:
            on_step(k, actions, env)
    return ended


@pytest.mark.parametrize('enemies', RUNS)
def test_reference_recorded_terminations(enemies):
    run = RUNS.index(enemies)
    assert replay(enemies, random_stream()[run]) == TERMINATIONS[enemies]


def test_random_stream_fixture_is_torch_seed_137():
    """The committed stream is what make_v1_actions.py draws (torch's CPU generator)."""
    torch = pytest.importorskip('torch')
    torch.manual_seed(137)
    want = random_stream()
    for run in range(3):
        for k in range(1, 300, 2):
            assert np.array_equal(torch.randint(0, 9, (37,)).numpy(), want[run, k // 2])


@pytest.mark.parametrize('mistake', [1, 2, 3])
def test_planted_mistakes_change_the_counts(mistake):
    """The counts bite: a monster's energy drawn before its cell at reset (1), the
    controller's ties kept by the later candidate (2), or the player's damage 1 + r(5) (3),
    each planted in the oracle, moves at least one run off the recorded counts."""
    lib = O.lib()
    lib.o_plant.argtypes = [O.C.c_int]
    stream = random_stream()
    try:
        lib.o_plant(mistake)
        got = [replay(e, stream[r]) for r, e in enumerate(RUNS)]
    finally:
        lib.o_plant(0)
    assert got != [TERMINATIONS[e] for e in RUNS], got


@pytest.mark.gpu
@pytest.mark.parametrize('enemies', RUNS)
def test_hip_reference_recorded_run(enemies):
    """The same run on the HIP environment. The reference feeds its CPU controller's actions
    to both simulators (test_learning.py:48-49); here the even steps take the HIP
    controller's own actions (Env.heuristic, d1_heuristic), which must equal the CPU
    controller's on every world (as v1 ids, and as joint actions mapped on the HIP world's
    own decoded row), and drive both. Every step the state rows (field by field), the state
    hash, out[] and the observation must equal the oracle's, and the HIP worlds' own
    episode ends must add up to the recorded count."""
    import torch
    from envstate import assert_same_worlds
    print(f'[v1 run] enemies={enemies}', flush=True)
    cfg = pkg.v1_config(enemies, sleep=False)
    gpu = pkg.Env(37, cfg, seed=91)
    cpu = O.OracleEnv(37, cfg, seed=91)
    stream = random_stream()[RUNS.index(enemies)]
    ended = 0
    for k in range(300):
        v1 = stream[k // 2] if k % 2 else cpu.heuristic_v1()
        f = gpu.fields()
        live = f['mhp'][:, :enemies] > 0
        actions = joint_actions(f['player'], lambda i, p: bool((live[i] & (f['pos'][i, :enemies] == p)).any()), v1)
        if k % 2 == 0:   # the HIP controller's own actions drive the step
            assert np.array_equal(gpu.heuristic(v1_ids=True).cpu().numpy(), v1), f'v1 controller at step {k}'
            hip = gpu.heuristic().cpu().numpy()
            assert np.array_equal(hip, actions), f'joint controller actions at step {k}'
            actions = hip
        cpu.step(actions)
        gpu.step(torch.from_numpy(actions).cuda())
        torch.cuda.synchronize()
        out = gpu.out.cpu().numpy()
        obs = gpu.obs.cpu().numpy()
        assert np.array_equal(gpu.hash.cpu().numpy().view(np.uint32), cpu.hash), f'hash at step {k}'
        assert np.array_equal(out.view(np.uint32), cpu.out.view(np.uint32)), f'out at step {k}'
        assert np.array_equal(obs, cpu.obs), f'observation at step {k}'
        assert_same_worlds(gpu.fields(), cpu.fields(), cfg, obs=obs, label=f'step {k}')
        ended += int(out[:, 1].sum())
    assert ended == TERMINATIONS[enemies]
    print(f'[v1 run] enemies={enemies}: {ended} terminations', flush=True)
