"""The fixed-panel evaluator of the learning task (dcss-auto_amd/learn.py:evaluate_panel)
on 32 generated levels x 32 episodes: every episode ends, freezing finished worlds does
not change any outcome (the reference's measurement, gpu-d1/PERFORMANCE.md:25-29, found
the same), per-map rates average to the panel's, and a repeat gives identical numbers."""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def panel(pkg):
    learn = importlib.import_module('dcss-auto_amd.learn')
    floors = pkg.Env(32, pkg.baseline_config(8), seed=21, hash=False).floors()
    maps = learn.LearnMaps(floors)
    env = learn.LearnEnv(1024, maps=maps, map_filter=-2, limit=256, clump=1)
    return learn, env


def test_generated_floors_hold_their_worlds(pkg):
    env = pkg.Env(64, pkg.baseline_config(8), seed=4, hash=False)
    floors = env.floors()
    assert floors.shape == (64, 5600) and set(np.unique(floors)) <= {0, 1}
    rows = env.state.cpu().numpy()
    player = rows[:, 28:30].copy().view('<i2')[:, 0]
    mons = rows[:, 96:96 + 64].copy().view('<i2').reshape(64, 8, 4)
    assert all(floors[i, player[i]] for i in range(64))
    for i in range(64):
        for pos, hp, _, _ in mons[i]:
            if hp > 0:
                assert floors[i, pos]
    print(f'[panel] floor cells per level {floors.sum(1).min()}..{floors.sum(1).max()}', flush=True)
    assert (floors.sum(1) >= 72).all()   # the generator's lower bound (room sizes x room count)


def test_panel_ends_and_freezing_changes_no_outcome(panel):
    learn, env = panel
    print('[panel] heuristic', flush=True)
    a = learn.evaluate_panel(env, 'heuristic', decisions=512, active=True)
    b = learn.evaluate_panel(env, 'heuristic', decisions=512, active=False)
    assert len(env.errors()) == 0
    assert a['unfinished'] == 0 and b['unfinished'] == 0
    for key in ('clear_rate', 'death_rate', 'kills', 'shaped_return'):
        assert a[key] == b[key], key
    assert a['maps'] == b['maps']
    assert abs(np.mean([m['clear_rate'] for m in a['maps']]) - a['clear_rate']) < 1e-6
    print(f"[panel] clear {a['clear_rate']:.3f} death {a['death_rate']:.3f} kills {a['kills']:.2f} "
          f"{a['seconds']:.3f} s frozen vs {b['seconds']:.3f} s", flush=True)


def test_panel_with_a_sampled_policy_repeats(panel):
    learn, env = panel
    policy = learn.MaskedPolicy().cuda()
    a = learn.evaluate_panel(env, policy, decisions=300)
    b = learn.evaluate_panel(env, policy, decisions=300)
    assert {k: v for k, v in a.items() if k != 'seconds'} == {k: v for k, v in b.items() if k != 'seconds'}
    assert 0.0 <= a['clear_rate'] <= 1.0 and 0.0 <= a['death_rate'] <= 1.0
