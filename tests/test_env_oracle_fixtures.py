"""The env oracle (oracle/d1_oracle.c), the checker of every C1/C2/C5 parity test, against
the reference's own hand-written fixtures, restated on this oracle's worlds. Each test names
the reference file it restates; the reference's asserted values are kept, and where the
reference reads a field this build does not have (its fp32 observation slots, its 45-wide
outcome row), the same fact is asserted through this build's state and outcome fields.

Configurations mirror the reference's: `Config c={}` with hp/count set (zero kinds, regen
and armour) for the v1 tests, the stairs-v2 learning configuration on map 1057 for the
stairs tests, and for the semantic tests the 12x5 test room that the reference's preflight
compiles around cell (40, 35) (branches/semantic-actions-v1/scripts/preflight.py:12,
branches/vision15-choice-practice-v1/scripts/map_compile.py:4-6)."""
import importlib

import numpy as np
import pytest

from oracle import oracle as O

pkg = importlib.import_module('dcss-auto_amd')
W = 80
WAIT, REST, DESCEND = 16, 17, 18
OPEN = np.ones(5600, np.uint8)


def v1_config(count, hp=20, limit=1024):
    """The reference tests' `Config c={}; c.hp=20; c.count=count` with v1's default rewards
    (gpu-d1/src/learn.cu:32-40,508: -1 milli per turn, +3000 clear, -1000 death)."""
    c = pkg.config.D1Config()
    c.count, c.hp, c.limit = count, hp, limit
    c.rng_mode, c.level_mode, c.roster_mode = pkg.config.RNG_PCG, pkg.config.LEVEL_SHARED, 0
    c.clear_on_kill_all, c.clear_milli, c.death_milli, c.kill_milli, c.step_milli = 1, 3000, 1000, 1000, -1
    c.explore_milli = 2
    return c


def room():
    """floor=[(x,y) for x in range(-2,10) for y in range(-2,3)] around (40, 35)."""
    f = np.zeros(5600, np.uint8)
    for x in range(-2, 10):
        for y in range(-2, 3):
            f[(35 + y) * W + 40 + x] = 1
    return f


# ---------------------------------------------------------------- gpu-d1/src/test_clear_reward.cu:4-21
@pytest.mark.parametrize('count', [8, 24, 40])
def test_clear_bonus_and_terminal_reset(count):
    """Every enemy dead: the next turn clears with +3 (CLEAR_PER_ENEMY_MILLI = 0, so the bonus
    does not scale with the enemy count) minus the 0.001 turn cost, then resets in place."""
    c = v1_config(count)
    w = O.OracleWorld(OPEN)
    w.seed_pcg(123, 1)
    w.reset(c)
    w.f['viewed'][:] = 1
    w.f['killed'] = count
    w.f['mhp'][:count] = 0
    out = w.transition(c, WAIT)
    assert out[1] == 1 and out[2] == 1 and out[6] == 0
    assert abs(out[0] - (3.0 - 0.001)) < 2e-6
    assert w.f['killed'] == 0 and w.f['hp'] == c.hp and w.f['episode'] == 1 and w.f['ticks'] == 0


# ---------------------------------------------------------------- gpu-d1/src/test_combat_ablations.cu:4-24
def test_death_penalty_and_auto_reset():
    """HP below zero: the turn ends the episode as a death with -(DEATH_MILLI + 1) milli, and
    the world is reset in place to full HP."""
    c = v1_config(1)
    w = O.OracleWorld(OPEN)
    w.seed_pcg(123, 1)
    w.reset(c)
    w.reset(c)
    w.f['viewed'][:] = 1
    w.f['hp'], w.f['regen'] = -100, 0
    out = w.transition(c, WAIT)
    assert out[6] == 1 and out[1] == 1 and w.f['hp'] == c.hp
    assert abs(out[0] - (-0.001 * (1000 + 1))) < 1e-6


def test_dead_enemy_leaves_the_observation():
    """The same file's observation half (:10-16): a living enemy is observed, a dead one is
    not. This build's window has no awake flag, so the living/dead half is what carries over:
    kind + 1 and HP on the enemy's cell while it lives, nothing once its HP is 0."""
    c = v1_config(1)
    w = O.OracleWorld(OPEN)
    w.seed_pcg(123, 1)
    w.reset(c)
    p0 = int(w.f['pos'][0])
    w.f['occ'][p0] = -1
    east = int(w.f['player']) + 1
    w.put(0, east, 10, awake=False, kind=3)
    o = w.obs(c)
    assert o[7, 8, 3] == 4 and o[7, 8, 4] == 10
    w.put(0, east, 10, awake=True, kind=3)
    assert np.array_equal(w.obs(c), o)          # awake or asleep: the same window
    w.f['mhp'][0] = 0
    o = w.obs(c)
    assert o[7, 8, 3] == 0 and o[7, 8, 4] == 0


# ---------------------------------------------------------------- branches/semantic-actions-v1/src/semantic_tests.cu:3-45
def isolated(hp=3):
    """semantic_tests.cu:3-7: an empty world (all enemies dead) with the player at (40, 35)
    of the test room, its view revealed."""
    c = pkg.config.reference_config(24, stairs=0)
    w = O.OracleWorld(room())
    w.f['player'], w.f['hp'], w.f['killed'] = 35 * W + 40, hp, 23
    w.f['energy'][:] = -30000
    w.reveal()
    return w, c


def test_rest_equals_repeated_waits():
    """:15-19: REST is the WAIT turns it stands for, RNG and regeneration included: the same
    world bytes, the reward their sum in turn order, as many turns."""
    base, c = isolated()
    macro, manual = base.copy(), base.copy()
    out = macro.transition(c, REST)
    count, reward = 0, np.float32(0)
    while True:
        step = manual.transition(c, WAIT)
        count += 1
        reward = np.float32(reward + step[0])
        if manual.f['hp'] >= c.hp:
            break
    manual.f['decisions'] = 1
    assert out[0] == reward and macro.f['ticks'] == count and count > 1
    assert np.array_equal(macro.state_bytes(), manual.state_bytes())


def test_sleep_radius_seven_rests_six_wakes():
    """:22-24: a sleeping enemy seven tiles away lets the REST run to full HP and stays
    asleep; at six tiles it wakes and interrupts the REST after one turn."""
    base, c = isolated()
    sleepy = base.copy()
    sleepy.put(0, 35 * W + 47, 8, awake=False)
    out = sleepy.transition(c, REST)
    assert not sleepy.f['awake'][0] and sleepy.f['hp'] == c.hp and sleepy.f['ticks'] > 1 and out[1] == 0
    waking = base.copy()
    waking.put(0, 35 * W + 46, 8, awake=False)
    waking.transition(c, REST)
    assert waking.f['ticks'] == 1 and waking.f['awake'][0]


def test_deadline_inside_rest():
    """:26-27: the physical deadline is exact inside a REST: one turn from 2047 ends the
    episode as a timeout at 2048 turns, and the world resets."""
    base, c = isolated()
    deadline = base.copy()
    deadline.f['ticks'] = 2047
    out = deadline.transition(c, REST)
    assert out[1] == 1 and out[7] == 1 and out[5] == 2048 and deadline.f['ticks'] == 0


@pytest.mark.parametrize('action', [8, 9, 13, 15, DESCEND, REST, 19, -1])
def test_invalid_action_is_one_wait(action):
    """:40-41: an invalid decision is one ordinary WAIT turn, not a zero-time transition. Here:
    ATTACK towards an empty cell, DESCEND off a stair, REST at full HP, ids outside 0..18;
    each leaves the world exactly as one WAIT does."""
    base, c = isolated(hp=18)
    a, b = base.copy(), base.copy()
    out_a = a.transition(c, action)
    out_b = b.transition(c, WAIT)
    assert a.f['ticks'] == 1
    assert np.array_equal(out_a, out_b) and np.array_equal(a.state_bytes(), b.state_bytes())


def test_move_into_visible_enemy_is_one_wait():
    """The joint-action rule beside it (branches/autoregressive-actions-v1/src/learn.cu:809-815):
    MOVE onto a visible enemy is invalid (that is ATTACK's job) and waits instead."""
    base, c = isolated(hp=18)
    base.put(0, 35 * W + 41, 8, awake=True)
    a, b = base.copy(), base.copy()
    a.transition(c, 1)       # MOVE east onto the enemy
    b.transition(c, WAIT)
    assert np.array_equal(a.state_bytes(), b.state_bytes())


# ---------------------------------------------------------------- branches/d1-stairs-v2/src/tests.cu:3-48
def stairs_world():
    c = pkg.config.reference_config(24)
    floor, cells = pkg.shared_map_arrays()
    w = O.OracleWorld(floor, cells)
    w.seed_pcg(123, 1)
    w.reset(c)
    return w, c


def harmless(w, c):
    """tests.cu:21: every enemy removed, the kill counter at REQUIRED."""
    f = w.f
    for i in range(c.count):
        f['occ'][f['pos'][i]] = -1
    f['mhp'][:c.count] = 0
    f['energy'][:c.count] = -30000
    f['killed'] = 24


def test_hidden_stairs_are_not_observed():
    """tests.cu:4-19: before any stair is seen, the window holds no stair, and moving the
    hidden stairs (permuted, or stair 0 onto an unseen cell) changes nothing observed."""
    w, c = stairs_world()
    o = w.obs(c)
    assert not o[..., 6].any()
    assert all(s >= 0 for s in w.f['stairs'])
    copy = w.copy()
    copy.f['stairs'][:] = np.roll(w.f['stairs'], -1)
    assert np.array_equal(copy.obs(c), o)
    seen = (w.f['viewed'] != 0) & (w.f['floor'] != 0)
    cells = np.flatnonzero(pkg.shared_map_arrays()[1])
    alternate = next(int(p) for p in cells if not seen[p] and p not in w.f['stairs'])
    copy.f['stairs'][0] = alternate
    assert np.array_equal(copy.obs(c), o)


def test_kill_all_does_not_end_and_invalid_descent_waits():
    """tests.cu:20-23: with the stairs task's rules, removing every enemy no longer ends the
    episode; DESCEND off a stair is one WAIT with the turn cost."""
    w, c = stairs_world()
    harmless(w, c)
    out = w.transition(c, WAIT)
    assert out[1] == 0 and out[3] == 24
    out = w.transition(c, DESCEND)
    assert out[1] == 0 and out[0] < 0


@pytest.mark.parametrize('k', [0, 1, 2])
def test_descent_from_each_stair(k):
    """tests.cu:24-30: on stair k the stair is observed under the player; standing is not
    descending; DESCEND ends the episode as a clear (no death, no timeout) with reward
    1 - 1e-5 > 0.9999."""
    w, c = stairs_world()
    for _ in range(k):       # the reference resets once per stair before this one
        w.reset(c)
    w.reset(c)
    harmless(w, c)
    w.f['player'] = w.f['stairs'][k]
    w.reveal()
    assert w.obs(c)[7, 7, 6] == 1
    out = w.transition(c, WAIT)
    assert out[1] == 0
    out = w.transition(c, DESCEND)
    assert out[1] == 1 and out[2] == 1 and out[6] == 0 and out[7] == 0 and out[0] > 0.9999


def test_stairs_deadline_is_a_timeout():
    """tests.cu:31-32: one turn from 2047 is a timeout at 2048 turns, not a clear."""
    w, c = stairs_world()
    harmless(w, c)
    w.f['ticks'] = 2047
    out = w.transition(c, WAIT)
    assert out[7] == 1 and out[2] == 0 and out[5] == 2048


def test_descent_leaves_enemies_alive():
    """tests.cu:45-47: descent succeeds before the enemies' next action and kills nothing."""
    w, c = stairs_world()
    w.reset(c)
    w.f['player'] = w.f['stairs'][0]
    w.reveal()
    out = w.transition(c, DESCEND)
    assert out[2] == 1 and out[3] == 0


# ---------------------------------------------------------------- gpu-d1/src/learn.cu:677-707 (learn_semantic_test)
def v1_world():
    """learn_semantic_test's world: the v1 rules on the fixture map with one monster,
    seed(123, 1), and the first floor cell p with a floor neighbour q (direction d)."""
    c = pkg.config.v1_config(1)
    floor, cells = pkg.shared_map_arrays()
    w = O.OracleWorld(floor, cells)
    w.seed_pcg(123, 1)
    w.reset(c)
    for p in np.flatnonzero(cells):
        for d, (dx, dy) in enumerate(((0, -1), (1, 0), (0, 1), (-1, 0), (1, -1), (1, 1), (-1, 1), (-1, -1))):
            x, y = int(p) % W + dx, int(p) // W + dy
            if 0 <= x < W and 0 <= y < 70 and floor[y * W + x]:
                return w, c, int(p), y * W + x, d


def test_v1_free_move_kill_deadline_and_death():
    w, c, p, q, d = v1_world()
    # free movement (:684-687)
    w.f['occ'][:] = -1
    w.f['player'], w.f['pos'][0], w.f['mhp'][0], w.f['energy'][0], w.f['killed'] = p, q, 0, -30000, 0
    out = w.transition(c, d)
    assert w.f['player'] == q and out[1] == 0
    # killing the last monster ends the episode before it can retaliate, then resets (:688-696):
    # +1000 kill, +3000 clear, -1 turn; the outcome row keeps the kill count and full HP
    for k in range(100):
        w.f['occ'][:] = -1
        w.f['player'], w.f['pos'][0], w.f['occ'][q], w.f['mhp'][0], w.f['energy'][0] = p, q, 0, 1, 79
        w.f['hp'], w.f['regen'], w.f['killed'], w.f['ticks'] = c.hp, 0, 0, 0
        out = w.transition(c, 8 + d)
        if out[2]:
            assert out[0] > 3.9 and out[3] == 1 and out[4] == c.hp
            break
        assert k < 99
    # a deadline is terminal with the timeout flag, not the death flag (:697-699)
    w.reset(c)
    w.f['ticks'], w.f['energy'][0] = c.limit - 1, -30000
    out = w.transition(c, WAIT)
    assert out[1] == 1 and out[7] == 1 and out[6] == 0 and w.f['ticks'] == 0
    # death terminates and reports the pre-reset HP (clamped at 0) (:700-702)
    w.reset(c)
    w.f['hp'], w.f['regen'] = -100, 0
    out = w.transition(c, WAIT)
    assert out[6] == 1 and out[4] == 0 and w.f['hp'] == c.hp


# ---------------------------------------------------------------- gpu-d1/scripts/test_learning.py:19-36,40-60
def v1_invariants(f, floor, c):
    """gpu-d1/scripts/test_learning.py:19-36 on every world of a batch."""
    for j in range(len(f)):
        s = f[j]
        live = [i for i in range(c.count) if s['mhp'][i] > 0]
        occ = s['occ']
        assert s['killed'] == c.count - len(live), j
        assert 0 < s['hp'] <= c.hp and 0 <= s['regen'] < 100 and 0 <= s['ticks'] < c.limit, j
        assert floor[s['player']] and occ[s['player']] == -1, j
        assert np.count_nonzero(occ >= 0) == len(live), j
        assert len({int(s['pos'][i]) for i in live}) == len(live), j
        for i in range(c.count):
            if i in live:
                p = int(s['pos'][i])
                assert floor[p] and occ[p] == i and s['energy'][i] < 80, (j, i)
            else:
                assert s['energy'][i] == -30000, (j, i)


@pytest.mark.parametrize('count', [1, 6, 8])
def test_v1_state_invariants_every_step(count):
    """The reference's learning test checks every world after the reset and between steps:
    the kill count equals the monsters no longer alive, 0 < HP <= 18, 0 <= regen < 100,
    0 <= ticks < 256, the player stands on a floor cell no monster occupies, there is one
    occupancy entry per living monster, at a distinct floor cell, holding its index, living
    monsters hold energy < 80 (every one that reached 80 has acted) and dead ones -30000.
    37 worlds, seed 91 and 1/6/8 enemies as there, controller and random decisions
    alternating over episode ends and resets; the invariants cover the reset's placement."""
    c = pkg.config.v1_config(count)
    env = O.OracleEnv(37, c, seed=91, threads=2)
    rng = np.random.default_rng(137)
    ends = 0
    for k in range(600):
        v1_invariants(env.fields(), env.floor, c)
        a = env.heuristic() if k % 2 == 0 else rng.integers(0, 19, 37).astype(np.int64)
        env.step(a)
        ends += int(env.out[:, 1].sum())
    v1_invariants(env.fields(), env.floor, c)
    assert ends > 0
