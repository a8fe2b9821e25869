"""HIP environment vs the CPU oracle: per-step state hash, out[], the uint8 observation
and every field of the state rows must be identical (integer/byte work is bit-exact;
reward floats too)."""
import numpy as np
import pytest
import torch

from envstate import assert_same_worlds
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CASES = [
    # name, config factory args, batch, steps, actions
    ('baseline8', ('baseline_config', 8), 64, 300, 16),
    ('reference24', ('reference_config', 24), 40, 300, 19),
    ('v1_8', ('v1_config', 8), 37, 300, 9),
    ('stress40', ('stress_config',), 24, 200, 16),
    ('crowd64', ('make_config', 64), 24, 150, 16),   # the largest layout: 41-64 monsters
    ('single', ('make_config', 1), 24, 150, 16),     # the smallest roster
]


def make(pkg, spec):
    fn = getattr(pkg, spec[0])
    return fn(*spec[1:])


def compare(gpu, cpu, step, name):
    torch.cuda.synchronize()
    gh = gpu.hash.cpu().numpy().view(np.uint32)
    bad = np.flatnonzero(gh != cpu.hash)
    go = gpu.obs.cpu().numpy()
    bad_obs = np.flatnonzero((go != cpu.obs).reshape(len(go), -1).any(1))
    gout = gpu.out.cpu().numpy()
    bad_out = np.flatnonzero((gout.view(np.uint32) != cpu.out.view(np.uint32)).any(1)) if step >= 0 else []
    if len(bad) or len(bad_obs) or len(bad_out):
        e = int((list(bad) + list(bad_obs) + list(bad_out))[0])
        f = cpu.fields()[e]
        msg = (f'{name} step {step}: {len(bad)} hash, {len(bad_obs)} obs, {len(bad_out)} out mismatches; env {e} '
               f'player {f["player"]} hp {f["hp"]} ticks {f["ticks"]} episode {f["episode"]} '
               f'out gpu {gout[e]} cpu {cpu.out[e]}')
        if e in bad_obs:
            d = np.argwhere(go[e] != cpu.obs[e])[:5]
            msg += f' obs diffs (dy,dx,ch) {d.tolist()} gpu {[int(go[e][tuple(i)]) for i in d]} ' \
                   f'cpu {[int(cpu.obs[e][tuple(i)]) for i in d]}'
        pytest.fail(msg)
    assert_same_worlds(gpu.fields(), cpu.fields(), gpu.cfg, obs=go, label=f'{name} step {step}')


@pytest.mark.parametrize('name,spec,batch,steps,nact', CASES)
def test_hip_matches_oracle(pkg, name, spec, batch, steps, nact):
    print(f'[parity] {name} batch={batch} steps={steps}', flush=True)
    cfg = make(pkg, spec)
    gpu = pkg.Env(batch, cfg, seed=91)
    cpu = O.OracleEnv(batch, cfg, seed=91, threads=8)
    compare(gpu, cpu, -1, name)
    rng = np.random.default_rng(137)
    dones = 0
    for k in range(steps):
        a = rng.integers(0, nact, batch).astype(np.int64) if k % 2 else cpu.heuristic()
        cpu.step(a)
        gpu.step(torch.from_numpy(a).to(gpu.device))
        compare(gpu, cpu, k, name)
        dones += int(cpu.out[:, 1].sum())
    assert dones > 0
    print(f'[parity] {name} ok, {dones} episode ends', flush=True)


@pytest.mark.parametrize('name,spec,batch,steps,nact', CASES)
def test_v1_controller_matches_oracle(pkg, name, spec, batch, steps, nact):
    """Env.heuristic (d1_heuristic, the v1 pursuit controller of gpu-d1/src/learn.cu:599-621)
    equals the oracle's o_heuristic_v1 on every world at every step, as v1 action ids and as
    the joint actions they stand for on each world (a bump into a living monster is ATTACK);
    the worlds are driven by the controller's joint actions on even steps and by random
    actions on odd ones, and stay equal to the oracle's field by field."""
    from test_v1_reference_run import joint_actions
    print(f'[v1 controller] {name} batch={batch}', flush=True)
    cfg = make(pkg, spec)
    gpu = pkg.Env(batch, cfg, seed=5)
    cpu = O.OracleEnv(batch, cfg, seed=5, threads=8)
    rng = np.random.default_rng(11)
    kinds = set()
    for k in range(min(steps, 120)):
        v1 = cpu.heuristic_v1()
        ids = gpu.heuristic(v1_ids=True).cpu().numpy()
        joint = gpu.heuristic().cpu().numpy()
        bad = np.flatnonzero(ids != v1)
        assert not len(bad), f'{name} step {k}: world {bad[0]} v1 action gpu {ids[bad[0]]} oracle {v1[bad[0]]}'
        f = cpu.fields()
        want = joint_actions(f['player'], lambda i, q: f['occ'][i][q] >= 0, v1)
        assert np.array_equal(joint, want), f'{name} step {k}: joint actions differ'
        kinds.update(np.where(want == 16, 2, np.where(want >= 8, 1, 0)).tolist())
        a = joint if k % 2 == 0 else rng.integers(0, nact, batch).astype(np.int64)
        cpu.step(a)
        gpu.step(torch.from_numpy(a).to(gpu.device))
        compare(gpu, cpu, k, name)
    assert {0, 1} <= kinds, f'{name}: controller cases seen {kinds}'   # moves and attacks
    # with every monster dead the controller waits (learn.cu:613: no target)
    for i in range(gpu.max_monsters):
        gpu.state[:, 96 + 8 * i + 2:96 + 8 * i + 4] = 0   # Mon.hp (int16) of monster i
    assert (gpu.heuristic(v1_ids=True) == 8).all() and (gpu.heuristic() == 16).all()


@pytest.mark.parametrize('spec', [('baseline_config', 8), ('reference_config', 8), ('v1_config', 8),
                                  ('reference_config', 24), ('stress_config',)])
def test_step_without_hash_is_the_same_step(pkg, spec):
    """Env(hash=False) passes no hash buffer and the digest is skipped. Every step's state
    rows, observation and out[] must equal those of the same worlds stepped with the digest
    (the path test_hip_matches_oracle checks against the oracle every step), over moves,
    REST, descents and episode ends, on generated levels and on map 1057, in the <= 8
    monster and the crowded builds; the hash tensor keeps its value."""
    print(f'[parity] hash off {spec}', flush=True)
    cfg = make(pkg, spec)
    n = 2048
    a = pkg.Env(n, cfg, seed=5)
    b = pkg.Env(n, cfg, seed=5, hash=False)
    h0 = b.hash.clone()
    g = torch.Generator().manual_seed(9)
    dones = 0
    for k in range(240):
        act = torch.randint(0, 19, (n,), generator=g).cuda()
        a.step(act)
        b.step(act)
        torch.cuda.synchronize()
        rows = torch.nonzero((a.state != b.state).any(1)).flatten().tolist()
        assert not rows, f'step {k}: state rows differ for worlds {rows[:8]}'
        assert torch.equal(a.obs, b.obs), f'step {k}: observation'
        assert torch.equal(a.out, b.out), f'step {k}: out'
        dones += int(a.out[:, 1].sum())
    assert torch.equal(b.hash, h0)
    assert dones > 0


def test_crowded_field_memo_standing_player(pkg):
    """The crowded layouts reuse the stored distance field while the player stands still.
    40-monster worlds (half awake) driven mostly by WAIT and REST, with a move or an attack
    now and then, so most steps reload the stored field (and every move recomputes it):
    state hash, out[] and the observation equal the oracle's every step."""
    print('[parity] crowded field memo', flush=True)
    cfg = pkg.stress_config()
    n = 96
    gpu = pkg.Env(n, cfg, seed=13)
    cpu = O.OracleEnv(n, cfg, seed=13, threads=8)
    rng = np.random.default_rng(3)
    for k in range(160):
        a = np.where(rng.random(n) < 0.85, rng.choice([16, 17], n), rng.integers(0, 16, n)).astype(np.int64)
        cpu.step(a)
        gpu.step(torch.from_numpy(a).to(gpu.device))
        compare(gpu, cpu, k, 'crowded memo')
    tag, whole = memo_heads(gpu)
    assert (tag >= 0).any() and (whole[tag >= 0] == 1).all()    # generated levels are connected


def memo_heads(env):
    """The crowded rows' distance-field memo head (after the header, view, monsters and the
    viewed, floor and cells bitmaps): the player cell the stored field is for (-1: none)
    and bit 31 of its second dword, set when the stored field reaches the whole floor and
    its reach plane is not stored."""
    off = 96 + 8 * env.max_monsters + 3 * 840
    head = env.state[:, off:off + 8].cpu().numpy().copy().view('<u4')
    return head[:, 0].view('<i4'), head[:, 1] >> 31


def pocket_level(pkg):
    """Map 1057 plus a 3 x 3 floor pocket walled off from the rest (rows 7-9, columns
    38-40, two wall cells from the nearest floor): floor that no search from the player
    reaches and that is not spawnable."""
    floor, cells = pkg.shared_map_arrays()
    f = floor.reshape(70, 80).copy()
    assert not f[5:12, 36:43].any()    # the pocket and a two-cell wall ring around it
    f[7:10, 38:41] = 1
    return f.reshape(-1), cells


@pytest.mark.parametrize('count', [8, 24])
def test_level_with_an_unreachable_floor_pocket(pkg, count):
    """On a level whose floor is not one connected region, the distance field reaches less
    than the whole floor, so the crowded layouts store the reach plane with the field
    instead of taking the floor bitmap for it. Worlds driven mostly by WAIT and REST (most
    steps reload the stored field), with moves now and then: state rows, hash, out[] and
    the observation equal the oracle's every step, in the <= 8 monster and the crowded
    builds."""
    print(f'[parity] pocket level count={count}', flush=True)
    cfg = pkg.reference_config(count)
    level = pocket_level(pkg)
    n = 64
    gpu = pkg.Env(n, cfg, seed=21, level=level)
    cpu = O.OracleEnv(n, cfg, seed=21, threads=8, level=level)
    assert gpu.floors().sum(1).tolist() == [int(level[0].sum())] * n
    compare(gpu, cpu, -1, 'pocket')
    rng = np.random.default_rng(8)
    dones = stored = 0
    for k in range(240):
        if k % 3 == 0:
            a = cpu.heuristic()
        else:
            a = np.where(rng.random(n) < 0.7, rng.choice([16, 17], n), rng.integers(0, 19, n)).astype(np.int64)
        cpu.step(a)
        gpu.step(torch.from_numpy(a).to(gpu.device))
        compare(gpu, cpu, k, f'pocket{count}')
        dones += int(cpu.out[:, 1].sum())
        if count > 8:
            tag, whole = memo_heads(gpu)
            assert not whole[tag >= 0].any(), f'step {k}: a stored field claims to reach the pocket'
            stored += int((tag >= 0).sum())
    assert dones > 0 and (count == 8 or stored > 0)


def test_v1_controller_with_unreachable_monsters(pkg):
    """The pocket level with the pocket spawnable: players and monsters that start inside
    it are walled off from the rest, so the v1 controller meets living monsters it cannot
    reach (it waits when none is reachable, learn.cu:613, and otherwise targets the nearest
    reachable one). Its actions equal the oracle's on every world at every step, and the
    worlds, driven by those actions and random ones, stay equal to the oracle's."""
    from test_v1_reference_run import joint_actions
    print('[v1 controller] unreachable monsters', flush=True)
    floor, cells = pocket_level(pkg)
    cells = cells.reshape(70, 80).copy()
    cells[7:10, 38:41] = 1
    level = (floor, cells.reshape(-1))
    cfg = pkg.v1_config(8, sleep=False)
    n = 256
    gpu = pkg.Env(n, cfg, seed=33, level=level)
    cpu = O.OracleEnv(n, cfg, seed=33, threads=8, level=level)
    pocket = np.zeros(5600, bool)
    pocket.reshape(70, 80)[7:10, 38:41] = True
    rng = np.random.default_rng(4)
    walled_waits = split = 0
    for k in range(60):
        v1 = cpu.heuristic_v1()
        ids = gpu.heuristic(v1_ids=True).cpu().numpy()
        bad = np.flatnonzero(ids != v1)
        assert not len(bad), f'step {k}: world {bad[0]} gpu {ids[bad[0]]} oracle {v1[bad[0]]}'
        f = cpu.fields()
        live = f['mhp'][:, :8] > 0
        inside = pocket[f['pos'][:, :8].clip(0)] & live
        player_in = pocket[f['player']]
        walled_waits += int(((v1 == 8) & live.any(1) & (player_in != inside.any(1))).sum())
        split += int((live.any(1) & (inside.any(1) != player_in)).sum())
        joint = joint_actions(f['player'], lambda i, q: f['occ'][i][q] >= 0, v1)
        assert np.array_equal(gpu.heuristic().cpu().numpy(), joint), f'step {k}: joint actions differ'
        a = joint if k % 2 == 0 else rng.integers(0, 19, n).astype(np.int64)
        cpu.step(a)
        gpu.step(torch.from_numpy(a).to(gpu.device))
        compare(gpu, cpu, k, 'unreachable')
    assert walled_waits > 0 and split > 0, (walled_waits, split)


@pytest.mark.parametrize('spec', [('baseline_config', 8), ('stress_config',)])
def test_frozen_worlds_match_the_oracle(pkg, spec):
    """step(actions, active=mask) with a random half of the worlds frozen each step: the
    frozen worlds' state rows, observations and out rows stay bit for bit as they were (no
    RNG draw, no reset), and every world equals the oracle stepped with the same mask."""
    print(f'[parity] active mask {spec}', flush=True)
    cfg = make(pkg, spec)
    n = 48
    gpu = pkg.Env(n, cfg, seed=33)
    cpu = O.OracleEnv(n, cfg, seed=33, threads=8)
    rng = np.random.default_rng(12)
    frozen_steps = 0
    for k in range(120):
        a = rng.integers(0, 16, n).astype(np.int64) if k % 3 else cpu.heuristic()
        on = rng.random(n) < 0.5
        torch.cuda.synchronize()
        before = (gpu.state.clone(), gpu.obs.clone(), gpu.out.clone())
        cpu.step(a, active=on)
        gpu.step(torch.from_numpy(a).to(gpu.device), active=torch.from_numpy(on).to(gpu.device))
        torch.cuda.synchronize()
        off = torch.from_numpy(~on).to(gpu.device)
        for name, x, y in zip(('state', 'obs', 'out'), before, (gpu.state, gpu.obs, gpu.out)):
            assert torch.equal(x[off], y[off]), f'step {k}: a frozen world changed its {name}'
        frozen_steps += int((~on).sum())
        compare(gpu, cpu, k, f'active {spec[0]}')
    assert frozen_steps > 0


def test_out_of_range_actions_match_the_oracle(pkg):
    """int64 actions outside the action set (negative, past 18, past 2^31, and values whose
    low 32 bits are a valid action, as the reference's int parameter truncates them) step
    every world exactly as the oracle does."""
    print('[parity] out-of-range actions', flush=True)
    cfg = pkg.baseline_config(8)
    n = 64
    gpu = pkg.Env(n, cfg, seed=44)
    cpu = O.OracleEnv(n, cfg, seed=44, threads=8)
    odd = np.array([-1, -7, 16, 17, 18, 19, 1000, 1001, 2**31 - 1, -2**31, 2**32 + 3, 2**32 + 17,
                    2**40 + 18, -(2**33) + 5, 2**62], np.int64)
    rng = np.random.default_rng(5)
    for k in range(80):
        a = np.where(rng.random(n) < 0.5, rng.choice(odd, n), rng.integers(0, 16, n)).astype(np.int64)
        cpu.step(a)
        gpu.step(torch.from_numpy(a).to(gpu.device))
        compare(gpu, cpu, k, 'odd actions')


@pytest.mark.parametrize('limit,stairs', [(3, 3), (1, 3), (5, 0)])
def test_short_deadlines_and_stair_counts(pkg, limit, stairs):
    """Episode deadlines of one, three and five turns (every episode times out, the worlds
    reset every few steps), with and without stairs: state, observation, out[] and hash
    equal the oracle's every step. Stair counts other than 0 and 3 are refused."""
    print(f'[parity] limit {limit} stairs {stairs}', flush=True)
    cfg = pkg.make_config(8, limit=limit, stairs=stairs, awake_pct=30)
    n = 40
    gpu = pkg.Env(n, cfg, seed=17)
    cpu = O.OracleEnv(n, cfg, seed=17, threads=8)
    rng = np.random.default_rng(21)
    dones = 0
    for k in range(90):
        a = rng.integers(0, 19, n).astype(np.int64) if k % 2 else cpu.heuristic()
        cpu.step(a)
        gpu.step(torch.from_numpy(a).to(gpu.device))
        compare(gpu, cpu, k, f'limit{limit}')
        dones += int(cpu.out[:, 1].sum())
    assert dones > 0
    with pytest.raises(RuntimeError, match='code -2'):
        pkg.Env(4, pkg.make_config(8, stairs=1))


def test_v1_controller_ties(pkg):
    """The v1 controller's tie-breaks, from the reference's rules (gpu-d1/src/learn.cu:599-621)
    on worlds edited in the HIP state rows: among equally weak adjacent monsters the first
    direction (N, E, S, W, NE, SE, SW, NW) is attacked, a weaker one wins over an earlier
    direction; among equally near monsters (floor BFS) the lowest index is the target, and
    the step is the first neighbour one layer closer to it."""
    print('[v1 controller] ties', flush=True)
    DX, DY = (0, 1, 0, -1, 1, 1, -1, -1), (-1, 0, 1, 0, -1, 1, 1, -1)
    cfg = pkg.v1_config(8, sleep=False)
    env = pkg.Env(64, cfg, seed=12)
    f = env.fields()
    floor = env.floors()[0].astype(bool)
    mon = 96   # Mon rows: pos, hp (int16), energy (int16), awake, kind

    def nb(p, d):
        x, y = p % 80 + DX[d], p // 80 + DY[d]
        return y * 80 + x if 0 <= x < 80 and 0 <= y < 70 else -1

    def bfs(src):
        dist = np.full(5600, 65535, np.int64)
        dist[src] = 0
        frontier = [src]
        while frontier:
            nxt = []
            for p in frontier:
                for d in range(8):
                    q = nb(p, d)
                    if q >= 0 and floor[q] and dist[q] == 65535:
                        dist[q] = dist[p] + 1
                        nxt.append(q)
            frontier = nxt
        return dist

    def place(w, cells_hp):
        """monsters 0.. on the given cells with the given HP; the rest dead"""
        for i in range(8):
            pos, hp = cells_hp[i] if i < len(cells_hp) else (0, 0)
            raw = np.array([pos, hp], np.int16).view(np.uint8)
            env.state[w, mon + 8 * i:mon + 8 * i + 4] = torch.from_numpy(raw.copy()).to(env.device)

    checked = 0
    for w in range(64):
        p = int(f['player'][w])
        free = [d for d in range(8) if nb(p, d) >= 0 and floor[nb(p, d)]]
        if len(free) < 2:
            continue
        da, db = free[0], free[-1]
        place(w, [(nb(p, db), 5), (nb(p, da), 5)])        # equal HP: the earlier direction
        assert int(env.heuristic(v1_ids=True)[w]) == da
        assert int(env.heuristic()[w]) == 8 + da
        place(w, [(nb(p, db), 4), (nb(p, da), 5)])        # weaker wins over the earlier direction
        assert int(env.heuristic(v1_ids=True)[w]) == db
        # two monsters at the same floor distance >= 3 in different places: the lower index is the target
        dist = bfs(p)
        for k in (3, 4, 5):
            ring = np.flatnonzero(dist == k)
            if len(ring) < 2:
                continue
            a, b = int(ring[-1]), int(ring[0])
            back = bfs(a)
            want = next(d for d in range(8) if nb(p, d) >= 0 and floor[nb(p, d)] and back[nb(p, d)] == k - 1)
            place(w, [(a, 9), (b, 9)])
            assert int(env.heuristic(v1_ids=True)[w]) == want, (w, k)
            back_b = bfs(b)
            want_b = next(d for d in range(8) if nb(p, d) >= 0 and floor[nb(p, d)] and back_b[nb(p, d)] == k - 1)
            place(w, [(b, 9), (a, 9)])
            assert int(env.heuristic(v1_ids=True)[w]) == want_b, (w, k)
            checked += 1
            break
    assert checked >= 16, checked
