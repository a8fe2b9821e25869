"""CPU pins of the learning-task restatement (oracle/learn_oracle.c) against the
reference's own semantic tests and fixtures, restated with the d1-stairs-v2 layout:

* gpu-d1/src/test_route_cue.cu            route cue: detour, unknown shortcut, direct
                                          route, adjacent, at-target, unreachable, absent
* gpu-d1/src/test_wall_observations.cu    reveal counts, remembered ring walls, the
                                          seven frontier-pointer fields (ring-memory branch)
* gpu-d1/branches/d1-stairs-v2/src/tests.cu  hidden stairs, descent, deadline, remembered
                                          stair cue, descent with enemies alive
* fixture tables: LOS of every origin and the fixture player's distance row.
No GPU needed."""
import numpy as np
import pytest

W, N = 80, 5600
FRONTIER_OBS, RING_OBS, STAIR_OBS = 718, 654, 999


@pytest.fixture(scope='module')
def O():
    from oracle import oracle
    oracle.learn_lib()
    return oracle


def blank(O, maps, hp=18):
    """A zeroed world on map 0: no enemies on the map, empty memory."""
    buf = np.zeros(O.lstate_dtype().itemsize, np.uint8)
    f = buf.view(O.lstate_dtype())[0]
    f['occ'][:] = -1
    f['frontier_slot'][:] = -1
    f['enemy_slot'][:] = -1
    f['stairs'][:] = [N - 1, N - 2, N - 3]
    return buf, f


def setv(f, name, v):
    f['scalars'][__import__('oracle.oracle', fromlist=['SCALARS']).SCALARS.index(name)] = v


def getv(f, name):
    return int(f['scalars'][__import__('oracle.oracle', fromlist=['SCALARS']).SCALARS.index(name)])


def observe(O, buf, maps, cfg):
    import ctypes as C
    o = np.zeros(1015, np.float32)
    m = np.zeros(19, np.float32)
    O.learn_lib().lo_observe(buf.ctypes.data, C.byref(cfg), C.byref(maps.tables()), o.ctypes.data, m.ctypes.data)
    return o, m


def known_distances(O, buf, maps, nearest_only=0):
    import ctypes as C
    ds = np.zeros(N, np.uint16)
    O.learn_lib().lo_known_distances(buf.ctypes.data, C.byref(maps.tables()), ds.ctypes.data, nearest_only)
    return ds


def test_fixture_tables(O, pkg, golden):
    """LOS of every origin equals fixture.bin's table; the all-pairs row of the fixture
    player equals fixture.bin's distance field (gpu-d1/src/bench.cu:131-134)."""
    m = pkg.data.map1057()
    maps = O.LearnTablesHost(m['floor'][None])
    assert np.array_equal(maps.los[0], np.load(golden / 'map1057_los.npz')['los'])
    row = maps.distance[maps.index[3631]]
    assert np.array_equal(row, m['dist'])


def test_route_cue(O, pkg):
    """gpu-d1/src/test_route_cue.cu: the cue follows known floor only."""
    import ctypes as C
    floor = np.zeros(N, np.uint8)
    maps = O.LearnTablesHost(floor[None])
    cfg = pkg.config.learn_config()
    buf, f = blank(O, maps)
    player = 20 * W + 20
    setv(f, 'player', player)
    setv(f, 'hp', 18)

    def known(x, y):
        p = y * W + x
        maps.floor[p] = 1
        f['viewed'][p] = 1
        f['seen'][p] = 1

    def check(target, expected):
        ds = known_distances(O, buf, maps)
        assert O.learn_lib().lo_route_first_step(player, target, ds.ctypes.data) == expected
        setv(f, 'frontier_count', 1)
        f['frontier_cells'][0] = target
        f['frontier_slot'][:] = -1
        f['frontier_slot'][target] = 0
        o, _ = observe(O, buf, maps, cfg)
        assert list(o[FRONTIER_OBS + 7:FRONTIER_OBS + 15]) == [float(d == expected) for d in range(8)]

    for x in range(18, 21):
        known(x, 20)
    for y in range(20, 25):
        known(18, y)
    for x in range(18, 25):
        known(x, 24)
    for y in range(20, 25):
        known(24, y)
    target = 20 * W + 24
    check(target, 3)                       # detour west around the known wall
    for x in range(21, 24):
        maps.floor[20 * W + x] = 1         # an unseen direct corridor changes nothing
    check(target, 3)
    for x in range(21, 24):
        known(x, 20)
    check(target, 1)                       # observed: east
    check(player + 1, 1)                   # adjacent
    check(player, -1)                      # at the target
    known(40, 40)
    check(40 * W + 40, -1)                 # unreachable
    setv(f, 'frontier_count', 0)
    o, _ = observe(O, buf, maps, cfg)
    assert not o[FRONTIER_OBS:FRONTIER_OBS + 15].any()   # absent


def test_wall_observations(O, pkg):
    """gpu-d1/src/test_wall_observations.cu (ring-memory-walls branch) with the
    d1-stairs-v2 radii: view 7 (225 cells), ring 8 (64 cells), pointer at 718."""
    import ctypes as C
    floor = np.ones(N, np.uint8)
    los = np.full((1, N, 10), 0xFFFFFFFF, np.uint32)   # every cell in range visible
    maps = O.LearnTablesHost(floor[None], los=los)
    cfg = pkg.config.learn_config()
    L = O.learn_lib()
    buf, f = blank(O, maps)
    player = 20 * W + 20
    setv(f, 'player', player)
    setv(f, 'hp', 18)
    t = maps.tables()
    maps.floor[player + 1] = 0
    assert L.lo_reveal(buf.ctypes.data, C.byref(t)) == 224     # walls are recorded, not rewarded
    assert f['viewed'][player + 1] and not f['seen'][player + 1]
    assert f['seen'][player] and L.lo_reveal(buf.ctypes.data, C.byref(t)) == 0
    p = player - 8 * W - 8                                       # first outer-ring entry
    f['viewed'][p] = 0
    maps.floor[p] = 1
    assert observe(O, buf, maps, cfg)[0][RING_OBS] == 0
    maps.floor[p] = 0
    assert observe(O, buf, maps, cfg)[0][RING_OBS] == 0
    f['viewed'][p] = 1
    assert observe(O, buf, maps, cfg)[0][RING_OBS] == -1
    maps.floor[p] = 1
    f['seen'][p] = 1
    assert observe(O, buf, maps, cfg)[0][RING_OBS] == 1
    # one seen anchor with one unknown neighbour: all seven pointer fields
    f['viewed'][:] = 1
    f['seen'][:] = 0
    f['frontier_slot'][:] = -1
    setv(f, 'frontier_count', 0)
    anchor, unknown = player + 6, player + 7
    f['seen'][anchor] = 1
    f['viewed'][unknown] = 0
    L.lo_refresh_frontier(buf.ctypes.data, C.byref(t), anchor)
    assert getv(f, 'frontier_count') == 1
    o, _ = observe(O, buf, maps, cfg)
    b = FRONTIER_OBS
    assert o[b] == 1 and o[b + 1] == np.float32(6 / 80) and o[b + 2] == 0 and o[b + 3] == np.float32(6 / 150)
    assert o[b + 4] == np.float32(1 / 8) and o[b + 5] == 1 and o[b + 6] == 0
    before = o.copy()
    maps.floor[unknown] = 0                                      # unknown terrain is either kind
    L.lo_refresh_frontier(buf.ctypes.data, C.byref(t), anchor)
    assert np.array_equal(observe(O, buf, maps, cfg)[0], before)
    f['viewed'][unknown] = 1
    L.lo_refresh_frontier(buf.ctypes.data, C.byref(t), anchor)
    o, _ = observe(O, buf, maps, cfg)
    assert getv(f, 'frontier_count') == 0
    assert not o[FRONTIER_OBS:FRONTIER_OBS + 15].any()


def pcg_seed(f, s, seq):
    """gpu-d1/src/sim.h:29-35 on the world's RNG words."""
    M, mask = 6364136223846793005, (1 << 64) - 1
    inc = ((seq << 1) | 1) & mask
    st = 0
    st = (st * M + inc) & mask
    st = (st + s) & mask
    st = (st * M + inc) & mask
    rng = f['rng'].view(np.uint64)
    rng[0], rng[1] = st, inc
    f['rng'][40:44] = 0   # mode 0 (PCG)


def test_stairs_semantics(O, pkg):
    """gpu-d1/branches/d1-stairs-v2/src/tests.cu on map 1057."""
    import ctypes as C
    maps = O.LearnTablesHost(pkg.data.map1057()['floor'][None])
    cfg = pkg.config.learn_config()
    L = O.learn_lib()
    t = maps.tables()
    buf, f = blank(O, maps)
    pcg_seed(f, 123, 1)
    w = buf.ctypes.data
    out = np.zeros(45, np.float32)

    def reset():
        L.lo_reset(w, C.byref(cfg), C.byref(t), 0)
        assert getv(f, 'error') == 0

    def transition(a):
        L.lo_transition(w, C.byref(cfg), C.byref(t), a, 2048, out.ctypes.data, 0)
        return out.copy()

    def harmless():
        for i in range(24):
            f['occ'][f['pos'][i]] = -1
            f['mhp'][i] = 0
            f['energy'][i] = -30000
        setv(f, 'killed', 24)

    reset()
    obs, mask = observe(O, buf, maps, cfg)
    stairs = [int(v) for v in f['stairs']]
    assert not any(f['seen'][s] for s in stairs) and not mask[18]
    assert not obs[STAIR_OBS:].any()
    # hidden stair placement changes no observation or mask
    copy = buf.copy()
    cf = copy.view(O.lstate_dtype())[0]
    cf['stairs'][:] = [stairs[1], stairs[2], stairs[0]]
    assert np.array_equal(observe(O, copy, maps, cfg)[0], obs)
    cells = maps.cells[:maps.ncells[0]]
    alternate = next(int(p) for p in cells if not f['seen'][p] and p not in stairs)
    cf['stairs'][0] = alternate
    assert np.array_equal(observe(O, copy, maps, cfg)[0], obs)
    # removing all enemies no longer ends the episode; invalid descent waits
    harmless()
    o = transition(16)
    assert not o[1] and o[3] == 24
    o = transition(18)
    assert not o[1] and o[0] < 0
    for k in range(3):
        reset()
        harmless()
        setv(f, 'player', int(f['stairs'][k]))
        L.lo_reveal(w, C.byref(t))
        obs, mask = observe(O, buf, maps, cfg)
        assert mask[18] and obs[STAIR_OBS + 15] and obs[STAIR_OBS] > 0
        assert not transition(16)[1]                    # standing is not descending
        o = transition(18)
        assert o[1] and o[2] and not o[6] and not o[7]
        assert o[44] == k + 1 and o[26] == 1 and o[0] > 0.9999
    reset()
    harmless()
    setv(f, 'ticks', 2047)
    o = transition(16)
    assert o[7] and not o[2] and o[5] == 2048
    # a stair remembered out of LOS keeps its cue; unknown floor is excluded
    reset()
    harmless()
    start, goal = getv(f, 'player'), int(f['stairs'][0])
    setv(f, 'player', goal)
    L.lo_reveal(w, C.byref(t))
    setv(f, 'player', start)
    obs, _ = observe(O, buf, maps, cfg)
    assert not L.lo_in_view(w, C.byref(t), goal) and obs[STAIR_OBS] > 0
    ds = known_distances(O, buf, maps)
    assert bool(obs[STAIR_OBS + 1]) == (L.lo_nearest_stair(w, ds.ctypes.data) >= 0)
    for p in cells:                                     # reveal a connected route
        setv(f, 'player', int(p))
        L.lo_reveal(w, C.byref(t))
    setv(f, 'player', start)
    obs, _ = observe(O, buf, maps, cfg)
    assert obs[STAIR_OBS + 1]
    dirs = np.flatnonzero(obs[STAIR_OBS + 7:STAIR_OBS + 15])
    assert len(dirs) == 1
    dx, dy = [0, 1, 0, -1, 1, 1, -1, -1][dirs[0]], [-1, 0, 1, 0, -1, 1, 1, -1][dirs[0]]
    assert f['viewed'][start + dy * W + dx]
    # descent can leave enemies alive and succeeds before their next action
    reset()
    setv(f, 'player', int(f['stairs'][0]))
    L.lo_reveal(w, C.byref(t))
    o = transition(18)
    assert o[2] and o[3] == 0 and o[9] + o[10] == 24


def test_frontier_list_is_the_anchor_set(O, pkg):
    """Invariant of the incremental list (learn.cu:281-296): after any sequence of steps
    its entries are exactly the anchor cells (seen floor with an unviewed neighbour),
    each once, and frontier_slot indexes them."""
    maps = O.LearnTablesHost(pkg.data.map1057()['floor'][None])
    env = O.OracleLearn(8, maps, seed=7)
    rng = np.random.default_rng(1)
    floor = maps.floor.reshape(70, 80).astype(bool)
    for step in range(120):
        a = env.heuristic() if step % 2 else rng.integers(0, 19, 8)
        env.step(a)
        for f in env.fields():
            n = int(f['scalars'][13])
            lst = f['frontier_cells'][:n].astype(int)
            viewed = f['viewed'].reshape(70, 80).astype(bool)
            pad = np.pad(~viewed, 1, constant_values=False)
            unviewed_nb = np.zeros_like(viewed)
            for dy in (-1, 0, 1):
                for dx in (-1, 0, 1):
                    if dx or dy:
                        unviewed_nb |= pad[1 + dy:71 + dy, 1 + dx:81 + dx]
            anchors = np.flatnonzero((floor & viewed & unviewed_nb).reshape(-1))
            assert sorted(lst) == list(anchors)
            assert np.array_equal(f['frontier_slot'][lst], np.arange(n))


# ---------------------------------------------------------------- branches/semantic-actions-v1/src/semantic_tests.cu:3-45
def semantic_room(O):
    """The 12x5 test room the reference's preflight compiles around (40, 35)
    (branches/semantic-actions-v1/scripts/preflight.py:12)."""
    f = np.zeros(N, np.uint8)
    for x in range(-2, 10):
        for y in range(-2, 3):
            f[(35 + y) * W + 40 + x] = 1
    return O.LearnTablesHost([f])


def isolated(O, maps, cfg, hp=3):
    """semantic_tests.cu:3-7: all-zero world, player at (40, 35), REQUIRED-1 kills, every
    enemy dead with -30000 energy, no stairs, the view revealed."""
    buf, f = blank(O, maps)
    f['stairs'][:] = -1
    f['energy'][:] = -30000
    setv(f, 'player', 35 * W + 40)
    setv(f, 'hp', hp)
    setv(f, 'killed', 23)
    setv(f, 'first_stair_tick', -1)
    import ctypes as C
    O.learn_lib().lo_reveal(buf.ctypes.data, C.byref(maps.tables()))
    return buf, f


def put(f, i, p, hp, awake):
    f['pos'][i], f['mhp'][i], f['awake'][i] = p, hp, int(awake)
    f['occ'][p] = i


def transition(O, buf, maps, cfg, action, limit=2048):
    import ctypes as C
    out = np.zeros(45, np.float32)
    O.learn_lib().lo_transition(buf.ctypes.data, C.byref(cfg), C.byref(maps.tables()), action, limit, out.ctypes.data, 0)
    return out


def test_semantic_rest_sleep_deadline_invalid(O, pkg):
    """The reference's semantic self-test on its 45-field outcome row: REST equals the WAIT
    turns it stands for (world bytes, reward, out[26] and out[35] turn counts, out[36]
    completed, out[37] not interrupted, out[40] the return at learn_return_gamma() = 1);
    a sleeper at seven tiles lets the REST complete, one at six wakes and interrupts it
    after one turn; the deadline is exact inside a REST; an ATTACK with no target is one
    WAIT turn."""
    maps = semantic_room(O)
    cfg = pkg.config.learn_config()
    base, f = isolated(O, maps, cfg)
    macro, manual = base.copy(), base.copy()
    out = transition(O, macro, maps, cfg, 17)
    count, reward = 0, np.float32(0)
    while True:
        step = transition(O, manual, maps, cfg, 16)
        count += 1
        reward = np.float32(reward + step[0])
        if getv(manual.view(O.lstate_dtype())[0], 'hp') >= cfg.hp:
            break
    setv(manual.view(O.lstate_dtype())[0], 'decisions', 1)
    assert count > 1 and out[0] == reward and out[40] == reward
    assert out[26] == count and out[35] == count and out[36] == 1 and out[37] == 0
    assert np.array_equal(macro, manual)

    sleepy = base.copy()
    s = sleepy.view(O.lstate_dtype())[0]
    put(s, 0, 35 * W + 47, 8, False)
    out = transition(O, sleepy, maps, cfg, 17)
    assert out[36] == 1 and out[37] == 0 and not s['awake'][0]
    waking = base.copy()
    s = waking.view(O.lstate_dtype())[0]
    put(s, 0, 35 * W + 46, 8, False)
    out = transition(O, waking, maps, cfg, 17)
    assert out[26] == 1 and out[37] == 1 and s['awake'][0]

    deadline = base.copy()
    s = deadline.view(O.lstate_dtype())[0]
    setv(s, 'ticks', 2047)
    out = transition(O, deadline, maps, cfg, 17)
    assert out[1] == 1 and out[7] == 1 and out[5] == 2048 and out[26] == 1 and getv(s, 'ticks') == 0

    invalid = base.copy()
    s = invalid.view(O.lstate_dtype())[0]
    out = transition(O, invalid, maps, cfg, 8)
    assert out[26] == 1 and getv(s, 'ticks') == 1


def test_controller_priority_order(O, pkg):
    """The stairs controller's rules in the order of gpu-d1/branches/d1-stairs-v2/src/
    learn.cu:876-888 (descend, attack the weakest adjacent visible enemy, rest, wait while an
    awake enemy is in view, the route to a remembered stair, engage, explore): worlds on map
    1057 in which two of them apply at once each get the earlier rule's action. Engage and
    explore exclude each other (engage needs an enemy in view, explore none: :459,471), and
    rest and wait do too. Each pair is shown to bite: the two rules swapped in the oracle
    (lo_plant 10-15) change that world's action."""
    import ctypes as C
    maps = O.LearnTablesHost(pkg.data.map1057()['floor'][None])
    cfg = pkg.config.learn_config()
    L = O.learn_lib()
    L.lo_plant.argtypes = [C.c_int]
    L.lo_heuristic_one.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    L.lo_route_first_step.argtypes = [C.c_int, C.c_int, C.c_void_p]
    L.lo_nearest_stair.argtypes = [C.c_void_p, C.c_void_p]
    t = maps.tables()
    floor = maps.floor[:N].astype(bool)
    DX, DY = (0, 1, 0, -1, 1, 1, -1, -1), (-1, 0, 1, 0, -1, 1, 1, -1)

    def nb(p, d):
        x, y = p % W + DX[d], p // W + DY[d]
        return y * W + x if 0 <= x < W and 0 <= y < 70 else -1

    # a floor cell whose eight neighbours are floor, and the map revealed from every cell
    player = next(p for p in range(N) if floor[p] and all(nb(p, d) >= 0 and floor[nb(p, d)] for d in range(8)))
    base, f = blank(O, maps)
    for p in maps.cells[:maps.ncells[0]]:
        setv(f, 'player', int(p))
        L.lo_reveal(base.ctypes.data, C.byref(t))
    setv(f, 'player', player)
    setv(f, 'hp', cfg.hp)
    ds = np.zeros(N, np.uint16)
    L.lo_known_distances(base.ctypes.data, C.byref(t), ds.ctypes.data, 0)
    stair = int(np.flatnonzero(floor & (ds < 65535))[np.argmax(ds[floor & (ds < 65535)])])   # the farthest known cell

    def world(on_stair=False, hp=None, enemy=None, awake=1, known_stair=False):
        buf = base.copy()
        g = buf.view(O.lstate_dtype())[0]
        if hp is not None:
            setv(g, 'hp', hp)
        if on_stair:
            g['stairs'][0] = player
        if known_stair:
            g['stairs'][0] = stair
            assert g['seen'][stair]
        if enemy is not None:
            g['pos'][0], g['mhp'][0], g['occ'][enemy], g['awake'][0], g['enemy_slot'][0] = enemy, 10, 0, awake, 0
            g['encountered'][0] = 1
            assert L.lo_in_view(buf.ctypes.data, C.byref(t), enemy)
        return buf

    def act(buf, plant=0):
        L.lo_plant(plant)
        try:
            return L.lo_heuristic_one(buf.ctypes.data, C.byref(cfg), C.byref(t))
        finally:
            L.lo_plant(0)

    def route(buf, goal):
        d = np.zeros(N, np.uint16)
        L.lo_known_distances(buf.ctypes.data, C.byref(t), d.ctypes.data, 0)
        return L.lo_route_first_step(player, goal, d.ctypes.data)

    adjacent = nb(player, 1)   # east
    # a visible cell two or three steps away whose route's first step differs from the stair's
    to_stair = route(world(known_stair=True), stair)
    assert to_stair >= 0
    far = next(p for p in range(N) if floor[p] and 2 <= max(abs(p % W - player % W), abs(p // W - player // W)) <= 3
               and L.lo_in_view(base.ctypes.data, C.byref(t), p) and route(base, p) not in (-1, to_stair))
    cases = [
        # (world, faithful action, planted swap, the swapped rule's action)
        (world(on_stair=True, enemy=adjacent), 18, 10, 8 + 1),                              # descend > attack
        (world(hp=cfg.hp - 8, enemy=adjacent, awake=0), 8 + 1, 11, 17),                     # attack > rest
        (world(enemy=adjacent, awake=1), 8 + 1, 12, 16),                                    # attack > wait
        (world(hp=cfg.hp - 8, known_stair=True), 17, 13, to_stair),                         # rest > stair route
        (world(enemy=far, awake=1, known_stair=True), 16, 14, to_stair),                    # wait > stair route
        (world(enemy=far, awake=0, known_stair=True), to_stair, 15, route(base, far)),      # stair route > engage
    ]
    for k, (buf, want, plant, swapped) in enumerate(cases):
        assert act(buf) == want, f'case {k}'
        assert act(buf, plant) == swapped != want, f'case {k}: planted swap {plant}'
