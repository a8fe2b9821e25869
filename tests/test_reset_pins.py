"""Pins of the resets' reservoir draws, which no reference-held log records: the three
stairs (gpu-d1/branches/d1-stairs-v2/src/learn.cu:425-438) in both oracles and the
learning task's clumps of three (learn.cu:378-400). What sampling fixes is checked, not
the oracle's code retyped:

* a copy of the RNG: the stairs and the clumps draw nothing from the play stream, so a
  reset with them leaves the player, the monsters' draws and the RNG state exactly as
  a reset without them;
* the eligibility bounds: every stair is at least 12 from the player and 8 from the
  earlier stairs, and both bounds are reached;
* the reservoir rule (candidate i of n kept when r(i) == 0): the choice is uniform over
  the eligible cells, which an exact chi-square of the chosen ranks checks.

Each check is shown to bite: mistakes planted in the oracle (o_plant, lo_plant) fail it.
No GPU needed."""
import ctypes as C
import importlib

import numpy as np
import pytest

from oracle import oracle as O

pkg = importlib.import_module('dcss-auto_amd')
W = 80
BATCH = 4096
CHI2_LIMIT = 1e-4     # the checks use fixed seeds, so they pass or fail deterministically


def cheb(a, b):
    a, b = np.asarray(a, np.int64), np.asarray(b, np.int64)
    return np.maximum(np.abs(a % W - b % W), np.abs(a // W - b // W))


def chi2_uniform_ranks(ranks, sizes, bins=10):
    """Chi-square p-value of ranks r in [0, n) against the uniform law, in `bins` bins of
    r / n; expected counts are summed exactly per sample (n need not divide by bins)."""
    from scipy.stats import chi2
    ranks, sizes = np.asarray(ranks), np.asarray(sizes)
    assert (ranks >= 0).all() and (ranks < sizes).all()
    got = np.bincount(ranks * bins // sizes, minlength=bins)
    want = np.zeros(bins)
    for n, k in zip(*np.unique(sizes, return_counts=True)):
        want += k * np.bincount(np.arange(n) * bins // n, minlength=bins) / n
    stat = ((got - want) ** 2 / want).sum()
    return chi2.sf(stat, bins - 1)


def chi2_small_ranks(ranks, sizes):
    """The same for small n (a clump member among 2-8 free neighbours): one cell per
    (n, rank), pooled over n."""
    from scipy.stats import chi2
    ranks, sizes = np.asarray(ranks), np.asarray(sizes)
    stat, df = 0.0, 0
    for n in np.unique(sizes):
        sel = ranks[sizes == n]
        if n < 2 or len(sel) < 20 * n:
            continue
        got = np.bincount(sel, minlength=n)
        want = len(sel) / n
        stat += ((got - want) ** 2 / want).sum()
        df += n - 1
    assert df > 0
    return chi2.sf(stat, df)


def stair_ranks(cells, player, occ, stairs):
    """Rank of each stair among its eligible cells, in cell-list order, and their count;
    None where a stair is not one of them (or missing)."""
    out = []
    for k in range(3):
        ok = (cheb(cells, player) >= 12) & (occ[cells] < 0)
        for q in range(k):
            ok &= cheb(cells, stairs[q]) >= 8
        eligible = cells[ok]
        where = np.flatnonzero(eligible == stairs[k])
        if len(where) != 1:
            return None
        out.append((int(where[0]), len(eligible)))
    return out


def uniformity(rows):
    """p-values of the three stairs' ranks over worlds given as (cells, player, occ,
    stairs); 0 for all three when a world's stairs are not eligible cells."""
    ranks, sizes = [[], [], []], [[], [], []]
    for row in rows:
        got = stair_ranks(*row)
        if got is None:
            return [0.0, 0.0, 0.0]
        for k, (r, n) in enumerate(got):
            ranks[k].append(r)
            sizes[k].append(n)
    return [chi2_uniform_ranks(ranks[k], sizes[k]) for k in range(3)]


# ---------------------------------------------------------------- env oracle (d1_oracle.c)
def env_worlds(stairs, seed=5):
    cfg = pkg.config.reference_config(stairs=stairs)
    return O.OracleEnv(BATCH, cfg, seed=seed, threads=8).fields()


def planted_env(mistake, stairs=3):
    lib = O.lib()
    lib.o_plant.argtypes = [C.c_int]
    try:
        lib.o_plant(mistake)
        return env_worlds(stairs)
    finally:
        lib.o_plant(0)


def env_stream_differs(with_stairs, without):
    keys = ('player', 'pos', 'mhp', 'energy', 'awake', 'rng_state', 'rng_inc', 'hp')
    return [k for k in keys if not np.array_equal(with_stairs[k], without[k])]


def env_support(f):
    s = f['stairs'].astype(np.int64)
    d_player = cheb(s[:, 0], f['player'])
    d_player = np.minimum(d_player, np.minimum(cheb(s[:, 1], f['player']), cheb(s[:, 2], f['player'])))
    spacing = np.minimum(np.minimum(cheb(s[:, 0], s[:, 1]), cheb(s[:, 0], s[:, 2])), cheb(s[:, 1], s[:, 2]))
    return int(d_player.min()), int(spacing.min())


def env_uniformity(f):
    return uniformity((w['cells'][:w['ncells']].astype(np.int64), int(w['player']), w['occ'],
                       w['stairs'].astype(np.int64)) for w in f)


@pytest.fixture(scope='module')
def env3():
    return env_worlds(3)


def test_env_stairs_draw_from_a_copy(env3):
    without = env_worlds(0)
    assert (without['stairs'] == -1).all() and (env3['stairs'] >= 0).all()
    assert env_stream_differs(env3, without) == []
    # planted: stairs drawn from the play stream move its state
    assert 'rng_state' in env_stream_differs(planted_env(4), without)


def test_env_stairs_eligibility_bounds(env3):
    assert env_support(env3) == (12, 8)
    assert env_support(planted_env(5))[0] == 13        # "more than 12" never reaches 12
    assert env_support(planted_env(6))[1] < 8          # the third stair too near the second


def test_env_stairs_uniform_over_eligible_cells(env3):
    p = env_uniformity(env3)
    assert min(p) > CHI2_LIMIT, p
    # planted: the draw bound counting every cell of the list skews the choice
    p = env_uniformity(planted_env(7))
    assert min(p) < 1e-12, p


# ---------------------------------------------------------------- learning task (learn_oracle.c)
@pytest.fixture(scope='module')
def maps():
    O.learn_lib()
    return O.LearnTablesHost(pkg.data.map1057()['floor'][None])


def learn_worlds(maps, clump, mistake=0, seed=7):
    L = O.learn_lib()
    L.lo_plant.argtypes = [C.c_int]
    try:
        L.lo_plant(mistake)
        e = O.OracleLearn(BATCH, maps, seed=seed, clump=clump, threads=8)
    finally:
        L.lo_plant(0)
    f = e.fields().copy()
    assert mistake or (e.scalar('error') == 0).all()   # a planted reservoir may place no stair
    return f


def sc(f, name):
    return f['scalars'][:, O.SCALARS.index(name)]


def learn_floor(maps):
    return pkg.data.map1057()['floor'].astype(bool)


def nb(p, a):
    dx, dy = [0, 1, 0, -1, 1, 1, -1, -1][a], [-1, 0, 1, 0, -1, 1, 1, -1][a]
    x, y = p % W + dx, p // W + dy
    return y * W + x if 0 <= x < W and 0 <= y < 70 else -1


def clump_ranks(maps, f):
    """Replays each world's clumps from its final positions: the anchor's rank among the
    cells with at least two free floor neighbours, each member's rank among the anchor's
    free neighbours in direction order, the smallest free-neighbour count of a chosen
    anchor, and the number of worlds whose placement is not such a replay (a reset that
    stopped with an error, or positions that break the rules)."""
    floor = learn_floor(maps)
    cells = maps.cells[:maps.ncells[0]].astype(np.int64)
    nbr = np.array([[nb(p, a) for a in range(8)] for p in cells])
    valid = nbr >= 0
    nbr = np.where(valid, nbr, 0)
    a_rank, a_size, m_rank, m_size, least, broken = [], [], [], [], 8, 0
    for w in f:
        player = int(w['scalars'][O.SCALARS.index('player')])
        if w['scalars'][O.SCALARS.index('error')]:
            broken += 1
            continue
        occ = np.full(5600, -1)
        pos = w['pos'].astype(np.int64)
        ranks = []
        for i in range(0, 24, 3):
            free = floor & (occ < 0)
            free[player] = False
            nfree = (valid & free[nbr]).sum(1)
            eligible = cells[free[cells] & (nfree >= 2)]
            r = np.flatnonzero(eligible == pos[i])
            if len(r) != 1:
                break
            ranks.append(('a', int(r[0]), len(eligible), int(nfree[np.searchsorted(cells, pos[i])])))
            occ[pos[i]] = i
            for k in (1, 2):
                cand = [nb(pos[i], a) for a in range(8)]
                cand = [q for q in cand if q >= 0 and floor[q] and q != player and occ[q] < 0]
                if pos[i + k] not in cand:
                    break
                ranks.append(('m', cand.index(pos[i + k]), len(cand), 0))
                occ[pos[i + k]] = i + k
            else:
                continue
            break
        if len(ranks) != 24:
            broken += 1
            continue
        for kind, r, n, nf in ranks:
            if kind == 'a':
                a_rank.append(r)
                a_size.append(n)
                least = min(least, nf)
            else:
                m_rank.append(r)
                m_size.append(n)
    return a_rank, a_size, m_rank, m_size, least, broken


def learn_stair_uniformity(maps, f):
    cells = maps.cells[:maps.ncells[0]].astype(np.int64)
    return uniformity((cells, int(w['scalars'][O.SCALARS.index('player')]), w['occ'], w['stairs'].astype(np.int64))
                      for w in f)


@pytest.fixture(scope='module')
def plain(maps):
    return learn_worlds(maps, 0)


@pytest.fixture(scope='module')
def clumped(maps):
    return learn_worlds(maps, 2)


def learn_stream_differs(a, b):
    keys = ('rng', 'energy', 'mhp', 'awake')
    out = [k for k in keys if not np.array_equal(a[k], b[k])]
    return out + [k for k in ('player', 'hp', 'map_id') if not np.array_equal(sc(a, k), sc(b, k))]


def test_learn_clumps_and_stairs_draw_from_copies(maps, plain, clumped):
    assert (sc(clumped, 'placement_clumped') == 1).all() and (sc(plain, 'placement_clumped') == 0).all()
    assert learn_stream_differs(plain, clumped) == []
    assert not np.array_equal(plain['pos'], clumped['pos'])
    bad = learn_worlds(maps, 2, mistake=1)
    assert 'rng' in learn_stream_differs(plain, bad)


def test_learn_stairs_bounds_and_uniformity(maps, plain, clumped):
    for f in (plain, clumped):
        s = f['stairs'].astype(np.int64)
        player = sc(f, 'player').astype(np.int64)
        d = np.min([cheb(s[:, k], player) for k in range(3)], axis=0)
        spacing = np.min([cheb(s[:, a], s[:, b]) for a, b in ((0, 1), (0, 2), (1, 2))], axis=0)
        assert d.min() == 12 and spacing.min() == 8
        p = learn_stair_uniformity(maps, f)
        assert min(p) > CHI2_LIMIT, p
    p = learn_stair_uniformity(maps, learn_worlds(maps, 0, mistake=2))
    assert min(p) < 1e-12, p


def test_learn_clumps_uniform_anchor_and_members(maps, clumped):
    a_rank, a_size, m_rank, m_size, least, broken = clump_ranks(maps, clumped)
    assert broken == 0
    assert least == 2                                  # "at least two free neighbours" is reached
    assert chi2_uniform_ranks(a_rank, a_size) > CHI2_LIMIT
    assert chi2_small_ranks(m_rank, m_size) > CHI2_LIMIT
    # planted: members drawn with the direction index as the bound (most resets then find
    # no member for some clump and stop with an error)
    bad = clump_ranks(maps, learn_worlds(maps, 2, mistake=3))
    assert bad[5] > BATCH // 2, bad[5]
    # planted: anchors needing three free neighbours never sit at two
    bad = clump_ranks(maps, learn_worlds(maps, 2, mistake=4))
    assert bad[5] == 0 and bad[4] == 3
