"""The env oracle's uint8 15x15x8 encoder (o_obs, and the reveal that feeds it) pinned channel
by channel against what the reference's data fixes, over thousands of stepped states:

* the view (channel 2) is the player cell's bitset in the reference's LOS table
  (tests/golden/map1057_los.npz, gpu-d1/fixtures/fixture.bin, verified against native
  Crawl for every pair, gpu-d1/RESULTS.md:80) within radius 7;
* the memory behind channels 0, 1, 6 and 7 is tracked here from the player's trajectory
  alone: the union of those views since the last episode start
  (gpu-d1/branches/d1-stairs-v2/src/learn.cu:298-333 marks exactly the viewed cells), and
  it must equal the oracle's own `viewed` bitmap;
* wall = out of bounds or remembered non-floor, floor = remembered floor (the reference's
  remembered-terrain rule, learn.cu:488-491), monster kind + 1 and HP exactly on visible
  living monsters, the player's clamped HP everywhere, stairs on remembered stair cells,
  frontier = remembered floor with an in-bounds unviewed neighbour (learn.cu:269-280);
* on the same worlds, the learning-task oracle's fp32 terrain, visible-monster HP and
  visible-mask planes and its frontier-anchor list (pinned by the reference's
  test_wall_observations.cu and route-cue fixtures in tests/test_learn_oracle.py) equal
  channel 1 - channel 0, channel 4 / 16, channel 2 and channel 7.

The generated-level run takes the view from the oracle's runtime ray scan, which
tests/test_oracle_pins.py pins against the same LOS table for all 5,600 origins of map 1057."""
import ctypes as C
import importlib

import numpy as np
import pytest

from conftest import ROOT
from oracle import oracle as O

pkg = importlib.import_module('dcss-auto_amd')
W, H = 80, 70
LOS = np.load(ROOT / 'tests' / 'golden' / 'map1057_los.npz')['los']
# learning-task fp32 observation offsets (gpu-d1/branches/d1-stairs-v2/src/learn.cu:101-112)
VC, PLAYER_OBS = 225, 2 * 225 + 40 * 5
VISIBLE_OBS = PLAYER_OBS + 4 + 8 * 8 + 15


def view_cells(bits, player):
    """Cells of a 17x17 LOS bitset (bit (dy+8)*17+dx+8) within Chebyshev 7, in bounds."""
    out = np.zeros(5600, bool)
    px, py = player % W, player // W
    for dy in range(-7, 8):
        for dx in range(-7, 8):
            x, y = px + dx, py + dy
            b = (dy + 8) * 17 + dx + 8
            if 0 <= x < W and 0 <= y < H and (int(bits[b // 32]) >> (b % 32)) & 1:
                out[y * W + x] = True
    return out


def neighbours_unviewed(viewed):
    """Per cell: some in-bounds 8-neighbour is not viewed."""
    v = viewed.reshape(H, W)
    pad = np.pad(~v, 1, constant_values=False)
    any_ = np.zeros((H, W), bool)
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            if dx or dy:
                any_ |= pad[1 + dy:1 + dy + H, 1 + dx:1 + dx + W]
    return any_.reshape(-1)


def expected_window(f, viewed, view, floor, count):
    """The window the encoder's rules give for world record f."""
    want = np.zeros((15, 15, 8), np.uint8)
    px, py = int(f['player']) % W, int(f['player']) // W
    want[..., 5] = min(max(int(f['hp']), 0), 255)
    monsters = {int(f['pos'][i]): i for i in range(count) if f['mhp'][i] > 0}
    stairs = {int(s) for s in f['stairs'] if s >= 0}
    frontier = viewed & (floor != 0) & neighbours_unviewed(viewed)
    for dy in range(-7, 8):
        for dx in range(-7, 8):
            x, y = px + dx, py + dy
            cell = want[dy + 7, dx + 7]
            if not (0 <= x < W and 0 <= y < H):
                cell[0] = 1
                continue
            p = y * W + x
            cell[0] = viewed[p] and not floor[p]
            cell[1] = viewed[p] and floor[p]
            cell[2] = view[p]
            if view[p] and p in monsters:
                i = monsters[p]
                cell[3], cell[4] = int(f['kind'][i]) + 1, min(int(f['mhp'][i]), 255)
            cell[6] = p in stairs and viewed[p] and floor[p]
            cell[7] = frontier[p]
    return want


def learn_planes(f, viewed, count, maps, cfg):
    """The learning-task oracle's observation of the same world (map 1057): its fp32 obs and
    its frontier-anchor set."""
    L = O.learn_lib()
    dt = O.lstate_dtype()
    buf = np.zeros(dt.itemsize, np.uint8)
    s = buf.view(dt)[0]
    sc = list(O.SCALARS)
    s['scalars'][sc.index('player')] = int(f['player'])
    s['scalars'][sc.index('hp')] = int(f['hp'])
    s['scalars'][sc.index('next_slot')] = count
    s['scalars'][sc.index('first_stair_tick')] = -1
    s['stairs'][:] = -1
    s['occ'][:] = -1
    s['frontier_slot'][:] = -1
    s['enemy_slot'][:] = -1
    for i in range(count):
        s['pos'][i], s['mhp'][i], s['awake'][i] = f['pos'][i], f['mhp'][i], f['awake'][i]
        if f['mhp'][i] > 0:
            s['occ'][int(f['pos'][i])] = i
            s['enemy_slot'][i] = i
    s['viewed'][:] = viewed
    s['seen'][:] = viewed & (maps.floor[:5600] != 0)
    tab = maps.tables()
    for p in range(5600):
        L.lo_refresh_frontier(buf.ctypes.data, C.byref(tab), p)
    obs = np.zeros(1015, np.float32)
    mask = np.zeros(19, np.float32)
    L.lo_observe(buf.ctypes.data, C.byref(cfg), C.byref(tab), obs.ctypes.data, mask.ctypes.data)
    n = int(s['scalars'][sc.index('frontier_count')])
    anchors = np.zeros(5600, bool)
    anchors[s['frontier_cells'][:n]] = True
    return obs, anchors


def window_cells(player):
    """(dy+7, dx+7, cell) for the in-bounds cells of the window."""
    px, py = player % W, player // W
    for dy in range(-7, 8):
        for dx in range(-7, 8):
            x, y = px + dx, py + dy
            if 0 <= x < W and 0 <= y < H:
                yield dy + 7, dx + 7, y * W + x


CASES = [  # name, config, worlds, steps
    ('stairs task, map 1057, PCG', lambda: pkg.config.reference_config(8), 64, 24),
    ('v1 kill-all, map 1057, PCG', lambda: pkg.config.v1_config(8), 64, 20),
    ('BASELINE generated levels, counter RNG', lambda: pkg.baseline_config(8), 32, 36),
]


@pytest.mark.parametrize('name,make,n,steps', CASES)
def test_encoder_channels_follow_the_rules(name, make, n, steps):
    cfg = make()
    env = O.OracleEnv(n, cfg, seed=29, threads=8)
    shared = cfg.level_mode == pkg.config.LEVEL_SHARED
    floor_1057 = pkg.shared_map_arrays()[0]
    maps = O.LearnTablesHost([floor_1057], los=LOS.reshape(1, 5600, 10)) if shared else None
    lcfg = pkg.config.learn_config(cfg.count) if shared else None
    fields = env.fields()
    floors = [floor_1057 if shared else fields[i]['floor'].copy() for i in range(n)]

    def view_of(i, player):
        bits = LOS[player] if shared else O.los_bitset(floors[i], player)
        return view_cells(bits, player)

    tracked = [view_of(i, int(fields[i]['player'])) for i in range(n)]
    rng = np.random.default_rng(5)
    checked = crossed = 0
    for k in range(steps + 1):
        if k:
            env.step(rng.integers(0, 19, n))
            fields = env.fields()
        for i in range(n):
            f = fields[i]
            player = int(f['player'])
            view = view_of(i, player)
            if k and env.out[i, 1]:
                tracked[i] = view
            elif k:
                tracked[i] = tracked[i] | view
            assert np.array_equal(f['viewed'] != 0, tracked[i]), (name, k, i, 'memory')
            want = expected_window(f, tracked[i], view, floors[i], cfg.count)
            got = env.obs[i]
            if not np.array_equal(got, want):
                bad = np.argwhere(got != want)[:4].tolist()
                pytest.fail(f'{name} step {k} world {i}: (dy,dx,ch) {bad}')
            checked += 1
            if shared and (k + i) % 6 == 0:
                obs, anchors = learn_planes(f, tracked[i], cfg.count, maps, lcfg)
                for wy, wx, p in window_cells(player):
                    j = wy * 15 + wx
                    assert obs[j] == float(got[wy, wx, 1]) - float(got[wy, wx, 0]), (name, k, i, 'terrain')
                    assert obs[VISIBLE_OBS + j] == got[wy, wx, 2], (name, k, i, 'visible')
                    assert obs[VC + j] == np.float32(got[wy, wx, 4]) / np.float32(16), (name, k, i, 'enemy hp')
                    assert anchors[p] == bool(got[wy, wx, 7]), (name, k, i, 'frontier')
                crossed += 1
    assert checked >= 1000
    assert crossed >= 200 or not shared


def test_stair_channel_near_every_stair():
    """Channel 6 where random walks rarely go: the player placed on every floor cell within
    Chebyshev 7 of each stair of a map-1057 episode, with a fresh memory of that one view;
    the whole window must follow the rules, the stair marked exactly when that view (the
    LOS table) holds it."""
    cfg = pkg.config.reference_config(24)
    floor, cells = pkg.shared_map_arrays()
    w = O.OracleWorld(floor, cells)
    w.seed_pcg(123, 1)
    w.reset(cfg)
    marked = hidden = 0
    for s in w.f['stairs']:
        sx, sy = int(s) % W, int(s) // W
        for p in np.flatnonzero(floor):
            if max(abs(int(p) % W - sx), abs(int(p) // W - sy)) > 7:
                continue
            v = w.copy()
            v.f['viewed'][:] = 0
            v.f['player'] = p
            v.reveal()
            view = view_cells(LOS[p], int(p))
            want = expected_window(v.f, view, view, floor, cfg.count)
            got = v.obs(cfg)
            assert np.array_equal(got, want), (int(s), int(p), np.argwhere(got != want)[:4].tolist())
            marked += int(view[s])
            hidden += int(not view[s])
    assert marked > 20 and hidden > 20
