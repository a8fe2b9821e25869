"""Runtime rule configuration (mirror of `D1Config` in include/d1hip.h) and presets.

The player stats and the six-kind roster come from the map-1057 fixture header
(gpu-d1/src/bench.cu:107-127; decoded values in gpu-d1/fixtures/native-1057.json
"roster"); the task switches replace the reference's compile-time -D flags
(gpu-d1/Makefile:14-95, gpu-d1/branches/d1-stairs-v2/scripts/assets.py:5).
"""
import ctypes as C

import numpy as np

from . import data


class D1Kind(C.Structure):
    _fields_ = [('speed', C.c_int32), ('damage', C.c_int32), ('tohit', C.c_int32), ('bypass', C.c_int32)]


class D1Config(C.Structure):
    _fields_ = ([('count', C.c_int32)] +
                [(k, C.c_int32) for k in ('hp', 'ac100', 'ev100', 'sh100', 'shield_limit', 'regen', 'repair')] +
                [('gdr', C.c_int32 * 2), ('kinds', D1Kind * 6)] +
                [(k, C.c_int32) for k in ('limit', 'rng_mode', 'level_mode', 'roster_mode', 'hp_lo', 'hp_hi',
                                           'awake_pct', 'wake_los', 'stairs', 'clear_on_kill_all',
                                           'explore_milli', 'kill_milli', 'clear_milli', 'death_milli',
                                           'step_milli')] +
                [('turn_cost', C.c_float)])

    def as_dict(self):
        out = {}
        for name, _ in self._fields_:
            v = getattr(self, name)
            if name == 'gdr':
                v = list(v)
            elif name == 'kinds':
                v = [[k.speed, k.damage, k.tohit, k.bypass] for k in v]
            out[name] = v
        return out


class D1Tables(C.Structure):
    _fields_ = [('floor', C.c_void_p), ('cells', C.c_void_p), ('ray_slots', C.c_void_p), ('nslots', C.c_int32)]


class D1WaitMap(C.Structure):
    _fields_ = [('floor', C.c_void_p), ('dist', C.c_void_p), ('starts', C.c_void_p), ('player', C.c_int32)]


class D1LKind(C.Structure):
    _fields_ = [('speed', C.c_int32), ('damage', C.c_int32), ('tohit', C.c_int32), ('bypass', C.c_int32)]


class D1LConfig(C.Structure):
    """sim::Config (gpu-d1/src/sim.h:64-67), the learning task's config (include/d1learn.h)."""
    _fields_ = ([(k, C.c_int32) for k in ('count', 'player', 'hp', 'ac100', 'ev100', 'sh100', 'shield_limit',
                                           'regen', 'repair')] +
                [('gdr', C.c_int32 * 2), ('kinds', D1LKind * 6)])


class D1LTables(C.Structure):
    """learn::Tables with MULTI_MAP (learn_env_ring_multi.py:11-17 ctypes layout)."""
    _fields_ = [('floor', C.c_void_p), ('cells', C.c_void_p), ('index', C.c_void_p), ('distance', C.c_void_p),
                ('ncells', C.c_int32), ('map_ncells', C.c_void_p), ('distance_offsets', C.c_void_p),
                ('n_maps', C.c_int32), ('map_filter', C.c_int32), ('los', C.c_void_p)]


def learn_config(enemies=24):
    """The reference wrapper's packing [enemies, *header[:7], 1, *gdr, *kinds]
    (gpu-d1/branches/d1-stairs-v2/scripts/learn_env_ring_multi.py:93-97) from map 1057's
    fixture header and roster."""
    m = data.map1057()
    header, kinds = m['header'], m['kinds']
    values = [enemies, *(int(v) for v in header[:7]), 1, *gdr_table(int(header[2])),
              *(int(v) for v in kinds.reshape(-1))]
    c = D1LConfig()
    C.memmove(C.addressof(c), (C.c_int32 * 35)(*values), 140)
    return c


RNG_PCG, RNG_COUNTER = 0, 1
LEVEL_SHARED, LEVEL_GENERATED = 0, 1


def gdr_table(ac100):
    """floor((65536*(ac+j))^(1/4)) by integer search, as gpu-d1/src/bench.cu:121-127."""
    out = []
    for j in range(2):
        ac, g = ac100 // 100 + j, 0
        while (g + 1) ** 4 <= 65536 * ac:
            g += 1
        out.append(g)
    return out


def make_config(count=8, *, limit=2048, rng_mode=RNG_COUNTER, level_mode=LEVEL_GENERATED, roster_mode=1,
                hp_lo=5, hp_hi=30, awake_pct=0, wake_los=1, stairs=3, clear_on_kill_all=1,
                explore_milli=2, kill_milli=1000, clear_milli=3000, death_milli=1000, step_milli=-1,
                turn_cost=0.0):
    """Defaults are the BASELINE rules: generated levels, counter RNG, random roster
    HP U[5,30], LOS sleep/wake, three stairs, v1 rewards (gpu-d1/src/learn.cu:32-40,508)."""
    m = data.map1057()
    header, kinds = m['header'], m['kinds']
    c = D1Config()
    c.count = count
    c.hp, c.ac100, c.ev100, c.sh100, c.shield_limit, c.regen = (int(v) for v in header[1:7])
    c.repair = 1
    c.gdr[:] = gdr_table(c.ac100)
    for k in range(6):
        c.kinds[k] = D1Kind(*(int(v) for v in kinds[k]))
    for name, v in dict(limit=limit, rng_mode=rng_mode, level_mode=level_mode, roster_mode=roster_mode,
                        hp_lo=hp_lo, hp_hi=hp_hi, awake_pct=awake_pct, wake_los=wake_los, stairs=stairs,
                        clear_on_kill_all=clear_on_kill_all, explore_milli=explore_milli,
                        kill_milli=kill_milli, clear_milli=clear_milli, death_milli=death_milli,
                        step_milli=step_milli).items():
        setattr(c, name, int(v))
    c.turn_cost = float(turn_cost)
    return c


def baseline_config(count=8):
    """C1-C3: generated 80x70 levels, counter RNG, up to 8 monsters, HP U[5,30], kinds U{0..5}."""
    return make_config(count)


def stress_config():
    """C5: 40 monsters, HP U[40,60], half awake at spawn."""
    return make_config(40, hp_lo=40, hp_hi=60, awake_pct=50)


def reference_config(count=24, *, stairs=3, wake_los=1, clear_on_kill_all=0):
    """The d1-stairs-v2 task on map 1057 with the reference's PCG stream and roster
    (gpu-d1/branches/d1-stairs-v2/scripts/assets.py:5: KILL_MILLI=0, CLEAR_MILLI=1000,
    DEATH_MILLI=0, EXPLORE_MILLI=0, TURN_COST=1e-5, 2048-turn deadline)."""
    return make_config(count, rng_mode=RNG_PCG, level_mode=LEVEL_SHARED, roster_mode=0, awake_pct=0,
                       wake_los=wake_los, stairs=stairs, clear_on_kill_all=clear_on_kill_all,
                       explore_milli=0, kill_milli=0, clear_milli=1000, death_milli=0, step_milli=0,
                       turn_cost=1e-5, limit=2048)


def v1_config(count=8, sleep=True):
    """The v1 floor-clear task of gpu-d1/src/learn.cu on map 1057: kill-all clears, no
    stairs, 256 turns. sleep=True is its SLEEP_ON + EXPLORE_REWARD + MARK_WALLS build
    (monsters start asleep and wake within Chebyshev 6); sleep=False is the default build
    (gpu-d1/Makefile:14-16, no defines: every monster awake from the start, rewards -0.001
    per turn, +1 per kill, +3 on clear, -1 on death, no exploration reward)."""
    return make_config(count, rng_mode=RNG_PCG, level_mode=LEVEL_SHARED, roster_mode=0,
                       awake_pct=0 if sleep else 100, wake_los=0, stairs=0, clear_on_kill_all=1, limit=256,
                       explore_milli=2 if sleep else 0)


def shared_map_arrays():
    """Byte-per-cell floor and spawnable-cell masks of map 1057 (cells = floor
    reachable from the fixture player, gpu-d1/scripts/learn_env.py:20-22)."""
    m = data.map1057()
    floor = m['floor'].astype(np.uint8)
    cells = ((floor != 0) & (m['dist'] < 65535)).astype(np.uint8)
    return floor, cells


def check_level(floor, cells):
    """A shared level given as (floor, cells) masks -> two contiguous uint8 [5600] arrays
    of 0/1; raises ValueError on a wrong size, or on a spawnable cell that is not floor."""
    floor = np.ascontiguousarray(floor, np.uint8).reshape(-1)
    cells = np.ascontiguousarray(cells, np.uint8).reshape(-1)
    if floor.size != 5600 or cells.size != 5600:
        raise ValueError('a level is 80 x 70 = 5600 cells')
    floor, cells = (floor != 0).astype(np.uint8), (cells != 0).astype(np.uint8)
    if np.any(cells > floor):
        raise ValueError('spawnable cells must be floor cells')
    if not cells.any():
        raise ValueError('a level needs at least one spawnable cell')
    return floor, cells
