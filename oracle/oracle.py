"""TEST INFRASTRUCTURE ONLY — ctypes wrapper of the CPU restatement (libd1oracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this.
"""
import ctypes as C
import importlib
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
pkg = importlib.import_module('dcss-auto_amd')
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = HERE / 'libd1oracle.so'
        if not path.exists():
            raise RuntimeError(f'{path} is not built; run __graft_entry__.build()')
        L = C.CDLL(str(path))
        p, i = C.c_void_p, C.c_int
        L.o_mix.restype = C.c_uint64
        L.o_mix.argtypes = [C.c_uint64]
        L.o_philox.argtypes = [p, p, p]
        L.o_set_rays.argtypes = [i, p, p]
        L.o_los_bitset.argtypes = [p, i, p]
        L.o_los.argtypes = [p, i, i, i]
        L.o_level_generate.argtypes = [C.c_uint64, C.c_uint32, p]
        L.o_init.argtypes = [p, i, p, p, p, C.c_uint64, p, p, i]
        L.o_step.argtypes = [p, i, p, p, p, p, p, p, i]
        L.o_obs.argtypes = [p, p, p]
        L.o_hash.restype = C.c_uint32
        L.o_hash.argtypes = [p, p]
        L.o_heuristic.argtypes = [p, p]
        L.o_rng_ops.argtypes = [i, C.c_uint64, C.c_uint64, i, p, p, p, p]
        L.o_wait_run.argtypes = [i, i, i, i, C.c_uint64, C.c_uint32, p, p, p, p, p, C.c_int32, p]
        r = pkg.data.rays()
        ends = np.ascontiguousarray(r['ends'], np.int8)
        masks = np.ascontiguousarray(r['masks'], np.uint64)
        L.o_set_rays(len(masks), ends.ctypes.data, masks.ctypes.data)
        _LIB = L
    return _LIB


def ptr(a):
    return None if a is None else a.ctypes.data


class OracleEnv:
    """Batch of worlds stepped by the CPU restatement; numpy buffers mirror the GPU Env."""

    def __init__(self, batch, cfg, seed=0, threads=1, level=None):
        self.L, self.batch, self.cfg, self.threads = lib(), batch, cfg, threads
        self.state = np.zeros((batch, self.L.o_state_bytes()), np.uint8)
        self.obs = np.zeros((batch, 15, 15, 8), np.uint8)
        self.out = np.zeros((batch, 8), np.float32)
        self.hash = np.zeros(batch, np.uint32)
        self.floor, self.cells = pkg.shared_map_arrays() if level is None else pkg.config.check_level(*level)
        self.reset(seed)

    def reset(self, seed):
        self.L.o_init(ptr(self.state), self.batch, C.byref(self.cfg), ptr(self.floor), ptr(self.cells),
                      seed, ptr(self.obs), ptr(self.hash), self.threads)
        return self.obs

    def step(self, actions, active=None):
        a = np.ascontiguousarray(actions, np.int64)
        act = None if active is None else np.ascontiguousarray(active, np.uint8)
        self.L.o_step(ptr(self.state), self.batch, C.byref(self.cfg), ptr(a), ptr(self.obs), ptr(self.out),
                      ptr(self.hash), ptr(act), self.threads)
        return self.obs, self.out

    def heuristic(self):
        n = self.state.shape[1]
        return np.array([self.L.o_heuristic(self.state[i:].ctypes.data, C.byref(self.cfg)) for i in range(self.batch)],
                        np.int64) if n else None

    def heuristic_v1(self):
        """The v1 pursuit controller (o_heuristic_v1): v1 actions 0-8, one per world."""
        self.L.o_heuristic_v1.argtypes = [C.c_void_p, C.c_void_p]
        return np.array([self.L.o_heuristic_v1(self.state[i:].ctypes.data, C.byref(self.cfg))
                         for i in range(self.batch)], np.int64)

    def fields(self, worlds=None):
        """Structured copy of the worlds (OState, oracle/d1_oracle.h): all, or a slice."""
        rows = self.state if worlds is None else self.state[worlds]
        return np.ascontiguousarray(rows).reshape(-1).view(ostate_dtype()).copy()


OSTATE_FIELDS = [('rng', 'u1', 48), ('env_id', '<u4'), ('t', '<u4'), ('episode', '<i4'), ('player', '<i4'),
                 ('hp', '<i4'), ('regen', '<i4'), ('blocks', '<i4'), ('ticks', '<i4'), ('killed', '<i4'),
                 ('decisions', '<i4'), ('floor_seen', '<i4'), ('first_stair_tick', '<i4'), ('stairs', '<i4', 3),
                 ('ncells', '<i4'), ('vis_origin', '<i4'), ('vis', '<u4', 10), ('pos', '<i2', 64),
                 ('mhp', '<i2', 64), ('energy', '<i2', 64), ('awake', 'u1', 64), ('kind', 'u1', 64),
                 ('occ', '<i2', 5600), ('viewed', 'u1', 5600), ('floor', 'u1', 5600), ('cells', '<i2', 5600),
                 ('rng_state', '<u8'), ('rng_inc', '<u8'), ('rng_mode', '<i4'), ('rng_k', '<u4'), ('rng_t', '<u4')]


def ostate_dtype():
    """OState as a numpy record, offsets read from the library (o_field_offset)."""
    L = lib()
    L.o_field_offset.argtypes = [C.c_int]
    off = [L.o_field_offset(k) for k in range(len(OSTATE_FIELDS) + 1)]
    formats = [(f[1], f[2]) if len(f) == 3 else f[1] for f in OSTATE_FIELDS]
    return np.dtype({'names': [f[0] for f in OSTATE_FIELDS], 'formats': formats, 'offsets': off[:-1],
                     'itemsize': off[-1]})


class OracleWorld:
    """One env world of the CPU restatement built by hand, for the restated reference
    fixtures: `f` is a writable record view of its OState."""

    def __init__(self, floor, cells=None):
        L = self.L = lib()
        L.o_world_map.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        L.o_reset.argtypes = [C.c_void_p, C.c_void_p]
        L.o_reveal.argtypes = [C.c_void_p]
        L.o_transition.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
        L.o_pcg_seed.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64]
        dt = ostate_dtype()
        self.buf = np.zeros(dt.itemsize, np.uint8)
        self.f = self.buf.view(dt)[0]
        floor = np.ascontiguousarray(floor, np.uint8)
        cells = floor if cells is None else np.ascontiguousarray(cells, np.uint8)
        L.o_world_map(self.ptr, floor.ctypes.data, cells.ctypes.data)

    @property
    def ptr(self):
        return self.buf.ctypes.data

    def seed_pcg(self, seed, seq):
        """The reference's RNG::seed(seed, seq) (gpu-d1/src/sim.h:29-35), on the world's stream."""
        self.L.o_pcg_seed(self.ptr, seed, seq)

    def reset(self, cfg):
        self.L.o_reset(self.ptr, C.byref(cfg))

    def reveal(self):
        return self.L.o_reveal(self.ptr)

    def transition(self, cfg, action):
        out = np.zeros(8, np.float32)
        self.L.o_transition(self.ptr, C.byref(cfg), action, out.ctypes.data)
        return out

    def put(self, i, p, hp, awake, kind=0):
        """Monster i on cell p (the reference's `put`, semantic_tests.cu:8)."""
        f = self.f
        f['pos'][i], f['mhp'][i], f['awake'][i], f['kind'][i] = p, hp, int(awake), kind
        f['occ'][p] = i

    def obs(self, cfg):
        o = np.zeros((15, 15, 8), np.uint8)
        self.L.o_obs(self.ptr, C.byref(cfg), o.ctypes.data)
        return o

    def copy(self):
        w = OracleWorld.__new__(OracleWorld)
        w.L, w.buf = self.L, self.buf.copy()
        w.f = w.buf.view(self.f.dtype)[0]
        return w

    def state_bytes(self):
        """The world's bytes without the view memo (vis_origin, vis), which is not state."""
        b = self.buf.copy()
        dt = self.f.dtype
        for name in ('vis_origin', 'vis'):
            off = dt.fields[name][1]
            b[off:off + dt.fields[name][0].itemsize] = 0
        return b


def level(seed, env):
    f = np.zeros(5600, np.uint8)
    lib().o_level_generate(seed, env, f.ctypes.data)
    return f


def los_bitset(floor, origin):
    out = np.zeros(10, np.uint32)
    lib().o_los_bitset(np.ascontiguousarray(floor, np.uint8).ctypes.data, origin, out.ctypes.data)
    return out


def philox(ctr, key):
    c = np.array(ctr, np.uint32)
    k = np.array(key, np.uint32)
    o = np.zeros(4, np.uint32)
    lib().o_philox(c.ctypes.data, k.ctypes.data, o.ctypes.data)
    return o


# ---------------------------------------------------------------- learning task (learn_oracle.c)
_LEARN_READY = False


def learn_lib():
    global _LEARN_READY
    L = lib()
    if not _LEARN_READY:
        p, i = C.c_void_p, C.c_int
        L.lo_state_bytes.argtypes = []
        L.lo_field_offset.argtypes = [i]
        L.lo_init.argtypes = [p, i, p, p, C.c_uint64, p, p, i, i]
        L.lo_step.argtypes = [p, i, p, p, p, i, p, p, p, p, i, i]
        L.lo_heuristic.argtypes = [p, i, p, p, p, i]
        L.lo_reset.argtypes = [p, p, p, i]
        L.lo_reveal.argtypes = [p, p]
        L.lo_refresh_frontier.argtypes = [p, p, i]
        L.lo_observe.argtypes = [p, p, p, p, p]
        L.lo_known_distances.argtypes = [p, p, p, i]
        L.lo_route_first_step.argtypes = [i, i, p]
        L.lo_nearest_stair.argtypes = [p, p]
        L.lo_in_view.argtypes = [p, p, i]
        L.lo_transition.argtypes = [p, p, p, i, i, p, i]
        L.lo_heuristic_one.argtypes = [p, p, p]
        L.lo_distance_table.argtypes = [p, p, i, p]
        L.lo_los_table.argtypes = [p, p]
        _LEARN_READY = True
    return L


class LearnTablesHost:
    """Host tables as the reference's wrappers build them: byte floor, row-major floor
    cells padded with -1, cell index, all-pairs floor BFS rows, LOS bitsets
    (gpu-d1/scripts/compile_corpus.py:18-93; learn_env_ring_multi.py:68-86)."""

    def __init__(self, floors, los=None):
        L = learn_lib()
        floors = np.ascontiguousarray(np.asarray(floors, np.uint8).reshape(-1, 5600))
        M = len(floors)
        self.floor = floors.reshape(-1).copy()
        self.cells = np.full(M * 5600, -1, np.int16)
        self.index = np.full(M * 5600, -1, np.int16)
        self.ncells = np.zeros(M, np.int32)
        rows = []
        for m, f in enumerate(floors):
            c = np.flatnonzero(f).astype(np.int16)
            self.cells[m * 5600:m * 5600 + len(c)] = c
            self.index[m * 5600 + c] = np.arange(len(c), dtype=np.int16)
            self.ncells[m] = len(c)
            d = np.empty((len(c), 5600), np.uint16)
            L.lo_distance_table(f.ctypes.data, c.ctypes.data, len(c), d.ctypes.data)
            rows.append(d)
        self.distance = np.ascontiguousarray(np.concatenate(rows))
        self.offsets = np.concatenate(([0], np.cumsum(self.ncells[:-1]))).astype(np.int32)
        if los is None:
            los = np.zeros((M, 5600, 10), np.uint32)
            for m, f in enumerate(floors):
                L.lo_los_table(np.ascontiguousarray(f).ctypes.data, los[m].ctypes.data)
        self.los = np.ascontiguousarray(los, np.uint32)
        self.n_maps = M

    def tables(self, map_filter=-1):
        return pkg.config.D1LTables(self.floor.ctypes.data, self.cells.ctypes.data, self.index.ctypes.data,
                                    self.distance.ctypes.data, int(self.ncells[0]), self.ncells.ctypes.data,
                                    self.offsets.ctypes.data, self.n_maps, map_filter, self.los.ctypes.data)


def lstate_dtype():
    L = learn_lib()
    off = [L.lo_field_offset(k) for k in range(15)]
    names = ['rng', 'scalars', 'stairs', 'pos', 'energy', 'mhp', 'awake', 'enemy_slot', 'encountered', 'occ', 'seen',
             'viewed', 'frontier_cells', 'frontier_slot']
    formats = [('u1', 48), ('<i4', 15), ('<i4', 3), ('<i2', 40), ('<i2', 40), ('<i2', 40), ('<i2', 40), ('<i2', 40),
               ('u1', 40), ('<i2', 5600), ('u1', 5600), ('u1', 5600), ('<i2', 5600), ('<i2', 5600)]
    return np.dtype({'names': names, 'formats': formats, 'offsets': off[:14], 'itemsize': off[14]})


SCALARS = ('map_id', 'player', 'hp', 'regen', 'blocks', 'ticks', 'killed', 'decisions', 'episode', 'next_slot',
           'floor_seen', 'first_stair_tick', 'placement_clumped', 'frontier_count', 'error')


class OracleLearn:
    """Batch of d1-stairs-v2 worlds stepped by the CPU restatement; numpy buffers mirror
    dcss-auto_amd.learn.LearnEnv."""

    def __init__(self, batch, maps, seed=0, clump=0, map_filter=-1, limit=2048, threads=1):
        self.L, self.batch, self.maps, self.clump = learn_lib(), batch, maps, clump
        self.limit, self.threads = limit, threads
        self.tab = maps.tables(map_filter)
        self.cfg = pkg.config.learn_config()
        self.dtype = lstate_dtype()
        self.state = np.zeros(batch * self.dtype.itemsize, np.uint8)
        self.obs = np.zeros((batch, 1015), np.float32)
        self.mask = np.zeros((batch, 19), np.float32)
        self.out = np.zeros((batch, 45), np.float32)
        self.reset(seed)

    def reset(self, seed):
        return self.L.lo_init(ptr(self.state), self.batch, C.byref(self.cfg), C.byref(self.tab), seed, ptr(self.obs),
                              ptr(self.mask), self.clump, self.threads)

    def step(self, actions, active=None):
        a = np.ascontiguousarray(actions, np.int64)
        act = None if active is None else np.ascontiguousarray(active, np.uint8)
        return self.L.lo_step(ptr(self.state), self.batch, C.byref(self.cfg), C.byref(self.tab), ptr(a), self.limit,
                              ptr(self.obs), ptr(self.mask), ptr(self.out), ptr(act), self.clump, self.threads)

    def heuristic(self):
        a = np.zeros(self.batch, np.int64)
        self.L.lo_heuristic(ptr(self.state), self.batch, C.byref(self.cfg), C.byref(self.tab), ptr(a), self.threads)
        return a

    def fields(self):
        """Writable structured view of the worlds (LState, oracle/d1_oracle.h)."""
        return self.state.view(self.dtype)

    def scalar(self, name):
        return self.fields()['scalars'][:, SCALARS.index(name)]

    def world(self, i):
        """Pointer to world i (for the single-world hooks)."""
        return self.state.ctypes.data + i * self.dtype.itemsize
