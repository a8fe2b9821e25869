"""The reference's d1-stairs-v2 learning task on the HIP `learn_*` library.

`LearnEnv` keeps the constructor, buffers and `reset / step / heuristic` of
gpu-d1/branches/d1-stairs-v2/scripts/learn_env_ring_multi.py:61-120, so a trainer
written against that wrapper runs unchanged: obs float [B, 1015], mask float [B, 19],
out float [B, 45], int64 actions, optional bool `active`. `LearnMaps` builds the
library's map tables on the device from byte floor maps: cells (all floor cells in
row-major order, the corpus compiler's rule, gpu-d1/scripts/compile_corpus.py:37-40),
and the LOS table by the HIP LOS compiler (`d1_los_table`). There is no host path:
the library refuses `gpu=0` and this module needs a GPU device.
"""
import ctypes as C
import time

import numpy as np
import torch

from . import _lib, data
from .config import D1LTables, D1Tables, learn_config

N = 5600


class LearnMaps:
    """Device map tables for one or more 80x70 byte floor maps (nonzero = floor)."""

    def __init__(self, floors=None, device='cuda'):
        if floors is None:
            floors = data.map1057()['floor'][None]
        floors = np.ascontiguousarray(np.asarray(floors, np.uint8).reshape(-1, N))
        self.n_maps = len(floors)
        cells = np.full((self.n_maps, N), -1, np.int16)
        ncells = np.zeros(self.n_maps, np.int32)
        for m, f in enumerate(floors):
            c = np.flatnonzero(f).astype(np.int16)
            cells[m, :len(c)] = c
            ncells[m] = len(c)
        self.device = torch.device(device)
        self.floor = torch.from_numpy(floors).to(self.device)
        self.cells = torch.from_numpy(cells).to(self.device)
        self.ncells = torch.from_numpy(ncells).to(self.device)
        self.cell_counts = ncells
        self.los = torch.empty((self.n_maps, N, 10), dtype=torch.int32, device=self.device)
        slots = np.ascontiguousarray(data.rays()['slots'], np.uint64)
        self._slots = torch.from_numpy(slots.view(np.int64)).to(self.device)
        rays = D1Tables(None, None, self._slots.data_ptr(), slots.shape[0])
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _lib.check(_lib.load().d1_los_table(self.floor.data_ptr(), self.n_maps, C.byref(rays), self.los.data_ptr(),
                                            stream), 'd1_los_table')

    @classmethod
    def from_maps(cls, maps, device='cuda'):
        """Tables from read_maps() output (corpus map files): their floors, with the LOS
        table the map files carry, as the reference's EnvV2 uploads them
        (gpu-d1/scripts/learn_env_v2.py:91-104)."""
        self = cls(np.stack([m['floor'] for m in maps]), device)
        los = np.ascontiguousarray(np.stack([m['los'] for m in maps]), np.uint32)
        self.los.copy_(torch.from_numpy(los.view(np.int32)).to(self.device))
        return self

    def tables(self, map_filter=-1):
        """The library's Tables struct; index/distance are not read by this library."""
        if not -2 <= map_filter < self.n_maps:
            raise ValueError('map_filter is -2 (balanced first episodes), -1 (random) or a map index')
        return D1LTables(self.floor.data_ptr(), self.cells.data_ptr(), None, None, int(self.cell_counts[0]),
                         self.ncells.data_ptr(), None, self.n_maps, map_filter, self.los.data_ptr())


class LearnEnv:
    def __init__(self, batch=512, enemies=24, seed=0, device='cuda', limit=2048, maps=None, map_filter=-1,
                 clump=0):
        if enemies != 24 or limit < 1:
            raise ValueError('the d1-stairs-v2 task places exactly 24 enemies')
        self.device = torch.device('cuda:0' if device == 'cuda' else device)
        if self.device.type != 'cuda':
            raise RuntimeError('the learning task runs on the GPU only (no host path)')
        self.batch, self.enemies, self.limit = batch, enemies, limit
        self.lib = _lib.load_learn(clump)
        self.maps = maps if maps is not None else LearnMaps(device=self.device)
        self.tables = self.maps.tables(map_filter)
        self.config = learn_config(enemies)
        assert C.sizeof(self.config) == self.lib.learn_config_bytes()
        self.state = torch.zeros((batch, self.lib.learn_state_bytes()), dtype=torch.uint8, device=self.device)
        self.obs = torch.empty((batch, self.lib.learn_obs_size()), device=self.device)
        self.action_size = self.lib.learn_action_size()
        self.out_size = self.lib.learn_out_size()
        self.mask = torch.empty((batch, self.action_size), device=self.device)
        self.out = torch.zeros((batch, self.out_size), device=self.device)
        self.actions = torch.empty(batch, dtype=torch.int64, device=self.device)
        self.reset(seed)

    @property
    def stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def check(self, code):
        if code:
            raise RuntimeError(f'learning task call failed with error {code}')

    def reset(self, seed):
        self.check(self.lib.learn_init(self.state.data_ptr(), self.batch, C.byref(self.config),
                                       C.byref(self.tables), seed, self.obs.data_ptr(), self.mask.data_ptr(),
                                       self.stream, 1))
        return self.obs

    def step(self, actions, active=None):
        assert actions.device == self.device and actions.dtype == torch.int64 and actions.is_contiguous()
        if active is not None:
            assert active.device == self.device and active.dtype == torch.bool and active.is_contiguous()
            assert active.shape == (self.batch,)
            self.check(self.lib.learn_step_active(self.state.data_ptr(), self.batch, C.byref(self.config),
                                                  C.byref(self.tables), actions.data_ptr(), self.limit,
                                                  self.obs.data_ptr(), self.mask.data_ptr(), self.out.data_ptr(),
                                                  active.data_ptr(), self.stream, 1))
            return self.obs, self.out
        self.check(self.lib.learn_step(self.state.data_ptr(), self.batch, C.byref(self.config),
                                       C.byref(self.tables), actions.data_ptr(), self.limit, self.obs.data_ptr(),
                                       self.mask.data_ptr(), self.out.data_ptr(), self.stream, 1))
        return self.obs, self.out

    def heuristic(self):
        self.check(self.lib.learn_heuristic(self.state.data_ptr(), self.batch, C.byref(self.config),
                                            C.byref(self.tables), self.actions.data_ptr(), self.stream, 1))
        return self.actions

    def errors(self):
        """Envs whose last reset found no clump anchor or stair cell (the reference asserts)."""
        return self.state[:, ROW_DTYPE.fields['error'][1]].nonzero().flatten()


# Row layout (d1_learn.hip): header, 24 enemies, viewed and floor bitmaps, frontier list.
ROW_DTYPE = np.dtype([
    ('rng_state', '<u8'), ('rng_inc', '<u8'), ('encountered', '<u8'),
    ('ticks', '<i4'), ('killed', '<i4'), ('decisions', '<i4'), ('floor_seen', '<i4'), ('episode', '<i4'),
    ('first_stair_tick', '<i4'), ('player', '<i2'), ('hp', '<i2'), ('regen', '<i2'), ('blocks', '<i2'),
    ('map_id', '<i2'), ('next_slot', '<i2'), ('frontier_count', '<i2'), ('stairs', '<i2', 3),
    ('clumped', 'u1'), ('error', 'u1'), ('pad', 'u1', 10),
    ('mon', [('pos', '<i2'), ('hp', '<i2'), ('energy', '<i2'), ('awake', 'u1'), ('slot', 'i1')], 24),
    ('viewed', '<u4', 210), ('floor', '<u4', 210), ('frontier', '<u2', N)])


def decode_rows(state):
    """Structured view of learn state rows (a [B, learn_state_bytes] uint8 array)."""
    a = np.ascontiguousarray(np.asarray(state, np.uint8))
    return np.frombuffer(a.tobytes(), dtype=np.dtype({'names': ROW_DTYPE.names,
                                                      'formats': [ROW_DTYPE.fields[n][0] for n in ROW_DTYPE.names],
                                                      'offsets': [ROW_DTYPE.fields[n][1] for n in ROW_DTYPE.names],
                                                      'itemsize': a.shape[1]}))


def bitmap_cells(words):
    """uint32 [210] rows-of-3-dwords bitmap -> bool [5600]."""
    w = np.asarray(words, np.uint32).reshape(70, 3)
    bits = ((w[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(70, 96)[:, :80]
    return bits.reshape(-1).astype(bool)


class MaskedPolicy(torch.nn.Module):
    """The policy shape of the reference's evaluation and pipeline benchmarks
    (gpu-d1/scripts/benchmark_pipeline.py:9-16): obs -> 128 tanh -> 128 tanh -> action
    logits with the invalid actions masked to -1e9, and a value."""

    def __init__(self, obs=1015, actions=19, width=128, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.body = torch.nn.Sequential(torch.nn.Linear(obs, width), torch.nn.Tanh(), torch.nn.Linear(width, width),
                                        torch.nn.Tanh())
        self.actor, self.critic = torch.nn.Linear(width, actions), torch.nn.Linear(width, 1)
        with torch.no_grad():
            for layer in (self.body[0], self.body[2], self.actor, self.critic):
                layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) / layer.in_features ** 0.5)
                layer.bias.zero_()

    def forward(self, obs, mask):
        h = self.body(obs)
        return self.actor(h).masked_fill(mask == 0, -1e9), self.critic(h).squeeze(-1)


@torch.no_grad()
def evaluate_panel(env, policy, decisions=1024, seed=900000, active=True, greedy=False):
    """The reference's fixed-panel evaluation (gpu-d1/scripts/benchmark_evaluation.py,
    gpu-d1/scripts/run_ring_ablations.py:231-267): reset the panel to `seed`, sample (or
    take the most likely) masked action of `policy` — or the task's heuristic controller
    when policy == 'heuristic' — for `decisions` steps with torch's RNG seeded to `seed`, freezing finished worlds through `active` when asked, and keep each world's
    first terminal out row. Returns the wall time, the outcome rates and the per-map
    rates (world i plays map i % n_maps under map_filter -2)."""
    env.reset(seed)
    n = env.batch
    live = torch.ones(n, dtype=torch.bool, device=env.device)
    terminal = torch.zeros_like(env.out)
    returns = torch.zeros(n, device=env.device)
    with torch.random.fork_rng(devices=[env.device]):
        torch.manual_seed(seed)
        torch.cuda.synchronize(env.device)
        start = time.perf_counter()
        for _ in range(decisions):
            if policy == 'heuristic':   # the task's own controller (learn_heuristic)
                action = env.heuristic()
            else:
                logits, _ = policy(env.obs, env.mask)
                action = logits.argmax(-1) if greedy else torch.distributions.Categorical(logits=logits).sample()
            _, out = env.step(action, active=live if active else None)
            returns += live * out[:, 0]
            ended = live & (out[:, 1] > 0)
            terminal[ended] = out[ended]
            live &= ~ended
        torch.cuda.synchronize(env.device)
        seconds = time.perf_counter() - start
    t, r, unfinished = terminal.cpu(), returns.cpu(), int(live.sum())

    def rates(tt, rr):
        return dict(clear_rate=tt[:, 2].mean().item(), death_rate=tt[:, 6].mean().item(),
                    kills=tt[:, 3].mean().item(), shaped_return=rr.mean().item())
    k = env.maps.n_maps
    return dict(seconds=seconds, unfinished=unfinished, **rates(t, r),
                maps=[rates(t[i::k], r[i::k]) for i in range(k)])
