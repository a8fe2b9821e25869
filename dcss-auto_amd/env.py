"""Batched D:1 environment on one GPU: the drop-in for the reference's ctypes `Env`
(gpu-d1/scripts/learn_env.py:56-117, gpu-d1/scripts/learn_env_ring_multi.py:45-119).

Same surface: ``Env(batch, ..., seed, device)``, ``reset(seed) -> obs``,
``step(actions, active=None) -> (obs, out)`` with ``out[:, 0]`` reward and
``out[:, 1]`` done, and the ``state/obs/out`` tensors as attributes. Calls run
asynchronously on PyTorch's current stream, as the reference's do
(gpu-d1/scripts/learn_env.py:83-85). Observations are uint8 [batch, 15, 15, 8];
``hash`` holds the per-env 32-bit state hash after every call (a parity digest the
reference does not have; ``Env(..., hash=False)`` skips it in step()).
"""
import ctypes as C

import numpy as np
import torch

from . import _lib, config as cfgmod, data


# The state row's 64-byte header (d1_env.hip `Hdr`), little-endian and packed.
HEADER = np.dtype([('rng_state', '<u8'), ('rng_inc', '<u8'), ('env_id', '<u4'), ('t', '<u4'), ('episode', '<i4'),
                   ('player', '<i2'), ('hp', '<i2'), ('regen', '<i2'), ('ncells', '<i2'), ('ticks', '<i4'),
                   ('killed', '<i4'), ('decisions', '<i4'), ('floor_seen', '<i4'), ('stairs', '<i2', 3),
                   ('blocks', '<i2'), ('first_stair_tick', '<i4')])
assert HEADER.itemsize == 64


def _bitmap_bytes(words):
    """[n, 840] bytes of 70 rows x 3 little-endian dwords (bit x of row y) -> [n, 5600] 0/1."""
    bits = np.unpackbits(words.reshape(len(words), 70, 12), axis=2, bitorder='little')
    return np.ascontiguousarray(bits[:, :, :80].reshape(len(words), 5600))


def decode_rows(raw, max_monsters):
    """State rows (uint8 [n, d1_state_bytes(max_monsters)], a host copy) -> one numpy record
    per world: the header scalars (rng_state is the PCG state, or the Philox key in counter
    mode), `view` [15, 15] (the player's field of view the row memoises, [dy+7][dx+7]), the
    monster fields pos/mhp/energy/awake/kind [max_monsters], and the `viewed`, `floor` and
    `cells` (spawnable) maps as [5600] bytes of 0/1. The rows of crowded layouts also carry a
    distance-field memo, which is a cache and is not decoded."""
    raw = np.ascontiguousarray(raw, np.uint8)
    n, m = len(raw), max_monsters
    dt = np.dtype(HEADER.descr + [('view', 'u1', (15, 15)), ('pos', '<i2', m), ('mhp', '<i2', m),
                                   ('energy', '<i2', m), ('awake', 'u1', m), ('kind', 'u1', m),
                                   ('viewed', 'u1', 5600), ('floor', 'u1', 5600), ('cells', 'u1', 5600)])
    out = np.zeros(n, dt)
    hdr = raw[:, :64].copy().view(HEADER).reshape(n)
    for name in HEADER.names:
        out[name] = hdr[name]
    quads = raw[:, 64:96].copy().view('<u8')                  # quadrants (+x,+y) (-x,+y) (-x,-y) (+x,-y)
    j = np.arange(64, dtype=np.uint64)
    tx, ty = (j % 8).astype(int), (j // 8).astype(int)
    for q, (sx, sy) in enumerate(((1, 1), (-1, 1), (-1, -1), (1, -1))):
        on = ((quads[:, q, None] >> j) & np.uint64(1)).astype(np.uint8)   # [n, 64]
        out['view'][:, sy * ty + 7, sx * tx + 7] |= on
    mon = raw[:, 96:96 + 8 * m].copy().reshape(n, m, 8)
    out['pos'] = mon[:, :, 0:2].copy().view('<i2')[..., 0]
    out['mhp'] = mon[:, :, 2:4].copy().view('<i2')[..., 0]
    out['energy'] = mon[:, :, 4:6].copy().view('<i2')[..., 0]
    out['awake'] = mon[:, :, 6]
    out['kind'] = mon[:, :, 7]
    o = 96 + 8 * m
    for name in ('viewed', 'floor', 'cells'):
        out[name] = _bitmap_bytes(raw[:, o:o + 840])
        o += 840
    return out


class Env:
    def __init__(self, batch=512, cfg=None, seed=0, device='cuda', max_monsters=None, hash=True, level=None):
        """`level` optionally replaces map 1057 as the shared level (level_mode shared): a
        (floor, cells) pair of 5600-byte 0/1 masks, row-major 80 x 70, where cells (the
        spawnable cells, a subset of the floor) is what player, monsters and stairs are
        placed on."""
        self.with_hash = hash
        self.device = torch.device('cuda:0' if device == 'cuda' else device)
        if self.device.type != 'cuda':
            raise ValueError('the HIP environment runs on a GPU device; the CPU restatement is test-only')
        self.lib = _lib.load()
        self.cfg = cfg if cfg is not None else cfgmod.baseline_config()
        self.batch = batch
        self.max_monsters = max_monsters or (8 if self.cfg.count <= 8 else 40 if self.cfg.count <= 40 else 64)
        if C.sizeof(cfgmod.D1Config) != self.lib.d1_config_bytes():
            raise RuntimeError('D1Config layout differs from the library')
        r = data.rays()
        self.ray_slots = torch.from_numpy(r['slots'].view(np.int64).copy()).to(self.device)
        floor, cells = cfgmod.shared_map_arrays() if level is None else cfgmod.check_level(*level)
        self.floor = torch.from_numpy(floor).to(self.device)
        self.cells = torch.from_numpy(cells).to(self.device)
        self.tables = cfgmod.D1Tables(self.floor.data_ptr(), self.cells.data_ptr(), self.ray_slots.data_ptr(),
                                      int(r['slots'].shape[0]))
        self.state = torch.zeros((batch, self.lib.d1_state_bytes(self.max_monsters)), dtype=torch.uint8,
                                 device=self.device)
        self.obs = torch.zeros((batch, 15, 15, 8), dtype=torch.uint8, device=self.device)
        self.out = torch.zeros((batch, 8), dtype=torch.float32, device=self.device)
        self.hash = torch.zeros(batch, dtype=torch.int32, device=self.device)
        self.reset(seed)

    def floors(self):
        """Each world's level floor as uint8 [batch, 5600] (1 = floor), unpacked from the
        state rows (the 840-byte floor bitmap after the header, view, monsters and
        viewed bitmap)."""
        off = 96 + 8 * self.max_monsters + 840
        return _bitmap_bytes(self.state[:, off:off + 840].cpu().numpy())

    def fields(self, worlds=None):
        """The worlds' state rows decoded on the host (decode_rows), all of them or the slice
        or index array `worlds`; the reference's tests read its rows the same way through a
        ctypes mirror of `State` (gpu-d1/scripts/test_learning.py:15-36)."""
        rows = self.state if worlds is None else self.state[worlds]
        return decode_rows(rows.cpu().numpy(), self.max_monsters)

    @property
    def stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def reset(self, seed):
        _lib.check(self.lib.d1_init(self.state.data_ptr(), self.batch, self.max_monsters, C.byref(self.cfg),
                                    C.byref(self.tables), seed, self.obs.data_ptr(), self.hash.data_ptr(),
                                    self.stream), 'd1_init')
        return self.obs

    def heuristic(self, v1_ids=False, out=None):
        """The v1 pursuit controller's action for every world (d1_heuristic; the reference's
        learn_env.py:114 heuristic(), gpu-d1/src/learn.cu:599-621), as int64 [batch]: the
        joint actions step() takes (a bump into a living monster is ATTACK d), or with
        `v1_ids` the v1 action ids (0-7 direction, 8 wait)."""
        if out is None:
            out = torch.empty(self.batch, dtype=torch.int64, device=self.device)
        elif not (out.device == self.device and out.dtype == torch.int64 and out.is_contiguous()
                  and out.shape == (self.batch,)):
            raise ValueError('out must be a contiguous int64 tensor of shape [batch] on the env device')
        _lib.check(self.lib.d1_heuristic(self.state.data_ptr(), self.batch, self.max_monsters, C.byref(self.cfg),
                                         0 if v1_ids else 1, out.data_ptr(), self.stream), 'd1_heuristic')
        return out

    def step_rows(self, lo, hi, actions):
        """Steps worlds lo..hi-1 only, with actions[lo:hi], writing their observation and
        out rows (the hash is not computed), on the current stream. Disjoint row ranges are
        independent, so they may be stepped on different streams."""
        if not (actions.device == self.device and actions.dtype == torch.int64 and actions.is_contiguous()
                and actions.shape == (self.batch,)):
            raise ValueError('actions must be a contiguous int64 tensor of shape [batch] on the env device')
        if not (0 <= lo < hi <= self.batch):
            raise ValueError(f'row range [{lo}, {hi}) outside [0, {self.batch})')
        rb = self.state.shape[1]
        _lib.check(self.lib.d1_step(self.state.data_ptr() + lo * rb, hi - lo, self.max_monsters, C.byref(self.cfg),
                                    C.byref(self.tables), actions.data_ptr() + lo * 8,
                                    self.obs.data_ptr() + lo * 1800, self.out.data_ptr() + lo * 4 * self.out.shape[1],
                                    None, None, self.stream), 'd1_step')
        return self.obs[lo:hi], self.out[lo:hi]

    def step(self, actions, active=None, obs=None):
        """`obs` optionally redirects this step's observation into another uint8
        [batch, 15, 15, 8]-shaped buffer (e.g. a rollout-buffer slice); self.obs then
        keeps the previous step's values."""
        if not (actions.device == self.device and actions.dtype == torch.int64 and actions.is_contiguous()
                and actions.shape == (self.batch,)):
            raise ValueError('actions must be a contiguous int64 tensor of shape [batch] on the env device')
        act = None
        if active is not None:
            if not (active.device == self.device and active.dtype == torch.bool and active.is_contiguous()
                    and active.shape == (self.batch,)):
                raise ValueError('active must be a contiguous bool tensor of shape [batch] on the env device')
            act = active.data_ptr()
        dst = self.obs
        if obs is not None:
            if not (obs.device == self.device and obs.dtype == torch.uint8 and obs.is_contiguous()
                    and obs.numel() == self.batch * 1800):
                raise ValueError('obs must be a contiguous uint8 buffer of batch*1800 bytes on the env device')
            dst = obs
        _lib.check(self.lib.d1_step(self.state.data_ptr(), self.batch, self.max_monsters, C.byref(self.cfg),
                                    C.byref(self.tables), actions.data_ptr(), dst.data_ptr(),
                                    self.out.data_ptr(), self.hash.data_ptr() if self.with_hash else None, act,
                                    self.stream), 'd1_step')
        return dst, self.out
