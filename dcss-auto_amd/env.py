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


class Env:
    def __init__(self, batch=512, cfg=None, seed=0, device='cuda', max_monsters=None, hash=True):
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
        floor, cells = cfgmod.shared_map_arrays()
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
        words = self.state[:, off:off + 840].cpu().numpy().view('<u4').reshape(self.batch, 70, 3)
        bits = np.unpackbits(words.view(np.uint8).reshape(self.batch, 70, 12), axis=2, bitorder='little')
        return np.ascontiguousarray(bits[:, :, :80].reshape(self.batch, 5600))

    @property
    def stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def reset(self, seed):
        _lib.check(self.lib.d1_init(self.state.data_ptr(), self.batch, self.max_monsters, C.byref(self.cfg),
                                    C.byref(self.tables), seed, self.obs.data_ptr(), self.hash.data_ptr(),
                                    self.stream), 'd1_init')
        return self.obs

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
