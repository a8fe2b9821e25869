"""The reference's monster-wait benchmark workload on the GPU (gpu-d1/src/bench.cu,
gpu-d1/src/sim.h:93-122,276-295): map 1057, a stationary player, `count` awake monsters
from the fixture spawn lists, one wave per world (libd1hip `d1_wait_*`)."""
import ctypes as C

import numpy as np
import torch

from . import _lib, config, data

SCENARIOS = {'contact': 0, 'approach': 1, 'mixed': 2}


class WaitWorlds:
    def __init__(self, n, count=8, scenario='mixed', seed=42, device='cuda'):
        self.lib = _lib.load()
        self.device = torch.device('cuda:0' if device == 'cuda' else device)
        self.n, self.count = n, count
        m = data.map1057()
        self.cfg = config.reference_config()
        self.floor = torch.from_numpy(m['floor'].astype(np.uint8)).to(self.device)
        self.dist = torch.from_numpy(m['dist'].view(np.int16).copy()).to(self.device)
        self.starts = torch.from_numpy(m['starts'].copy()).to(self.device)
        self.map = config.D1WaitMap(self.floor.data_ptr(), self.dist.data_ptr(), self.starts.data_ptr(),
                                    int(m['header'][0]))
        self.worlds = torch.zeros((n, self.lib.d1_wait_bytes()), dtype=torch.uint8, device=self.device)
        _lib.check(self.lib.d1_wait_init(self.worlds.data_ptr(), n, count, C.byref(self.cfg), C.byref(self.map), seed,
                                         SCENARIOS[scenario], self.stream), 'd1_wait_init')

    @property
    def stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def run(self, steps, trace=False):
        out = torch.empty((self.n, steps), dtype=torch.int32, device=self.device) if trace else None
        _lib.check(self.lib.d1_wait_run(self.worlds.data_ptr(), self.n, self.count, C.byref(self.cfg),
                                        C.byref(self.map), steps, None if out is None else out.data_ptr(),
                                        self.stream), 'd1_wait_run')
        return out
