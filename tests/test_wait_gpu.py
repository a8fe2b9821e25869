"""The GPU monster-wait kernel against golden traces produced by the reference's own
gpu-d1/src/sim.h (tests/golden/sim_ref.npz): 72 runs (1-64 monsters; contact,
approach and mixed spawns; scan and heap scheduling) x 257 waits, digest per wait."""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_wait_kernel_matches_reference_traces(golden):
    wait = importlib.import_module('dcss-auto_amd.wait')
    g = np.load(golden / 'sim_ref.npz')
    names = {0: 'contact', 1: 'approach', 2: 'mixed'}
    runs = {}
    for meta, want in zip(g['wait_meta'], g['wait_trace']):
        count, scenario, fixture, heap, world, seed, prewarm = (int(v) for v in meta)
        key = (count, scenario, seed)
        if key not in runs:
            print(f'[wait] count={count} scenario={names[scenario]}', flush=True)
            w = wait.WaitWorlds(3, count, names[scenario], seed=seed)
            runs[key] = w.run(g['wait_trace'].shape[1], trace=True).cpu().numpy()
        np.testing.assert_array_equal(runs[key][world], want,
                                      err_msg=f'count={count} scenario={scenario} heap={heap} world={world}')


def test_wait_chunking_is_invisible():
    """4 calls of 16 waits == 1 call of 64 (state fully round-trips through HBM)."""
    wait = importlib.import_module('dcss-auto_amd.wait')
    a, b = wait.WaitWorlds(128, 8, 'mixed', seed=7), wait.WaitWorlds(128, 8, 'mixed', seed=7)
    ta = a.run(64, trace=True)
    tb = torch.cat([b.run(16, trace=True) for _ in range(4)], 1)
    assert torch.equal(ta, tb) and torch.equal(a.worlds, b.worlds)
