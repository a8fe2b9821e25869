#!/usr/bin/env python3
"""Write tests/golden/sim_ref.npz from the reference's own rule core.

Builds oracle/_ref/simref (the reference's gpu-d1/src/sim.h compiled from where
it lies, driven by oracle/ref/simref.cpp) and stores its outputs as data:
  mix_in/mix_out      splitmix64 finaliser
  rng_*               PCG32 op streams (op 0 next, 1 r(b), 2 avg(n), 3 round(n,d) with arg=n<<8|d)
  wait_meta/wait_trace monster-wait trajectories on map 1057 (count, scenario, fixture,
                      heap, world, seed, prewarm) -> per-step world digests
  config/kinds        the fixture Config the harness decoded
Run in a container that has /root/reference; the .npz is committed.
"""
import json
import pathlib
import subprocess
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]


def main(reference='/root/reference/gpu-d1'):
    subprocess.run(['make', '-s', '-C', str(ROOT / 'oracle'), 'ref', f'REF={reference}'], check=True)
    raw = subprocess.run([str(ROOT / 'oracle/_ref/simref'), f'{reference}/fixtures/fixture.bin'],
                         check=True, capture_output=True, text=True).stdout
    d = json.loads(raw)
    out = dict(
        mix_in=np.array([int(a) for a, _ in d['mix']], np.uint64),
        mix_out=np.array([int(b) for _, b in d['mix']], np.uint64),
        rng_seed=np.array([int(r['seed']) for r in d['rng']], np.uint64),
        rng_seq=np.array([r['seq'] for r in d['rng']], np.uint64),
        rng_ops=np.array([r['ops'] for r in d['rng']], np.int32),
        rng_args=np.array([r['args'] for r in d['rng']], np.int32),
        rng_results=np.array([r['results'] for r in d['rng']], np.int32),
        rng_final=np.array([int(r['final_state']) for r in d['rng']], np.uint64),
        wait_meta=np.array([[w[k] for k in ('count', 'scenario', 'fixture', 'heap', 'world', 'seed', 'prewarm')]
                            for w in d['wait']], np.int64),
        wait_trace=np.array([w['trace'] for w in d['wait']], np.int32),
        config=np.array(d['config'], np.int32),
        kinds=np.array(d['kinds'], np.int32),
    )
    np.savez_compressed(ROOT / 'tests/golden/sim_ref.npz', **out)
    print({k: v.shape for k, v in out.items()})


if __name__ == '__main__':
    main(*sys.argv[1:])
