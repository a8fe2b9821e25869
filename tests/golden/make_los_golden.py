#!/usr/bin/env python3
"""Write tests/golden/map1057_los.npz: the reference's LOS bitsets for every origin of
map 1057 (fixture.bin, 5600 x 10 uint32, bit (dy+8)*17+dx+8; layout
gpu-d1/src/bench.cu:131), checked by its author against native Crawl for all
1,618,400 pairs (gpu-d1/RESULTS.md:80). Data only; committed."""
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]


def main(reference='/root/reference/gpu-d1'):
    raw = (pathlib.Path(reference) / 'fixtures/fixture.bin').read_bytes()
    los = np.frombuffer(raw, '<u4', 56000, 132 + 5600 + 11200).reshape(5600, 10)
    np.savez_compressed(ROOT / 'tests/golden/map1057_los.npz', los=los)


if __name__ == '__main__':
    main(*sys.argv[1:])
