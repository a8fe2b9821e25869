#!/usr/bin/env python3
"""Derive the library's static data files from the reference's map-1057 fixtures.

Run once in a container that has the reference checkout; the outputs are small
binary files committed beside this script, so nothing at run time reads the
reference.

Inputs (reference data, not code):
  gpu-d1/fixtures/native-1057.rays  ray endpoints + per-cell blocker bitsets exported
                                    from native Crawl (format read by
                                    gpu-d1/scripts/compile_fixture.py:20-27)
  gpu-d1/fixtures/fixture.bin       map 1057: header, roster, floor, distance field,
                                    LOS bitsets, spawn lists (gpu-d1/src/bench.cu:107-136)

Outputs:
  los_rays.npz   ends  int8[428,2]   ray endpoint (x, y) in the +x/+y quadrant
                 masks uint64[428]   bit j set when inside-blocker cell j=(y*8+x) lies on the ray
                 slots uint64[11,64] per-target ray masks, slot-major, padded by repeating
                                     the target's first ray (so a wave can test every
                                     slot without a per-lane count); target j=(y*8+x)
                 nslots int8[64]     real ray count per target
  map1057.npz    floor uint8[5600], dist uint16[5600] (distance from the fixture player),
                 header int32[8], kinds int32[6,4], starts int16[128]
"""
import pathlib
import struct
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent


def main(reference=pathlib.Path('/root/reference/gpu-d1')):
    fixtures = reference / 'fixtures'
    lines = (fixtures / 'native-1057.rays').read_text().splitlines()
    nrays = int(lines[0])
    ends = np.array([tuple(map(int, l.split())) for l in lines[1:1 + nrays]], np.int8)
    inside = []
    for l in lines[1 + nrays:]:
        x, y, flag, bits = l.split()
        if int(flag):
            inside.append((int(x), int(y), int(bits[::-1], 2)))
    # The inside blockers of this export are exactly the 8x8 block x,y in [0,7],
    # listed y-major; the kernels index blocker j as (x=j%8, y=j/8).
    assert [(x, y) for x, y, _ in inside] == [(j % 8, j // 8) for j in range(64)]
    masks = np.zeros(nrays, np.uint64)
    for j, (_, _, bits) in enumerate(inside):
        for i in range(nrays):
            if bits >> i & 1:
                masks[i] |= np.uint64(1 << j)
    per = [[] for _ in range(64)]
    for i, (x, y) in enumerate(ends):
        if x < 8 and y < 8:
            per[y * 8 + x].append(int(masks[i]))
    per[0] = [0]                      # the origin is always visible
    nslots = max(len(v) for v in per)
    slots = np.zeros((nslots, 64), np.uint64)
    for j, v in enumerate(per):
        assert v, f'target {j} has no ray'
        for k in range(nslots):
            slots[k, j] = v[k] if k < len(v) else v[0]
    np.savez_compressed(HERE / 'los_rays.npz', ends=ends, masks=masks, slots=slots,
                        nslots=np.array([len(v) for v in per], np.int8))

    raw = (fixtures / 'fixture.bin').read_bytes()
    assert struct.unpack_from('<I', raw)[0] == 0x44314750
    header = np.frombuffer(raw, '<i4', 8, 4).copy()
    kinds = np.frombuffer(raw, '<i4', 24, 36).reshape(6, 4).copy()
    floor = np.frombuffer(raw, np.uint8, 5600, 132).copy()
    dist = np.frombuffer(raw, '<u2', 5600, 5732).copy()
    starts = np.frombuffer(raw, '<i2', 128, 5732 + 11200 + 224000).copy()
    np.savez_compressed(HERE / 'map1057.npz', floor=floor, dist=dist, header=header,
                        kinds=kinds, starts=starts)
    print('rays', nrays, 'slots', slots.shape, 'floor cells', int(floor.sum()))


if __name__ == '__main__':
    main(*map(pathlib.Path, sys.argv[1:]))
