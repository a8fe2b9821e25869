"""The reference's on-disk map formats and the map compiler.

``map-SEED.bin`` — one compiled map of a corpus (written by
gpu-d1/scripts/compile_corpus.py:88-95, read by gpu-d1/scripts/learn_env_v2.py:26-60):

    u32 magic 0x44325650, u32 seed, u32 ncells; i32 hp, ac100, ev100, sh100
    u8  floor[5600]                      1 = floor ('.' in the native export)
    i16 cells[5600]                      the floor cells in row-major order, then -1
    i16 index[5600]                      position of a cell in `cells`, -1 off floor
    u16 distance[ncells][5600]           BFS distance from each floor cell, 65535 unreached
    u32 los[5600][10]                    17x17 bitset of cells seen from each origin

``fixture.bin`` — the wait benchmark's map (written by gpu-d1/scripts/compile_fixture.py:73-80,
read by gpu-d1/src/bench.cu:107-136):

    u32 magic 0x44314750; i32 player, hp, ac100, ev100, sh100, shield_limit, regen, 0
    i32 kinds[6][4]                      speed, damage, to_hit, bypass
    u8  floor[5600]; u16 dist[5600]      distance from the player, 65535 unreached
    u32 los[5600][10]; i16 spawns[128]   64 contact + 64 approach cells

The compiler builds both from a floor map and its stats: the distance rows come from
``d1_distance_rows`` and the LOS bitsets from ``d1_los_table`` (HIP kernels); the cell
lists, the fixture's player and its spawn lists follow the reference's rules.
"""
import ctypes as C
import hashlib
import pathlib
import struct

import numpy as np
import torch

from . import _lib, data
from .config import D1Tables

N, W, H = 5600, 80, 70
MAP_MAGIC = 0x44325650
FIXTURE_MAGIC = 0x44314750


def _raw(src):
    return bytes(src) if isinstance(src, (bytes, bytearray, memoryview)) else pathlib.Path(src).read_bytes()


# ---------------------------------------------------------------- map-SEED.bin
def read_map(src):
    """Parse a map file (path or bytes) into a dict of arrays and stats."""
    raw = _raw(src)
    magic, seed, ncells = struct.unpack_from('<3I', raw)
    if magic != MAP_MAGIC or ncells > N:
        raise ValueError('not a corpus map file (bad magic or cell count)')
    size = 28 + N + 2 * N + 2 * N + ncells * 2 * N + N * 40
    if len(raw) != size:
        raise ValueError(f'map file has {len(raw)} bytes, the header implies {size}')
    hp, ac100, ev100, sh100 = struct.unpack_from('<4i', raw, 12)
    off = 28
    floor = np.frombuffer(raw, np.uint8, N, off).copy(); off += N
    cells = np.frombuffer(raw, '<i2', N, off).astype(np.int16); off += 2 * N
    index = np.frombuffer(raw, '<i2', N, off).astype(np.int16); off += 2 * N
    distance = np.frombuffer(raw, '<u2', ncells * N, off).astype(np.uint16).reshape(ncells, N); off += ncells * 2 * N
    los = np.frombuffer(raw, '<u4', N * 10, off).astype(np.uint32).reshape(N, 10)
    return dict(seed=seed, ncells=ncells, hp=hp, ac100=ac100, ev100=ev100, sh100=sh100, floor=floor, cells=cells,
                index=index, distance=distance, los=los)


def write_map(m):
    """The bytes of a map file (the inverse of read_map)."""
    out = bytearray(struct.pack('<3I', MAP_MAGIC, m['seed'], m['ncells']))
    out += struct.pack('<4i', m['hp'], m['ac100'], m['ev100'], m['sh100'])
    out += np.asarray(m['floor'], np.uint8).tobytes()
    out += np.asarray(m['cells'], '<i2').tobytes()
    out += np.asarray(m['index'], '<i2').tobytes()
    out += np.asarray(m['distance'], '<u2').tobytes()
    out += np.asarray(m['los'], '<u4').tobytes()
    return bytes(out)


def read_maps(root, map_limit=None):
    """All map-*.bin of a corpus directory (or its `all/` subdirectory), by seed; with
    map_limit, the nested seed-independent subset of gpu-d1/scripts/learn_env_v2.py:26-47
    (the first map, then the others ordered by sha256 of their file name)."""
    def key(path):
        try:
            return int(path.stem.split('-', 1)[1])
        except (IndexError, ValueError):
            return path.name
    root = pathlib.Path(root)
    paths = sorted(root.glob('map-*.bin'), key=key)
    if not paths and (root / 'all').is_dir():
        paths = sorted((root / 'all').glob('map-*.bin'), key=key)
    if map_limit is not None:
        if not 1 <= map_limit <= len(paths):
            raise ValueError(f'map_limit must be 1..{len(paths)}')
        paths = paths[:1] + sorted(paths[1:], key=lambda p: hashlib.sha256(p.name.encode()).digest())
        paths = sorted(paths[:map_limit], key=key)
    if not paths:
        raise ValueError('the corpus holds no map-*.bin file')
    maps = []
    for path in paths:
        m = read_map(path)
        m['path'] = path.name
        maps.append(m)
    return maps


# ---------------------------------------------------------------- fixture.bin
def read_fixture(src):
    raw = _raw(src)
    if len(raw) != 4 + 32 + 96 + N + 2 * N + 40 * N + 256 or struct.unpack_from('<I', raw)[0] != FIXTURE_MAGIC:
        raise ValueError('not a fixture file (bad magic or size)')
    head = struct.unpack_from('<8i', raw, 4)
    off = 36
    kinds = np.frombuffer(raw, '<i4', 24, off).astype(np.int32).reshape(6, 4); off += 96
    floor = np.frombuffer(raw, np.uint8, N, off).copy(); off += N
    dist = np.frombuffer(raw, '<u2', N, off).astype(np.uint16); off += 2 * N
    los = np.frombuffer(raw, '<u4', 10 * N, off).astype(np.uint32).reshape(N, 10); off += 40 * N
    spawns = np.frombuffer(raw, '<i2', 128, off).astype(np.int16)
    return dict(player=head[0], hp=head[1], ac100=head[2], ev100=head[3], sh100=head[4], shield_limit=head[5],
                regen=head[6], kinds=kinds, floor=floor, dist=dist, los=los, spawns=spawns)


def write_fixture(f):
    out = bytearray(struct.pack('<I8i', FIXTURE_MAGIC, f['player'], f['hp'], f['ac100'], f['ev100'], f['sh100'],
                                f['shield_limit'], f['regen'], 0))
    out += np.asarray(f['kinds'], '<i4').tobytes()
    out += np.asarray(f['floor'], np.uint8).tobytes()
    out += np.asarray(f['dist'], '<u2').tobytes()
    out += np.asarray(f['los'], '<u4').tobytes()
    out += np.asarray(f['spawns'], '<i2').tobytes()
    return bytes(out)


# ---------------------------------------------------------------- compiler (HIP kernels)
def distance_rows(floor, sources, device='cuda'):
    """BFS distance rows uint16 [len(sources), 5600] over the 8-connected floor (d1_distance_rows)."""
    dev = torch.device(device)
    fl = torch.from_numpy(np.ascontiguousarray(floor, np.uint8).reshape(N)).to(dev)
    src = torch.from_numpy(np.ascontiguousarray(sources, np.int16)).to(dev)
    out = torch.empty((len(src), N), dtype=torch.int16, device=dev)
    if len(src):
        _lib.check(_lib.load().d1_distance_rows(fl.data_ptr(), src.data_ptr(), len(src), out.data_ptr(),
                                                torch.cuda.current_stream(dev).cuda_stream), 'd1_distance_rows')
    return out.cpu().numpy().view(np.uint16)


def los_table(floor, device='cuda'):
    """The 17x17 LOS bitsets uint32 [5600, 10] of one map with the native ray table (d1_los_table)."""
    dev = torch.device(device)
    fl = torch.from_numpy(np.ascontiguousarray(floor, np.uint8).reshape(N)).to(dev)
    slots = np.ascontiguousarray(data.rays()['slots'], np.uint64)
    slots_dev = torch.from_numpy(slots.view(np.int64)).to(dev)
    rays = D1Tables(None, None, slots_dev.data_ptr(), slots.shape[0])
    los = torch.empty((N, 10), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().d1_los_table(fl.data_ptr(), 1, C.byref(rays), los.data_ptr(),
                                        torch.cuda.current_stream(dev).cuda_stream), 'd1_los_table')
    return los.cpu().numpy().view(np.uint32)


def compile_map(floor, seed, hp, ac100, ev100, sh100, device='cuda'):
    """A corpus map from a floor map and the player stats (gpu-d1/scripts/compile_corpus.py
    :18-104 without the native-export parsing): cell list, index, distance rows, LOS."""
    floor = (np.asarray(floor).reshape(N) != 0).astype(np.uint8)
    cells_list = np.flatnonzero(floor).astype(np.int16)
    cells = np.full(N, -1, np.int16)
    cells[:len(cells_list)] = cells_list
    index = np.full(N, -1, np.int16)
    index[cells_list] = np.arange(len(cells_list), dtype=np.int16)
    return dict(seed=int(seed), ncells=len(cells_list), hp=int(hp), ac100=int(ac100), ev100=int(ev100),
                sh100=int(sh100), floor=floor, cells=cells, index=index,
                distance=distance_rows(floor, cells_list, device), los=los_table(floor, device))


def compile_fixture(floor, hp, ac100, ev100, sh100, shield_limit, regen, kinds, device='cuda'):
    """The wait benchmark's fixture (gpu-d1/scripts/compile_fixture.py:50-80): the player is
    the floor cell with 8 floor neighbours closest (L1) to (40, 35), ties to the lower
    index; dist is its BFS field; the spawns are the 64 nearest reachable cells by
    (distance, index) and the 64 reachable cells at distance >= 10 nearest to distance
    18 by (|distance - 18|, index)."""
    floor = (np.asarray(floor).reshape(N) != 0).astype(np.uint8)
    f2 = np.zeros((H + 2, W + 2), np.uint8)
    f2[1:-1, 1:-1] = floor.reshape(H, W)
    nb = sum(f2[1 + dy:H + 1 + dy, 1 + dx:W + 1 + dx] for dy in (-1, 0, 1) for dx in (-1, 0, 1)
             if dy or dx).reshape(N)
    cand = np.flatnonzero((floor == 1) & (nb == 8))
    if not len(cand):
        raise ValueError('no floor cell with eight floor neighbours')
    px, py = cand % W, cand // W
    player = int(cand[np.lexsort((cand, np.abs(px - 40) + np.abs(py - 35)))[0]])
    dist = distance_rows(floor, [player], device)[0]
    reach = np.flatnonzero((dist > 0) & (dist < 65535))
    if len(reach) < 128:
        raise ValueError('fewer than 128 reachable cells')
    d = dist[reach].astype(np.int64)
    contact = reach[np.lexsort((reach, d))][:64]
    far = d >= 10
    approach = reach[far][np.lexsort((reach[far], np.abs(d[far] - 18)))][:64]
    if len(approach) != 64:
        raise ValueError('fewer than 64 approach cells')
    return dict(player=player, hp=int(hp), ac100=int(ac100), ev100=int(ev100), sh100=int(sh100),
                shield_limit=int(shield_limit), regen=int(regen), kinds=np.asarray(kinds, np.int32).reshape(6, 4),
                floor=floor, dist=dist, los=los_table(floor, device),
                spawns=np.concatenate([contact, approach]).astype(np.int16))


def compile_map1057(device='cuda'):
    """map-1057.bin and fixture.bin rebuilt from this package's map-1057 data (floor,
    player stats and roster as exported by native Crawl)."""
    d = data.map1057()
    _, hp, ac, ev, sh, limit, regen, _ = (int(v) for v in d['header'])
    m = compile_map(d['floor'], 1057, hp, ac, ev, sh, device)
    f = compile_fixture(d['floor'], hp, ac, ev, sh, limit, regen, d['kinds'], device)
    return write_map(m), write_fixture(f)


# ---------------------------------------------------------------- native exports -> corpus
def read_native(prefix):
    """The floor and stats of a native export native-SEED.{json,markers}, with the
    eligibility rules of gpu-d1/scripts/compile_corpus.py:19-27 (no unsupported terrain,
    every map marker a plain feature)."""
    import json
    prefix = pathlib.Path(prefix)
    d = json.loads(prefix.with_suffix('.json').read_text())
    if d['unsupported_tiles']:
        raise ValueError(f'{prefix}: unsupported terrain')
    for line in prefix.with_suffix('.markers').read_text().splitlines():
        if line.strip() and line.split()[0] != '0':
            raise ValueError(f'{prefix}: active map marker')
    floor = np.frombuffer(''.join(d['map']).encode(), np.uint8) == ord('.')
    if floor.size != N:
        raise ValueError(f'{prefix}: unexpected map size')
    return dict(floor=floor.astype(np.uint8), seed=d['seed'], hp=d['hp'], ac100=d['ac100'], ev100=d['ev100'],
                sh100=d['sh100'], roster=d['roster'])


def native_los(prefix):
    """The native LOS table of an export (native-SEED.los: 289 bytes of 0/1 per origin)
    packed as the map files' uint32 [5600, 10] bitsets."""
    raw = np.frombuffer(pathlib.Path(prefix).with_suffix('.los').read_bytes(), np.uint8)
    if raw.size != N * 289:
        raise ValueError(f'{prefix}: missing native LOS table')
    bits = np.zeros((N, 320), np.uint8)
    bits[:, :289] = raw.reshape(N, 289) != 0
    return np.packbits(bits.reshape(N, 10, 32)[:, :, ::-1], axis=2).view('>u4').reshape(N, 10).astype(np.uint32)


def compile_native(prefix, device='cuda', check_los=True):
    """map-SEED.bin bytes of a native export, its LOS table checked against the export's
    own (gpu-d1/scripts/compile_corpus.py:56-86 raises on any mismatch as well)."""
    n = read_native(prefix)
    m = compile_map(n['floor'], n['seed'], n['hp'], n['ac100'], n['ev100'], n['sh100'], device)
    if check_los:
        bad = np.flatnonzero((m['los'] != native_los(prefix)).any(1))
        if len(bad):
            raise ValueError(f'{prefix}: LOS mismatch at {len(bad)} origins, first {int(bad[0])}')
    return write_map(m), m


def main(argv=None):
    """Compile native exports into a corpus directory with its manifest, as
    gpu-d1/scripts/compile_corpus.py:106-129 (same arguments)."""
    import argparse
    import json
    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument('--sources', type=pathlib.Path, action='append', required=True)
    ap.add_argument('--output', type=pathlib.Path, required=True)
    ap.add_argument('--seeds', default='1057,1080,1235,1363,1589,1609')
    args = ap.parse_args(argv)
    rows = []
    for seed in map(int, args.seeds.split(',')):
        src = next((r / f'native-{seed}' for r in args.sources if (r / f'native-{seed}.json').exists()), None)
        if src is None:
            raise FileNotFoundError(f'no native export for seed {seed} in {args.sources}')
        raw, m = compile_native(src)
        args.output.mkdir(parents=True, exist_ok=True)
        (args.output / f'map-{seed}.bin').write_bytes(raw)
        rows.append(dict(seed=seed, cells=m['ncells'], sha256=hashlib.sha256(raw).hexdigest(),
                         player_hp=m['hp'], monster_roster=read_native(src)['roster']))
    (args.output / 'manifest.json').write_text(json.dumps({
        'format': 'gpu-d1-v2-map-corpus', 'magic': MAP_MAGIC, 'maps': rows,
        'sources': args.seeds, 'static_only': True}, indent=2) + '\n')
    print(json.dumps(rows, indent=2))
