"""Map file formats (dcss-auto_amd/maps.py): byte layout round trips, rejected files and
the corpus subset rule of gpu-d1/scripts/learn_env_v2.py:26-47. No GPU needed."""
import importlib

import numpy as np
import pytest


@pytest.fixture(scope='module')
def maps():
    return importlib.import_module('dcss-auto_amd.maps')


def synthetic_map(M, seed, rng):
    floor = (rng.random(5600) < 0.3).astype(np.uint8)
    cells_list = np.flatnonzero(floor).astype(np.int16)[:20]
    floor[:] = 0
    floor[cells_list] = 1
    cells = np.full(5600, -1, np.int16)
    cells[:len(cells_list)] = cells_list
    index = np.full(5600, -1, np.int16)
    index[cells_list] = np.arange(len(cells_list))
    return dict(seed=seed, ncells=len(cells_list), hp=18, ac100=681, ev100=794, sh100=906, floor=floor, cells=cells,
                index=index, distance=rng.integers(0, 65536, (len(cells_list), 5600)).astype(np.uint16),
                los=rng.integers(0, 2 ** 32, (5600, 10)).astype(np.uint32))


def test_map_round_trip_and_layout(maps):
    rng = np.random.default_rng(1)
    m = synthetic_map(maps, 1057, rng)
    raw = maps.write_map(m)
    # header then floor, cells, index, distance rows, LOS (gpu-d1/scripts/compile_corpus.py:89-95)
    assert len(raw) == 28 + 5600 + 11200 + 11200 + m['ncells'] * 11200 + 224000
    assert raw[:4] == (0x44325650).to_bytes(4, 'little') and int.from_bytes(raw[8:12], 'little') == m['ncells']
    back = maps.read_map(raw)
    for k in m:
        assert np.array_equal(np.asarray(back[k]), np.asarray(m[k])), k
    with pytest.raises(ValueError):
        maps.read_map(b'\0' * len(raw))                        # bad magic
    with pytest.raises(ValueError):
        maps.read_map(raw[:-4])                                # truncated


def test_fixture_round_trip(maps):
    rng = np.random.default_rng(2)
    f = dict(player=3645, hp=18, ac100=681, ev100=794, sh100=906, shield_limit=2, regen=23,
             kinds=rng.integers(0, 30, (6, 4)).astype(np.int32), floor=(rng.random(5600) < .3).astype(np.uint8),
             dist=rng.integers(0, 65536, 5600).astype(np.uint16), los=rng.integers(0, 2 ** 32, (5600, 10)).astype(np.uint32),
             spawns=rng.integers(0, 5600, 128).astype(np.int16))
    raw = maps.write_fixture(f)
    assert len(raw) == 241188                                  # gpu-d1/src/bench.cu:107-136
    back = maps.read_fixture(raw)
    for k in f:
        assert np.array_equal(np.asarray(back[k]), np.asarray(f[k])), k
    with pytest.raises(ValueError):
        maps.read_fixture(raw[:-2])


def test_corpus_subsets_are_nested(maps, tmp_path):
    """map_limit picks the first map by seed and then a fixed, seed-independent order of
    the others: every smaller subset is contained in every larger one."""
    rng = np.random.default_rng(3)
    seeds = [1057, 1080, 1235, 1363, 1589, 1609, 1733]
    for s in seeds:
        (tmp_path / f'map-{s}.bin').write_bytes(maps.write_map(synthetic_map(maps, s, rng)))
    everything = [m['seed'] for m in maps.read_maps(tmp_path)]
    assert everything == sorted(seeds)
    prev = set()
    for k in range(1, len(seeds) + 1):
        got = [m['seed'] for m in maps.read_maps(tmp_path, map_limit=k)]
        assert got == sorted(got) and got[0] == 1057 and len(got) == k
        assert prev <= set(got)
        prev = set(got)
    with pytest.raises(ValueError):
        maps.read_maps(tmp_path, map_limit=0)
    (tmp_path / 'all').mkdir()
    with pytest.raises(ValueError):
        maps.read_maps(tmp_path / 'all')                       # empty corpus


REF = __import__('pathlib').Path('/root/reference/gpu-d1/fixtures')


@pytest.mark.skipif(not (REF / 'native-1057.json').exists(), reason='the reference checkout is not present')
def test_native_export_parses_to_the_package_map(maps):
    """native-1057.json/.markers parse to this package's map-1057 floor and stats, and the
    native .los packs to the fixture's LOS words for a few origins (CPU only)."""
    data = importlib.import_module('dcss-auto_amd.data')
    n = maps.read_native(REF / 'native-1057')
    d = data.map1057()
    assert np.array_equal(n['floor'], d['floor'])
    assert (n['hp'], n['ac100'], n['ev100'], n['sh100']) == tuple(int(v) for v in d['header'][1:5])
    los = maps.native_los(REF / 'native-1057')
    fixture = maps.read_fixture(REF / 'fixture.bin')
    assert np.array_equal(los, fixture['los'])


def test_shared_level_checks():
    """The optional shared level of Env(level=...): 5600-cell masks, spawnable cells inside
    the floor, at least one spawnable cell; map 1057 passes unchanged."""
    config = importlib.import_module('dcss-auto_amd.config')
    floor, cells = config.shared_map_arrays()
    f, c = config.check_level(floor, cells)
    assert np.array_equal(f, floor) and np.array_equal(c, cells)
    f2, c2 = config.check_level(floor.reshape(70, 80) * 3, cells.astype(bool))
    assert np.array_equal(f2, floor) and np.array_equal(c2, cells)
    with pytest.raises(ValueError, match='5600'):
        config.check_level(floor[:5599], cells[:5599])
    bad = cells.copy()
    bad[np.flatnonzero(floor == 0)[0]] = 1
    with pytest.raises(ValueError, match='floor'):
        config.check_level(floor, bad)
    with pytest.raises(ValueError, match='spawnable'):
        config.check_level(floor, np.zeros(5600, np.uint8))
