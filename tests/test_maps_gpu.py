"""The map compiler (dcss-auto_amd/maps.py on d1_distance_rows + d1_los_table): map-1057
rebuilt from this package's data is byte-identical to the reference's compiled files —
the sha256 values the reference's manifests record for them."""
import hashlib
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# gpu-d1/fixtures/d1-corpus-388/manifest.json:9 (map-1057.bin, written by compile_corpus.py)
MAP1057_SHA256 = '9a89eff1b7e19eed9cea6784256dd8c8b5ba1f24c37a05ccdf79274793acb281'
# gpu-d1/fixtures/manifest.json:3 (fixture.bin, written by compile_fixture.py)
FIXTURE_SHA256 = 'af72ec047fb96bee6c32fda79e495776fd0132f9103fc27fea187f4717cee3ec'


def test_map1057_round_trip_sha256():
    maps = importlib.import_module('dcss-auto_amd.maps')
    data = importlib.import_module('dcss-auto_amd.data')
    print('[maps] compile map 1057', flush=True)
    map_bytes, fixture_bytes = maps.compile_map1057()
    assert hashlib.sha256(map_bytes).hexdigest() == MAP1057_SHA256
    assert hashlib.sha256(fixture_bytes).hexdigest() == FIXTURE_SHA256
    f = maps.read_fixture(fixture_bytes)
    d = data.map1057()
    assert f['player'] == int(d['header'][0])
    assert np.array_equal(f['dist'], d['dist']) and np.array_equal(f['spawns'], d['starts'])
    m = maps.read_map(map_bytes)
    assert m['ncells'] == 836 and np.array_equal(m['los'], f['los'])
    # the fixture's distance field is the player's row of the all-pairs table
    assert np.array_equal(m['distance'][m['index'][f['player']]], f['dist'])


def test_distance_rows_are_a_metric():
    """On a random cave: d(p, p) = 0, symmetry, and neighbours differ by at most one."""
    maps = importlib.import_module('dcss-auto_amd.maps')
    rng = np.random.default_rng(4)
    floor = (rng.random(5600) < 0.55).astype(np.uint8)
    cells = np.flatnonzero(floor)[:300].astype(np.int16)
    d = maps.distance_rows(floor, cells).astype(np.int64)
    assert np.all(d[np.arange(len(cells)), cells] == 0)
    sub = d[:, cells]
    assert np.array_equal(sub, sub.T)
    assert np.all(d[:, ~floor.astype(bool)] == 65535)
    fin = d < 65535
    grid = d.reshape(len(cells), 70, 80)
    for dy, dx in ((0, 1), (1, 0), (1, 1), (1, -1)):   # every 8-neighbour pair once
        x0, x1 = max(0, -dx), 80 - max(0, dx)
        a = grid[:, 0:70 - dy, x0:x1]
        b = grid[:, dy:70, x0 + dx:x1 + dx]
        both = (a < 65535) & (b < 65535)
        assert np.all(np.abs(a - b)[both] <= 1)
    # a source outside the map leaves its row unreached
    assert np.all(maps.distance_rows(floor, [-1, 5600]) == 65535)
    assert fin.any()


def test_learn_maps_from_files_equal_computed(tmp_path):
    maps = importlib.import_module('dcss-auto_amd.maps')
    learn = importlib.import_module('dcss-auto_amd.learn')
    map_bytes, _ = maps.compile_map1057()
    (tmp_path / 'map-1057.bin').write_bytes(map_bytes)
    loaded = learn.LearnMaps.from_maps(maps.read_maps(tmp_path))
    computed = learn.LearnMaps(maps.read_map(map_bytes)['floor'][None])
    torch.cuda.synchronize()
    assert torch.equal(loaded.los, computed.los) and torch.equal(loaded.floor, computed.floor)
