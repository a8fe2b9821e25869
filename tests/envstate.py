"""Full-state comparison of HIP env rows (Env.fields(), dcss-auto_amd/env.py:decode_rows)
with the CPU restatement's worlds (OracleEnv.fields()), the check the reference's parity
run makes every step with torch.equal(cpu.state, gpu.state) (gpu-d1/scripts/test_learning.py:53).

Every field a row holds is compared: the RNG (PCG state and increment, or the Philox key
in counter mode), the header scalars (blocks and ncells included, which the state hash
leaves out), the monsters, the viewed memory, the level's floor and spawnable cells, the
occupancy the oracle keeps (rebuilt from the row's living monsters) and the memoised
player view (against the observation's visible channel, which the oracle's LOS fixes)."""
import numpy as np

SCALARS = ('env_id', 't', 'episode', 'player', 'hp', 'regen', 'blocks', 'ticks', 'killed', 'decisions',
           'floor_seen', 'first_stair_tick', 'ncells')


def _first(bad):
    w = np.flatnonzero(bad)
    return f'{len(w)} worlds, first {w[:4].tolist()}'


def assert_same_worlds(got, want, cfg, obs=None, label=''):
    """got: decoded HIP rows; want: oracle records of the same worlds; obs: the HIP
    observations of those worlds (uint8 [n, 15, 15, 8]) when the view is to be checked."""
    n, c = len(want), cfg.count
    assert len(got) == n
    for k in SCALARS:
        bad = got[k].astype(np.int64) != want[k].astype(np.int64)
        assert not bad.any(), f'{label}: {k} differs in {_first(bad)}'
    bad = (got['stairs'].astype(np.int64) != want['stairs'].astype(np.int64)).any(1)
    assert not bad.any(), f'{label}: stairs differ in {_first(bad)}'
    rng = want['rng'].reshape(n, 48)
    if cfg.rng_mode == 0:
        state, inc = rng[:, 0:8].copy().view('<u8')[:, 0], rng[:, 8:16].copy().view('<u8')[:, 0]
        bad = (got['rng_state'] != state) | (got['rng_inc'] != inc)
    else:
        key = rng[:, 16:24].copy().view('<u8')[:, 0]   # key0 | key1 << 32
        bad = got['rng_state'] != key
    assert not bad.any(), f'{label}: RNG state differs in {_first(bad)}'
    for k in ('pos', 'mhp', 'energy', 'awake', 'kind'):
        bad = (got[k][:, :c].astype(np.int64) != want[k][:, :c].astype(np.int64)).any(1)
        assert not bad.any(), f'{label}: monster {k} differs in {_first(bad)}'
    for k in ('viewed', 'floor'):
        bad = ((got[k] != 0) != (want[k] != 0)).any(1)
        assert not bad.any(), f'{label}: {k} map differs in {_first(bad)}'
    cells = np.zeros((n, 5600), bool)
    for i in range(n):
        cells[i, want['cells'][i, :want['ncells'][i]]] = True
    bad = ((got['cells'] != 0) != cells).any(1)
    assert not bad.any(), f'{label}: spawnable cells differ in {_first(bad)}'
    occ = np.full((n, 5600), -1, np.int64)
    live = got['mhp'][:, :c] > 0
    w, i = np.nonzero(live)
    occ[w, got['pos'][:, :c][w, i]] = i
    bad = (occ != want['occ']).any(1)
    assert not bad.any(), f'{label}: occupancy differs in {_first(bad)}'
    if obs is not None:
        bad = ((obs[..., 2] != 0) != (got['view'] != 0)).reshape(n, -1).any(1)
        assert not bad.any(), f'{label}: memoised view differs from the visible channel in {_first(bad)}'
