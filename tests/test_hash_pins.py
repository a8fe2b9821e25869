"""The per-world state digest (o_hash in oracle/d1_oracle.c, state_hash in the HIP step).

It is a sum mod 2^32 of fmix32(word ^ index * 0x9E3779B9) over the canonical words, and
fmix32 is a bijection, so a change of any one canonical word changes the sum. These tests
check that every canonical field is in fact one of those words (a field dropped from the
digest would let a divergence in it pass the per-step hash comparison unseen), and record
which stored fields the digest leaves out: the GPU parity tests compare those through the
decoded state rows (tests/envstate.py) instead."""
import ctypes as C
import importlib

import numpy as np
import pytest

from oracle import oracle as O

pkg = importlib.import_module('dcss-auto_amd')


def worlds(cfg, n=4, steps=40):
    env = O.OracleEnv(n, cfg, seed=17)
    rng = np.random.default_rng(1)
    for _ in range(steps):
        env.step(rng.integers(0, 19, n))
    return env


def digest(buf, cfg):
    L = O.lib()
    return L.o_hash(buf.ctypes.data, C.byref(cfg))


def edits(cfg, f):
    """(name, edit) pairs, each changing one canonical word of record `f`."""
    def set_(name, idx=None):
        def go(r):
            if idx is None:
                r[name] = r[name] + 1
            else:
                r[name][idx] = r[name][idx] + 1
        return go
    out = [(k, set_(k)) for k in ('player', 'hp', 'regen', 'ticks', 'killed', 'decisions', 'floor_seen',
                                  'episode', 't', 'first_stair_tick')]
    out += [(f'stairs[{k}]', set_('stairs', k)) for k in range(3)]
    if cfg.rng_mode == 0:
        out += [('pcg state low word', lambda r: r.__setitem__('rng_state', r['rng_state'] ^ np.uint64(1))),
                ('pcg state high word', lambda r: r.__setitem__('rng_state', r['rng_state'] ^ np.uint64(1 << 40)))]
    for i in range(cfg.count):
        for k in ('pos', 'mhp', 'energy', 'awake', 'kind'):
            out.append((f'{k}[{i}]', set_(k, i)))
    return out


@pytest.mark.parametrize('which', ['baseline', 'reference', 'stress'])
def test_every_canonical_field_changes_the_digest(which):
    cfg = {'baseline': pkg.baseline_config(8), 'reference': pkg.reference_config(24),
           'stress': pkg.stress_config()}[which]
    env = worlds(cfg)
    dt = O.ostate_dtype()
    for w in range(env.batch):
        base = env.state[w].copy()
        h0 = digest(base, cfg)
        for name, edit in edits(cfg, base.view(dt)[0]):
            buf = base.copy()
            edit(buf.view(dt)[0])
            assert digest(buf, cfg) != h0, (which, w, name)
        # every cell of the viewed memory is a bit of one of the 210 row words
        for p in range(5600):
            buf = base.copy()
            r = buf.view(dt)[0]
            r['viewed'][p] ^= 1
            assert digest(buf, cfg) != h0, (which, w, 'viewed', p)


def test_fields_left_out_of_the_digest():
    """The digest covers the trajectory's state, not the level or the caches: blocks (cleared
    at the start of every turn), ncells, the spawnable-cell list and the floor (fixed per
    world), the occupancy map (derived from the monsters), the PCG increment (fixed per
    world) and the counter RNG's key (fixed per run) leave it unchanged, so the parity tests
    compare them from the decoded rows."""
    cfg = pkg.baseline_config(8)
    env = worlds(cfg)
    dt = O.ostate_dtype()
    base = env.state[0].copy()
    h0 = digest(base, cfg)

    def key_edit(r):
        r['rng'][16] ^= 1

    for name, edit in (('blocks', lambda r: r.__setitem__('blocks', r['blocks'] + 1)),
                       ('ncells', lambda r: r.__setitem__('ncells', r['ncells'] - 1)),
                       ('occ', lambda r: r['occ'].__setitem__(0, 5)),
                       ('floor', lambda r: r['floor'].__setitem__(0, 1 - r['floor'][0])),
                       ('rng_inc', lambda r: r.__setitem__('rng_inc', r['rng_inc'] + np.uint64(2))),
                       ('counter key', key_edit)):
        buf = base.copy()
        edit(buf.view(dt)[0])
        assert digest(buf, cfg) == h0, name
