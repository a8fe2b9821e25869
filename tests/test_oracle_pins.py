"""Pins of the CPU oracle (oracle/d1_oracle.c) against the reference's own outputs,
published known answers and closed-form properties. No GPU needed."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O


def test_philox_known_answers():
    # Random123 kat_vectors, philox4x32 with 10 rounds.
    assert list(O.philox([0, 0, 0, 0], [0, 0])) == [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]
    assert list(O.philox([0xffffffff] * 4, [0xffffffff] * 2)) == [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]
    assert list(O.philox([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0])) == \
        [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]


def test_mix_matches_reference(golden):
    g = np.load(golden / 'sim_ref.npz')
    L = O.lib()
    for x, y in zip(g['mix_in'], g['mix_out']):
        assert L.o_mix(int(x)) == int(y)


def test_pcg_op_streams_match_reference(golden):
    """next / r (incl. the rejection path at huge bounds) / avg / round, gpu-d1/src/sim.h:21-60."""
    g = np.load(golden / 'sim_ref.npz')
    L = O.lib()
    for s in range(len(g['rng_seed'])):
        ops = np.ascontiguousarray(g['rng_ops'][s])
        args = np.ascontiguousarray(g['rng_args'][s])
        res = np.zeros_like(ops)
        final = np.zeros(1, np.uint64)
        L.o_rng_ops(0, int(g['rng_seed'][s]), int(g['rng_seq'][s]), len(ops), ops.ctypes.data, args.ctypes.data,
                    res.ctypes.data, final.ctypes.data)
        np.testing.assert_array_equal(res, g['rng_results'][s])
        assert int(final[0]) == int(g['rng_final'][s])


def test_bounded_draw_is_unbiased_lemire():
    """Closed form: the counter-mode r(b) over Philox words equals floor(x*b/2^32) unless rejected."""
    L = O.lib()
    n = 2000
    ops = np.ones(n, np.int32)
    args = np.full(n, 6, np.int32)
    res = np.zeros(n, np.int32)
    final = np.zeros(1, np.uint64)
    L.o_rng_ops(1, 5, 3, n, ops.ctypes.data, args.ctypes.data, res.ctypes.data, final.ctypes.data)
    words = []
    for k in range(n):
        words.append(O.philox([k >> 2, 0, 3, 0], [5, 0])[k & 3])
    expect = (np.array(words, np.uint64) * 6) >> 32
    np.testing.assert_array_equal(res, expect.astype(np.int32))   # no rejection at b=6 in this stream
    assert int(final[0]) == n


def test_wait_workload_matches_reference(golden, pkg):
    """Full monster-wait trajectories (scheduler, melee, pathing with repair BFS, reset)
    against the reference's own sim.h: 72 runs x 257 steps, scan and heap scheduling."""
    g = np.load(golden / 'sim_ref.npz')
    L = O.lib()
    m = pkg.data.map1057()
    floor = np.ascontiguousarray(m['floor'])
    dist = np.ascontiguousarray(m['dist'])
    starts = np.ascontiguousarray(m['starts'])
    cfg = np.ascontiguousarray(g['config'])
    kinds = np.ascontiguousarray(g['kinds'])
    trace = np.zeros(g['wait_trace'].shape[1], np.int32)
    for meta, want in zip(g['wait_meta'], g['wait_trace']):
        count, scenario, fixture, heap, world, seed, prewarm = (int(v) for v in meta)
        L.o_wait_run(count, len(trace), heap, fixture, seed, world, floor.ctypes.data, dist.ctypes.data,
                     starts.ctypes.data, cfg.ctypes.data, kinds.ctypes.data, prewarm, trace.ctypes.data)
        np.testing.assert_array_equal(trace, want, err_msg=f'count={count} scenario={scenario} heap={heap} world={world}')


def test_fixture_decode(golden, pkg):
    g = np.load(golden / 'sim_ref.npz')
    c = pkg.reference_config()
    assert [c.hp, c.ac100, c.ev100, c.sh100, c.shield_limit, c.regen, c.repair, c.gdr[0], c.gdr[1]] == \
        list(g['config'][2:])
    assert [v for k in c.kinds for v in (k.speed, k.damage, k.tohit, k.bypass)] == list(g['kinds'])
    assert C.sizeof(pkg.D1Config) == 4 * 50


def test_los_matches_native_export_all_origins(golden, pkg):
    """The runtime ray scan reproduces the reference's LOS bitsets (native Crawl LOS) for
    every one of the 5600 origins of map 1057."""
    want = np.load(golden / 'map1057_los.npz')['los']
    floor = pkg.data.map1057()['floor']
    for p in range(5600):
        got = O.los_bitset(floor, p)
        assert np.array_equal(got, want[p]), p


def test_point_los_agrees_with_bitset(pkg):
    floor = pkg.data.map1057()['floor']
    L = O.lib()
    rng = np.random.default_rng(3)
    f = np.ascontiguousarray(floor)
    for p in rng.choice(np.flatnonzero(floor), 60, replace=False):
        bits = O.los_bitset(floor, int(p))
        for dy in range(-7, 8):
            for dx in range(-7, 8):
                x, y = p % 80 + dx, p // 80 + dy
                if not (0 <= x < 80 and 0 <= y < 70):
                    continue
                b = (dy + 8) * 17 + dx + 8
                assert L.o_los(f.ctypes.data, int(p), y * 80 + x, 7) == (bits[b // 32] >> (b % 32)) & 1


def _components(floor):
    from collections import deque
    seen = np.zeros(5600, bool)
    comps = 0
    for s in np.flatnonzero(floor):
        if seen[s]:
            continue
        comps += 1
        q = deque([s]); seen[s] = True
        while q:
            p = q.popleft()
            x, y = p % 80, p // 80
            for dx in (-1, 0, 1):
                for dy in (-1, 0, 1):
                    if 0 <= x + dx < 80 and 0 <= y + dy < 70:
                        r = (y + dy) * 80 + x + dx
                        if floor[r] and not seen[r]:
                            seen[r] = True; q.append(r)
    return comps


def test_generated_levels_are_connected_rooms():
    sizes = []
    for env in range(40):
        f = O.level(12345, env).reshape(70, 80)
        assert not f[0].any() and not f[-1].any() and not f[:, 0].any() and not f[:, -1].any()
        assert _components(f.ravel()) == 1
        sizes.append(int(f.sum()))
        assert np.array_equal(f, O.level(12345, env).reshape(70, 80))
    assert min(sizes) > 150 and max(sizes) < 2500
    assert len(set(sizes)) > 20
