"""D4 camera augmentation (dcss-auto_amd/symmetry.py, d1_obs_d4): the window permutation
equals numpy's flips and quarter turns, the action tables follow the geometry, the
wrapper steps the world with the mapped actions, and a group-averaged policy is
invariant (the reference's D4 check, gpu-d1/branches/autoregressive-actions-v1/scripts/
preflight.py:18-24)."""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def numpy_d4(w, g):
    """w [15 rows (y), 15 cols (x), 8]: mirror x (flip columns) when g >= 4, then g % 4
    clockwise quarter turns ((x, y) -> (-y, x) with y pointing down)."""
    if g >= 4:
        w = np.flip(w, 1)
    return np.rot90(w, -(g % 4), axes=(0, 1))


def test_window_permutation_matches_numpy():
    S = importlib.import_module('dcss-auto_amd.symmetry')
    print('[d4] permutation', flush=True)
    rng = np.random.default_rng(0)
    n = 333
    obs = rng.integers(0, 256, (n, 15, 15, 8), dtype=np.uint8)
    groups = rng.integers(0, 8, n).astype(np.int32)
    out = S.observation(torch.from_numpy(obs).cuda(), torch.from_numpy(groups).cuda()).cpu().numpy()
    for i in range(n):
        assert np.array_equal(out[i], numpy_d4(obs[i], groups[i])), (i, groups[i])
    # the group acts faithfully: 8 distinct images, g = 0 is the identity, inverses undo
    forward, inverse = S.tables()
    x = torch.from_numpy(obs[:1]).cuda().repeat(8, 1, 1, 1).contiguous()
    imgs = S.observation(x, torch.arange(8, dtype=torch.int32, device='cuda'))
    assert len({bytes(imgs[g].cpu().numpy()) for g in range(8)}) == 8 and torch.equal(imgs[0], x[0])
    inv_g = torch.tensor([next(h for h in range(8) if all(S.xy(*S.xy(1, 2, g), h) == (1, 2) and
                                                          S.xy(*S.xy(0, 1, g), h) == (0, 1) for _ in [0]))
                          for g in range(8)], dtype=torch.int32, device='cuda')
    assert torch.equal(S.observation(imgs, inv_g), x)


def test_action_tables_follow_the_window():
    """A monster one cell away in world direction d appears in the camera window at the
    cell of camera direction forward[g][d]; attacking it there maps back to 8 + d."""
    S = importlib.import_module('dcss-auto_amd.symmetry')
    forward, inverse = S.tables()
    for g in range(8):
        assert sorted(forward[g].tolist()) == list(range(19)) and forward[g, 16:].tolist() == [16, 17, 18]
        for d, (dx, dy) in enumerate(S.DIRECTIONS):
            w = np.zeros((15, 15, 8), np.uint8)
            w[7 + dy, 7 + dx, 3] = 1
            cw = numpy_d4(w, g)
            cy, cx = [int(v[0]) for v in np.nonzero(cw[:, :, 3])]
            cam = forward[g, 8 + d].item()
            assert S.DIRECTIONS[cam - 8] == (cx - 7, cy - 7)
            assert inverse[g, cam].item() == 8 + d and inverse[g, forward[g, d]].item() == d


def test_episode_symmetry_steps_the_world(pkg):
    S = importlib.import_module('dcss-auto_amd.symmetry')
    print('[d4] wrapper', flush=True)
    cfg = pkg.baseline_config(8)
    world = pkg.Env(400, cfg, seed=3, hash=False)
    twin = pkg.Env(400, cfg, seed=3, hash=False)
    sym = S.EpisodeSymmetry(twin, seed=9)
    g = torch.Generator().manual_seed(1)
    ended_any = False
    for _ in range(200):
        cam = torch.randint(0, 19, (400,), generator=g).cuda()
        groups = sym.groups.clone()
        world.step(sym.inverse[groups.long()].gather(1, cam[:, None]).squeeze(1))
        obs, out = sym.step(cam)
        ended = out[:, 1] > 0
        ended_any |= bool(ended.any())
        assert torch.equal(world.state, twin.state)
        assert torch.equal(sym.groups[~ended], groups[~ended])          # groups change only at episode ends
        assert torch.equal(obs, S.observation(world.obs, sym.groups))
    assert ended_any
    snap = sym.snapshot()
    before = sym.obs.clone()
    sym.step(torch.randint(0, 19, (400,), generator=g).cuda())
    twin.state.copy_(world.state)
    sym.restore(snap)
    assert torch.equal(sym.obs, before)


def test_group_averaged_policy_is_invariant():
    """p(a | o) = mean_g softmax(L(T_g o))[forward_g[a]] (the reference's d4_exact head on
    this build's fused forward): p(. | T_h o) permuted by forward_h equals p(. | o)."""
    S = importlib.import_module('dcss-auto_amd.symmetry')
    P = importlib.import_module('dcss-auto_amd.policy')
    print('[d4] invariance', flush=True)
    model = P.Policy(seed=5).cuda().to(torch.bfloat16)
    forward, _ = S.tables()
    fwd16 = forward[:, :16].cuda()
    obs = torch.randint(0, 40, (64, 15, 15, 8), dtype=torch.uint8, device='cuda')

    def averaged(o):
        n = o.shape[0]
        groups = torch.arange(8, dtype=torch.int32, device='cuda').repeat_interleave(n)
        with torch.no_grad():
            logits, _ = model(S.observation(o.repeat(8, 1, 1, 1).contiguous(), groups))
        p = torch.softmax(logits.view(8, n, 16).double(), -1)
        return torch.stack([p[g][:, fwd16[g]] for g in range(8)]).mean(0)

    base = averaged(obs)
    for h in range(8):
        seen = averaged(S.observation(obs, torch.full((64,), h, dtype=torch.int32, device='cuda')))
        torch.testing.assert_close(seen[:, fwd16[h]], base, rtol=1e-9, atol=1e-12)
