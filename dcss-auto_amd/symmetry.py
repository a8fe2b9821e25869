"""D4 camera augmentation, fixed per episode: the reference's EpisodeSymmetry
(gpu-d1/branches/autoregressive-actions-v1/scripts/symmetry.py:10-102) restated for this
build's uint8 15x15x8 observation and its 19 actions (0-7 move, 8-15 attack in the
direction order N, E, S, W, NE, SE, SW, NW; 16 wait, 17 rest, 18 descend).

Group g (0..7) mirrors x when g >= 4, then turns g % 4 quarter turns (x, y) -> (-y, x)
(x east, y south). The observation permutation runs on the GPU (d1_obs_d4); actions
chosen in the camera frame map back to the world frame through the inverse direction
permutation, as the reference's to_world does."""
import torch

from . import _lib

DIRECTIONS = ((0, -1), (1, 0), (0, 1), (-1, 0), (1, -1), (1, 1), (-1, 1), (-1, -1))
N_ACTIONS = 19


def xy(x, y, g):
    """(x, y) under group element g."""
    if g >= 4:
        x = -x
    for _ in range(g % 4):
        x, y = -y, x
    return x, y


def tables():
    """forward[g][a]: the camera-frame action of world action a; inverse = its inverse."""
    forward = torch.zeros((8, N_ACTIONS), dtype=torch.int64)
    for g in range(8):
        for a in range(N_ACTIONS):
            if a < 16:
                forward[g, a] = 8 * (a // 8) + DIRECTIONS.index(xy(*DIRECTIONS[a % 8], g))
            else:
                forward[g, a] = a
    return forward, forward.argsort(1)


def observation(obs, groups, out=None):
    """uint8 [n, 15, 15, 8] observations seen through per-env camera groups (int32 [n])."""
    n = obs.shape[0]
    if obs.dtype != torch.uint8 or obs.numel() != n * 1800 or not obs.is_contiguous():
        raise ValueError('observations must be contiguous uint8 [n, 15, 15, 8]')
    if groups.dtype != torch.int32 or groups.shape != (n,) or not groups.is_contiguous():
        raise ValueError('groups must be int32 [n]')
    if out is None:
        out = torch.empty_like(obs)
    _lib.check(_lib.load().d1_obs_d4(obs.data_ptr(), groups.data_ptr(), n, out.data_ptr(),
                                     torch.cuda.current_stream(obs.device).cuda_stream), 'd1_obs_d4')
    return out


class EpisodeSymmetry:
    """An Env seen through a camera group per world, drawn at reset and redrawn when the
    world's episode ends (a fixed-size draw per step, so no device synchronisation)."""

    def __init__(self, base, seed):
        self.base = base
        forward, inverse = tables()
        self.forward, self.inverse = forward.to(base.device), inverse.to(base.device)
        self.rng = torch.Generator(device=base.device)
        self.rng.manual_seed(seed)
        self.groups = self._draw()
        self.obs = torch.empty_like(base.obs)
        self.refresh()

    def __getattr__(self, name):
        return getattr(self.base, name)

    def _draw(self):
        return torch.randint(8, (self.base.batch,), generator=self.rng, device=self.base.device, dtype=torch.int32)

    def refresh(self):
        observation(self.base.obs, self.groups, out=self.obs)

    def to_world(self, actions):
        return self.inverse[self.groups.long()].gather(1, actions[:, None]).squeeze(1)

    def reset(self, seed):
        self.base.reset(seed)
        self.groups = self._draw()
        self.refresh()
        return self.obs

    def step(self, actions, active=None):
        _, out = self.base.step(self.to_world(actions), active=active)
        ended = out[:, 1] > 0
        if active is not None:
            ended &= active
        self.groups = torch.where(ended, self._draw(), self.groups)
        self.refresh()
        return self.obs, out

    def snapshot(self):
        return dict(groups=self.groups.cpu(), rng=self.rng.get_state(), raw_obs=self.base.obs.cpu())

    def restore(self, state):
        self.groups = state['groups'].to(self.base.device)
        self.rng.set_state(state['rng'])
        self.base.obs.copy_(state['raw_obs'])
        self.refresh()
