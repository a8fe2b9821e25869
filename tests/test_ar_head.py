"""Autoregressive verb x target head. CPU: the factorisation identities the reference
checks for its type x direction head (gpu-d1/branches/autoregressive-actions-v1/scripts/
preflight.py:25-35) — entropy and log-prob equal those of the joint categorical.
GPU: the HIP two-stage sampler against an inverse-CDF restatement."""
import importlib

import numpy as np
import pytest
import torch
from torch.distributions import Categorical


def test_ar_distribution_matches_joint_categorical():
    P = importlib.import_module('dcss-auto_amd.policy')
    g = torch.Generator().manual_seed(1)
    verb = torch.randn(64, 8, generator=g, requires_grad=True)
    target = torch.randn(64, 8, 25, generator=g, requires_grad=True)
    dist = P.ARDistribution(verb.double(), target.double())
    joint = Categorical(probs=dist.probs)
    torch.testing.assert_close(dist.probs.sum(1), torch.ones(64, dtype=torch.float64))
    torch.testing.assert_close(dist.entropy(), joint.entropy())
    for _ in range(20):
        a = joint.sample()
        torch.testing.assert_close(dist.log_prob(a // 25, a % 25), joint.log_prob(a))
    (-dist.log_prob(torch.zeros(64, dtype=torch.long), torch.ones(64, dtype=torch.long)).mean()
     - 0.01 * dist.entropy().mean()).backward()
    assert torch.isfinite(verb.grad).all() and torch.isfinite(target.grad).all()


def test_ar_policy_shapes_and_verb_conditioning():
    P = importlib.import_module('dcss-auto_amd.policy')
    m = P.ARPolicy(seed=2)
    obs = torch.randint(0, 9, (5, 15, 15, 8), dtype=torch.uint8)
    v, t, val = m(obs)
    assert v.shape == (5, 8) and t.shape == (5, 8, 25) and val.shape == (5,)
    assert not torch.allclose(t[:, 0], t[:, 1])            # the embedding conditions the target head


@pytest.mark.gpu
def test_ar_sampler_matches_inverse_cdf():
    from oracle import oracle as O
    P = importlib.import_module('dcss-auto_amd.policy')
    n, seed, t = 2048, 99, 3
    g = torch.Generator().manual_seed(7)
    vl = torch.randn(n, 8, generator=g) * 2
    tl = torch.randn(n, 8, 25, generator=g) * 2
    verb, target, action, logp = (x.cpu() for x in P.sample_ar(vl.cuda(), tl.cuda(), seed, t))
    key = [seed & 0xFFFFFFFF, seed >> 32]
    words = np.array([O.philox([0, t, i, 3], key)[:2] for i in range(n)], np.uint64)
    u = torch.from_numpy(((words >> 8).astype(np.float64) / 16777216.0))
    pv = torch.softmax(vl.double(), 1)
    cv = torch.cumsum(pv, 1)
    ref_v = (u[:, :1] < cv).double().argmax(1)
    pt = torch.softmax(tl.double(), 2)[torch.arange(n), verb.long()]
    ct = torch.cumsum(pt, 1)
    ref_t = (u[:, 1:] < ct).double().argmax(1)
    near = ((cv - u[:, :1]).abs() < 1e-5).any(1) | ((ct - u[:, 1:]).abs() < 1e-5).any(1)
    assert torch.equal(verb.long()[~near], ref_v[~near]) and torch.equal(target.long()[~near], ref_t[~near])
    ref_lp = P.ARDistribution(vl.double(), tl.double()).log_prob(verb.long(), target.long())
    torch.testing.assert_close(logp.double(), ref_lp, rtol=1e-5, atol=1e-5)
    dirs = {(0, -1): 0, (1, 0): 1, (0, 1): 2, (-1, 0): 3, (1, -1): 4, (1, 1): 5, (-1, 1): 6, (-1, -1): 7}
    for v, tg, a in zip(verb.tolist(), target.tolist(), action.tolist()):
        if v <= 1:
            d = dirs.get((tg % 5 - 2, tg // 5 - 2))
            assert a == (-1 if d is None else d + 8 * v)
        else:
            assert a == {2: 16, 3: 17, 4: 18}.get(v, 16)
