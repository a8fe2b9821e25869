"""Sampler and GAE kernels vs fp32 PyTorch restatements of the reference's math
(gpu-d1/scripts/run_ring_ablations.py:350-362). Tolerance: 1e-5 relative (fp32)."""
import importlib

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def philox_u(seed, t, n):
    key = [seed & 0xFFFFFFFF, seed >> 32]
    w = np.array([O.philox([0, t, i, 3], key)[0] for i in range(n)], np.uint64)
    return torch.from_numpy(((w >> 8).astype(np.float64) / 16777216.0).astype(np.float32))


@pytest.mark.parametrize('k', [16, 19, 8])
def test_sampler_matches_inverse_cdf(k):
    pol = importlib.import_module('dcss-auto_amd.policy')
    print(f'[sampler] k={k}', flush=True)
    n, seed, t = 4096, 77, 5
    g = torch.Generator().manual_seed(k)
    logits = torch.randn(n, k, generator=g) * 2.0
    logits[:, 0] -= 30.0        # a near-impossible action
    a, lp = pol.sample(logits.cuda(), seed, t)
    a, lp = a.cpu(), lp.cpu()
    u = philox_u(seed, t, n)
    p = torch.softmax(logits.double(), 1)
    c = torch.cumsum(p, 1)
    ref = (u.double()[:, None] < c).float().argmax(1)
    ref = torch.where((u.double()[:, None] < c).any(1), ref, torch.full_like(ref, k - 1))
    near = ((c - u.double()[:, None]).abs() < 1e-5).any(1)
    assert torch.equal(a[~near], ref[~near])
    ref_lp = torch.log_softmax(logits.double(), 1).gather(1, a[:, None]).squeeze(1)
    torch.testing.assert_close(lp.double(), ref_lp, rtol=1e-5, atol=1e-5)
    # the empirical distribution follows the probabilities
    freq = torch.bincount(a, minlength=k).double() / n
    assert (freq - p.mean(0)).abs().max() < 0.03


def test_sampler_is_a_counter_rng():
    pol = importlib.import_module('dcss-auto_amd.policy')
    logits = torch.zeros(1000, 16, device='cuda')
    a1, _ = pol.sample(logits, 3, 9)
    a2, _ = pol.sample(logits, 3, 9)
    a3, _ = pol.sample(logits, 3, 10)
    assert torch.equal(a1, a2) and not torch.equal(a1, a3)
    sub, _ = pol.sample(logits[:100], 3, 9)          # env i's draw does not depend on the batch size
    assert torch.equal(sub, a1[:100])


def gae_reference(r, d, v, boot, gamma=0.99, lam=0.95):
    """The reference loop, fp32 elementwise (gpu-d1/scripts/run_ring_ablations.py:355-360)."""
    T = r.shape[0]
    adv = torch.empty_like(r)
    nextv = boot.clone()
    gae = torch.zeros_like(boot)
    for t in reversed(range(T)):
        live = 1 - d[t]
        delta = r[t] + gamma * nextv * live - v[t]
        gae = delta + gamma * lam * live * gae
        adv[t], nextv = gae, v[t]
    return adv, adv + v


@pytest.mark.parametrize('T,n', [(128, 4096), (7, 1000), (1, 33)])
def test_gae_matches_reference_loop(T, n):
    pol = importlib.import_module('dcss-auto_amd.policy')
    print(f'[gae] T={T} n={n}', flush=True)
    g = torch.Generator().manual_seed(T * n)
    r = torch.where(torch.rand(T, n, generator=g) < 0.97, torch.zeros(T, n), torch.rand(T, n, generator=g) * 2 - 1)
    d = (torch.rand(T, n, generator=g) < 0.01).to(torch.uint8)
    v = torch.randn(T, n, generator=g)
    boot = torch.randn(n, generator=g)
    ra, rr = gae_reference(r, d.float(), v, boot)
    adv, ret = pol.gae(r.cuda(), d.cuda(), v.cuda(), boot.cuda())
    torch.testing.assert_close(adv.cpu(), ra, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ret.cpu(), rr, rtol=1e-5, atol=1e-6)
    exact = (adv.cpu() == ra).float().mean().item()
    print(f'[gae] bit-exact fraction {exact:.6f}', flush=True)


def test_gae_properties_closed_form():
    """gamma=lam=1, no dones: adv[t] = sum_{s>=t} r[s] + boot - v[t]."""
    pol = importlib.import_module('dcss-auto_amd.policy')
    T, n = 16, 256
    r = torch.randint(-3, 4, (T, n)).float()
    v = torch.randint(-3, 4, (T, n)).float()
    boot = torch.randint(-3, 4, (n,)).float()
    d = torch.zeros(T, n, dtype=torch.uint8)
    adv, _ = pol.gae(r.cuda(), d.cuda(), v.cuda(), boot.cuda(), gamma=1.0, lam=1.0)
    want = torch.flip(torch.cumsum(torch.flip(r, [0]), 0), [0]) + boot - v
    assert torch.equal(adv.cpu(), want)
    d[5] = 1      # a done cuts the bootstrap and the accumulation at t=5
    adv, _ = pol.gae(r.cuda(), d.cuda(), v.cuda(), boot.cuda(), gamma=1.0, lam=1.0)
    assert torch.equal(adv.cpu()[5], r[5] - v[5])


def test_widening_is_exact():
    pol = importlib.import_module('dcss-auto_amd.policy')
    x = torch.arange(256, dtype=torch.uint8).repeat(4096 * 7 // 256 + 16)[: 4096 * 7].cuda()
    y = pol.widen(x, torch.bfloat16)
    assert torch.equal(y.float().cpu(), x.float().cpu())


def test_policy_forward_matches_fp32_reference():
    """bf16 trunk vs an fp32 restatement with the same (bf16-rounded) weights: 2e-2."""
    pol = importlib.import_module('dcss-auto_amd.policy')
    model = pol.Policy(seed=3).cuda().to(torch.bfloat16)
    obs = torch.randint(0, 20, (512, 15, 15, 8), dtype=torch.uint8, device='cuda')
    with torch.no_grad():
        logits, value = model(obs)
        x = obs.reshape(512, -1).float()
        w = {k: v.float() for k, v in model.state_dict().items()}
        h = torch.relu(x @ w['l1.weight'].t() + w['l1.bias'])
        h = torch.relu(h @ w['l2.weight'].t() + w['l2.bias'])
        out = h @ w['head.weight'].t() + w['head.bias']
    torch.testing.assert_close(logits, out[:, :16], rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(value, out[:, 16], rtol=2e-2, atol=2e-2)
