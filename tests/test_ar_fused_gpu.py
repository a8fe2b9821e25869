"""The fused autoregressive policy kernel (d1_policy_fwd_sample_ar): ARPolicy's bf16
forward (trunk, verb head, value, verb-embedding-conditioned target MLP) and the two-stage
counter-RNG draw in one launch.

Checked against (1) an fp32 restatement of the network on the CPU and the bf16 torch forward
(ARPolicy.forward) at the bf16 bar, 2e-2 of the output scale, for the verb logits, the value
and the drawn verb's target logits; (2) the standalone two-stage sampler d1_sample_ar on the
kernel's own logits, bit for bit (verb, target, env action, log-probability); (3) the inverse
CDF of the oracle's Philox uniforms, and log-softmax of the kernel's logits (1e-5, the fp32
bar). Batches of 1, 255, 4,133 (ragged tails) and C5's 262,144."""
import importlib

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def run_fused(P, model, obs, seed, t, t_dev=None):
    n = obs.shape[0]
    out = dict(action=torch.empty(n, dtype=torch.int64, device='cuda'), logp=torch.empty(n, device='cuda'),
               value=torch.empty(n, device='cuda'), verb=torch.empty(n, dtype=torch.int32, device='cuda'),
               target=torch.empty(n, dtype=torch.int32, device='cuda'),
               verb_logits=torch.empty((n, P.N_VERBS), device='cuda'),
               target_logits=torch.empty((n, P.N_TARGETS), device='cuda'))
    P.policy_fwd_sample_ar(obs, model.packed(), seed, t, out['action'], out['logp'], out['value'], t_dev=t_dev,
                           verb=out['verb'], target=out['target'], verb_logits=out['verb_logits'],
                           target_logits=out['target_logits'])
    torch.cuda.synchronize()
    return out


def restated(model, x, verb):
    """fp32 CPU restatement of the network for rows x, target head at the given verbs."""
    f = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    h = torch.relu(x @ f['l1.weight'].T + f['l1.bias'])
    h = torch.relu(h @ f['l2.weight'].T + f['l2.bias'])
    vz = h @ f['verb.weight'].T + f['verb.bias']
    val = (h @ f['value.weight'].T + f['value.bias'])[:, 0]
    w = f['t1.weight']
    ht = h @ w[:, :h.shape[1]].T + f['t1.bias']
    ev = f['embedding'] @ w[:, h.shape[1]:].T
    z = torch.tanh(ht + ev[verb])
    return vz, val, z @ f['t2.weight'].T + f['t2.bias']


def close(got, want, what):
    scale = float(want.abs().max()) + 1e-6
    err = float((got - want).abs().max())
    assert err <= 2e-2 * scale, f'{what}: max error {err:.3g} vs scale {scale:.3g}'


@pytest.mark.parametrize('n', [1, 255, 4133])
def test_fused_ar_head(n):
    print(f'[ar fused] n={n}', flush=True)
    P = importlib.import_module('dcss-auto_amd.policy')
    model = P.ARPolicy(seed=5).cuda().to(torch.bfloat16)
    with torch.no_grad():   # spread the target logits so the draws are not near-uniform
        model.t2.weight.mul_(20)
        model.embedding.mul_(10)
    g = torch.Generator(device='cuda').manual_seed(n)
    obs = torch.randint(0, 24, (n, 1800), dtype=torch.uint8, device='cuda', generator=g)
    seed, t = 0x1234_5678_9ABC, 37
    out = run_fused(P, model, obs, seed, t)
    vl, tl = out['verb_logits'].cpu(), out['target_logits'].cpu()
    verb, target = out['verb'].cpu().long(), out['target'].cpu().long()

    # (1) the network: fp32 restatement, and the bf16 torch forward
    vz, val, tz = restated(model, obs.float().cpu(), verb)
    close(vl, vz, 'verb logits vs fp32')
    close(out['value'].cpu(), val, 'value vs fp32')
    close(tl, tz, 'target logits vs fp32')
    with torch.no_grad():
        tv, tt, tval = model(obs)
    rows = torch.arange(n)
    close(vl, tv.cpu(), 'verb logits vs torch bf16')
    close(out['value'].cpu(), tval.cpu(), 'value vs torch bf16')
    close(tl, tt.cpu()[rows, verb], 'target logits vs torch bf16')

    # (2) the standalone two-stage sampler on the kernel's own logits: bit for bit
    full = tt.clone()
    full[rows.cuda(), verb.cuda()] = out['target_logits']
    v2, t2, a2, lp2 = P.sample_ar(out['verb_logits'], full.contiguous(), seed, t)
    assert torch.equal(v2, out['verb']) and torch.equal(t2, out['target'])
    assert torch.equal(a2, out['action']) and torch.equal(lp2, out['logp'])

    # (3) the inverse CDF of the oracle's uniforms; log-probabilities from the kernel's logits
    key = [seed & 0xFFFFFFFF, seed >> 32]
    pick = np.unique(np.linspace(0, n - 1, min(n, 600)).astype(int))
    w = np.array([O.philox([0, t, int(i), 3], key)[:2] for i in pick], np.uint64)
    u = (w >> 8).astype(np.float64) / 16777216.0
    pv = torch.softmax(vl[pick].double(), 1).numpy()
    pt = torch.softmax(tl[pick].double(), 1).numpy()
    cv, ct = np.cumsum(pv, 1), np.cumsum(pt, 1)
    want_v = np.array([int(np.argmax(u[j, 0] < cv[j])) if (u[j, 0] < cv[j]).any() else 7 for j in range(len(pick))])
    want_t = np.array([int(np.argmax(u[j, 1] < ct[j])) if (u[j, 1] < ct[j]).any() else 24 for j in range(len(pick))])
    clear = (np.abs(cv - u[:, :1]).min(1) > 1e-5) & (np.abs(ct - u[:, 1:]).min(1) > 1e-5)
    assert clear.mean() > 0.9
    assert np.array_equal(verb.numpy()[pick][clear], want_v[clear])
    assert np.array_equal(target.numpy()[pick][clear], want_t[clear])
    lp = torch.log_softmax(vl.double(), 1)[rows, verb] + torch.log_softmax(tl.double(), 1)[rows, target]
    assert torch.allclose(out['logp'].cpu().double(), lp, rtol=1e-5, atol=1e-6)
    assert len(set(verb.tolist())) > 1 or n == 1


def test_fused_ar_device_counter_and_full_size():
    """C5's size (262,144 rows), the counter step read on the device (t_dev + t_add equal to
    the host step), and a batch of zero."""
    print('[ar fused] 262144', flush=True)
    P = importlib.import_module('dcss-auto_amd.policy')
    model = P.ARPolicy(seed=1).cuda().to(torch.bfloat16)
    n = 262144
    g = torch.Generator(device='cuda').manual_seed(3)
    obs = torch.randint(0, 2, (n, 1800), dtype=torch.uint8, device='cuda', generator=g)
    a = run_fused(P, model, obs, 11, 300)
    t_dev = torch.tensor([290], dtype=torch.int32, device='cuda')
    n_ = obs.shape[0]
    action, logp, value = (torch.empty(n_, dtype=torch.int64, device='cuda'), torch.empty(n_, device='cuda'),
                           torch.empty(n_, device='cuda'))
    P.policy_fwd_sample_ar(obs, model.packed(), 11, 10, action, logp, value, t_dev=t_dev)
    torch.cuda.synchronize()
    assert torch.equal(action, a['action']) and torch.equal(logp, a['logp']) and torch.equal(value, a['value'])
    rows = torch.arange(0, n, 509)
    vz, val, tz = restated(model, obs[rows].float().cpu(), a['verb'][rows].cpu().long())
    close(a['verb_logits'][rows].cpu(), vz, 'verb logits')
    close(a['target_logits'][rows].cpu(), tz, 'target logits')
    empty = torch.empty((0, 1800), dtype=torch.uint8, device='cuda')
    z = torch.empty(0, device='cuda')
    P.policy_fwd_sample_ar(empty, model.packed(), 11, 0, torch.empty(0, dtype=torch.int64, device='cuda'), z, z)
