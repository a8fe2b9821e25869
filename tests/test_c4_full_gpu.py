"""C4 at its own size: the PPO update over a T=128 x N=65,536
rollout buffer (8,388,608 samples; 15.1 GB of uint8 observations) filled by 128 env steps of
65,536 generated-level worlds (8 monsters, uniform random actions; rewards and dones from the
env, synthetic values and old log-probabilities).

* GAE (HIP) against the fp32 restatement of the reference loop
  (gpu-d1/scripts/run_ring_ablations.py:354-360) on a 512-column slice: 1e-5.
* The first minibatch through FastPPO against bf16-autocast autograd on the same 8,192 rows
  of a shuffled order (almost all of them past byte 2^32 of the buffer): gradients within
  the bf16 bar (2e-2 of each gradient's scale).
* The kernel's loss terms against an fp64 recomputation from the head outputs the kernel
  itself computed (FastPPO.record_head): within 1e-5 of the sum of the terms' magnitudes,
  the fp32 bar of the reference's loss (train_clear.py:160-172); the head outputs against
  autograd's bf16 forward at the bf16 bar.
* Graph replays against eager steps over the first 32 minibatches: parameters, Adam step
  and cursor bit for bit.
* A whole update through the graph: 4 epochs x 1,024 minibatches = 4,096 Adam steps, the
  cursor back at 0 and run to 1,024 in every epoch, finite loss terms and parameters."""
import importlib

import pytest
import torch

from test_policy_gpu import gae_reference

pytestmark = pytest.mark.gpu

T, N, MB = 128, 65536, 8192


@pytest.fixture(scope='module')
def c4():
    pkg = importlib.import_module('dcss-auto_amd')
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    print('[c4] filling the 128 x 65,536 buffer', flush=True)
    buf = ppo.RolloutBuffer(T, N)
    env = pkg.Env(N, pkg.baseline_config(8), seed=41, hash=False)
    g = torch.Generator(device='cuda').manual_seed(41)
    actions = torch.empty(N, dtype=torch.int64, device='cuda')
    for t in range(T):
        actions.random_(0, 16, generator=g)
        buf.actions[t].copy_(actions)
        _, out = env.step(actions, obs=buf.obs[t])
        buf.rewards[t].copy_(out[:, 0])
        buf.dones[t].copy_((out[:, 1] > 0).to(torch.uint8))
    buf.logp.copy_(-torch.rand(T, N, device='cuda', generator=g) * 3)
    buf.values.normal_(generator=g)
    buf.bootstrap.normal_(generator=g)
    torch.cuda.synchronize()
    assert int(buf.dones.sum()) > 0 and float(buf.rewards.abs().sum()) > 0
    return pkg, P, ppo, buf


def test_gae_slice_matches_reference_loop(c4):
    _, P, _, buf = c4
    adv, ret = P.gae(buf.rewards, buf.dones, buf.values, buf.bootstrap)
    cols = slice(N - 512, N)
    ra, rr = gae_reference(buf.rewards[:, cols].cpu(), buf.dones[:, cols].float().cpu(), buf.values[:, cols].cpu(),
                           buf.bootstrap[cols].cpu())
    torch.testing.assert_close(adv[:, cols].cpu(), ra, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ret[:, cols].cpu(), rr, rtol=1e-5, atol=1e-6)


def test_first_minibatch_gradients_and_loss_terms(c4):
    _, P, ppo, buf = c4
    model = P.Policy(seed=12).cuda()
    ref = P.Policy(seed=12).cuda()
    fast = ppo.FastPPO(model, minibatch=MB, graph=False)
    fast.record_head()
    adv, ret = fast.advantages(buf)
    obs, actions, logp = fast._views(buf)
    perm = torch.randperm(T * N, device='cuda', generator=torch.Generator(device='cuda').manual_seed(5))
    rows = perm[:MB]
    assert int((rows >= (1 << 32) // 1800).sum()) > MB // 2   # offsets past 2^32 bytes in the gather
    fast.set_order(perm)
    fast._step(obs, actions, logp, adv, ret)
    torch.cuda.synchronize()
    assert fast.cursor[0].item() == 1

    # gradients vs bf16 autocast autograd on the same rows
    ref.zero_grad(set_to_none=True)
    with torch.autocast('cuda', dtype=torch.bfloat16):
        logits, value = ref(obs[rows])
    loss, *_ = ppo.ppo_loss(logits, value, actions[rows], logp[rows], adv[rows], ret[rows])
    loss.backward()
    for name, prm in ref.named_parameters():
        gk = fast.flat.view(fast.flat.g, name).float()
        scale = prm.grad.abs().max().item() + 1e-12
        err = (gk - prm.grad).abs().max().item() / scale
        assert err < 2e-2, (name, err)

    # loss terms vs fp64 from the kernel's own head outputs
    z = fast.head_out.double()
    assert torch.isfinite(z).all()
    lsm = torch.log_softmax(z[:, :16], 1)
    a = actions[rows]
    lpa = lsm.gather(1, a[:, None])[:, 0]
    ratio = torch.exp(lpa - logp[rows].double())
    A = adv[rows].double()
    pg = -torch.minimum(ratio * A, ratio.clamp(1 - fast.clip, 1 + fast.clip) * A)
    vl = 0.5 * (z[:, 16] - ret[rows].double()) ** 2
    ent = -(lsm.exp() * lsm).sum(1)
    want = torch.stack([pg.sum(), vl.sum(), ent.sum()])
    scale = torch.stack([pg.abs().sum(), vl.abs().sum(), ent.abs().sum()])   # the surrogate sum can cancel
    got = fast.loss_parts.view(-1, 4)[:, :3].double().sum(0)
    assert ((got - want).abs() <= 1e-5 * scale + 1e-6).all(), (got.tolist(), want.tolist())
    # and the head outputs themselves vs autograd's bf16 forward on the same rows
    zr = torch.cat([logits.float(), value.float()[:, None]], 1).double()
    assert (z - zr).abs().max().item() <= 2e-2 * (zr.abs().max().item() + 1e-6)


def test_graph_matches_eager_then_full_update(c4):
    _, P, ppo, buf = c4
    eager = ppo.FastPPO(P.Policy(seed=13).cuda(), minibatch=MB, graph=False)
    graphed = ppo.FastPPO(P.Policy(seed=13).cuda(), minibatch=MB, graph=True, graph_steps=16)
    graphed._capture(buf)
    adv, ret = eager.advantages(buf)
    graphed._adv.copy_(adv)
    graphed._ret.copy_(ret)
    obs, actions, logp = eager._views(buf)
    perm = torch.randperm(T * N, device='cuda', generator=torch.Generator(device='cuda').manual_seed(6))
    eager.set_order(perm)
    graphed.set_order(perm)
    for r in range(2):
        for _ in range(16):
            eager._step(obs, actions, logp, adv, ret)
        graphed._g.replay()
        torch.cuda.synchronize()
        assert torch.equal(eager.flat.p, graphed.flat.p), f'replay {r}'
        assert torch.equal(eager.step_t, graphed.step_t) and torch.equal(eager.cursor[:1], graphed.cursor[:1])
    assert graphed.cursor[0].item() == 32 and graphed.step_t[0].item() == 32

    # a whole update on a fresh trainer: 4 epochs x 1,024 minibatches through the graph
    print('[c4] full update', flush=True)
    fast = ppo.FastPPO(P.Policy(seed=14).cuda(), minibatch=MB, graph=True, graph_steps=16)
    p0 = fast.flat.p.clone()
    cursors = []
    orig = fast.set_order

    def spy(perm_):
        if fast._g is not None and fast.perm is not None:
            cursors.append(fast.cursor[0].item())
        orig(perm_)
    fast.set_order = spy
    terms = fast.update(buf, generator=torch.Generator(device='cuda').manual_seed(7))
    torch.cuda.synchronize()
    cursors.append(fast.cursor[0].item())
    assert fast.step_t[0].item() == 4 * (T * N // MB) == 4096
    assert cursors[-4:] == [T * N // MB] * 4, cursors
    assert fast.nonfinite_steps() == 0
    assert torch.isfinite(terms).all() and torch.isfinite(fast.flat.p).all()
    assert not torch.equal(fast.flat.p, p0)
