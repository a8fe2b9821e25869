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


def reference_loss(logits, values, actions, old_logp, adv, ret, clip=0.2):
    """The reference's loss expression (gpu-d1/scripts/run_ring_ablations.py:365-367) with
    C4's coefficients (value 0.5 x 0.5*MSE = the reference's .25*MSE, entropy 0.01)."""
    from torch.distributions import Categorical
    dist = Categorical(logits=logits)
    ratio = (dist.log_prob(actions) - old_logp).exp()
    pg = -torch.minimum(ratio * adv, ratio.clamp(1 - clip, 1 + clip) * adv).mean()
    return pg + .25 * (values - ret).square().mean() - 0.01 * dist.entropy().mean()


def _fwd_reference(obs, w1, b1, w2, b2, w3, b3, round_hidden=True):
    """fp32 restatement of the bf16 forward: fp32 products and sums, each layer's output
    rounded to bf16 where the bf16 torch forward rounds it (round_hidden=False: pure fp32)."""
    r = (lambda x: x.to(torch.bfloat16).float()) if round_hidden else (lambda x: x)
    h = r(torch.relu(obs.float() @ w1.float().T + b1.float()))
    h = r(torch.relu(h @ w2.float().T + b2.float()))
    return r(h @ w3.float().T + b3.float())


@pytest.mark.parametrize('M', [1, 255, 1000, 4096 + 37])
def test_policy_fwd_matches_fp32_reference(M):
    """The fused uint8 -> MFMA forward (three layers, one launch) vs the fp32 restatement
    with random weights AND biases of a scale where a misplaced bias, a permuted hidden unit
    or a transposed weight moves the output by far more than the tolerance: within 2e-2 of
    the output scale against pure fp32, and within 1e-2 against the restatement that
    rounds h1/h2/out to bf16 like the kernel; also against torch's own bf16 GEMM chain."""
    P = importlib.import_module('dcss-auto_amd.policy')
    print(f'[policy_fwd] M={M}', flush=True)
    g = torch.Generator().manual_seed(M)
    obs = torch.randint(0, 60, (M, 1800), dtype=torch.uint8, generator=g).cuda()
    w1 = (torch.randn(256, 1800, generator=g) * 0.02).to(torch.bfloat16).cuda()
    b1 = (torch.randn(256, generator=g) * 5).to(torch.bfloat16).cuda()
    w2 = (torch.randn(256, 256, generator=g) * 0.1).to(torch.bfloat16).cuda()
    b2 = (torch.randn(256, generator=g) * 5).to(torch.bfloat16).cuda()
    w3 = (torch.randn(17, 256, generator=g) * 0.1).to(torch.bfloat16).cuda()
    b3 = (torch.randn(17, generator=g) * 5).to(torch.bfloat16).cuda()
    wpk = P.pack_weights(w1, w2, w3)
    logits, value = P.policy_fwd(obs, wpk, b1, b2, b3)
    out = torch.cat([logits, value[:, None]], 1)
    exact = _fwd_reference(obs, w1, b1, w2, b2, w3, b3, round_hidden=False)
    scale = exact.abs().max().clamp_min(1e-3)
    assert ((out - exact).abs().max() / scale).item() < 2e-2
    emul = _fwd_reference(obs, w1, b1, w2, b2, w3, b3)
    assert ((out - emul).abs().max() / scale).item() < 1e-2
    with torch.no_grad():
        h = torch.relu(torch.addmm(b1, obs.to(torch.bfloat16), w1.T))
        h = torch.relu(torch.addmm(b2, h, w2.T))
        tb = torch.addmm(b3, h, w3.T).float()
    assert ((out - tb).abs().max() / scale).item() < 2e-2
    # a different batch size sees the same per-sample outputs (no cross-sample leakage)
    if M > 1:
        l2_, v2_ = P.policy_fwd(obs[: M // 2], wpk, b1, b2, b3)
        assert torch.equal(l2_, logits[: M // 2]) and torch.equal(v2_, value[: M // 2])


def test_policy_module_uses_fused_forward_and_repacks():
    """Policy.forward (bf16, no grad, uint8) runs the fused kernel, and a weight update
    through copy_ is picked up by the packed-weight cache."""
    P = importlib.import_module('dcss-auto_amd.policy')
    model = P.Policy(seed=4).cuda().to(torch.bfloat16)
    obs = torch.randint(0, 30, (777, 15, 15, 8), dtype=torch.uint8, device='cuda')
    with torch.no_grad():
        logits, value = model(obs)
        wpk = model.packed()[0]
        ref = _fwd_reference(obs.reshape(777, -1), model.l1.weight, model.l1.bias, model.l2.weight, model.l2.bias,
                             model.head.weight, model.head.bias)
        scale = ref.abs().max().clamp_min(1e-3)
        assert ((torch.cat([logits, value[:, None]], 1) - ref).abs().max() / scale).item() < 1e-2
        model.l2.bias.copy_(torch.randn(256, device='cuda').to(torch.bfloat16))
        logits2, value2 = model(obs)
        assert model.packed()[0] is not wpk
        ref = _fwd_reference(obs.reshape(777, -1), model.l1.weight, model.l1.bias, model.l2.weight, model.l2.bias,
                             model.head.weight, model.head.bias)
        scale = ref.abs().max().clamp_min(1e-3)
        assert ((torch.cat([logits2, value2[:, None]], 1) - ref).abs().max() / scale).item() < 1e-2


def test_ppo_loss_matches_reference_fp32():
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    g = torch.Generator().manual_seed(5)
    n = 8192
    logits = torch.randn(n, 16, generator=g) * 3
    values = torch.randn(n, generator=g)
    actions = torch.randint(0, 16, (n,), generator=g)
    old = torch.log_softmax(logits + 0.3 * torch.randn(n, 16, generator=g), 1).gather(1, actions[:, None]).squeeze(1)
    adv = torch.randn(n, generator=g)
    ret = torch.randn(n, generator=g)
    want = reference_loss(logits.double(), values.double(), actions, old.double(), adv.double(), ret.double())
    got, *_ = ppo.ppo_loss(logits.cuda(), values.cuda(), actions.cuda(), old.cuda(), adv.cuda(), ret.cuda())
    torch.testing.assert_close(got.double().cpu(), want, rtol=1e-5, atol=1e-6)


def test_ppo_update_runs_and_improves_surrogate():
    """One bf16-autocast PPO update on a small buffer: finite, weights move, the clipped
    objective on the same data goes down."""
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    torch.manual_seed(0)
    T, N = 8, 2048
    buf = ppo.RolloutBuffer(T, N)
    buf.obs.random_(0, 20)
    model = P.Policy(seed=1).cuda()
    with torch.no_grad():
        logits, v = model(buf.obs.view(T * N, -1).to(torch.float32))
    buf.actions.copy_(torch.randint(0, 16, (T, N), device='cuda'))
    buf.logp.copy_(torch.log_softmax(logits, 1).gather(1, buf.actions.view(-1, 1)).view(T, N))
    buf.values.copy_(v.view(T, N))
    buf.rewards.copy_(torch.where(torch.rand(T, N, device='cuda') < 0.5, 1.0, -1.0) * (buf.actions == 3))
    trainer = ppo.PPO(model, epochs=2, minibatch=4096)
    before = [p.detach().clone() for p in model.parameters()]
    loss = trainer.update(buf)
    assert torch.isfinite(loss)
    assert any(not torch.equal(a, b) for a, b in zip(before, model.parameters()))


def _small_buffer(T, N, seed=3):
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    buf = ppo.RolloutBuffer(T, N)
    torch.manual_seed(seed)
    buf.obs.random_(0, 20)
    buf.actions.random_(0, 16)
    buf.logp.copy_(-torch.rand(T, N, device='cuda') * 3)
    buf.values.normal_()
    buf.rewards.copy_(torch.randn(T, N, device='cuda') * (torch.rand(T, N, device='cuda') < 0.1))
    buf.dones.copy_((torch.rand(T, N, device='cuda') < 0.05).to(torch.uint8))
    buf.bootstrap.normal_()
    return buf


def _autograd_grads(model, ppo, obs, actions, logp, adv, ret, inds):
    model.zero_grad(set_to_none=True)
    with torch.autocast('cuda', dtype=torch.bfloat16):
        logits, value = model(obs[inds])
    loss, pg, vl, ent = ppo.ppo_loss(logits, value, actions[inds], logp[inds], adv[inds], ret[inds])
    loss.backward()
    return torch.stack([pg, vl, ent]).float()


@pytest.mark.parametrize('mb', [1024, 4096, 8192])
def test_fast_ppo_gradients_match_autograd(mb):
    """The fused minibatch step (libd1hip d1_ppo_step) vs torch autograd under bf16 autocast
    on the same minibatch, taken through a shuffled order: gradients within the bf16 bar
    (2e-2 relative to the gradient scale), loss terms within 2e-2; the Adam step from zero
    moments (no clipping) moves every weight by lr * g / (|g| + eps), checked to 1e-6. A
    second step, after the model takes the updated weights, checks the weight copies the
    step keeps for its own next call the same way. Minibatches of 1,024, 4,096 and 8,192
    samples give the weight-gradient kernels 1, 4 and 8 sample splits (4, 16 and 32 for dW3)."""
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    T, N = 4, 4096
    buf = _small_buffer(T, N)
    model = P.Policy(seed=4).cuda()
    fast = ppo.FastPPO(model, minibatch=mb, graph=False, max_grad_norm=1e9)
    p0 = fast.flat.p.clone()
    adv, ret = fast.advantages(buf)
    obs, actions, logp = fast._views(buf)
    perm = torch.randperm(T * N, device='cuda', generator=torch.Generator(device='cuda').manual_seed(1))
    fast.set_order(perm)
    for step in range(2):
        fast._step(obs, actions, logp, adv, ret)
        assert fast.cursor[0].item() == step + 1
        want = _autograd_grads(model, ppo, obs, actions, logp, adv, ret, perm[step * mb:(step + 1) * mb])
        torch.testing.assert_close(fast.loss_terms(), want, rtol=2e-2, atol=1e-4)
        for name, prm in model.named_parameters():
            g = fast.flat.view(fast.flat.g, name).float()
            scale = prm.grad.abs().max().item() + 1e-12
            err = (g - prm.grad).abs().max().item() / scale
            assert err < 2e-2, (step, name, err)
        if step == 0:
            g = fast.flat.g.float()
            torch.testing.assert_close(fast.flat.p, p0 - fast.lr * g / (g.abs() + fast.eps), rtol=0, atol=1e-6)
            fast.flat.load_into(model)


def test_fast_ppo_graph_replays_match_eager():
    """A graph of two minibatch steps vs eager steps over two epochs, with eager torch
    reductions between replays: parameters, step count and cursor agree bit for bit after
    every replay; a replay past the end of the order changes nothing."""
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    T, N, mb = 4, 4096, 4096
    n = T * N
    buf = _small_buffer(T, N)
    eager = ppo.FastPPO(P.Policy(seed=2).cuda(), minibatch=mb, graph=False)
    graphed = ppo.FastPPO(P.Policy(seed=2).cuda(), minibatch=mb, graph=True, graph_steps=2)
    graphed._capture(buf)
    adv, ret = eager.advantages(buf)
    graphed._adv.copy_(adv)
    graphed._ret.copy_(ret)
    obs, actions, logp = eager._views(buf)
    for epoch in range(2):
        perm = torch.randperm(n, device='cuda')
        eager.set_order(perm)
        graphed.set_order(perm)
        for r in range(2):
            eager._step(obs, actions, logp, adv, ret)
            eager._step(obs, actions, logp, adv, ret)
            graphed._g.replay()
            torch.cuda.synchronize()
            _ = torch.randn(1000, device='cuda').sum().item()      # eager reductions between replays
            assert torch.equal(eager.flat.p, graphed.flat.p), f'epoch {epoch} replay {r}'
            assert torch.equal(eager.step_t, graphed.step_t)
            assert torch.equal(eager.cursor[:1], graphed.cursor[:1])
    assert graphed.cursor[0].item() == n // mb
    # past the end: the kernels still load their operands (only their stores wait for the
    # cursor check), and no output or state changes
    F = graphed.flat
    before = [x.clone() for x in (F.p, F.pb, F.g, F.m, F.v, graphed.step_t, graphed.loss_parts)]
    graphed._g.replay()
    torch.cuda.synchronize()
    after = (F.p, F.pb, F.g, F.m, F.v, graphed.step_t, graphed.loss_parts)
    for name, x, y in zip(('p', 'pb', 'g', 'm', 'v', 'step', 'loss_parts'), before, after):
        assert torch.equal(x, y), name
    assert graphed.cursor[0].item() == n // mb


def test_fast_ppo_update_tracks_autograd_ppo():
    """A whole update (GAE, 2 epochs x 4 minibatches, same shuffles) through FastPPO and
    through the autograd PPO: every parameter moves the same way (cosine of the two
    parameter deltas > 0.9) and the loss terms stay finite."""
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    T, N, mb = 4, 4096, 4096
    buf = _small_buffer(T, N, seed=7)
    ref_model = P.Policy(seed=6).cuda()
    p0 = {k: v.detach().clone() for k, v in ref_model.named_parameters()}
    fast = ppo.FastPPO(P.Policy(seed=6).cuda(), minibatch=mb, epochs=2)
    ref = ppo.PPO(ref_model, minibatch=mb, epochs=2)
    fast_terms = fast.update(buf, generator=torch.Generator(device='cuda').manual_seed(11))
    ref.update(buf, generator=torch.Generator(device='cuda').manual_seed(11))
    for name, prm in ref_model.named_parameters():
        d_ref = (prm.detach() - p0[name]).flatten()
        d_fast = (fast.flat.view(fast.flat.p, name) - p0[name]).flatten()
        cos = torch.nn.functional.cosine_similarity(d_ref, d_fast, dim=0).item()
        assert cos > 0.9, (name, cos)
    assert torch.isfinite(fast_terms).all()


@pytest.mark.parametrize('M', [1, 255, 4133])
def test_fused_sample_matches_forward_then_sampler(M):
    """d1_policy_fwd_sample == d1_policy_fwd followed by d1_sample / d1_sample_dev, bit for
    bit (actions, log-probabilities, value and logits), at a host step and a device step."""
    P = importlib.import_module('dcss-auto_amd.policy')
    print(f'[fused sample] M={M}', flush=True)
    model = P.Policy(seed=8).cuda().to(torch.bfloat16)
    with torch.no_grad():
        for layer in (model.l1, model.l2, model.head):
            layer.bias.copy_(torch.randn(layer.bias.shape) * 3)   # logits of varied scale
    wpk, b1, b2, b3 = model.packed()
    obs = torch.randint(0, 60, (M, 1800), dtype=torch.uint8, device='cuda')
    logits, value = P.policy_fwd(obs, wpk, b1, b2, b3)
    a_ref, lp_ref = P.sample(logits, 1234, 77)
    a = torch.empty(M, dtype=torch.int64, device='cuda')
    lp = torch.empty(M, device='cuda')
    v = torch.empty(M, device='cuda')
    lg = torch.empty(M, 16, device='cuda')
    P.policy_fwd_sample(obs, wpk, b1, b2, b3, 1234, 77, a, lp, v, logits=lg)
    assert torch.equal(a, a_ref) and torch.equal(lp, lp_ref) and torch.equal(v, value) and torch.equal(lg, logits)
    t_dev = torch.tensor([70], dtype=torch.int32, device='cuda')
    P.policy_fwd_sample(obs, wpk, b1, b2, b3, 1234, 7, a, lp, v, t_dev=t_dev)   # logits not written
    assert torch.equal(a, a_ref) and torch.equal(lp, lp_ref)
    if M >= 100:   # the rows do not all draw one action
        assert len(torch.unique(a_ref)) > 4
