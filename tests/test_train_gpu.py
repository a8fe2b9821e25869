"""The training loop (dcss-auto_amd/train.py): graph-captured rollouts equal eager ones,
a resumed run equals the uninterrupted run bit for bit (the reference's
gpu-d1/scripts/test_resume.py checks the same of its trainer), also when the worker loop is
stopped by SIGTERM, a non-finite loss stops the update with the last finite weights,
evaluation ends every episode, and the device-counter sampler equals the host-counter one."""
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


def make_trainer(pkg, graph, n=2048, T=8, seed=11):
    train = importlib.import_module('dcss-auto_amd.train')
    P = importlib.import_module('dcss-auto_amd.policy')
    env = pkg.Env(n, pkg.baseline_config(8), seed=seed, hash=False)
    model = P.Policy(seed=2).cuda()
    return train.Trainer(env, model, horizon=T, minibatch=8192, epochs=2, graph=graph)


def assert_same_state(a, b):
    assert a.keys() == b.keys()
    for key in a:
        if key in ('hparams', 'format'):
            assert a[key] == b[key]
        else:
            assert torch.equal(a[key], b[key]), key


def test_sample_dev_matches_sample():
    P = importlib.import_module('dcss-auto_amd.policy')
    print('[train] sample_dev', flush=True)
    g = torch.Generator().manual_seed(3)
    logits = (torch.randn(5000, 16, generator=g) * 2).cuda()
    a1, l1 = P.sample(logits, 99, 12)
    t_dev = torch.tensor([5], dtype=torch.int32, device='cuda')
    a2 = torch.empty_like(a1)
    l2 = torch.empty_like(l1)
    P.sample_dev(logits, 99, t_dev, 7, a2, l2)
    assert torch.equal(a1, a2) and torch.equal(l1, l2)
    # a counter near 2^32 wraps as uint32 on both paths
    a3, l3 = P.sample(logits, 99, 2)
    t_dev.fill_(-1)
    P.sample_dev(logits, 99, t_dev, 3, a2, l2)
    assert torch.equal(a3, a2) and torch.equal(l3, l2)


def _buffers(tr):
    b = tr.buf
    return [b.obs, b.actions, b.logp, b.values, b.rewards, b.dones, b.bootstrap, tr.next_obs, tr.env.state, tr.t_dev]


def test_graph_rollout_matches_eager(pkg):
    """Three rollout+update rounds: the graph-replayed rollout equals eager launches bit for
    bit every round, with eager torch work (GAE reductions, the PPO update) in between."""
    print('[train] graph vs eager', flush=True)
    eager = make_trainer(pkg, graph=False)
    graph = make_trainer(pkg, graph=True)
    for r in range(3):
        eager.rollout()
        graph.rollout()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(_buffers(eager), _buffers(graph))):
            assert torch.equal(a, b), f'round {r}: buffer {i} differs'
        eager.update()
        graph.update()
    assert torch.equal(eager.ppo.flat.p, graph.ppo.flat.p)
    assert eager.buf.dones.sum() > 0 or eager.buf.rewards.abs().sum() > 0


def test_resume_is_bit_exact(pkg, tmp_path):
    """4 updates uninterrupted == 2 updates, save, a fresh trainer (other env seed) that
    loads the checkpoint, 2 more updates: weights, Adam state, live worlds, observations,
    counters and the shuffle generator all equal."""
    print('[train] resume', flush=True)
    full = make_trainer(pkg, graph=True)
    full.train(4)
    half = make_trainer(pkg, graph=True)
    half.train(2)
    half.save(tmp_path / 'ckpt.pt')
    resumed = make_trainer(pkg, graph=True, seed=12345)
    resumed.load(tmp_path / 'ckpt.pt')
    resumed.train(2)
    torch.cuda.synchronize()
    a, b = full.state_dict(), resumed.state_dict()
    assert_same_state(a, b)
    assert int(a['updates']) == 4 and int(a['decisions']) == 4 * 8 * 2048
    # the weights moved, and sync_model writes them into the module
    model = resumed.sync_model()
    assert torch.equal(model.l1.weight.detach().reshape(-1), resumed.ppo.flat.view(resumed.ppo.flat.p, 'l1.weight').reshape(-1))


def test_load_into_a_trained_graph_trainer(pkg, tmp_path):
    """A graph-mode trainer that has already trained (its PPO graph captured, its packed
    weight copies current) loads another run's checkpoint: the next updates equal those of
    a fresh trainer resumed from the same checkpoint, bit for bit (the captured PPO graph
    must not step on the pre-load weights)."""
    print('[train] load into a trained trainer', flush=True)
    src = make_trainer(pkg, graph=True)
    src.train(2)
    src.save(tmp_path / 'ckpt.pt')
    busy = make_trainer(pkg, graph=True, seed=999)
    busy.model.l1.weight.data.mul_(0.5)            # a different run: other weights, other worlds
    busy.ppo.flat.p.mul_(0.5)
    busy.ppo.flat.pb.copy_(busy.ppo.flat.p)
    busy.ppo._packed = False
    busy._repack()
    busy.train(2)                                   # captures both graphs on the other weights
    busy.load(tmp_path / 'ckpt.pt')
    busy.train(2)
    fresh = make_trainer(pkg, graph=True, seed=4321)
    fresh.load(tmp_path / 'ckpt.pt')
    fresh.train(2)
    torch.cuda.synchronize()
    assert_same_state(fresh.state_dict(), busy.state_dict())


def test_checkpoint_refuses_other_settings(pkg, tmp_path):
    """A checkpoint records the trainer settings that decide the next update (sampler seed,
    horizon, batch, minibatch, epochs, optimiser and loss coefficients); loading it into a
    trainer built with other settings raises instead of silently diverging."""
    print('[train] checkpoint settings', flush=True)
    train = importlib.import_module('dcss-auto_amd.train')
    P = importlib.import_module('dcss-auto_amd.policy')
    src = make_trainer(pkg, graph=False)
    src.save(tmp_path / 'ckpt.pt')
    env = pkg.Env(2048, pkg.baseline_config(8), seed=11, hash=False)
    other = train.Trainer(env, P.Policy(seed=2).cuda(), horizon=8, minibatch=8192, epochs=2, graph=False, lr=1e-3)
    with pytest.raises(ValueError, match='lr'):
        other.load(tmp_path / 'ckpt.pt')
    reseeded = train.Trainer(env, P.Policy(seed=2).cuda(), horizon=8, minibatch=8192, epochs=2, graph=False, seed=8)
    with pytest.raises(ValueError, match='seed'):
        reseeded.load(tmp_path / 'ckpt.pt')


def test_evaluation_ends_every_episode(pkg):
    print('[train] evaluation', flush=True)
    tr = make_trainer(pkg, graph=False, n=1024)
    ev = pkg.Env(256, pkg.baseline_config(8), seed=5, hash=False)
    for mode in ('greedy', 'sampled'):
        m = tr.evaluate(ev, mode)
        print(f'[train] {mode}: {m}', flush=True)
        assert 0.0 <= m['clear_rate'] <= 1.0 and 0.0 <= m['death_rate'] <= 1.0 and 0.0 <= m['timeout_rate'] <= 1.0
        assert abs(m['clear_rate'] + m['death_rate'] + m['timeout_rate'] - 1.0) < 1e-6   # every episode ended one way
        assert m['turns'] >= 1
    # the same evaluation twice gives the same numbers (reset + counter RNG)
    assert tr.evaluate(ev, 'sampled') == tr.evaluate(ev, 'sampled')


def test_non_finite_loss_leaves_the_last_finite_weights(pkg):
    """A NaN reward makes every advantage NaN: FastPPO skips every minibatch step, keeps the
    weights, moments, Adam step and packed copies of the last finite update, and update
    raises as the reference's loop does; after clear_nonfinite training goes on."""
    print('[train] non-finite loss', flush=True)
    tr = make_trainer(pkg, graph=True)
    tr.rollout()
    tr.update()
    F = tr.ppo.flat
    keep = [F.p.clone(), F.pb.clone(), F.m.clone(), F.v.clone(), tr.ppo.step_t[:1].clone(), tr.wpk.clone()]
    tr.rollout()
    tr.buf.rewards[3, 17] = float('nan')
    with pytest.raises(RuntimeError, match='Non-finite'):
        tr.update()
    steps = 2 * (8 * 2048 // 8192)
    assert tr.ppo.nonfinite_steps() == steps
    for i, (a, b) in enumerate(zip(keep, [F.p, F.pb, F.m, F.v, tr.ppo.step_t[:1], tr.wpk])):
        assert torch.equal(a, b), i
    tr.ppo.clear_nonfinite()
    tr.rollout()
    tr.update()
    assert tr.ppo.nonfinite_steps() == 0 and not torch.equal(F.p, keep[0]) and bool(torch.isfinite(F.p).all())
    assert float(tr.ppo.step_t[0]) == float(keep[4][0]) + steps


def test_autograd_ppo_raises_on_a_non_finite_loss():
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo_mod = importlib.import_module('dcss-auto_amd.ppo')
    model = P.Policy(seed=3).cuda()
    ppo = ppo_mod.PPO(model)
    obs = torch.randint(0, 40, (64, 1800), dtype=torch.uint8, device='cuda')
    act = torch.randint(0, 16, (64,), device='cuda')
    logp = torch.full((64,), -2.77, device='cuda')
    adv = torch.randn(64, device='cuda')
    adv[5] = float('inf')
    before = model.l1.weight.detach().clone()
    with pytest.raises(RuntimeError, match='Non-finite'):
        ppo.minibatch_step(obs, act, logp, adv, torch.zeros(64, device='cuda'))
    assert torch.equal(model.l1.weight, before)


def test_worker_loop_stop_and_resume_is_bit_exact(pkg, tmp_path):
    """run() to 4 updates == run() stopped by SIGTERM after update 2 (status 130), then the
    same call on a fresh trainer (other env seed), which resumes from the checkpoint."""
    import os
    import signal
    print('[train] worker loop stop/resume', flush=True)
    target = 4 * 8 * 2048
    full = make_trainer(pkg, graph=True)
    assert full.run(target, handle_signals=False) == 0
    ck = tmp_path / 'latest.pt'
    first = make_trainer(pkg, graph=True)

    def hook(t, terms):
        if t.updates == 2:
            os.kill(os.getpid(), signal.SIGTERM)

    assert first.run(target, checkpoint=ck, on_update=hook) == 130
    resumed = make_trainer(pkg, graph=True, seed=12345)
    assert resumed.run(target, checkpoint=ck) == 0
    torch.cuda.synchronize()
    assert_same_state(full.state_dict(), resumed.state_dict())
