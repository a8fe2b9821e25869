"""d1_ppo_step_static (the PPO minibatch step on the library's own per-GPU work buffer,
allocating nothing) against the existing entry points d1_ppo_prepare + d1_ppo_step on a
private work buffer: two calls in a row, the second with a smaller minibatch and buffer
while the static buffer still holds the first call's contents. Every output (fp32 masters,
bf16 copy, gradients, Adam moments and step, loss partials, cursor) must agree bit for
bit; a minibatch above the static limit is refused with D1_E_SCRATCH before any launch."""
import ctypes as C
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu


def _buffer(T, N, seed):
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    buf = ppo.RolloutBuffer(T, N)
    g = torch.Generator(device='cuda').manual_seed(seed)
    buf.obs.random_(0, 20, generator=g)
    buf.actions.random_(0, 16, generator=g)
    buf.logp.copy_(-torch.rand(T, N, device='cuda', generator=g) * 3)
    buf.values.normal_(generator=g)
    buf.rewards.copy_(torch.randn(T, N, device='cuda', generator=g) * (torch.rand(T, N, device='cuda', generator=g) < 0.1))
    buf.dones.copy_((torch.rand(T, N, device='cuda', generator=g) < 0.05).to(torch.uint8))
    buf.bootstrap.normal_(generator=g)
    return buf


def _outputs(fast):
    F = fast.flat
    return {'p': F.p, 'pb': F.pb, 'g': F.g, 'm': F.m, 'v': F.v, 'step': fast.step_t, 'loss_parts': fast.loss_parts,
            'cursor': fast.cursor[:1]}


def _pair(mb, state_from=None):
    P = importlib.import_module('dcss-auto_amd.policy')
    ppo = importlib.import_module('dcss-auto_amd.ppo')
    ref = ppo.FastPPO(P.Policy(seed=21).cuda(), minibatch=mb, graph=False)
    new = ppo.FastPPO(P.Policy(seed=21).cuda(), minibatch=mb, graph=False)
    if state_from is not None:   # continue from the previous call's parameters and Adam state
        for fast in (ref, new):
            for name in ('p', 'pb', 'm', 'v'):
                getattr(fast.flat, name).copy_(getattr(state_from.flat, name))
            fast.step_t.copy_(state_from.step_t)
    return ref, new


def _call_both(ref, new, buf, perm, cursor):
    _lib = importlib.import_module('dcss-auto_amd._lib')
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    adv, ret = ref.advantages(buf)
    obs, actions, logp = ref._views(buf)
    for fast in (ref, new):
        fast.set_order(perm)
        fast.cursor[0] = cursor
    ref._step(obs, actions, logp, adv, ret)           # d1_ppo_prepare (first use) + d1_ppo_step
    new._packed = True                               # build the struct without touching new.work ...
    args = new._struct(obs, actions, logp, adv, ret)
    args.work, args.work_bytes = None, 0             # ... and hand the static entry point no buffer
    print(f'[no-alloc] mb={new.minibatch} n={obs.shape[0]} cursor={cursor}', flush=True)
    _lib.check(lib.d1_ppo_step_static(C.byref(args), stream), 'd1_ppo_step_static')
    torch.cuda.synchronize()
    want, got = _outputs(ref), _outputs(new)
    for name in want:
        assert torch.equal(want[name], got[name]), (new.minibatch, name)
    assert ref.cursor[0].item() == cursor + 1


def test_static_step_matches_prepare_plus_step():
    torch.manual_seed(0)
    # call 1: the largest minibatch the static buffer takes
    ref1, new1 = _pair(8192)
    buf1 = _buffer(4, 4096, seed=5)
    perm1 = torch.randperm(4 * 4096, device='cuda', generator=torch.Generator(device='cuda').manual_seed(7))
    _call_both(ref1, new1, buf1, perm1, cursor=1)
    # call 2: smaller minibatch and buffer, continuing from call 1's state; the static buffer
    # still holds call 1's (larger) contents
    ref2, new2 = _pair(2048, state_from=ref1)
    buf2 = _buffer(2, 2048, seed=6)
    perm2 = torch.randperm(2 * 2048, device='cuda', generator=torch.Generator(device='cuda').manual_seed(8))
    _call_both(ref2, new2, buf2, perm2, cursor=1)


def test_static_step_refuses_oversize_minibatch():
    _lib = importlib.import_module('dcss-auto_amd._lib')
    args = _lib.D1PPOStep(mb=16384, n=32768)
    assert _lib.load().d1_ppo_step_static(C.byref(args), None) == -4   # D1_E_SCRATCH, nothing launched
    assert _lib.load().d1_ppo_step_static(None, None) == -1


def test_static_step_allocates_nothing_and_replays_from_a_graph():
    """After its first call on the device (made outside capture, as the header requires), a
    static call leaves the device's free memory unchanged, and static calls captured in a HIP
    graph replay equal to eager d1_ppo_prepare + d1_ppo_step calls, bit for bit, with eager
    torch work between the replays."""
    _lib = importlib.import_module('dcss-auto_amd._lib')
    lib = _lib.load()
    ref, new = _pair(4096)
    buf = _buffer(6, 4096, seed=9)   # six minibatches: two eager steps, then three replays
    perm = torch.randperm(6 * 4096, device='cuda', generator=torch.Generator(device='cuda').manual_seed(3))
    adv, ret = ref.advantages(buf)
    obs, actions, logp = ref._views(buf)
    for fast in (ref, new):
        fast.set_order(perm)
    new._packed = True
    args = new._struct(obs, actions, logp, adv, ret)
    args.work, args.work_bytes = None, 0
    print('[no-alloc] first static call (outside capture)', flush=True)
    ref._step(obs, actions, logp, adv, ret)
    _lib.check(lib.d1_ppo_step_static(C.byref(args), torch.cuda.current_stream().cuda_stream), 'static')
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    ref._step(obs, actions, logp, adv, ret)
    _lib.check(lib.d1_ppo_step_static(C.byref(args), torch.cuda.current_stream().cuda_stream), 'static')
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0, 'a static call changed the free device memory'
    want, got = _outputs(ref), _outputs(new)
    for name in want:
        assert torch.equal(want[name], got[name]), ('eager', name)
    print('[no-alloc] capture', flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.check(lib.d1_ppo_step_static(C.byref(args), torch.cuda.current_stream().cuda_stream), 'static')
    for r in range(3):
        ref._step(obs, actions, logp, adv, ret)
        g.replay()
        torch.cuda.synchronize()
        assert float(adv.abs().sum()) > 0   # eager reductions between the replays
        want, got = _outputs(ref), _outputs(new)
        for name in want:
            assert torch.equal(want[name], got[name]), ('replay', r, name)
