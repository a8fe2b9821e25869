"""PPO update over a resident rollout buffer.

Follows the reference's update (gpu-d1/scripts/run_ring_ablations.py:354-372;
gpu-d1/scripts/train_clear.py:149-172): reverse-time GAE, advantages normalised over
the whole buffer (unbiased std + 1e-8), then `epochs` passes of shuffled minibatches
with the clipped surrogate, a value loss and an entropy bonus, gradient-norm clipping
at 0.5 and Adam (lr 3e-4, eps 1e-5). C4's coefficients are clip 0.2, value 0.5 x
(0.5 * MSE) — the reference's 0.25 * MSE — and entropy 0.01. The trunk runs under bf16
autocast while the optimizer keeps fp32 master weights; GAE is the HIP kernel.
"""
import torch

from . import policy as P

OBS = P.OBS


class RolloutBuffer:
    """[T, N] rollout storage; observations stay uint8 (15.1 GB at T=128, N=65,536)."""

    def __init__(self, T, N, device='cuda', obs_bytes=OBS):
        self.T, self.N = T, N
        self.obs = torch.empty((T, N, obs_bytes), dtype=torch.uint8, device=device)
        self.actions = torch.zeros((T, N), dtype=torch.int64, device=device)
        self.logp = torch.zeros((T, N), dtype=torch.float32, device=device)
        self.values = torch.zeros((T, N), dtype=torch.float32, device=device)
        self.rewards = torch.zeros((T, N), dtype=torch.float32, device=device)
        self.dones = torch.zeros((T, N), dtype=torch.uint8, device=device)
        self.bootstrap = torch.zeros(N, dtype=torch.float32, device=device)


def ppo_loss(logits, values, actions, old_logp, adv, returns, clip=0.2, vcoef=0.5, ecoef=0.01):
    """Clipped surrogate + vcoef * 0.5*MSE - ecoef * entropy, in fp32 (logits upcast)."""
    logp_all = torch.log_softmax(logits.float(), -1)
    logp = logp_all.gather(1, actions[:, None]).squeeze(1)
    ratio = torch.exp(logp - old_logp)
    pg = -torch.minimum(ratio * adv, ratio.clamp(1 - clip, 1 + clip) * adv).mean()
    vloss = 0.5 * (values.float() - returns).square().mean()
    entropy = -(logp_all.exp() * logp_all).sum(-1).mean()
    return pg + vcoef * vloss - ecoef * entropy, pg.detach(), vloss.detach(), entropy.detach()


class PPO:
    def __init__(self, model, lr=3e-4, eps=1e-5, clip=0.2, vcoef=0.5, ecoef=0.01, max_grad_norm=0.5,
                 epochs=4, minibatch=8192, gamma=0.99, lam=0.95, autocast=True):
        self.model = model
        self.opt = torch.optim.Adam(model.parameters(), lr=lr, eps=eps, fused=True)
        self.clip, self.vcoef, self.ecoef, self.max_grad_norm = clip, vcoef, ecoef, max_grad_norm
        self.epochs, self.minibatch, self.gamma, self.lam, self.autocast = epochs, minibatch, gamma, lam, autocast

    def advantages(self, buf):
        adv, ret = P.gae(buf.rewards, buf.dones, buf.values, buf.bootstrap, self.gamma, self.lam)
        flat = adv.flatten()
        return (flat - flat.mean()) / (flat.std() + 1e-8), ret.flatten()

    def minibatch_step(self, obs, actions, old_logp, adv, ret):
        with torch.autocast('cuda', dtype=torch.bfloat16, enabled=self.autocast):
            logits, value = self.model(obs)
        loss, pg, vl, ent = ppo_loss(logits, value, actions, old_logp, adv, ret, self.clip, self.vcoef, self.ecoef)
        if not torch.isfinite(loss).item():   # as the reference's update loop (run_ring_ablations.py:369-370)
            raise RuntimeError('Non-finite PPO loss')
        self.opt.zero_grad(set_to_none=True)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(self.model.parameters(), self.max_grad_norm)
        self.opt.step()
        return loss.detach()

    def update(self, buf, generator=None):
        adv, ret = self.advantages(buf)
        n = buf.T * buf.N
        obs = buf.obs.view(n, -1)
        actions, logp = buf.actions.flatten(), buf.logp.flatten()
        last = None
        for _ in range(self.epochs):
            perm = torch.randperm(n, device=obs.device, generator=generator)
            for inds in perm.split(self.minibatch):
                last = self.minibatch_step(obs.index_select(0, inds), actions[inds], logp[inds], adv[inds],
                                           ret[inds])
        return last


# ----------------------------------------------------------------------------------------
# Graph-safe PPO: one libd1hip call (d1_ppo_step) per minibatch over flat parameter buffers.
# The step picks its minibatch from a device-side cursor, so a HIP graph holding several
# calls walks consecutive minibatches of the epoch's sample order.

_PARAMS = (('l1.weight', (256, 1800)), ('l1.bias', (256,)), ('l2.weight', (256, 256)), ('l2.bias', (256,)),
           ('head.weight', (17, 256)), ('head.bias', (17,)))


class FlatParams:
    """fp32 master weights, their bf16 copy, bf16 gradients and Adam moments, each one
    flat buffer; segments start on 64-element boundaries."""

    def __init__(self, policy, device):
        self.offsets, off = {}, 0
        for name, shape in _PARAMS:
            numel = 1
            for d in shape:
                numel *= d
            self.offsets[name] = (off, shape, numel)
            off += (numel + 63) // 64 * 64
        self.n = off
        self.p = torch.zeros(off, dtype=torch.float32, device=device)
        state = policy.state_dict()
        for name, (o, shape, numel) in self.offsets.items():
            self.p[o:o + numel].copy_(state[name].reshape(-1).float())
        self.pb = self.p.to(torch.bfloat16)
        self.g = torch.zeros(off, dtype=torch.bfloat16, device=device)
        self.m = torch.zeros(off, dtype=torch.float32, device=device)
        self.v = torch.zeros(off, dtype=torch.float32, device=device)

    def view(self, buf, name):
        o, shape, numel = self.offsets[name]
        return buf[o:o + numel].view(shape)

    def load_into(self, policy):
        with torch.no_grad():
            for name, (o, shape, numel) in self.offsets.items():
                dict(policy.named_parameters())[name].copy_(self.p[o:o + numel].view(shape))


class FastPPO:
    """PPO update with the minibatch step in libd1hip (four kernels: fused per-sample
    forward/loss/backward, grouped split-K weight gradients, fixed-order reduction, clip +
    Adam). Same interface and semantics as PPO with bf16 autocast; `minibatch` must be a
    multiple of 1024. With graph=True, `graph_steps` consecutive minibatch steps are
    captured in one HIP graph per buffer and replayed.

    A minibatch whose loss or gradient norm is not finite changes nothing, and neither does
    any later one until `clear_nonfinite()`; `update` then raises RuntimeError, as the
    reference's loop does at the first non-finite loss (run_ring_ablations.py:369-370),
    leaving the weights and Adam state of the last finite step."""

    def __init__(self, policy, lr=3e-4, eps=1e-5, clip=0.2, vcoef=0.5, ecoef=0.01, max_grad_norm=0.5,
                 epochs=4, minibatch=8192, gamma=0.99, lam=0.95, graph=True, graph_steps=16):
        from . import _lib
        if minibatch <= 0 or minibatch % 1024:
            raise ValueError('FastPPO needs a minibatch that is a multiple of 1024')
        dev = next(policy.parameters()).device
        self.flat = F = FlatParams(policy, dev)
        self.lr, self.eps, self.clip, self.vcoef, self.ecoef = lr, eps, clip, vcoef, ecoef
        self.max_grad_norm, self.epochs, self.minibatch, self.gamma, self.lam = max_grad_norm, epochs, minibatch, gamma, lam
        self.graph, self.graph_steps, self.dev = graph, graph_steps, dev
        self.step_t = torch.zeros(3, dtype=torch.float32, device=dev)   # Adam step, scratch, skipped steps
        self.cursor = torch.zeros(2, dtype=torch.int32, device=dev)
        self.loss_parts = torch.zeros(minibatch // 32 * 4, dtype=torch.float32, device=dev)
        nbytes = _lib.load().d1_ppo_work_bytes(minibatch)
        _lib.check(0 if nbytes > 0 else nbytes, 'd1_ppo_work_bytes')
        self.work = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        self.perm = None
        self.head_out = None   # [minibatch, 17] fp32: when set, each step writes its head outputs here
        self._packed = False
        self._g = self._g_buf = None
        self._args = self._args_key = None

    def _struct(self, obs, actions, logp, adv, ret):
        from . import _lib
        key = (obs.data_ptr(), actions.data_ptr(), logp.data_ptr(), adv.data_ptr(), ret.data_ptr(),
               self.perm.data_ptr(), obs.shape[0], 0 if self.head_out is None else self.head_out.data_ptr())
        if self._args_key != key:
            F = self.flat
            if obs.shape[1] != OBS or not obs.is_contiguous() or obs.dtype != torch.uint8:
                raise ValueError('observations must be contiguous uint8 [n, 1800]')
            off = {name: o for name, (o, _, _) in F.offsets.items()}
            self._args = _lib.D1PPOStep(
                obs=obs.data_ptr(), perm=self.perm.data_ptr(), cursor=self.cursor.data_ptr(),
                actions=actions.data_ptr(), logp_old=logp.data_ptr(), adv=adv.data_ptr(), ret=ret.data_ptr(),
                n=obs.shape[0], mb=self.minibatch, p=F.p.data_ptr(), pb=F.pb.data_ptr(), g=F.g.data_ptr(),
                m=F.m.data_ptr(), v=F.v.data_ptr(), nparams=F.n, off_w1=off['l1.weight'], off_b1=off['l1.bias'],
                off_w2=off['l2.weight'], off_b2=off['l2.bias'], off_w3=off['head.weight'],
                off_b3=off['head.bias'], step=self.step_t.data_ptr(), loss_parts=self.loss_parts.data_ptr(), work=self.work.data_ptr(),
                work_bytes=self.work.numel(), clip=self.clip, vcoef=self.vcoef, ecoef=self.ecoef,
                max_grad_norm=self.max_grad_norm, lr=self.lr, beta1=0.9, beta2=0.999, eps=self.eps,
                z_out=None if self.head_out is None else self.head_out.data_ptr())
            self._args_key = key
        if not self._packed:   # kernel-ordered weight copies in the work buffer, from pb
            _lib.check(_lib.load().d1_ppo_prepare(self._args, torch.cuda.current_stream(self.dev).cuda_stream),
                       'd1_ppo_prepare')
            self._packed = True
        return self._args

    def record_head(self, on=True):
        """Have every following minibatch step write the head outputs its loss was computed
        from (16 logits + value, bf16-rounded, as fp32) into self.head_out [minibatch, 17]
        (NaN until a step writes it). A captured graph holds the buffer it was captured
        with, so this drops it and the next update captures again."""
        self._g = self._g_buf = None
        self.head_out = torch.full((self.minibatch, 17), float('nan'), device=self.dev) if on else None

    def set_order(self, perm):
        """Sample order of the next minibatches (int64 [n] on the device); resets the cursor
        so the next step takes perm[0:minibatch]."""
        if self.perm is None or self.perm.shape != perm.shape:
            self.perm = torch.empty_like(perm, dtype=torch.int64)
        self.perm.copy_(perm)
        self.cursor.zero_()

    def _step(self, obs, actions, logp, adv, ret):
        """One minibatch: samples perm[cursor*mb : (cursor+1)*mb]; advances the cursor."""
        from . import _lib
        args = self._struct(obs, actions, logp, adv, ret)
        _lib.check(_lib.load().d1_ppo_step(args, torch.cuda.current_stream(self.dev).cuda_stream), 'd1_ppo_step')

    def nonfinite_steps(self):
        """Minibatch steps skipped since the first non-finite loss or gradient norm."""
        return int(self.step_t[2].item())

    def clear_nonfinite(self):
        self.step_t[2].zero_()

    def loss_terms(self):
        """(pg, value, entropy) means of the last minibatch (reads device partials)."""
        return self.loss_parts.view(-1, 4)[:, :3].sum(0) / self.minibatch

    def _views(self, buf):
        n = buf.T * buf.N
        return buf.obs.view(n, -1), buf.actions.view(n), buf.logp.view(n)

    def _graph_len(self, n):
        steps = n // self.minibatch
        k = max(1, min(self.graph_steps, steps))
        while steps % k:
            k -= 1
        return k

    def _capture(self, buf):
        n = buf.T * buf.N
        if n < self.minibatch:
            raise ValueError('the buffer holds fewer samples than one minibatch')
        self._adv = torch.zeros(n, device=self.dev)
        self._ret = torch.zeros(n, device=self.dev)
        if self.perm is None or self.perm.numel() != n:
            self.perm = torch.zeros(n, dtype=torch.int64, device=self.dev)
        obs, actions, logp = self._views(buf)
        args = self._struct(obs, actions, logp, self._adv, self._ret)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(self._graph_len(n)):
                self._step(obs, actions, logp, self._adv, self._ret)
        self._g, self._g_buf, self._g_args = g, buf, args

    def advantages(self, buf):
        adv, ret = P.gae(buf.rewards, buf.dones, buf.values, buf.bootstrap, self.gamma, self.lam)
        flat = adv.flatten()
        return (flat - flat.mean()) / (flat.std() + 1e-8), ret.flatten()

    def update(self, buf, generator=None):
        adv, ret = self.advantages(buf)
        n = buf.T * buf.N
        obs, actions, logp = self._views(buf)
        if self.graph:
            if self._g is None or self._g_buf is not buf:
                self._capture(buf)
            self._adv.copy_(adv)
            self._ret.copy_(ret)
            adv, ret = self._adv, self._ret
            if not self._packed:   # weights replaced outside the step (a checkpoint load): the graph
                self._struct(obs, actions, logp, adv, ret)   # only replays, so rebuild its weight copies here
        steps = n // self.minibatch            # a ragged tail is dropped (T*N is a multiple in C4)
        for _ in range(self.epochs):
            self.set_order(torch.randperm(n, device=self.dev, generator=generator))
            if self.graph:
                for _ in range(steps // self._graph_len(n)):
                    self._g.replay()
            else:
                for _ in range(steps):
                    self._step(obs, actions, logp, adv, ret)
        if self.nonfinite_steps():
            raise RuntimeError('Non-finite PPO loss')
        return self.loss_terms()
