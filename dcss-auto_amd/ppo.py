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
# Graph-safe PPO: explicit forward/backward over flat parameter buffers. Everything in the
# minibatch step is a GEMM (hipBLASLt through torch) or a libd1hip kernel; no torch
# reductions run inside the step, so the step can be captured in a HIP graph and replayed.

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
    def __init__(self, policy, lr=3e-4, eps=1e-5, clip=0.2, vcoef=0.5, ecoef=0.01, max_grad_norm=0.5,
                 epochs=4, minibatch=8192, gamma=0.99, lam=0.95, graph=True, nparts=512):
        dev = next(policy.parameters()).device
        self.flat = FlatParams(policy, dev)
        self.lr, self.eps, self.clip, self.vcoef, self.ecoef = lr, eps, clip, vcoef, ecoef
        self.max_grad_norm, self.epochs, self.minibatch, self.gamma, self.lam = max_grad_norm, epochs, minibatch, gamma, lam
        self.graph, self.nparts, self.dev = graph, nparts, dev
        mb = minibatch
        self.step_t = torch.zeros(2, dtype=torch.float32, device=dev)
        self.norm_parts = torch.zeros(nparts, dtype=torch.float32, device=dev)
        self.loss_parts = torch.zeros(((mb + 255) // 256) * 4, dtype=torch.float32, device=dev)
        self.idx = torch.zeros(mb, dtype=torch.int64, device=dev)
        self.xb = torch.empty((mb, OBS), dtype=torch.bfloat16, device=dev)
        self.act = torch.empty(mb, dtype=torch.int32, device=dev)
        self.old = torch.empty(mb, dtype=torch.float32, device=dev)
        self.adv_mb = torch.empty(mb, dtype=torch.float32, device=dev)
        self.ret_mb = torch.empty(mb, dtype=torch.float32, device=dev)
        self.dz = torch.empty((mb, 17), dtype=torch.bfloat16, device=dev)
        self.colblocks = 512
        self.colpart = torch.zeros(self.colblocks * 256, dtype=torch.float32, device=dev)
        self.splitk = 16 if mb % 16 == 0 else 1
        self.kpart = torch.empty(self.splitk * 256 * OBS, dtype=torch.bfloat16, device=dev)
        self._g = self._g_buf = None

    # one minibatch whose indices are in self.idx; buffers are flattened [T*N, ...] views
    def _step(self, obs, actions, logp, adv, ret):
        from . import _lib
        L, F, s = _lib.load(), self.flat, torch.cuda.current_stream(self.dev).cuda_stream
        mb = self.minibatch
        _lib.check(L.d1_ppo_gather(obs.data_ptr(), obs.shape[1], self.idx.data_ptr(), mb, actions.data_ptr(),
                                   logp.data_ptr(), adv.data_ptr(), ret.data_ptr(), self.xb.data_ptr(),
                                   self.act.data_ptr(), self.old.data_ptr(), self.adv_mb.data_ptr(),
                                   self.ret_mb.data_ptr(), s), 'd1_ppo_gather')
        W1, b1 = F.view(F.pb, 'l1.weight'), F.view(F.pb, 'l1.bias')
        W2, b2 = F.view(F.pb, 'l2.weight'), F.view(F.pb, 'l2.bias')
        W3, b3 = F.view(F.pb, 'head.weight'), F.view(F.pb, 'head.bias')
        h1 = torch._addmm_activation(b1, self.xb, W1.t())
        h2 = torch._addmm_activation(b2, h1, W2.t())
        z = torch.addmm(b3, h2, W3.t())
        _lib.check(L.d1_ppo_loss(z.data_ptr(), 17, 16, self.act.data_ptr(), self.old.data_ptr(),
                                 self.adv_mb.data_ptr(), self.ret_mb.data_ptr(), mb, self.clip, self.vcoef, self.ecoef,
                                 self.dz.data_ptr(), self.loss_parts.data_ptr(), s), 'd1_ppo_loss')
        G = lambda name: F.view(F.g, name)   # noqa: E731
        cb, cp = self.colblocks, self.colpart.data_ptr()
        self._wgrad(self.dz, h2, G('head.weight'))
        _lib.check(L.d1_colsum(self.dz.data_ptr(), mb, 17, 17, cp, cb, G('head.bias').data_ptr(), s), 'd1_colsum')
        dh2 = torch.mm(self.dz, W3)
        _lib.check(L.d1_relu_bwd_bias(dh2.data_ptr(), h2.data_ptr(), mb, 256, cp, cb, G('l2.bias').data_ptr(), s),
                   'd1_relu_bwd_bias')
        self._wgrad(dh2, h1, G('l2.weight'))
        dh1 = torch.mm(dh2, W2)
        _lib.check(L.d1_relu_bwd_bias(dh1.data_ptr(), h1.data_ptr(), mb, 256, cp, cb, G('l1.bias').data_ptr(), s),
                   'd1_relu_bwd_bias')
        self._wgrad(dh1, self.xb, G('l1.weight'))
        _lib.check(L.d1_adam_clip(F.p.data_ptr(), F.pb.data_ptr(), F.g.data_ptr(), F.m.data_ptr(), F.v.data_ptr(),
                                  F.n, self.norm_parts.data_ptr(), self.nparts, self.max_grad_norm, self.lr, 0.9,
                                  0.999, self.eps, self.step_t.data_ptr(), s), 'd1_adam_clip')

    def _wgrad(self, dy, x, out):
        """out = dy^T @ x with the batch (K) dimension split S ways: one bf16 bmm into
        [S, M, N] partials (right operand contiguous), then a libd1hip partial sum."""
        from . import _lib
        S = self.splitk
        if S == 1:
            torch.mm(dy.t(), x, out=out)
            return
        mb, M = dy.shape
        N = x.shape[1]
        part = self.kpart[:S * M * N].view(S, M, N)
        torch.bmm(dy.view(S, mb // S, M).transpose(1, 2), x.view(S, mb // S, N), out=part)
        _lib.check(_lib.load().d1_sum_partials(part.data_ptr(), S, M * N, out.data_ptr(),
                                               torch.cuda.current_stream(self.dev).cuda_stream), 'd1_sum_partials')

    def loss_terms(self):
        """(pg, value, entropy) means of the last minibatch (reads device partials)."""
        parts = self.loss_parts.view(-1, 4)[:, :3].sum(0) / self.minibatch
        return parts

    def _views(self, buf):
        n = buf.T * buf.N
        return buf.obs.view(n, -1), buf.actions.view(n), buf.logp.view(n)

    def _capture(self, buf):
        n = buf.T * buf.N
        if n % self.minibatch:
            raise ValueError('T*N must be a multiple of the minibatch size')
        self._adv = torch.zeros(n, device=self.dev)
        self._ret = torch.zeros(n, device=self.dev)
        obs, actions, logp = self._views(buf)
        saved = [t.clone() for t in (self.flat.p, self.flat.pb, self.flat.m, self.flat.v, self.step_t)]
        side = torch.cuda.Stream(device=self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                self._step(obs, actions, logp, self._adv, self._ret)
        torch.cuda.current_stream(self.dev).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._step(obs, actions, logp, self._adv, self._ret)
        for dst, src in zip((self.flat.p, self.flat.pb, self.flat.m, self.flat.v, self.step_t), saved):
            dst.copy_(src)
        self._g, self._g_buf = g, buf

    def advantages(self, buf):
        adv, ret = P.gae(buf.rewards, buf.dones, buf.values, buf.bootstrap, self.gamma, self.lam)
        flat = adv.flatten()
        return (flat - flat.mean()) / (flat.std() + 1e-8), ret.flatten()

    def update(self, buf, generator=None):
        adv, ret = self.advantages(buf)
        n = buf.T * buf.N
        if self.graph:
            if self._g is None or self._g_buf is not buf:
                self._capture(buf)
            self._adv.copy_(adv)
            self._ret.copy_(ret)
        obs, actions, logp = self._views(buf)
        for _ in range(self.epochs):
            perm = torch.randperm(n, device=self.dev, generator=generator)
            for inds in perm.split(self.minibatch):
                if len(inds) != self.minibatch:
                    continue               # a ragged tail is dropped (T*N is a multiple in C4)
                self.idx.copy_(inds)
                if self.graph:
                    self._g.replay()
                else:
                    self._step(obs, actions, logp, adv, ret)
        return self.loss_terms()
