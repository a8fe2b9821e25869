"""Rollout policy: bf16 MLP trunk 1800 -> 256 -> 256 (ReLU) with a 16-logit policy head
and a scalar value head, plus the counter-RNG categorical sampler and GAE kernels.

The reference's policy is an fp32 MLP with tanh and orthogonal init
(gpu-d1/scripts/run_ring_ablations.py:209-223); this one follows BASELINE's C3
architecture: N(0, 0.02) weights, zero biases. The bf16 inference forward on uint8
observations (the rollout's) is one HIP MFMA kernel in libd1hip.so (d1_policy_fwd) on
weights packed once per update; other dtypes and the autograd path use torch. Sampling and
GAE are HIP kernels in libd1hip.so.
"""
import torch
from torch import nn

from . import _lib

OBS = 1800
N_ACTIONS = 16


class Policy(nn.Module):
    def __init__(self, width=256, n_actions=N_ACTIONS, obs=OBS, seed=0):
        super().__init__()
        self.l1 = nn.Linear(obs, width)
        self.l2 = nn.Linear(width, width)
        self.head = nn.Linear(width, n_actions + 1)   # logits | value
        self.n_actions = n_actions
        g = torch.Generator().manual_seed(seed)
        for layer in (self.l1, self.l2, self.head):
            with torch.no_grad():
                layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) * 0.02)
                layer.bias.zero_()

    def forward(self, obs_u8):
        """obs uint8 [B, 15, 15, 8] (or [B, 1800]) -> (fp32 logits [B, A], fp32 value [B])."""
        dtype = self.l1.weight.dtype
        if obs_u8.is_cuda and torch.is_autocast_enabled('cuda'):
            dtype = torch.get_autocast_dtype('cuda')
        flat = obs_u8.reshape(obs_u8.shape[0], -1)
        if flat.dtype == torch.uint8 and flat.is_cuda and dtype == torch.bfloat16 and not torch.is_grad_enabled() \
                and flat.shape[1] == OBS and self.l1.out_features == 256 and self.n_actions == N_ACTIONS:
            return policy_fwd(flat, *self.packed(dtype))
        x = widen(flat, dtype)
        if x.is_cuda and x.dtype == torch.bfloat16 and not torch.is_grad_enabled():
            # bias + ReLU in the hipBLASLt epilogue
            h = torch._addmm_activation(self.l1.bias, x, self.l1.weight.t())
            h = torch._addmm_activation(self.l2.bias, h, self.l2.weight.t())
        else:
            h = torch.relu(self.l1(x))
            h = torch.relu(self.l2(h))
        out = self.head(h).float()
        return out[:, :self.n_actions], out[:, self.n_actions]

    def packed(self, dtype=torch.bfloat16, refresh=False):
        """(packed bf16 weights, b1, b2, b3) for d1_policy_fwd, rebuilt when a parameter's
        storage or version counter changes (optimizer steps and copy_ bump it; writes through
        .data do not: pass refresh=True after those)."""
        params = (self.l1.weight, self.l2.weight, self.head.weight, self.l1.bias, self.l2.bias, self.head.bias)
        key = (dtype,) + tuple((q.data_ptr(), q._version) for q in params)
        if refresh or getattr(self, '_packed_key', None) != key:
            w1, w2, w3, b1, b2, b3 = (q.detach().to(dtype).contiguous() for q in params)
            self._packed_val = (pack_weights(w1, w2, w3), b1, b2, b3)
            self._packed_key = key
        return self._packed_val


def pack_weights(w1, w2, w3, out=None):
    """bf16 w1 [256, 1800], w2 [256, 256], w3 [17, 256] -> the operand-ordered buffer that
    d1_policy_fwd reads (d1_policy_pack); `out` repacks into an existing buffer."""
    for w, shape in ((w1, (256, OBS)), (w2, (256, 256)), (w3, (N_ACTIONS + 1, 256))):
        if w.dtype != torch.bfloat16 or tuple(w.shape) != shape or not w.is_contiguous() or not w.is_cuda:
            raise ValueError(f'expected a contiguous CUDA bf16 tensor of shape {shape}')
    L = _lib.load()
    wpk = out if out is not None else torch.empty(L.d1_policy_packed_elems(), dtype=torch.bfloat16, device=w1.device)
    if wpk.dtype != torch.bfloat16 or wpk.numel() != L.d1_policy_packed_elems() or not wpk.is_contiguous():
        raise ValueError('the packed buffer must hold d1_policy_packed_elems() contiguous bf16 values')
    _lib.check(L.d1_policy_pack(w1.data_ptr(), w2.data_ptr(), w3.data_ptr(), wpk.data_ptr(),
                                torch.cuda.current_stream(w1.device).cuda_stream), 'd1_policy_pack')
    return wpk


def policy_fwd(obs_u8, wpk, b1, b2, b3, logits=None, value=None):
    """The fused bf16 policy forward on uint8 obs [B, 1800]: (fp32 logits [B, 16], fp32 value [B])."""
    obs_u8 = obs_u8.contiguous()
    n = obs_u8.shape[0]
    assert obs_u8.dtype == torch.uint8 and obs_u8.shape[1] == OBS
    for b, size in ((b1, 256), (b2, 256), (b3, N_ACTIONS + 1)):
        assert b.dtype == torch.bfloat16 and b.shape == (size,) and b.is_contiguous()
    if logits is None:
        logits = torch.empty((n, N_ACTIONS), dtype=torch.float32, device=obs_u8.device)
    if value is None:
        value = torch.empty(n, dtype=torch.float32, device=obs_u8.device)
    L = _lib.load()
    _lib.check(L.d1_policy_fwd(obs_u8.data_ptr(), n, wpk.data_ptr(), b1.data_ptr(), b2.data_ptr(), b3.data_ptr(),
                               logits.data_ptr(), value.data_ptr(),
                               torch.cuda.current_stream(obs_u8.device).cuda_stream), 'd1_policy_fwd')
    return logits, value


def policy_fwd_sample(obs_u8, wpk, b1, b2, b3, seed, t, actions, logp, value, t_dev=None, logits=None):
    """policy_fwd and the counter-RNG sample of each row in one kernel (d1_policy_fwd_sample):
    the same actions/log-probs as sample() / sample_dev() on policy_fwd's logits at step
    t (+ t_dev[0] when given, int32 device tensor read as uint32)."""
    obs_u8 = obs_u8.contiguous()
    n = obs_u8.shape[0]
    assert obs_u8.dtype == torch.uint8 and obs_u8.shape[1] == OBS
    for b, size in ((b1, 256), (b2, 256), (b3, N_ACTIONS + 1)):
        assert b.dtype == torch.bfloat16 and b.shape == (size,) and b.is_contiguous()
    assert actions.dtype == torch.int64 and logp.dtype == torch.float32 and value.dtype == torch.float32
    assert actions.numel() == n and logp.numel() == n and value.numel() == n
    if t_dev is not None and t_dev.dtype != torch.int32:
        raise ValueError('t_dev must be an int32 device tensor')
    L = _lib.load()
    _lib.check(L.d1_policy_fwd_sample(obs_u8.data_ptr(), n, wpk.data_ptr(), b1.data_ptr(), b2.data_ptr(), b3.data_ptr(),
                                      seed, t_dev.data_ptr() if t_dev is not None else None, t & 0xFFFFFFFF,
                                      logits.data_ptr() if logits is not None else None, value.data_ptr(),
                                      actions.data_ptr(), logp.data_ptr(),
                                      torch.cuda.current_stream(obs_u8.device).cuda_stream), 'd1_policy_fwd_sample')
    return actions, logp, value


def widen(obs_u8, dtype):
    """uint8 observations -> `dtype`; the bf16 case runs the HIP widening kernel."""
    if obs_u8.dtype != torch.uint8:
        return obs_u8.to(dtype)
    if dtype == torch.bfloat16 and obs_u8.is_cuda and obs_u8.is_contiguous() and obs_u8.numel() % 16 == 0 \
            and obs_u8.data_ptr() % 16 == 0:
        out = torch.empty(obs_u8.shape, dtype=dtype, device=obs_u8.device)
        L = _lib.load()
        _lib.check(L.d1_obs_to_bf16(obs_u8.data_ptr(), out.data_ptr(), obs_u8.numel(),
                                    torch.cuda.current_stream(obs_u8.device).cuda_stream), 'd1_obs_to_bf16')
        return out
    return obs_u8.to(dtype)


def sample(logits, seed, t, actions=None, logp=None):
    """Counter-RNG categorical sample of fp32 logits [B, K] (row stride honoured)."""
    if logits.dtype != torch.float32 or logits.stride(1) != 1:
        raise ValueError('logits must be fp32 with unit column stride')
    n, k = logits.shape
    if actions is None:
        actions = torch.empty(n, dtype=torch.int64, device=logits.device)
    if logp is None:
        logp = torch.empty(n, dtype=torch.float32, device=logits.device)
    L = _lib.load()
    _lib.check(L.d1_sample(logits.data_ptr(), n, k, logits.stride(0), seed, t & 0xFFFFFFFF, actions.data_ptr(),
                           logp.data_ptr(), torch.cuda.current_stream(logits.device).cuda_stream), 'd1_sample')
    return actions, logp


def sample_dev(logits, seed, t_dev, t_add, actions, logp):
    """sample() with the counter step read on the device: t = t_dev[0] + t_add (int32
    tensor, read as uint32), so a captured graph draws a new step on every replay."""
    if logits.dtype != torch.float32 or logits.stride(1) != 1:
        raise ValueError('logits must be fp32 with unit column stride')
    if t_dev.dtype != torch.int32 or not t_dev.is_cuda:
        raise ValueError('t_dev must be an int32 device tensor')
    n, k = logits.shape
    L = _lib.load()
    _lib.check(L.d1_sample_dev(logits.data_ptr(), n, k, logits.stride(0), seed, t_dev.data_ptr(), t_add & 0xFFFFFFFF,
                               actions.data_ptr(), logp.data_ptr(),
                               torch.cuda.current_stream(logits.device).cuda_stream), 'd1_sample_dev')
    return actions, logp


def gae(reward, done, value, bootstrap, gamma=0.99, lam=0.95, adv=None, returns=None):
    """HIP reverse-time GAE over [T, N] fp32 rewards/values and uint8 dones."""
    T, n = reward.shape
    for t_ in (reward, value):
        assert t_.dtype == torch.float32 and t_.is_contiguous() and t_.shape == (T, n)
    assert done.dtype == torch.uint8 and done.is_contiguous() and done.shape == (T, n)
    assert bootstrap.dtype == torch.float32 and bootstrap.shape == (n,) and bootstrap.is_contiguous()
    if adv is None:
        adv = torch.empty_like(reward)
    if returns is None:
        returns = torch.empty_like(reward)
    L = _lib.load()
    _lib.check(L.d1_gae(reward.data_ptr(), done.data_ptr(), value.data_ptr(), bootstrap.data_ptr(), T, n,
                        float(gamma), float(gamma * lam), adv.data_ptr(), returns.data_ptr(),
                        torch.cuda.current_stream(reward.device).cuda_stream), 'd1_gae')
    return adv, returns


# ----------------------------------------------------------------------------------------
# Autoregressive verb x target head (BASELINE C5), generalising the reference's
# type-then-direction head (gpu-d1/branches/autoregressive-actions-v1/scripts/tactical_models.py:8-58):
# verb logits from the trunk, a learned verb embedding, and a target MLP on
# [trunk, embedding(verb)] evaluated for every verb in one pass.
N_VERBS, N_TARGETS, EMBED, TARGET_HIDDEN = 8, 25, 16, 64


class ARPolicy(nn.Module):
    def __init__(self, width=256, obs=OBS, seed=0):
        super().__init__()
        self.l1 = nn.Linear(obs, width)
        self.l2 = nn.Linear(width, width)
        self.verb = nn.Linear(width, N_VERBS)
        self.value = nn.Linear(width, 1)
        self.embedding = nn.Parameter(torch.zeros(N_VERBS, EMBED))
        self.t1 = nn.Linear(width + EMBED, TARGET_HIDDEN)
        self.t2 = nn.Linear(TARGET_HIDDEN, N_TARGETS)
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for layer in (self.l1, self.l2, self.verb, self.value, self.t1, self.t2):
                layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) * 0.02)
                layer.bias.zero_()
            self.embedding.copy_(torch.randn(N_VERBS, EMBED, generator=g) * 0.1)

    def forward(self, obs_u8):
        """-> verb logits [B, 8], target logits [B, 8, 25] (one row per verb), value [B] (fp32)."""
        dtype = self.l1.weight.dtype
        if obs_u8.is_cuda and torch.is_autocast_enabled('cuda'):
            dtype = torch.get_autocast_dtype('cuda')
        x = widen(obs_u8.reshape(obs_u8.shape[0], -1), dtype)
        h = torch.relu(self.l1(x))
        h = torch.relu(self.l2(h))
        w = self.t1.weight                         # [64, 256 + 16]: trunk part and embedding part
        ht = torch.nn.functional.linear(h, w[:, :h.shape[1]], self.t1.bias)            # [B, 64]
        ev = torch.nn.functional.linear(self.embedding.to(ht.dtype), w[:, h.shape[1]:])  # [8, 64]
        z = torch.tanh(ht[:, None, :] + ev[None])                                       # [B, 8, 64]
        targets = self.t2(z)                                                             # [B, 8, 25]
        return self.verb(h).float(), targets.float(), self.value(h).float().squeeze(-1)

    def packed(self, refresh=False):
        """(packed weights, b1, b2, b3, bt) for policy_fwd_sample_ar (bf16 parameters only),
        rebuilt when a parameter's storage or version counter changes (as Policy.packed).
        The head holds the verb logits in rows 0-7 and the value in row 16; ev, the verb
        embeddings through t1's embedding columns, is computed here by the same bf16 linear
        as forward() computes it."""
        params = (self.l1.weight, self.l2.weight, self.verb.weight, self.value.weight, self.embedding,
                  self.t1.weight, self.t2.weight, self.l1.bias, self.l2.bias, self.verb.bias, self.value.bias,
                  self.t1.bias, self.t2.bias)
        if any(q.dtype != torch.bfloat16 or not q.is_cuda for q in params):
            raise ValueError('the fused AR forward takes a CUDA model in bfloat16')
        key = tuple((q.data_ptr(), q._version) for q in params)
        if refresh or getattr(self, '_packed_key', None) != key:
            with torch.no_grad():
                dev, width = self.l1.weight.device, self.l2.out_features
                w3 = torch.zeros((N_ACTIONS + 1, width), dtype=torch.bfloat16, device=dev)
                w3[:N_VERBS] = self.verb.weight
                w3[N_ACTIONS] = self.value.weight[0]
                b3 = torch.zeros(N_ACTIONS + 1, dtype=torch.bfloat16, device=dev)
                b3[:N_VERBS] = self.verb.bias
                b3[N_ACTIONS] = self.value.bias[0]
                t1w = self.t1.weight.detach()
                ev = torch.nn.functional.linear(self.embedding.detach(), t1w[:, width:]).contiguous()
                bt = torch.cat([self.t1.bias.detach(), self.t2.bias.detach()]).contiguous()
                L = _lib.load()
                wpk = torch.empty(L.d1_policy_ar_packed_elems(), dtype=torch.bfloat16, device=dev)
                args = [self.l1.weight.detach().contiguous(), self.l2.weight.detach().contiguous(), w3,
                        t1w.contiguous(), self.t2.weight.detach().contiguous(), ev]
                _lib.check(L.d1_policy_ar_pack(*(a.data_ptr() for a in args), wpk.data_ptr(),
                                               torch.cuda.current_stream(dev).cuda_stream), 'd1_policy_ar_pack')
                self._packed_val = (wpk, self.l1.bias.detach().contiguous(), self.l2.bias.detach().contiguous(),
                                    b3, bt)
                self._packed_key = key
        return self._packed_val


def policy_fwd_sample_ar(obs_u8, packed, seed, t, action, logp, value, t_dev=None, verb=None, target=None,
                         verb_logits=None, target_logits=None):
    """ARPolicy's forward and its two-stage counter-RNG sample in one kernel
    (d1_policy_fwd_sample_ar) on uint8 obs [B, 1800]: the verb, target, env action and
    log-probability sample_ar() would draw from the same logits at step t (+ t_dev[0] when
    given), without the [B, 8, 25] target logits (only the drawn verb's row is formed)."""
    obs_u8 = obs_u8.reshape(obs_u8.shape[0], OBS).contiguous()
    n = obs_u8.shape[0]
    assert obs_u8.dtype == torch.uint8
    wpk, b1, b2, b3, bt = packed
    assert action.dtype == torch.int64 and logp.dtype == torch.float32 and value.dtype == torch.float32
    assert action.numel() == n and logp.numel() == n and value.numel() == n
    for x, dt, width in ((verb, torch.int32, 1), (target, torch.int32, 1), (verb_logits, torch.float32, N_VERBS),
                         (target_logits, torch.float32, N_TARGETS)):
        if x is not None and (x.dtype != dt or x.numel() != n * width or not x.is_contiguous()):
            raise ValueError('optional outputs: contiguous int32 verb/target [B], fp32 verb_logits [B, 8] and '
                             'target_logits [B, 25]')
    if t_dev is not None and t_dev.dtype != torch.int32:
        raise ValueError('t_dev must be an int32 device tensor')
    ptr = lambda x: None if x is None else x.data_ptr()
    L = _lib.load()
    _lib.check(L.d1_policy_fwd_sample_ar(obs_u8.data_ptr(), n, wpk.data_ptr(), b1.data_ptr(), b2.data_ptr(),
                                         b3.data_ptr(), bt.data_ptr(), seed, ptr(t_dev), t & 0xFFFFFFFF,
                                         value.data_ptr(), action.data_ptr(), logp.data_ptr(), ptr(verb),
                                         ptr(target), ptr(verb_logits), ptr(target_logits),
                                         torch.cuda.current_stream(obs_u8.device).cuda_stream),
               'd1_policy_fwd_sample_ar')
    return action, logp, value


class ARDistribution:
    """p(verb) p(target | verb) with the factorised log-prob and entropy
    (tactical_models.py:8-30): log p = log p(v) + log p(t|v); H = H(v) + sum_v p(v) H(t|v)."""

    def __init__(self, verb_logits, target_logits):
        self.lv = torch.log_softmax(verb_logits, -1)
        self.lt = torch.log_softmax(target_logits, -1)

    @property
    def probs(self):
        return (self.lv.exp()[:, :, None] * self.lt.exp()).flatten(1)

    def log_prob(self, verb, target):
        lt = self.lt.gather(1, verb[:, None, None].expand(-1, 1, self.lt.shape[2])).squeeze(1)
        return self.lv.gather(1, verb[:, None]).squeeze(1) + lt.gather(1, target[:, None]).squeeze(1)

    def entropy(self):
        pv = self.lv.exp()
        ht = -(self.lt.exp() * self.lt).sum(-1)
        return -(pv * self.lv).sum(-1) + (pv * ht).sum(-1)


def sample_ar(verb_logits, target_logits, seed, t):
    """HIP two-stage sample -> (verb int32, target int32, env action int64, logp fp32)."""
    n, nv = verb_logits.shape
    nt = target_logits.shape[2]
    assert verb_logits.dtype == torch.float32 and target_logits.dtype == torch.float32
    assert verb_logits.stride(1) == 1 and target_logits.is_contiguous()
    dev = verb_logits.device
    verb = torch.empty(n, dtype=torch.int32, device=dev)
    target = torch.empty(n, dtype=torch.int32, device=dev)
    action = torch.empty(n, dtype=torch.int64, device=dev)
    logp = torch.empty(n, dtype=torch.float32, device=dev)
    L = _lib.load()
    _lib.check(L.d1_sample_ar(verb_logits.data_ptr(), nv, verb_logits.stride(0), target_logits.data_ptr(), nt,
                              nv * nt, n, seed, t & 0xFFFFFFFF, verb.data_ptr(), target.data_ptr(), action.data_ptr(),
                              logp.data_ptr(), torch.cuda.current_stream(dev).cuda_stream), 'd1_sample_ar')
    return verb, target, action, logp
