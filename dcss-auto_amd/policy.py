"""Rollout policy: bf16 MLP trunk 1800 -> 256 -> 256 (ReLU) with a 16-logit policy head
and a scalar value head, plus the counter-RNG categorical sampler and GAE kernels.

The reference's policy is an fp32 MLP with tanh and orthogonal init
(gpu-d1/scripts/run_ring_ablations.py:209-223); this one follows BASELINE's C3
architecture: N(0, 0.02) weights, zero biases. The trunk GEMMs run on hipBLASLt
through torch in bf16 with fp32 accumulation; sampling and GAE are HIP kernels in
libd1hip.so.
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
        x = widen(obs_u8.reshape(obs_u8.shape[0], -1), dtype)
        if x.is_cuda and x.dtype == torch.bfloat16 and not torch.is_grad_enabled():
            # bias + ReLU in the hipBLASLt epilogue
            h = torch._addmm_activation(self.l1.bias, x, self.l1.weight.t())
            h = torch._addmm_activation(self.l2.bias, h, self.l2.weight.t())
        else:
            h = torch.relu(self.l1(x))
            h = torch.relu(self.l2(h))
        out = self.head(h).float()
        return out[:, :self.n_actions], out[:, self.n_actions]


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
