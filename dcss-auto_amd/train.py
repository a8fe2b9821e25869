"""PPO training loop on the batched environment: the drop-in for the reference's worker
loop (gpu-d1/scripts/run_ring_ablations.py:185-388, gpu-d1/scripts/train_clear.py).

One update = a T-step rollout (policy forward from the uint8 observation with the
counter-RNG sample in the same kernel, env step; each writes straight into the rollout
buffer) followed by FastPPO.update (GAE, advantage normalisation, epochs of shuffled
minibatches). With
graph=True the whole rollout — T x (forward + sample, step, reward/done copies), the
bootstrap value and the step-counter advance — is captured once in a HIP graph and
replayed; the sampler reads its counter step from the device, so every replay draws new
actions.

`run` is the worker loop around them: resume, periodic and stop-time checkpoints, a
SIGTERM/SIGINT stop at an update boundary (exit status 130), an abort on a non-finite loss.

Checkpoints hold everything the next update reads: fp32 master weights, their bf16 copy,
Adam moments and step, the live worlds (`env.state`) and their current observation, the
sampler's step counter and the minibatch-shuffle generator. A run resumed from one is
bit-identical to the uninterrupted run (the reference's gpu-d1/scripts/test_resume.py
checks the same for its trainer: weights, optimizer, live worlds, observations, RNGs).
"""
import os
import signal
import threading

import torch

from . import _lib
from . import policy as P
from . import ppo as ppo_mod

# Checkpoint layout version: 2 added the trainer-settings record and grew crowded env state
# rows (more than 8 monsters) by the 2,656-byte distance-field memo; 3 added the monsters'
# stuck-cache radii to that memo (rows of 40 monsters 5,632 -> 5,696 bytes); version-1 files
# carry no 'format' key.
CHECKPOINT_FORMAT = 3


class Trainer:
    def __init__(self, env, model, horizon=128, minibatch=8192, epochs=4, lr=3e-4, eps=1e-5, clip=0.2,
                 vcoef=0.5, ecoef=0.01, max_grad_norm=0.5, gamma=0.99, lam=0.95, seed=7, graph=True,
                 ppo_graph=True):
        if env.batch * horizon < minibatch:
            raise ValueError('a rollout must hold at least one minibatch')
        self.env, self.model, self.T, self.N = env, model, horizon, env.batch
        self.dev = env.device
        self.ppo = ppo_mod.FastPPO(model, lr=lr, eps=eps, clip=clip, vcoef=vcoef, ecoef=ecoef,
                                   max_grad_norm=max_grad_norm, epochs=epochs, minibatch=minibatch, gamma=gamma,
                                   lam=lam, graph=ppo_graph)
        self.buf = ppo_mod.RolloutBuffer(horizon, self.N, device=self.dev)
        self.seed = seed
        self.graph = graph
        # everything besides the tensors that decides what the next update computes: a
        # checkpoint made with other values would not resume the same run
        self.hparams = dict(seed=seed, horizon=horizon, batch=self.N, minibatch=minibatch, epochs=epochs, lr=lr,
                            eps=eps, clip=clip, vcoef=vcoef, ecoef=ecoef, max_grad_norm=max_grad_norm, gamma=gamma,
                            lam=lam)
        self.next_obs = env.obs.reshape(self.N, -1).clone()       # the observation the next rollout starts from
        self.t_dev = torch.zeros(1, dtype=torch.int32, device=self.dev)   # sampler counter step
        self.logits = torch.empty((self.N, P.N_ACTIONS), dtype=torch.float32, device=self.dev)
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(seed)
        self.wpk = torch.empty(_lib.load().d1_policy_packed_elems(), dtype=torch.bfloat16, device=self.dev)
        F = self.ppo.flat
        self.bias = tuple(F.view(F.pb, name) for name in ('l1.bias', 'l2.bias', 'head.bias'))
        self._repack()
        self._g = None
        self.updates = 0
        self.decisions = 0

    # ---- rollout
    def _repack(self):
        """Pack the current bf16 weights (FastPPO's copy, refreshed by every Adam step) for
        the rollout forward, in place: a captured rollout keeps reading the same buffer."""
        F = self.ppo.flat
        P.pack_weights(F.view(F.pb, 'l1.weight'), F.view(F.pb, 'l2.weight'), F.view(F.pb, 'head.weight'),
                       out=self.wpk)

    def _rollout_body(self):
        buf, env = self.buf, self.env
        b1, b2, b3 = self.bias
        buf.obs[0].copy_(self.next_obs)
        for k in range(self.T):   # forward + sample in one kernel, the counter step read on the device
            P.policy_fwd_sample(buf.obs[k], self.wpk, b1, b2, b3, self.seed, k, buf.actions[k], buf.logp[k],
                                buf.values[k], t_dev=self.t_dev)
            dst = buf.obs[k + 1] if k + 1 < self.T else self.next_obs
            env.step(buf.actions[k], obs=dst)
            buf.rewards[k].copy_(env.out[:, 0])
            buf.dones[k].copy_(env.out[:, 1])
        P.policy_fwd(self.next_obs, self.wpk, b1, b2, b3, logits=self.logits, value=buf.bootstrap)
        self.t_dev.add_(self.T)

    def rollout(self):
        """Fill the buffer with T decisions per world (eager launches, or one graph replay)."""
        if not self.graph:
            self._rollout_body()
        else:
            if self._g is None:   # capture records the launches without running them
                torch.cuda.synchronize(self.dev)
                self._g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self._g):
                    self._rollout_body()
                torch.cuda.synchronize(self.dev)
            self._g.replay()
        self.decisions += self.T * self.N
        return self.buf

    # ---- update
    def update(self):
        """One PPO update over the filled buffer; returns (pg, value, entropy) of the last minibatch."""
        terms = self.ppo.update(self.buf, generator=self.gen)
        self._repack()
        self.updates += 1
        return terms

    def train(self, updates):
        terms = None
        for _ in range(updates):
            self.rollout()
            terms = self.update()
        return terms

    def run(self, decisions, checkpoint=None, checkpoint_every=None, on_update=None, handle_signals=True):
        """The reference's worker loop (gpu-d1/scripts/run_ring_ablations.py:291-295,341-388):
        resume from `checkpoint` when that file exists, then rollout + update until
        `decisions` decisions have been trained, persisting to `checkpoint` every
        `checkpoint_every` decisions and at the end. SIGTERM or SIGINT (when called from
        the main thread with handle_signals) stops at the next update boundary, persists
        and returns 130 — rerunning the same call resumes; a finished run returns 0. A
        non-finite loss raises RuntimeError from `update`, with nothing persisted past the
        last finite update. `on_update(trainer, terms)` runs after every update (logging,
        milestone evaluation)."""
        if checkpoint is not None and os.path.exists(checkpoint):
            self.load(checkpoint)
        stop = [False]
        previous = {}
        if handle_signals and threading.current_thread() is threading.main_thread():
            def interrupt(*_):
                stop[0] = True
            for sig in (signal.SIGTERM, signal.SIGINT):
                previous[sig] = signal.signal(sig, interrupt)
        try:
            every = checkpoint_every or 0
            next_save = (self.decisions // every + 1) * every if every else None
            while self.decisions < decisions and not stop[0]:
                self.rollout()
                terms = self.update()
                if on_update is not None:
                    on_update(self, terms)
                if checkpoint is not None and next_save is not None and self.decisions >= next_save and not stop[0]:
                    self.save(checkpoint)
                    next_save = (self.decisions // every + 1) * every if every else None
            if checkpoint is not None:
                self.save(checkpoint)
            return 130 if stop[0] else 0
        finally:
            for sig, handler in previous.items():
                signal.signal(sig, handler)

    def sync_model(self):
        """Copy the fp32 master weights into the nn.Module."""
        self.ppo.flat.load_into(self.model)
        return self.model

    # ---- checkpoint / resume
    def state_dict(self):
        F = self.ppo.flat
        cpu = lambda t: t.detach().to('cpu', copy=True)
        return dict(p=cpu(F.p), pb=cpu(F.pb), m=cpu(F.m), v=cpu(F.v), adam_step=cpu(self.ppo.step_t),
                    env_state=cpu(self.env.state), next_obs=cpu(self.next_obs), t=cpu(self.t_dev),
                    gen=self.gen.get_state(), updates=torch.tensor(self.updates), decisions=torch.tensor(self.decisions),
                    hparams=dict(self.hparams), format=CHECKPOINT_FORMAT)

    def load_state_dict(self, sd):
        F = self.ppo.flat
        if sd.get('format') != CHECKPOINT_FORMAT:
            raise ValueError(f"checkpoint format {sd.get('format', 1)} is not this trainer's ({CHECKPOINT_FORMAT}): "
                             'it was written by an older version (no settings record, or env state rows of '
                             'crowded layouts in an older memo layout) and cannot be resumed')
        saved = sd.get('hparams')
        if saved != self.hparams:
            diff = sorted(k for k in set(self.hparams) | set(saved or {})
                          if (saved or {}).get(k) != self.hparams.get(k))
            raise ValueError(f'checkpoint was made with other trainer settings: {diff}')
        for dst, key in ((F.p, 'p'), (F.pb, 'pb'), (F.m, 'm'), (F.v, 'v'), (self.ppo.step_t, 'adam_step'),
                         (self.env.state, 'env_state'), (self.next_obs, 'next_obs'), (self.t_dev, 't')):
            if dst.shape != sd[key].shape or dst.dtype != sd[key].dtype:
                raise ValueError(f'checkpoint field {key} does not match this trainer')
            dst.copy_(sd[key])
        self.gen.set_state(sd['gen'])
        self.updates, self.decisions = int(sd['updates']), int(sd['decisions'])
        self.ppo._packed = False   # FastPPO rebuilds its kernel-ordered weight copies from pb before its next step
        self._repack()

    def save(self, path):
        """Write the checkpoint atomically: a reader sees the previous file or the new one."""
        path = os.fspath(path)
        tmp = f'{path}.tmp{os.getpid()}'
        torch.save(self.state_dict(), tmp)
        os.replace(tmp, path)

    def load(self, path):
        self.load_state_dict(torch.load(path, map_location='cpu', weights_only=True))

    # ---- evaluation
    @torch.no_grad()
    def evaluate(self, env, mode='sampled', seed=900000, max_decisions=None):
        """Run every world of `env` (reset to `seed`) to the end of one episode with the
        current policy, freezing finished worlds through the `active` mask, as the
        reference's evaluate (gpu-d1/scripts/run_ring_ablations.py:231-267). mode 'greedy'
        takes the most likely action, 'sampled' draws from the policy."""
        if mode not in ('sampled', 'greedy'):
            raise ValueError("mode is 'sampled' or 'greedy'")
        env.reset(seed)
        n = env.batch
        active = torch.ones(n, dtype=torch.bool, device=self.dev)
        terminal = torch.zeros_like(env.out)
        returns = torch.zeros(n, device=self.dev)
        actions = torch.zeros(n, dtype=torch.int64, device=self.dev)
        logp = torch.empty(n, device=self.dev)
        logits = torch.empty((n, P.N_ACTIONS), device=self.dev)
        value = torch.empty(n, device=self.dev)
        b1, b2, b3 = self.bias
        limit = max_decisions if max_decisions is not None else env.cfg.limit + 1
        for step in range(limit):
            P.policy_fwd(env.obs.reshape(n, -1), self.wpk, b1, b2, b3, logits=logits, value=value)
            if mode == 'greedy':
                torch.argmax(logits, dim=1, out=actions)
            else:
                P.sample(logits, seed, step, actions, logp)
            _, out = env.step(actions, active=active)
            returns += active * out[:, 0]
            ended = active & (out[:, 1] > 0)
            terminal[ended] = out[ended]
            active &= ~ended
            if not bool(active.any()):
                break
        if bool(active.any()):
            raise RuntimeError('an evaluation episode did not end within the decision limit')
        t, r = terminal.cpu(), returns.cpu()
        return dict(clear_rate=t[:, 2].mean().item(), kills=t[:, 3].mean().item(), death_rate=t[:, 6].mean().item(),
                    timeout_rate=t[:, 7].mean().item(), turns=t[:, 5].mean().item(), shaped_return=r.mean().item())
