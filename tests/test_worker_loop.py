"""The trainer's worker loop (Trainer.run, the reference's gpu-d1/scripts/
run_ring_ablations.py:291-295,341-388) on the CPU: a SIGTERM stops at the next update
boundary with a checkpoint and status 130, the same call resumes to the end, periodic
checkpoints land on their boundaries, and a non-finite loss aborts without persisting past
the last finite update. The rollout/update pair is a host stand-in, so no GPU is needed;
the GPU trainer's own checkpoint contents are checked in test_train_gpu.py."""
import importlib
import os
import signal

import pytest
import torch


class FakeTrainer:
    """Trainer.run over a counter 'model': each update adds 1 to the weight."""

    def __init__(self, T=4, N=8, bad_at=None):
        train = importlib.import_module('dcss-auto_amd.train')
        self.run = train.Trainer.run.__get__(self)
        self.save_impl = train.Trainer.save
        self.T, self.N, self.bad_at = T, N, bad_at
        self.decisions, self.updates, self.w = 0, 0, 0
        self.saves = []

    def rollout(self):
        self.decisions += self.T * self.N

    def update(self):
        if self.bad_at is not None and self.updates + 1 == self.bad_at:
            raise RuntimeError('Non-finite PPO loss')
        self.w += 1
        self.updates += 1
        return torch.tensor([0.0, 0.0, 0.0])

    def state_dict(self):
        return dict(decisions=torch.tensor(self.decisions), updates=torch.tensor(self.updates), w=torch.tensor(self.w))

    def save(self, path):
        self.saves.append(self.decisions)
        self.save_impl(self, path)

    def load(self, path):
        sd = torch.load(path, weights_only=True)
        self.decisions, self.updates, self.w = int(sd['decisions']), int(sd['updates']), int(sd['w'])


def test_sigterm_stops_at_an_update_boundary_and_resumes(tmp_path):
    ck = tmp_path / 'latest.pt'
    tr = FakeTrainer()

    def hook(t, terms):
        if t.updates == 3:
            os.kill(os.getpid(), signal.SIGTERM)

    before = signal.getsignal(signal.SIGTERM)
    assert tr.run(40 * 32, checkpoint=ck, on_update=hook) == 130
    assert signal.getsignal(signal.SIGTERM) is before            # handlers restored
    sd = torch.load(ck, weights_only=True)
    assert int(sd['updates']) == 3 and int(sd['w']) == 3 and int(sd['decisions']) == 3 * 32
    resumed = FakeTrainer()
    assert resumed.run(40 * 32, checkpoint=ck) == 0               # the same call resumes
    assert resumed.updates == 40 and resumed.w == 40 and int(torch.load(ck, weights_only=True)['updates']) == 40
    assert not [p for p in os.listdir(tmp_path) if '.tmp' in p]  # atomic writes leave no partial file


def test_periodic_checkpoints_fall_on_their_boundaries(tmp_path):
    tr = FakeTrainer()
    assert tr.run(10 * 32, checkpoint=tmp_path / 'c.pt', checkpoint_every=100) == 0
    # 32 decisions per update: boundaries 100, 200, 300 are crossed at 128, 224, 320; the
    # final save at 320 follows
    assert tr.saves == [128, 224, 320, 320]


def test_non_finite_loss_aborts_without_persisting(tmp_path):
    ck = tmp_path / 'c.pt'
    tr = FakeTrainer(bad_at=5)
    with pytest.raises(RuntimeError, match='Non-finite'):
        tr.run(10 * 32, checkpoint=ck, checkpoint_every=64)
    sd = torch.load(ck, weights_only=True)
    assert int(sd['updates']) == 4 and int(sd['w']) == 4           # the last finite update


def test_run_without_checkpoint_or_signals():
    tr = FakeTrainer()
    assert tr.run(5 * 32, handle_signals=False) == 0 and tr.updates == 5
