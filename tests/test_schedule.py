"""The routed-block budget schedule of training (dash_attention.py:272-341), host
logic only: endpoints, the geometric path, which calls move the clock."""

from types import SimpleNamespace

import torch

from ananta_ocr_amd.dash_attention import KSchedule


def test_geometric_path_and_endpoints():
    ks = KSchedule()
    ks.k_start, ks.k_end, ks.steps = 64, 12, 1000
    assert ks.k_for(0) == 64
    assert ks.k_for(1000) == 12 and ks.k_for(5000) == 12 and ks.k_for(-3) == 64
    # 64 * (12/64)^(1/2) = 27.71...
    assert ks.k_for(500) == 28
    seq = [ks.k_for(s) for s in range(0, 1001, 50)]
    assert all(a >= b for a, b in zip(seq, seq[1:]))
    ks.k_start, ks.k_end = 8, 32                     # an increasing schedule is clamped too
    assert ks.k_for(0) == 8 and ks.k_for(2000) == 32


def test_only_the_leader_in_training_moves_the_clock():
    ks = KSchedule()
    ks.k_start, ks.k_end, ks.steps = 64, 12, 4
    a, b = ks.register(), ks.register()
    ks.advance(b, True)                               # not the leader
    assert ks.micro == 0 and ks.k == 64
    ks.advance(a, False)                              # eval
    assert ks.micro == 0
    ks.advance(a, True)                               # no trainer state: micro-batch clock
    assert ks.micro == 1 and ks.step == 1 and ks.k == ks.k_for(1)


def test_attached_trainer_state_is_the_clock():
    ks = KSchedule()
    ks.k_start, ks.k_end, ks.steps = 64, 12, 100
    sid = ks.register()
    ks.attach(SimpleNamespace(global_step=100))
    ks.advance(sid, True)
    assert ks.step == 100 and ks.k == 12


def test_replay_inside_backward_does_not_advance():
    ks = KSchedule()
    sid = ks.register()
    x = torch.ones(2, requires_grad=True)

    class Probe(torch.autograd.Function):
        @staticmethod
        def forward(ctx, t):
            return t.clone()

        @staticmethod
        def backward(ctx, g):
            ks.advance(sid, True)                      # as a checkpoint recompute would
            return g

    ks.state = SimpleNamespace(global_step=0)
    Probe.apply(x).sum().backward()
    assert ks.micro == 0
