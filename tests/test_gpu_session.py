"""The step loop driving the HIP operator on the GPU: a toy transformer whose forward runs
two attention layers of the operator on per-step drifted inputs."""

from __future__ import annotations

import dataclasses

import pytest
import torch

from gpu_util import SMALL
from recap_amd import EXACT, REFRESH, REUSE, SPARSE, Operator, OperatorConfig, RecapSession
from recap_amd.config import GeometryConfig, RecapConfig, ScheduleConfig
from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
from recap_amd.synthetic import make_qkv, perturb

pytestmark = pytest.mark.gpu

LAYERS = 2


def make_operator(wl):
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=wl.text_first)
    return Operator.build(OperatorConfig(head_density=wl.density),
                          SparseGeometry.build(layout, 128), n_layers=LAYERS)


class ToyTransformer:
    """forward(t): the sum of LAYERS attention layers of the operator at step t's inputs."""

    def __init__(self, op, inputs):
        self.op, self.inputs = op, inputs

    def forward(self, t):
        q, k, v = self.inputs[t]
        out = None
        for layer in range(LAYERS):
            o = self.op.attend(layer, q, k, v).float()
            out = o if out is None else out + o
        return (out,)


def test_session_drives_the_operator_and_extrapolates(cuda):
    wl = SMALL["text-last-d128"]
    steps = 14
    base = make_qkv(wl, seed=4, device=cuda)
    inputs, cur = [], base
    for t in range(steps):
        cur = tuple(perturb(x, 0.002, seed=i, step=t + 1) for i, x in enumerate(cur))
        inputs.append(cur)
    cfg = dataclasses.replace(
        RecapConfig(), sync_step_timing=False,
        geometry=GeometryConfig(grid=wl.grid, text_tokens=wl.text_tokens),
        schedule=ScheduleConfig(num_steps=steps, tau=0.5, detail_tau_mult=1.0))
    op = make_operator(wl)
    tr = ToyTransformer(op, inputs)
    session = RecapSession(cfg, op)
    session.install(tr)
    outs, gains = [], []
    for t in range(steps):
        outs.append(tr.forward(t)[0])
        gains.append(session.gain)  # changes only on computed steps
    actions = [row["a"] for row in session.actions]
    print("schedule:", actions, "gain", session.gain, flush=True)
    assert {REFRESH, SPARSE, REUSE} <= set(actions), actions
    assert actions[0] == EXACT

    # An independent operator driven by hand with the same decisions gives the same
    # outputs on every computed step; a reused step is o + g h v from the last two
    # computed outputs, with the gain fitted up to the previous step.
    ref_op = make_operator(wl)
    ref = ToyTransformer(ref_op, inputs)
    computed = []  # (t, output)
    for t, action in enumerate(actions):
        if action == REUSE:
            (t1, o1), (t0, o0) = computed[-1], computed[-2]
            v = (o1 - o0) / float(t1 - t0)
            expected = o1 + v * (gains[t - 1] * float(t - t1))
            torch.testing.assert_close(outs[t], expected, rtol=1e-6, atol=1e-6)
            continue
        ref_op.begin_step(t, action)
        out = ref.forward(t)[0]
        assert torch.equal(out, outs[t]), (t, action)
        computed.append((t, out))
