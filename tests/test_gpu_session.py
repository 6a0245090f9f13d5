"""The step loop driving the HIP operator on the GPU: a toy transformer whose forward runs
two attention layers of the operator on per-step drifted inputs, against the same loop
driving the HIP operator by hand and the same loop driving the CPU oracle."""

from __future__ import annotations

import dataclasses
import math

import pytest
import torch

import oracle as O
from gpu_util import SMALL, assert_parity, assert_sparse_parity, inject, metrics
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


class OracleSessionOperator:
    """The operator surface the step loop uses (n_streams, reset, begin_step, set_stream,
    banks_valid, attend, drain_validation) over the CPU oracle.  After each refresh the GPU
    operator's refinement state of that layer is handed to the oracle, so every later sparse
    call runs on identical state; ``check(step, kind, layer, inputs, oracle_out)`` sees
    every computed call."""

    n_streams = 1

    def __init__(self, wl, perm, gpu_op, check):
        self.wl, self.perm, self.gpu_op, self.check = wl, perm, gpu_op, check
        self.reset()

    def reset(self):
        wl = self.wl
        self.ref = O.OracleOperator(wl.grid, wl.text_tokens, wl.text_first, wl.density,
                                    permutation=self.perm)
        self.refreshed: dict[int, int] = {}
        self.pending: list[tuple[int, torch.Tensor]] = []
        self.step, self.kind = 0, None

    def begin_step(self, step, kind):
        self.step, self.kind = step, kind

    def set_stream(self, stream):
        assert stream == 0

    @property
    def banks_valid(self):
        return len(self.refreshed) == LAYERS

    def attend(self, layer, q, k, v):
        qc, kc, vc = (x.cpu() for x in (q, k, v))
        ref = self.ref
        if self.kind == EXACT:
            b, h, n, d = qc.shape
            dense, _ = O.dense_attention(ref._banks(qc), ref._banks(kc), ref._banks(vc),
                                         1.0 / math.sqrt(d))
            out32 = O.restore(dense, ref.inv).reshape(b, h, n, d)
            out = out32.to(qc.dtype)
        elif self.kind == REFRESH:
            out = ref.refresh(layer, qc, kc, vc)
            out32 = ref.last["out_f32"]
            stats = ref.layers[layer].pending_stats
            if stats is not None:
                self.pending.append((self.step - self.refreshed[layer], stats))
            self.refreshed[layer] = self.step
            inject(ref, self.gpu_op, layer, self.wl)
        else:
            out = ref.sparse(layer, qc, kc, vc)
            out32 = ref.last["out_f32"]
        self.check(self.step, self.kind, layer, (qc, kc, vc), out32)
        return out.to(q.device)

    def drain_validation(self):
        if not self.pending:
            return None
        num, den = torch.stack([s for _, s in self.pending]).double().sum(dim=0).tolist()
        age = min(a for a, _ in self.pending)
        self.pending = []
        return age, math.sqrt(num / den) if den > 0 else float("inf")


class RecordingTransformer(ToyTransformer):
    """ToyTransformer whose forward keeps each layer's output, by (step, layer)."""

    def __init__(self, op, inputs):
        super().__init__(op, inputs)
        self.calls = {}

    def forward(self, t):
        q, k, v = self.inputs[t]
        outs = []
        for layer in range(LAYERS):
            o = self.op.attend(layer, q, k, v)
            self.calls[(t, layer)] = o.detach().clone()
            outs.append(o.float())
        return (torch.stack(outs),)


def test_session_with_the_gpu_operator_matches_the_session_with_the_oracle(cuda):
    """The step loop driving the HIP operator against the same loop driving the CPU oracle
    (the GPU's refinement state handed over after each refresh): the same action at every
    step, every computed call within the parity bar of the oracle's (the sparse calls with
    the gate and head-rounding alternates), validation errors within 2e-3 with the same
    ages and verdicts, and the fitted gains within 2e-3 (fits to step differences of bf16
    outputs that each side rounds its own way; the inputs move 2% per step, well above
    that rounding)."""
    wl = SMALL["text-last-d128"]
    steps = 14
    base = make_qkv(wl, seed=4, device=cuda)
    # A straight path base + 0.02 t xi: the outputs move ~2% per step, well above the bf16
    # rounding of either side, so both sessions fit their gains to the same motion.
    inputs = [tuple(perturb(x, 0.02 * t, seed=i, step=1) for i, x in enumerate(base))
              for t in range(steps)]
    cfg = dataclasses.replace(
        RecapConfig(), sync_step_timing=False,
        geometry=GeometryConfig(grid=wl.grid, text_tokens=wl.text_tokens),
        schedule=ScheduleConfig(num_steps=steps, tau=0.5, detail_tau_mult=1.0))
    perm = hilbert_permutation(wl.grid)
    gpu_op = make_operator(wl)
    gpu_tr = RecordingTransformer(gpu_op, inputs)
    gpu_session = RecapSession(cfg, gpu_op)
    gpu_session.install(gpu_tr)

    checked = {EXACT: 0, REFRESH: 0, SPARSE: 0}

    def check(t, kind, layer, qkv, want):
        got = gpu_tr.calls[(t, layer)]
        what = f"step {t} {kind} layer {layer}"
        if kind == SPARSE:
            assert_sparse_parity(got, oracle_op.ref, gpu_op, *qkv, wl, cuda, what, layer=layer)
        else:
            assert_parity(got.cpu().float(), want, what)
        checked[kind] += 1

    oracle_op = OracleSessionOperator(wl, perm, gpu_op, check)
    oracle_tr = RecordingTransformer(oracle_op, inputs)
    oracle_session = RecapSession(cfg, oracle_op)
    oracle_session.install(oracle_tr)

    gains = []
    for t in range(steps):
        out_g = gpu_tr.forward(t)[0]
        out_o = oracle_tr.forward(t)[0]
        a_g, a_o = gpu_session.actions[-1]["a"], oracle_session.actions[-1]["a"]
        print(f"  step {t}: {a_g} / {a_o}, gain {gpu_session.gain:.4f} / "
              f"{oracle_session.gain:.4f}", flush=True)
        row_g, row_o = gpu_session.actions[-1], oracle_session.actions[-1]
        if "m" in row_g:
            print(f"    miss m {row_g['m']} / {row_o.get('m')}", flush=True)
        assert a_g == a_o, (t, a_g, a_o)
        gains.append((gpu_session.gain, oracle_session.gain))
        if a_g == REUSE:
            m, _ = metrics(out_g.cpu(), out_o.cpu())
            print(f"    reused output: max-abs between the two sessions {m:.3e}", flush=True)
    val_g = [r["validation"] for r in gpu_session.actions if "validation" in r]
    val_o = [r["validation"] for r in oracle_session.actions if "validation" in r]
    print(f"  validations gpu {val_g} oracle {val_o}; checked calls {checked}", flush=True)
    assert [v["age"] for v in val_g] == [v["age"] for v in val_o]
    assert [v["passed"] for v in val_g] == [v["passed"] for v in val_o]
    for vg, vo in zip(val_g, val_o):
        assert abs(vg["error"] - vo["error"]) < 2e-3
    actions = [r["a"] for r in gpu_session.actions]
    print(f"  schedule {actions}", flush=True)
    assert {EXACT, REFRESH, SPARSE, REUSE} <= set(actions) and checked[SPARSE] > 0
    # the gains are fits to differences of bf16 outputs, each side rounded its own way
    assert max(abs(a - b) for a, b in gains) <= 2e-3, gains


def test_two_stream_session_with_host_banks_equals_resident(cuda):
    """Two transformer calls per step (two guidance branches, as Wan runs them,
    recap/models/wan.py:22) through the step loop, once with resident banks and once with
    host banks: the same actions, and every output equal bit for bit."""
    from recap_amd import HostBankOperator

    wl = SMALL["video-ragged-d128"]
    steps = 12
    base = [make_qkv(wl, seed=30 + s, device=cuda) for s in range(2)]
    inputs = [[tuple(perturb(x, 0.02 * t, seed=10 * s + i, step=1) for i, x in enumerate(base[s]))
               for s in range(2)] for t in range(steps)]
    cfg = dataclasses.replace(
        RecapConfig(), sync_step_timing=False,
        geometry=GeometryConfig(grid=wl.grid, text_tokens=wl.text_tokens),
        schedule=ScheduleConfig(num_steps=steps, tau=0.5, detail_tau_mult=1.0))
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=wl.text_first)
    geo = SparseGeometry.build(layout, 128)

    class TwoCalls:
        def __init__(self, op):
            self.op, self.calls = op, 0

        def forward(self, t):
            q, k, v = inputs[t][self.calls % 2]
            self.calls += 1
            return (torch.stack([self.op.attend(layer, q, k, v).float()
                                 for layer in range(LAYERS)]),)

    runs = []
    for cls, host in ((Operator, False), (HostBankOperator, True)):
        op = cls.build(OperatorConfig(head_density=wl.density, host_banks=host), geo,
                       n_layers=LAYERS, n_streams=2)
        tr = TwoCalls(op)
        session = RecapSession(cfg, op, calls_per_step=2)
        session.install(tr)
        outs = [tr.forward(t)[0] for t in range(steps) for _ in range(2)]
        if host:
            op.finish()
            print(f"  pager counts {op.pager_counts()}", flush=True)
        runs.append(([r["a"] for r in session.actions], outs))
    print(f"  schedule {runs[0][0]}", flush=True)
    assert runs[0][0] == runs[1][0]
    assert {REFRESH, SPARSE} <= set(runs[0][0])
    for i, (a, b) in enumerate(zip(runs[0][1], runs[1][1])):
        assert torch.equal(a, b), i
