#!/usr/bin/env python3
"""Benchmark of the corrected sparse-attention call on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload hunyuan-720p] [--no-sequence]
                    [--no-secondary]

One "step" is one corrected SPARSE call (Operator.attend after a REFRESH) at the
HunyuanVideo-720p shape: B=1, 24 heads x 128, 118,800 video + 256 text tokens, 128-token
blocks, 20% density, bf16, inputs resident in HBM and drifted 2% from the refresh inputs.
The timed region is K calls bracketed by torch.cuda.synchronize(); per-stage durations come
from HIP events recorded on the same stream inside the timed calls.  The default run then adds
the other reference shapes (Wan2.1-480p and CogVideoX-1.5: sparse call and dense SDPA, under
"workloads") and the ten-step schedule with refinement banks paged through pinned host memory
(20 layers, REFRESH at steps 0 and 5; ms_per_step_host_banks, copy_overlap_fraction).  Prints
one JSON line.
"""

from __future__ import annotations

import argparse
import gc
import hashlib
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ms per corrected sparse-attn call @Hunyuan 720p shape; eff. TFLOP/s vs dense"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of the attention kernel, measured with rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes scaled by a plain copy of known size (the file records the commands).
TRAFFIC_FILE = ROOT / "profiles" / "attention_hunyuan720p_traffic.md"
COPY_CAL_BYTES = 1 << 30
# The other reference shapes the default run also times (sparse call and dense SDPA).
SECONDARY = ("wan2.1-480p", "cogvideox1.5")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def kept_flops(kmask, n_tokens: int, dim: int) -> float:
    """4 d sum over kept (i, j) block pairs of n_i n_j (ragged counts)."""
    import torch
    tb = kmask.shape[-1]
    n = torch.full((tb,), 128.0, dtype=torch.float64, device=kmask.device)
    n[-1] = n_tokens - 128 * (tb - 1)
    pair = n.view(-1, 1) * n.view(1, -1)
    return float((kmask.to(torch.float64) * pair).sum()) * 4.0 * dim


def elapsed_stages(events: dict) -> dict:
    names = ["start", "pack", "closure", "coarse", "attention"]
    out = {}
    for a, b in zip(names[:-1], names[1:]):
        pairs = list(zip(events[a], events[b]))
        out[b] = sum(s.elapsed_time(e) for s, e in pairs) / len(pairs)
    return out


def recorded_traffic(workload: str) -> float | None:
    """HBM bytes per attention launch from the committed rocprof summary, if it covers
    this workload (a line 'traffic_bytes_per_launch <workload> <bytes>')."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.strip().strip("`").split()
        if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == workload:
            return float(parts[2])
    return None


def gemm_peak_tflops(n: int = 8192, reps: int = 10) -> float:
    """Measured bf16 GEMM rate of the vendor library (torch.matmul -> hipBLASLt) on random
    N(0,1) operands: the practical MFMA ceiling on this box (random data draws more power
    than the published peak assumes)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(7)
    a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
    b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
    for _ in range(3):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        torch.matmul(a, b)
    e.record()
    torch.cuda.synchronize()
    return 2.0 * n ** 3 * reps / (s.elapsed_time(e) / 1e3) / 1e12


def copy_calibration(reps: int = 5) -> int:
    """A plain device copy of COPY_CAL_BYTES, the known-size reference for the FETCH_SIZE /
    WRITE_SIZE counters: each dispatch reads and writes exactly COPY_CAL_BYTES."""
    import torch
    x = torch.empty(COPY_CAL_BYTES // 2, dtype=torch.bfloat16, device="cuda").normal_()
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_CAL_BYTES, "dispatches": reps}), flush=True)
    return 0


def step_sequence(wl, layers: int, steps: int, refresh_at: tuple, drift: float) -> dict:
    """The multi-step schedule with paged refinement banks (one JSON object).

    Every step runs `layers` attention layers; steps in `refresh_at` are REFRESH, the others
    SPARSE; inputs drift by `drift` (fresh N(0,1) noise) each step and are shared by the
    layers (each layer keeps its own banks).  Run twice: banks in pinned host memory paged
    through two GPU slots with layer-ahead prefetch (HostBankOperator), and banks resident
    on the GPU (Operator).  copy-overlap fraction = 1 - exposed / total copy time, where
    total = the HIP-event durations of every host<->device bank copy on its stream and
    exposed = the paged run's extra time over the resident run."""
    import torch

    from recap_amd import HostBankOperator, Operator, OperatorConfig, REFRESH, SPARSE
    from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
    from recap_amd.synthetic import make_qkv, perturb

    dev = torch.device("cuda:0")
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=wl.text_first)
    geometry = SparseGeometry.build(layout, 128)

    def step_inputs():
        """The drifting inputs step by step (each step's from the previous one); generated
        outside the timed region of its step, and identical for both runs."""
        x = make_qkv(wl, seed=0, device=dev)
        for step in range(steps):
            x = tuple(perturb(t, drift, seed=i, step=step + 1) for i, t in enumerate(x))
            yield x

    def run(cls, host: bool):
        cfg = OperatorConfig(head_density=wl.density, host_banks=host)
        op = cls.build(cfg, geometry, n_layers=layers)
        if host:
            op.record_copies = True
            op.preallocate_host(layers, wl.heads, wl.dim)
        times, outs = [], None
        for step, (q, k, v) in enumerate(step_inputs()):
            kind = REFRESH if step in refresh_at else SPARSE
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            op.begin_step(step, kind)
            for layer in range(layers):
                out = op.attend(layer, q, k, v)
                if layer == layers - 1:
                    outs = out
            end.record()
            torch.cuda.synchronize()
            times.append((kind, start.elapsed_time(end)))
            log(f"[sequence] {'host' if host else 'gpu'} banks step {step} {kind}: "
                f"{times[-1][1]:.1f} ms")
        copy_ms = 0.0
        host_bytes = 0
        counts = {}
        if host:
            op.finish()
            copy_ms, _ = op.copy_time()
            host_bytes = op.peak_bank_bytes()
            counts = op.pager_counts()
        del op
        torch.cuda.empty_cache()
        return times, copy_ms, host_bytes, outs.clone(), counts

    # Untimed warm-up of both operators on two layers and two steps: the process's first
    # refresh pays one-time costs (code loading, first-call setup, ~0.15 s), which would
    # otherwise land on whichever timed run goes first and read as exposed copy time.
    for cls, host in ((HostBankOperator, True), (Operator, False)):
        op = cls.build(OperatorConfig(head_density=wl.density, host_banks=host), geometry,
                       n_layers=2)
        for step, (q, k, v) in zip(range(2), step_inputs()):
            op.begin_step(step, REFRESH if step == 0 else SPARSE)
            for layer in range(2):
                op.attend(layer, q, k, v)
        if host:
            op.finish()
        del op
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    t_host, copy_ms, host_bytes, out_host, counts = run(HostBankOperator, True)
    t_gpu, _, _, out_gpu, _ = run(Operator, False)
    total_host = sum(t for _, t in t_host)
    total_gpu = sum(t for _, t in t_gpu)
    exposed = max(0.0, total_host - total_gpu)
    mean = lambda xs: sum(xs) / len(xs) if xs else None  # noqa: E731
    return {
        "sequence": f"{wl.name}: {layers} layers x {steps} steps, REFRESH at "
                    f"{list(refresh_at)}, SPARSE otherwise, {drift:.0%} input drift per step",
        "ms_per_step_host_banks": round(total_host / steps, 2),
        "ms_per_step_gpu_banks": round(total_gpu / steps, 2),
        "ms_per_refresh_step_host_banks": round(mean([t for k, t in t_host if k == REFRESH]), 2),
        "ms_per_sparse_step_host_banks": round(mean([t for k, t in t_host if k == SPARSE]), 2),
        "copy_ms_total": round(copy_ms, 2),
        "exposed_copy_ms": round(exposed, 2),
        "copy_overlap_fraction": round(1.0 - exposed / copy_ms, 4) if copy_ms > 0 else None,
        "host_bank_bytes": host_bytes,
        "pager_counts": counts,
        "outputs_identical": bool(torch.equal(out_host, out_gpu)),
    }


def refresh_calls(wl, count: int) -> dict:
    """A first REFRESH (selection, basis, capture) and then ``count`` revalidating REFRESH
    calls on inputs drifted 3% each, which score the previous refinement, select again and
    decide the rerank; per-call wall time from HIP events (one JSON object)."""
    import torch

    from recap_amd import Operator, OperatorConfig, REFRESH
    from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
    from recap_amd.synthetic import make_qkv, perturb

    dev = torch.device("cuda:0")
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=wl.text_first)
    op = Operator.build(OperatorConfig(head_density=wl.density), SparseGeometry.build(layout, 128),
                        n_layers=1)
    x = make_qkv(wl, seed=0, device=dev)
    times = []
    for call in range(count + 1):
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        op.begin_step(call, REFRESH)
        op.attend(0, *x)
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
        log(f"[refresh] call {call}: {times[-1]:.1f} ms")
        x = tuple(perturb(t, 0.03, seed=i, step=call + 1) for i, t in enumerate(x))
    age, error = op.drain_validation()
    return {"refresh": f"{wl.name}: a first REFRESH, then {count} revalidating REFRESH calls "
                       "(3% drift each)", "first_ms": round(times[0], 2),
            "revalidating_ms": [round(t, 2) for t in times[1:]], "last_validation_error":
            round(error, 6)}


def band_sweep(wl, keeps=(4, 16, 48, 96, 186, 280), reps: int = 10) -> dict:
    """The merge kernel's time against the kept tiles per row, on the workload's inputs with
    synthetic band masks (each video query block keeps the ``keep`` key blocks centred on
    itself; the kernel-mask expansion adds the text rows and columns): the work items stay
    fixed while the tile steps grow, which separates the per-step cost from the per-item
    one.  The drift weight is fixed at 0.5 (no drift inputs)."""
    import torch

    from recap_amd import kernels as K
    from recap_amd.layout import Layout, hilbert_permutation
    from recap_amd.synthetic import make_qkv

    dev = torch.device("cuda:0")
    q, k, v = make_qkv(wl, seed=0, device=dev)
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=wl.text_first)
    rowmap = layout.rowmap(dev)
    geo = K.Geometry(wl.tokens, wl.video_tokens)
    kv = K.kv_pack(k, v, rowmap, geo)
    banks, nb, rows, d = wl.heads, geo.nb, geo.rows, wl.dim
    g = torch.Generator(device=dev).manual_seed(1)
    go = torch.randn(banks, rows, d, device=dev, generator=g).to(q.dtype)
    gl = torch.randn(banks, rows, device=dev, generator=g)
    det = (0.1 * torch.randn(banks, rows, d, device=dev, generator=g)).to(torch.float16)
    dl = torch.randn(banks, rows, device=dev, generator=g)
    idx = torch.arange(nb, device=dev)
    out = []
    for keep in keeps:
        lo = (idx - keep // 2).clamp(0, max(nb - keep, 0))
        part = (idx[None, :] >= lo[:, None]) & (idx[None, :] < lo[:, None] + keep)
        kmask = K.kernel_block_mask(part[None].expand(banks, nb, nb).contiguous(), geo)
        steps = int(kmask.sum())
        call = lambda: K.sparse_merge_attn(q, kv, rowmap, kmask, geo, d ** -0.5, go, gl,  # noqa: E731
                                           det, dl, None, None, alpha_override=0.5)
        for _ in range(3):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        log(f"[band] keep {keep}: {steps} tile steps, {ms:.3f} ms, {ms * 1e6 / steps:.2f} ns/step")
        out.append({"keep": keep, "tile_steps": steps, "ms": round(ms, 4),
                    "ns_per_step": round(ms * 1e6 / steps, 3)})
    return {"band_sweep": wl.name, "items": banks * geo.tb, "points": out}


def cpu_baseline(op, q1, k1, v1, wl, heads: int) -> dict:
    """The oracle's sparse call on the host for ``heads`` of the heads (all query blocks),
    timed with the operator's refinement state; heads are independent and cost the same,
    so the whole call is that time x (all heads / sampled heads)."""
    import torch

    import oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    bank = op.banks[0][0]
    layer = op.layers[0][0]
    perm = op.layout.permutation.numpy()
    fwd, _ = O.gather_indices(perm, wl.text_tokens, wl.text_first)
    geo = O.block_geometry(wl.video_tokens, wl.tokens)
    nb, rows = geo["nb"], geo["rows"]
    q, k, v = (x[:, :heads].cpu() for x in (q1, k1, v1))
    part = bank.partition[:, :heads].cpu().reshape(heads, nb, nb)
    kmask = bank.head_kernel_mask[:heads].cpu()
    det, dl = bank.value[:heads].cpu().float(), bank.log_mass[:heads].cpu()
    glref, basis = bank.coarse_lse[:heads].cpu(), layer.basis[:heads].cpu()
    scale = 1.0 / math.sqrt(wl.dim)

    t0 = time.perf_counter()
    ql, kl, vl = (O.reorder(x, fwd)[0] for x in (q, k, v))
    km, counts = O.pool_blocks(kl, wl.video_tokens)
    vm, _ = O.pool_blocks(vl, wl.video_tokens)
    _, var = O.rotated_moments(kl, basis, counts, wl.video_tokens)
    cvk = O.value_key_covariance(kl, vl, km, counts, wl.video_tokens)
    w = O.fold_rank(var, 4)
    qv = ql[:, :wl.video_tokens].float()
    qsq = O.rotated_query_square(qv, basis, torch.bfloat16)
    drift = O.value_drift(qv, cvk, scale, torch.bfloat16)
    oh, lh = O.block_sparse_attention(ql, kl, vl, kmask, scale, acc=torch.float32)
    go, gl = O.coarse_tail(ql, qsq, drift, km, vm, w, counts, part, scale, 2.0,
                           wl.video_tokens, torch.bfloat16)
    go, gl = go[:, :rows], gl[:, :rows]
    center = O.drift_center(gl, glref)
    merged = O.sparse_merge(oh, lh, go, gl, det, dl, rows, glref, center)
    O.restore(merged.to(torch.bfloat16).unsqueeze(0), torch.argsort(fwd))
    seconds = time.perf_counter() - t0
    return {
        "value": round(seconds * 1e3 * wl.heads / heads, 1),
        "unit": "ms/call",
        "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"oracle (torch CPU, fp32 attention) sparse call on {heads} of {wl.heads} "
                   f"heads, all {rows // 128} query blocks: {seconds:.2f} s measured, scaled "
                   f"x{wl.heads / heads:g} (heads are independent and equal in cost)"),
        "cpu": cpu_model(),
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the machine type where that is absent."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def time_sparse_calls(op, q, k, v, steps: int, warmup: int) -> tuple[float, float, dict]:
    """(mean ms per SPARSE call over ``steps`` timed calls after ``warmup`` untimed ones,
    median ms per call, mean ms per stage) with HIP events recorded on the launch stream.
    Python's garbage collector is paused over the timed calls: a collection pauses the host
    for ~10-20 ms, which drains the launch queue of a short call (1.7 ms at the Wan shape)."""
    import torch

    from recap_amd import SPARSE

    op.begin_step(1, SPARSE)
    for _ in range(warmup):
        op.attend(0, q, k, v)
    torch.cuda.synchronize()
    op.stage_events = {}
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gc.collect()
    gc.disable()
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        op.attend(0, q, k, v)
    end.record()
    torch.cuda.synchronize()
    gc.enable()
    ms = start.elapsed_time(end) / steps
    stages = elapsed_stages(op.stage_events)
    ev = op.stage_events
    per_call = sorted(a.elapsed_time(b) for a, b in zip(ev["start"], ev["attention"]))
    op.stage_events = None
    return ms, per_call[len(per_call) // 2], stages


def dense_sdpa_ms(q, k, v, reps: int) -> float:
    """torch SDPA (the reference's EXACT path) on the same inputs, mean of ``reps``."""
    import torch
    import torch.nn.functional as F

    F.scaled_dot_product_attention(q, k, v)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        F.scaled_dot_product_attention(q, k, v)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def secondary_workload(wl, steps: int, warmup: int, dense_reps: int) -> dict:
    """One other reference shape, timed like the headline: a REFRESH, then ``steps`` SPARSE
    calls on inputs drifted 2%, and dense SDPA on the same inputs (one JSON object)."""
    import torch

    from recap_amd import Operator, OperatorConfig, REFRESH
    from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
    from recap_amd.synthetic import make_qkv, perturb

    dev = torch.device("cuda:0")
    q0, k0, v0 = make_qkv(wl, seed=0, device=dev)
    q1, k1, v1 = (perturb(x, 0.02, seed=0, step=1) for x in (q0, k0, v0))
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=wl.text_first)
    op = Operator.build(OperatorConfig(head_density=wl.density), SparseGeometry.build(layout, 128),
                        n_layers=1)
    op.begin_step(0, REFRESH)
    op.attend(0, q0, k0, v0)
    del q0, k0, v0
    ms, median_ms, stages = time_sparse_calls(op, q1, k1, v1, steps, warmup)
    kept = kept_flops(op.banks[0][0].head_kernel_mask, wl.tokens, wl.dim)
    dense = dense_sdpa_ms(q1, k1, v1, dense_reps)
    out = {"config": {"heads": wl.heads, "head_dim": wl.dim, "tokens": wl.tokens,
                      "text_tokens": wl.text_tokens, "text_first": wl.text_first,
                      "density": wl.density},
           "ms_per_call": round(ms, 4), "median_ms_per_call": round(median_ms, 4),
           "stages_ms": {k: round(v, 4) for k, v in stages.items()},
           "roofline_frac": round(kept / (stages["attention"] / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
           "kept_block_tflop": round(kept / 1e12, 4),
           "dense_sdpa_ms": round(dense, 3),
           "speedup_vs_dense_sdpa": round(dense / ms, 2),
           "effective_tflops": round(wl.dense_flops() / 1e12 / (ms / 1e3), 2)}
    del op
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="hunyuan-720p")
    ap.add_argument("--dense-reps", type=int, default=3)
    ap.add_argument("--cpu-heads", type=int, default=3,
                    help="heads of the CPU baseline sample (0 = skip)")
    ap.add_argument("--profile", action="store_true",
                    help="only the sparse calls (no dense comparator, no CPU baseline)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy (counter calibration under rocprofv3)")
    ap.add_argument("--sequence", action="store_true",
                    help="run only the step sequence with paged banks (20 layers, 10 steps, "
                         "REFRESH at 0 and 5, 3%% drift) and print its JSON line")
    ap.add_argument("--layers", type=int, default=20, help="layers of the step sequence")
    ap.add_argument("--no-sequence", action="store_true",
                    help="skip the paged step sequence of the default run")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other reference shapes (Wan2.1, CogVideoX) of the default run")
    ap.add_argument("--band-sweep", action="store_true",
                    help="run only the merge kernel with synthetic band masks of 4-280 kept "
                         "blocks per row (per-step against per-item cost) and print its JSON")
    ap.add_argument("--refresh", type=int, default=0, metavar="K",
                    help="run only K revalidating REFRESH calls after a first one (the "
                         "selection, the capture with validation, the rerank overlap) and "
                         "print their timing; a profiling target for those kernels")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} is not supported in this build "
              "(the operator shards over heads with no exchange; multi-GPU runs are not "
              "measured here)", file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration()

    import torch

    from recap_amd import Operator, OperatorConfig, REFRESH
    from recap_amd import _lib
    from recap_amd import kernels as K
    from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
    from recap_amd.synthetic import WORKLOADS, make_qkv, perturb

    _lib.load()
    wl = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    if args.sequence:
        print(json.dumps(step_sequence(wl, args.layers, 10, (0, 5), 0.03)), flush=True)
        return 0
    if args.refresh > 0:
        print(json.dumps(refresh_calls(wl, args.refresh)), flush=True)
        return 0
    if args.band_sweep:
        print(json.dumps(band_sweep(wl)), flush=True)
        return 0
    log(f"[bench] workload {wl.name}: heads={wl.heads} d={wl.dim} N={wl.tokens}")
    q0, k0, v0 = make_qkv(wl, seed=0, device=dev)
    q1, k1, v1 = (perturb(x, 0.02, seed=0, step=1) for x in (q0, k0, v0))
    digest = hashlib.sha256()
    for x in (q1, k1, v1):  # the timed calls' inputs, native [B, H, N, d] bf16 bytes
        digest.update(x.contiguous().view(torch.uint16).cpu().numpy().tobytes())
    input_sha256 = digest.hexdigest()
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=wl.text_first)
    op = Operator.build(OperatorConfig(head_density=wl.density), SparseGeometry.build(layout, 128),
                        n_layers=1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    op.begin_step(0, REFRESH)
    op.attend(0, q0, k0, v0)
    torch.cuda.synchronize()
    refresh_ms = (time.perf_counter() - t0) * 1e3
    log(f"[bench] first refresh (dense + selection + basis + capture) {refresh_ms:.1f} ms")

    ms, median_ms, stages = time_sparse_calls(op, q1, k1, v1, args.steps, args.warmup)
    log(f"[bench] sparse call {ms:.3f} ms (median {median_ms:.3f}); stages {stages}")

    # Stage-1 selection (REFRESH-only in the reference) on the same inputs, timed alone so
    # that "call + fresh selection" can be reported.
    layer = op.layers[0][0]
    rowmap = op.layout.rowmap(dev)
    geo = op._geometry(q1)
    kv = K.kv_pack(k1, v1, rowmap, geo)
    op._select(layer, q1, kv, geo, rowmap)
    torch.cuda.synchronize()
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(3):
        op._select(layer, q1, kv, geo, rowmap)
    s1.record()
    torch.cuda.synchronize()
    select_ms = s0.elapsed_time(s1) / 3
    log(f"[bench] fresh selection {select_ms:.3f} ms")

    dense_tflop = wl.dense_flops() / 1e12
    kept = kept_flops(op.banks[0][0].head_kernel_mask, wl.tokens, wl.dim)
    attn_ms = stages["attention"]
    result = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) + 3-D sinusoidal positional field on Q/K, seed 0, 2% drift "
                "between the refresh and the timed sparse calls",
        "generator": "recap_amd.synthetic.make_qkv(workload, seed=0) then "
                     "perturb(x, 0.02, seed=0, step=1) for q, k, v",
        "input_sha256": input_sha256,
        "config": {"workload": wl.name, "batch": 1, "heads": wl.heads, "head_dim": wl.dim,
                   "tokens": wl.tokens, "video_tokens": wl.video_tokens,
                   "text_tokens": wl.text_tokens, "block": 128, "density": wl.density},
        "median_ms_per_call": round(median_ms, 4),
        "select_ms": round(select_ms, 4),
        "ms_per_call_with_fresh_selection": round(ms + select_ms, 4),
        "effective_tflops": round(dense_tflop / (ms / 1e3), 2),
        "dense_equivalent_tflop": round(dense_tflop, 3),
        "kept_block_tflop": round(kept / 1e12, 3),
        "stages_ms": {k: round(v, 4) for k, v in stages.items()},
        "refresh_ms_first_call": round(refresh_ms, 2),
        "roofline": {
            "bound": "mfma", "kernel": "attention_kernel (merge epilogue)",
            "achieved": round(kept / (attn_ms / 1e3) / 1e12, 2),
            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(kept / (attn_ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "traffic": recorded_traffic(wl.name),
        },
    }
    if not args.profile:
        dense_ms = dense_sdpa_ms(q1, k1, v1, args.dense_reps)
        result["dense_sdpa_ms"] = round(dense_ms, 3)
        result["speedup_vs_dense_sdpa"] = round(dense_ms / ms, 2)
        gemm = gemm_peak_tflops()
        result["gemm_bf16_tflops_measured"] = round(gemm, 1)
        result["roofline"]["frac_of_measured_gemm"] = round(
            result["roofline"]["achieved"] / gemm, 4)
        log(f"[bench] hipBLASLt bf16 GEMM 8192^3 (random operands): {gemm:.0f} TFLOP/s")
        log(f"[bench] dense SDPA {dense_ms:.2f} ms ({dense_tflop / dense_ms * 1e3:.0f} TFLOP/s)")
        if args.cpu_heads > 0:
            log("[bench] CPU baseline sample ...")
            result["cpu_baseline"] = cpu_baseline(op, q1, k1, v1, wl, args.cpu_heads)
            log(f"[bench] CPU baseline {result['cpu_baseline']['value']} ms/call "
                f"({result['cpu_baseline']['sample']})")
        if not args.no_secondary:
            # The other reference shapes: sparse call and dense SDPA only (no sequence, no
            # CPU leg); the headline above is unchanged.
            del op, q0, k0, v0, kv
            op = q0 = k0 = v0 = kv = None
            torch.cuda.empty_cache()
            result["workloads"] = {}
            for name in SECONDARY:
                if name == wl.name:
                    continue
                log(f"[bench] secondary workload {name} ...")
                sec = secondary_workload(WORKLOADS[name], args.steps, args.warmup,
                                         args.dense_reps)
                result["workloads"][name] = sec
                log(f"[bench] {name}: {sec['ms_per_call']} ms/call, attention frac "
                    f"{sec['roofline_frac']}, {sec['speedup_vs_dense_sdpa']}x dense SDPA")
        if not args.no_sequence:
            # The ten-step schedule with paged refinement banks: REFRESH at steps 0 and 5,
            # SPARSE otherwise, 3% drift, args.layers layers; paged vs resident banks.
            del op, q0, k0, v0, kv
            torch.cuda.empty_cache()
            seq = step_sequence(wl, args.layers, 10, (0, 5), 0.03)
            result["ms_per_step_host_banks"] = seq["ms_per_step_host_banks"]
            result["copy_overlap_fraction"] = seq["copy_overlap_fraction"]
            result["sequence"] = seq
            log(f"[bench] sequence: {seq['ms_per_step_host_banks']} ms/step paged, "
                f"{seq['ms_per_step_gpu_banks']} resident, copy overlap "
                f"{seq['copy_overlap_fraction']}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
