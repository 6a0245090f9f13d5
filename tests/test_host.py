"""Host-side checks that need no GPU: the C ABI library loads and exports every symbol
the header declares, host-only entry points, argument validation, config and layout."""

import json
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
from recap_amd import _lib, config as C, kernels as K
from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
from recap_amd.synthetic import WORKLOADS

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "recap_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(recap_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES)
    assert lib.recap_abi_version() == _lib.ABI_VERSION


def test_library_defines_its_own_symbols():
    """Every symbol of the library's own namespace that it references is defined in it: a
    HIP host pass can drop a kernel's launch stub without an error, which would otherwise
    show only when a GPU process loads the library."""
    from recap_amd.build_lib import LIB, undefined_own_symbols
    assert LIB.exists(), "build librecap_hip.so first (python -m recap_amd.build_lib)"
    assert undefined_own_symbols(LIB) == []


def test_noalloc_capture_size_limit_is_checked_on_the_host():
    """recap_refresh_capture_noalloc rejects a validation whose partial pairs exceed its
    static scratch before it touches a device (the pointers here are never dereferenced)."""
    d, n_video = 128, 128 * 64
    per_bank = int(_lib.load().recap_capture_partials(1, d, n_video))
    banks = _lib.CAPTURE_NOALLOC_MAX_PAIRS // per_bank + 1
    with pytest.raises(ValueError, match="static scratch holds"):
        _lib.call("recap_refresh_capture_noalloc", 16, _lib.RECAP_BF16, 1, banks, d,
                  banks * n_video * d, n_video * d, d, 16, 16, 16, 16, 16, 16, n_video,
                  n_video, 16, 16, 16, 16, 16, None)


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_native_hilbert_matches_oracle(name):
    grid = WORKLOADS[name].grid
    np.testing.assert_array_equal(hilbert_permutation(grid), O.hilbert_permutation(grid))


@pytest.mark.parametrize("grid", [(1, 1, 1), (1, 1, 7), (3, 5, 2), (2, 16, 16)])
def test_native_hilbert_small_grids(grid):
    np.testing.assert_array_equal(hilbert_permutation(grid), O.hilbert_permutation(grid))


def test_argument_validation_before_launch():
    # Every check below fires on the host before any HIP call.
    with pytest.raises(ValueError, match="head dim"):
        _lib.call("recap_pool_blocks", 16, _lib.RECAP_BF16, 1, 1, 96, 0, 0, 96, 16, 256, 256, 16,
                  None)
    with pytest.raises(ValueError, match="dtype"):
        _lib.call("recap_pool_blocks", 16, 7, 1, 1, 64, 0, 0, 64, 16, 256, 256, 16, None)
    with pytest.raises(ValueError, match="16-byte"):
        _lib.call("recap_pool_blocks", 18, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 256, 256, 16,
                  None)
    with pytest.raises(ValueError, match="n_tokens"):
        _lib.call("recap_kv_pack", 16, 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 0, 0, 64, 16,
                  100, 200, 16, 16, 16, 16, None)
    with pytest.raises(ValueError, match="keep"):
        _lib.call("recap_topk_blocks", 16, 1, 10, 11, 0, 16, None)
    with pytest.raises(ValueError, match="flag"):
        _lib.call("recap_closure_stats", 16, 16, 16, _lib.RECAP_BF16, 16, 16, 1, 64, 256, 256, 8,
                  _lib.CLOSURE_SCATTER, 16, 16, 16, None)
    with pytest.raises(ValueError, match="drift weight"):
        _lib.call("recap_sparse_merge_attn", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16, 16,
                  16, 256, 256, 0.125, 16, 16, 16, 16, None, None, -1.0, 16, 0, 0, 64, None, None)
    with pytest.raises(ValueError, match="work_queue"):
        _lib.call("recap_sparse_merge_attn", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16, 16,
                  16, 256, 256, 0.125, 16, 16, 16, 16, None, None, 0.5, 16, 0, 0, 64, 20, None)
    assert _lib.load().recap_attn_queue_words() == 256
    with pytest.raises(ValueError, match="kernel blocks"):
        _lib.call("recap_dense_attn", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16, 16,
                  2049 * 128, 0.125, 16, 0, 0, 64, 16, None)
    for bad in (0.0, -0.125, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="scale"):
            _lib.call("recap_dense_attn", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16, 16,
                      256, bad, 16, 0, 0, 64, 16, None)
        with pytest.raises(ValueError, match="scale"):
            _lib.call("recap_block_sparse_attn", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16,
                      16, 16, 256, bad, 16, 16, None)
    with pytest.raises(ValueError, match="scale"):
        _lib.call("recap_block_scores", 16, 16, 1, 4, 64, -0.125, 16, None)
    with pytest.raises(ValueError, match="theta"):
        _lib.call("recap_coarse_tail", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16, 16, 16,
                  16, 16, 16, 256, 256, 0.125, -1.0, 4, None, 16, 16, 16, None)
    with pytest.raises(ValueError, match="rank"):
        _lib.call("recap_coarse_tail", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16, 16, 16,
                  16, 16, 16, 256, 256, 0.125, 2.0, 65, None, 16, 16, 16, None)
    with pytest.raises(ValueError, match="video blocks"):   # the coarse kernel's row limit
        _lib.call("recap_coarse_tail", 16, _lib.RECAP_BF16, 1, 1, 64, 0, 0, 64, 16, 16, 16, 16,
                  16, 16, 16, 4097 * 128, 4097 * 128, 0.125, 2.0, 4, None, 16, 16, 16, None)
    width = _lib.load().recap_coarse_w_width
    assert width(_lib.RECAP_BF16, 128, 4) == 16 and width(_lib.RECAP_BF16, 64, 13) == 16
    assert width(_lib.RECAP_BF16, 128, 0) == 128 and width(_lib.RECAP_BF16, 128, 14) == 128
    assert width(_lib.RECAP_F16, 128, 4) == 128 and width(_lib.RECAP_BF16, 96, 4) == -1
    with pytest.raises(ValueError, match="matrix order"):
        _lib.call("recap_symmetric_eigen", 16, 2, 129, 16, 16, None)
    with pytest.raises(ValueError, match="matrix order"):
        _lib.call("recap_symmetric_eigen", 16, 2, 0, 16, 16, None)
    need = _lib.load().recap_pool_select_workspace_size(2, 4, 64)
    assert need == 2048 + 256  # 2*4*64 fp32 means, then 2*4*4 fp32 scores, 256-byte aligned
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("recap_pool_select", 16, _lib.RECAP_BF16, 1, 2, 64, 0, 0, 64, 16, 512, 512,
                  16, 0.125, 0.25, 16, need - 1, 16, 16, None)
    with pytest.raises(ValueError, match="density"):
        _lib.call("recap_pool_select", 16, _lib.RECAP_BF16, 1, 2, 64, 0, 0, 64, 16, 512, 512,
                  16, 0.125, 1.5, 16, need, 16, 16, None)
    with pytest.raises(ValueError, match="video blocks"):   # before any of its four stages
        _lib.call("recap_pool_select", 16, _lib.RECAP_BF16, 1, 2, 64, 0, 0, 64, 16,
                  4097 * 128, 4097 * 128, 16, 0.125, 0.25, 16, 1 << 40, 16, 16, None)


def test_workspace_queries():
    lib = _lib.load()
    assert lib.recap_closure_groups(118800, 8) == 117
    assert lib.recap_closure_groups(0, 8) == -1
    assert lib.recap_capture_partials(24, 128, 118800) == 24 * 118784 // 16
    assert lib.recap_capture_partials(2, 64, 4096) == 2 * 4096 // 32


def test_geometry_matches_reference_shapes():
    hun = K.Geometry(119056, 118800)
    assert (hun.nb, hun.tb, hun.ds, hun.rows) == (929, 931, 928, 118784)
    cog = K.Geometry(45106, 44880)
    assert (cog.nb, cog.tb, cog.ds, cog.rows) == (351, 353, 350, 44800)
    wan = K.Geometry(32760, 32760)
    assert (wan.nb, wan.tb, wan.ds, wan.rows) == (256, 256, 256, 32640)
    assert wan.counts("cpu")[-1] == 120


def test_xcd_runs_is_a_bijection_keeping_runs_on_one_xcd():
    # Host restatement of the attention work-item remap in csrc/common.hpp (xcd_runs):
    # workgroup b runs on XCD b % 8; in the full rounds every run of `run` consecutive items
    # lands on one XCD, and run r on XCD r % 8.
    def remap(bid, n, run):
        full = n // (8 * run) * (8 * run)
        if bid >= full:
            return bid
        xcd, slot = bid & 7, bid >> 3
        return (slot // run * 8 + xcd) * run + slot % run

    for n in (1, 7, 8, 513, 931, 22344, 931 * 24 + 5):
        for run in (1, 16, 64):
            items = [remap(b, n, run) for b in range(n)]
            assert sorted(items) == list(range(n))
            full = n // (8 * run) * (8 * run)
            assert all((items[b] // run) % 8 == b % 8 for b in range(full))


def test_xcd_linear_is_a_bijection():
    # Host restatement of the device work-item remap in csrc/common.hpp.
    for n in (1, 7, 8, 9, 22344, 931 * 24 + 5):
        seen = set()
        for bid in range(n):
            xcd, slot = bid & 7, bid >> 3
            per, rem = n >> 3, n & 7
            seen.add(xcd * per + min(xcd, rem) + slot)
        assert seen == set(range(n))


def test_layout_rowmap_and_round_trip():
    perm = hilbert_permutation((2, 8, 8))
    for text_first in (False, True):
        layout = Layout.from_permutation(perm, text_tokens=9, text_first=text_first)
        fwd, inv = O.gather_indices(perm, 9, text_first)
        assert torch.equal(layout.rowmap("cpu").long(), fwd)
        x = torch.randn(1, 2, 137, 4)
        assert torch.equal(layout.restore(layout.reorder(x)), x)
        with pytest.raises(ValueError):
            layout.reorder(torch.randn(1, 2, 100, 4))
    geo = SparseGeometry.build(Layout.from_permutation(perm, text_tokens=0, text_first=False), 128)
    assert geo.n_blocks == 1 and geo.block_counts.tolist() == [128.0]


def test_config_loader_and_profiles(tmp_path):
    for model in C.MODELS:
        for preset in C.PRESETS:
            raw = {"model": model, "preset": preset,
                   "operating_point": {"B": 20, "tau_pred": 0.1, "tau_detail": 0.2}}
            path = tmp_path / f"{model}_{preset}.json"
            path.write_text(json.dumps(raw))
            cfg = C.load_config(path)
            assert cfg.schedule.budget == 20
            assert cfg.schedule.detail_tau_mult == pytest.approx(2.0)
            assert cfg.operating_point.tau_detail == pytest.approx(0.2)
    cfg = C.config_from_dict({"model": "hunyuan", "preset": "fast",
                              "operating_point": {"B": 17, "tau_pred": 0.2, "tau_detail": 0.2}})
    assert cfg.operator.head_density == 0.2 and cfg.operator.bank_chunks == 4
    assert cfg.geometry.grid == (33, 45, 80) and cfg.operator.host_banks
    bad = [
        ({"model": "x", "preset": "fast", "operating_point": {"B": 5, "tau_pred": 1, "tau_detail": 1}}, "unsupported"),
        ({"model": "hunyuan", "preset": "fast", "operating_point": {"B": 2, "tau_pred": 1, "tau_detail": 1}}, "at least 3"),
        ({"model": "hunyuan", "preset": "fast", "operating_point": {"B": 99, "tau_pred": 1, "tau_detail": 1}}, "num_steps"),
        ({"model": "hunyuan", "preset": "fast", "operating_point": {"B": 5, "tau_pred": 1}}, "exactly"),
        ({"model": "hunyuan", "preset": "fast", "extra": 1, "operating_point": {"B": 5, "tau_pred": 1, "tau_detail": 1}}, "unknown"),
    ]
    for raw, msg in bad:
        with pytest.raises(ValueError, match=msg):
            C.config_from_dict(raw)
    for field, value in [("head_density", 1.0), ("closure_gate_theta", 0.0), ("closure_rank", -1),
                         ("rerank_min_overlap", 1.5), ("bank_chunks", 0)]:
        with pytest.raises(ValueError):
            C.OperatorConfig(**{field: value}).validate()
    with pytest.raises(ValueError, match="128"):
        C.GeometryConfig(grid=(1, 2, 3), block_size=64).validate()
    # the schedule's relations between fields
    for kw, msg in [({"prefix_floor": 3, "prefix_cap": 2}, "prefix_cap"),
                    ({"budget": 5, "tail_exact": 5}, "budget"),
                    ({"num_steps": 3, "tail_exact": 3}, "num_steps"),
                    ({"budget": 2}, "budget"), ({"tau": 0.0}, "tau")]:
        with pytest.raises(ValueError, match=msg):
            C.ScheduleConfig(**kw).validate()
    C.ScheduleConfig(prefix_floor=3, prefix_cap=0, budget=5, tail_exact=4).validate()
    # operating points: B an int (not a bool) >= 3, tolerances finite and positive
    for point in [(True, 0.1, 0.1), (3.0, 0.1, 0.1), (3, float("inf"), 0.1), (3, 0.1, -1.0)]:
        with pytest.raises(ValueError):
            C.OperatingPoint(*point).validate()
    # profile sections: objects only, known keys only, values read per field
    profile = {"geometry": {"grid": [2, "4", 8], "text_tokens": "16"},
               "operator": {"head_density": 0.3}, "schedule": {"budget": "7"}}
    cfg = C.config_from_profile("hunyuan", profile)
    assert cfg.geometry.grid == (2, 4, 8) and cfg.geometry.text_tokens == 16
    assert cfg.schedule.budget == 7 and cfg.operator.block_size == 128
    with pytest.raises(TypeError, match="object"):
        C.config_from_profile("hunyuan", {**profile, "operator": [1]})
    with pytest.raises(ValueError, match="unknown key"):
        C.config_from_profile("hunyuan", {**profile, "operator": {"density": 0.3}})
    with pytest.raises(ValueError, match="grid"):
        C.config_from_profile("hunyuan", {"geometry": {"text_tokens": 3}})


def test_operator_host_errors():
    from recap_amd.operator import Operator, REFRESH
    from recap_amd.config import OperatorConfig
    layout = Layout.from_permutation(hilbert_permutation((2, 8, 8)), text_tokens=0, text_first=False)
    geo = SparseGeometry.build(layout, 128)
    op = Operator.build(OperatorConfig(head_density=0.5), geo, n_layers=2, n_streams=2)
    with pytest.raises(ValueError, match="kind"):
        op.begin_step(0, "bogus")
    with pytest.raises(ValueError, match="stream"):
        op.set_stream(2)
    with pytest.raises(ValueError):
        Operator.build(OperatorConfig(), geo, n_layers=0)
    op.begin_step(3, REFRESH)
    assert op.kind == REFRESH and op.step == 3 and not op.banks_valid
    assert op.drain_validation() is None and op.peak_bank_bytes() == 0
    with pytest.raises(ValueError, match="GPU"):
        op.attend(0, torch.zeros(1, 1, 128, 64, dtype=torch.bfloat16),
                  torch.zeros(1, 1, 128, 64, dtype=torch.bfloat16),
                  torch.zeros(1, 1, 128, 64, dtype=torch.bfloat16))


def test_attention_branches_over_disjoint_keys_merge_to_the_full_softmax():
    # AttentionBranch.merge: softmax over keys A and over keys B, merged in LSE space,
    # equals the softmax over A and B together (closed form, fp64 reference).
    from recap_amd import AttentionBranch

    g = torch.Generator().manual_seed(0)
    q = torch.randn(3, 17, 16, generator=g, dtype=torch.float64)
    k = torch.randn(3, 40, 16, generator=g, dtype=torch.float64)
    v = torch.randn(3, 40, 16, generator=g, dtype=torch.float64)
    logits = q @ k.transpose(-1, -2) * 0.25

    def branch(idx):
        sub = logits[..., idx]
        return AttentionBranch(torch.softmax(sub, -1) @ v[:, idx], torch.logsumexp(sub, -1))

    a, b = branch(list(range(0, 40, 3))), branch([i for i in range(40) if i % 3])
    full = branch(list(range(40)))
    merged = a.merge(b)
    torch.testing.assert_close(merged.output, full.output.float().double(), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(merged.lse.double(), full.lse, atol=1e-5, rtol=1e-5)
    # A branch with no keys (lse -inf) drops out.
    empty = AttentionBranch(torch.zeros_like(a.output), torch.full_like(a.lse, float("-inf")))
    same = a.merge(empty)
    torch.testing.assert_close(same.output, a.output.float().double(), atol=1e-6, rtol=1e-6)


def test_last_error_is_per_thread():
    """recap_last_error() reports the calling thread's own last failure: a failing call in
    one thread leaves another thread's message untouched (callers on distinct host threads
    and streams do not see each other's errors)."""
    import threading

    lib = _lib.load()
    lib.recap_symmetric_eigen(16, 2, 0, 16, 16, None)   # matrix order 0: this thread's error
    mine = lib.recap_last_error().decode()
    assert "matrix order" in mine
    seen = {}

    def other():
        seen["before"] = lib.recap_last_error().decode()
        lib.recap_topk_blocks(16, 1, 10, 11, 0, 16, None)    # keep > blocks
        seen["after"] = lib.recap_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "matrix order" not in seen["before"] and "keep" in seen["after"]
    assert lib.recap_last_error().decode() == mine


def test_no_refined_rows_needs_no_row_buffers():
    """A video of fewer than 128 tokens has no refined rows (R = 0): the coarse tail, the
    capture (without validation) and the drift centre accept empty (NULL) row buffers and
    return before any launch, as the reference handles empty tensors; with R > 0 the same
    NULL buffers are rejected."""
    lib = _lib.load()
    # recap_coarse_tail(q, dtype, B, H, d, strides, rowmap, partition, kbar, vbar, w, u_t,
    # cvk_t, n_tokens, n_video, scale, theta, rank, glref, go, gl, drift_partial, stream)
    args = lambda n: (16, _lib.RECAP_BF16, 1, 2, 64, 0, 0, 64, 16, 16, 16, 16, 16, 16, 16,  # noqa: E731
                      n + 40, n, 0.125, 2.0, 4, None, None, None, None, None)
    assert lib.recap_coarse_tail(*args(100)) == _lib.RECAP_OK
    with pytest.raises(ValueError, match="go and gl"):
        _lib.call("recap_coarse_tail", *args(300))
    # recap_refresh_capture(dense_out, dtype, B, H, d, out strides, dense_lse, head_out,
    # head_lse, go, gl, rowmap, n_tokens, n_video, det, dl, glref, center, stat_partial,
    # stats, stream)
    cap = lambda n: (16, _lib.RECAP_BF16, 1, 2, 64, 0, 0, 64, 16, 16, 16, None, None, 16,  # noqa: E731
                     n + 40, n, None, None, None, None, None, None, None)
    assert lib.recap_refresh_capture(*cap(100)) == _lib.RECAP_OK
    with pytest.raises(ValueError, match="NULL"):
        _lib.call("recap_refresh_capture", *cap(300))
    assert lib.recap_drift_center(None, 2, 100, 16, None) == _lib.RECAP_OK
    with pytest.raises(ValueError, match="NULL"):
        _lib.call("recap_drift_center", None, 2, 300, 16, None)


def test_operator_rejects_mixed_qkv_dtypes():
    """Q, K and V of different element types raise ValueError before any launch (the
    kernels read them in one type; the reference's kernels and SDPA refuse them too); the
    kernel wrappers check Q against the packed K/V tiles and the coarse tables."""
    from recap_amd import REFRESH, Operator, OperatorConfig

    layout = Layout.from_permutation(hilbert_permutation((1, 4, 32)), text_tokens=0,
                                     text_first=False)
    op = Operator.build(OperatorConfig(head_density=0.25), SparseGeometry.build(layout, 128),
                        n_layers=1)
    op.begin_step(0, REFRESH)
    q = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="dtypes differ"):
        op.attend(0, q, q.to(torch.float16), q.to(torch.float16))
    kv = K.PackedKV(*(torch.empty(0, dtype=torch.float16) for _ in range(2)),
                    *(torch.empty(0) for _ in range(2)), torch.float16, 64)
    with pytest.raises(ValueError, match="packed K/V tiles"):
        K.block_sparse_attn(q, kv, None, torch.empty(0, dtype=torch.bool), None, 0.125)
    tables = {n: torch.empty(0, dtype=torch.float16) for n in ("kbar", "vbar", "w", "u_t", "cvk_t")}
    with pytest.raises(ValueError, match="table kbar"):
        K.coarse_tail(q, None, torch.empty(0), None, tables, 0.125, 2.0)
