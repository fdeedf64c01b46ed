"""Host-side logic on the CPU: the algorithmic traffic model and the profile summaries of
bench.py (the measurement path), and the configuration mirror."""

from __future__ import annotations

import csv
import importlib.util
import os

import pytest

from pulsar_engine import traffic
from pulsar_engine.config import PulsarConfig

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_attention_bytes_count_a_sequences_key_blocks_once():
    cfg = PulsarConfig()
    es, hk, hd = 2, cfg.n_kv_heads, cfg.head_dim
    counts = [[0] * cfg.n_routed_experts for _ in range(cfg.n_core)]
    pos = 3000
    one = traffic.step_bytes(cfg, es, [(0, 2, pos)], counts, 1)["attention"]
    two = traffic.step_bytes(cfg, es, [(0, 2, pos), (0, 0, pos + 1)], counts, 2)["attention"]
    W = cfg.sliding_window
    n_local = sum(cfg.is_local(L) for L in range(cfg.n_core))
    n_global = cfg.n_core - n_local
    kv = lambda keys: keys * hk * hd * 2 * es  # noqa: E731
    # per row: query in, output and gate; bf16 (fused post-processing): raw key and value
    # in, key and value to the cache
    act = (cfg.q_dim + cfg.n_heads + cfg.q_dim) * es + 4 * hk * hd * es
    assert one == n_local * kv(W) + n_global * kv(pos + 1) + cfg.n_core * act
    # the speculative row adds one key per layer and its own activations, not a second cache read
    assert two - one == n_local * kv(1) + n_global * kv(1) + cfg.n_core * act
    # two different sequences read two caches
    other = traffic.step_bytes(cfg, es, [(0, 2, pos), (1, 0, pos + 1)], counts, 2)["attention"]
    assert other - one == n_local * kv(W) + n_global * kv(pos + 2) + cfg.n_core * act
    # with a separate post-processing kernel its bytes are a class of their own
    sep = traffic.step_bytes(cfg, es, [(0, 2, pos)], counts, 1, fused_post=False)
    assert one - sep["attention"] == cfg.n_core * 4 * hk * hd * es
    assert sep["qk_post"] == cfg.n_core * (cfg.qkv_dim * es * 2 + 2 * hk * hd * es)


def test_weight_bytes_follow_pulses_and_touched_experts():
    cfg = PulsarConfig()
    es = 2
    counts = [[0] * cfg.n_routed_experts for _ in range(cfg.n_core)]
    for L in range(cfg.n_core):
        counts[L][3] = 2
    b1 = traffic.step_bytes(cfg, es, [(0, 1, 10), (1, 1, 10)], counts, 0)
    b2 = traffic.step_bytes(cfg, es, [(0, 1, 10), (1, 0, 10)], counts, 0)
    per_pulse_qkv = cfg.n_core * (cfg.qkv_dim + cfg.n_heads) * cfg.d_model * es
    assert b2["qkv_gate_gemm"] - b1["qkv_gate_gemm"] == per_pulse_qkv
    assert b1["routed_gate_up"] == cfg.n_core * (2 * cfg.d_expert * cfg.d_model * es
                                                 + 2 * (cfg.d_model + cfg.d_expert) * es)
    assert "lm_head" not in b1
    assert traffic.step_bytes(cfg, es, [(0, 2, 10)], counts, 1)["lm_head"] > cfg.vocab_size * cfg.d_model * es


def _write_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        w.writeheader()
        w.writerows(rows)


def test_rocprof_summary_splits_warm_prefill_and_decode(tmp_path):
    b = _bench()
    rows = []
    t = 0
    trace = [("void pulsar::attn_prefill_mfma_kernel(pulsar::AttnArgs)", 900),   # cold prefill
             ("pulsar::controller_kernel(pulsar::ControllerArgs)", 5),
             ("pulsar::prefill_embed_kernel(x)", 70),                             # warm prefill
             ("pulsar::attn_prefill_mfma_kernel(pulsar::AttnArgs)", 480),
             ("void gemm_bf16_wide_kernel<1, 0>(GemmArgs)", 250),
             ("pulsar::controller_kernel(pulsar::ControllerArgs)", 5),
             ("pulsar::attn_decode_unit_kernel(pulsar::AttnArgs)", 10),         # decode
             ("pulsar::attn_decode_unit_kernel(pulsar::AttnArgs)", 12),
             ("pulsar::controller_kernel(pulsar::ControllerArgs)", 6)]
    for name, dur in trace:
        rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + dur * 1000})
        t += dur * 1000 + 100
    (tmp_path / "x").mkdir()
    _write_csv(tmp_path / "x" / "run_kernel_trace.csv", rows)
    out = b.rocprof_summary(str(tmp_path))
    assert "prefill" not in out and "gemm_bf16_wide" not in out
    assert "| `attn_decode_unit_kernel` | 2 | 11.00 |" in out
    assert "| `controller_kernel` | 1 | 6.00 |" in out
    pre = b.rocprof_summary(str(tmp_path), "prefill")
    assert "| `attn_prefill_mfma_kernel` | 1 | 480.00 |" in pre
    assert "| `gemm_bf16_wide_kernel<1, 0>` | 1 | 250.00 |" in pre
    assert "controller_kernel" not in pre and "decode" not in pre


def test_pmc_summary_calibrates_and_feeds_traffic(tmp_path, monkeypatch):
    b = _bench()
    for ctr, per_copy, per_kernel in (("FETCH_SIZE", 131072.0, 1000.0), ("WRITE_SIZE", 262144.0, 50.0)):
        d = tmp_path / ctr
        d.mkdir()
        _write_csv(d / "bench_counter_collection.csv", [
            {"Kernel_Name": "pulsar::controller_kernel(x)", "Counter_Value": 1.0},
            {"Kernel_Name": "pulsar::attn_decode_unit_kernel(x)", "Counter_Value": per_kernel},
            {"Kernel_Name": "pulsar::attn_decode_unit_kernel(x)", "Counter_Value": per_kernel * 3}])
        c = tmp_path / (ctr + "_copy")
        c.mkdir()
        _write_csv(c / "copy_counter_collection.csv", [
            {"Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Value": per_copy}])
    out = b.pmc_summary(str(tmp_path / "FETCH_SIZE"), str(tmp_path / "WRITE_SIZE"),
                        str(tmp_path / "FETCH_SIZE_copy"), str(tmp_path / "WRITE_SIZE_copy"), 256)
    assert "scale factor 2.0000" in out and "scale factor 1.0000" in out
    prof = tmp_path / "traffic.md"
    prof.write_text(out)
    monkeypatch.setattr(b, "TRAFFIC_PROFILE", str(prof))
    # fetch: mean 2000 KiB x 2 (calibration) ; write: mean 100 KiB x 1
    assert b.recorded_traffic(["attn_decode_unit_kernel"]) == 4000 * 1024 + 100 * 1024
    assert b.recorded_traffic(["not_profiled"]) is None


def test_kernel_trace_fraction_follows_the_committed_table(tmp_path):
    """The roofline's kernel-trace fraction: a class's dispatch-weighted average over every
    template of the class in a committed summary table, against the class's bytes per
    launch."""
    b = _bench()
    table = tmp_path / "trace.md"
    table.write_text("\n".join([
        "| kernel | dispatches | avg us | total ms | share | busy dispatches | busy avg us |",
        "|---|---|---|---|---|---|---|",
        "| `attn_decode_unit_kernel<32, 2>` | 30 | 10.00 | 0.30 | 50% | 30 | 10.00 |",
        "| `attn_decode_unit_kernel<8, 2>` | 10 | 20.00 | 0.20 | 30% | 10 | 20.00 |",
        "| `moe_combine_rows_kernel<bf16, 16, 4>` | 40 | 4.00 | 0.16 | 20% | 40 | 4.00 |"]))
    assert b.recorded_kernel_us("attention", str(table)) == pytest.approx(12.5)
    assert b.recorded_kernel_us("moe_combine", str(table)) == pytest.approx(4.0)
    assert b.recorded_kernel_us("router", str(table)) is None
    roof = {"bytes_per_launch": 10_000_000}
    b.trace_fraction(roof, "attention", str(table))
    assert roof["kernel_trace_us"] == 12.5
    assert roof["frac_kernel_trace"] == pytest.approx(10e6 / 12.5e-6 / 8e12, abs=1e-4)
    # the committed headline summary exists and names the dominant class
    assert b.recorded_kernel_us("attention", b.BLOCK_TRACE_PROFILE) is not None


def test_config_from_dict_keeps_reference_names():
    cfg = PulsarConfig.from_dict({"d_model": 512, "n_heads": 8, "n_kv_heads": 2})
    assert (cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim) == (512, 8, 2, 64)
    with pytest.warns(RuntimeWarning):
        PulsarConfig.from_dict({"not_a_field": 1})


@pytest.mark.parametrize("T", [5, 16, 23])
def test_prefill_flops_count_each_query_key_pair(T):
    """The attention term against a brute-force count of the (query, key) pairs of every
    layer (local layers: top-left aligned last-window keys when T exceeds the window), and
    the projection term against a hand count of one token's multiply-adds."""
    from pulsar_engine.config import tiny_config

    cfg = tiny_config()  # window 16
    W = cfg.sliding_window
    pairs = 0
    for L in range(cfg.n_core):
        for t in range(T):
            if cfg.is_local(L) and T > W:
                lo, hi = T - W, T - W + min(t, W - 1)
            else:
                lo, hi = 0, t
            pairs += hi - lo + 1
    f = traffic.prefill_flops(cfg, 2, T)
    assert f["attention"] == cfg.default_pulses * 2 * cfg.n_heads * 4 * cfg.head_dim * pairs
    D = cfg.d_model
    macs = ((cfg.qkv_dim + cfg.n_heads) * D + D * cfg.q_dim + cfg.n_routed_experts * D
            + 2 * cfg.d_shared * D + D * cfg.d_shared
            + cfg.top_k * (2 * cfg.d_expert * D + D * cfg.d_expert))
    assert f["projections"] == 2 * macs * cfg.n_core * cfg.default_pulses * 2 * T
    assert f["total"] == sum(v for k, v in f.items() if k != "total")


def test_poisson_binomial_pvalue_against_binomial_and_brute_force():
    from scipy.stats import binomtest

    from conftest import poisson_binomial_pvalue

    # equal probabilities: the binomial test with the same two-sided rule
    for n, p, k in ((40, 0.3, 5), (40, 0.3, 12), (64, 0.95, 64), (64, 0.95, 55)):
        want = binomtest(k, n, p, alternative="two-sided").pvalue
        assert abs(poisson_binomial_pvalue([p] * n, k) - want) < 1e-9, (n, p, k)
    # unequal probabilities: enumerate all 2^n outcomes
    import itertools

    ps = [0.1, 0.5, 0.9, 0.7, 0.2]
    dist = [0.0] * 6
    for bits in itertools.product((0, 1), repeat=5):
        pr = 1.0
        for b, p in zip(bits, ps):
            pr *= p if b else 1 - p
        dist[sum(bits)] += pr
    for k in range(6):
        want = sum(d for d in dist if d <= dist[k] * (1 + 1e-9))
        assert abs(poisson_binomial_pvalue(ps, k) - want) < 1e-12


def test_chi_square_pvalue_detects_a_shifted_distribution():
    import numpy as np

    from conftest import chi_square_pvalue

    rng = np.random.default_rng(0)
    p = np.array([0.5, 0.3, 0.15, 0.04, 0.01])
    good = rng.choice(5, size=3000, p=p)
    assert chi_square_pvalue(good, p) > 1e-3
    bad = rng.choice(5, size=3000, p=[0.45, 0.35, 0.15, 0.04, 0.01])
    assert chi_square_pvalue(bad, p) < 1e-4
    # mass missing from probs is pooled: samples there count against the rest category
    assert chi_square_pvalue(good, p[:4]) > 1e-3


def test_op_wrappers_check_operands_before_the_library_is_called(monkeypatch):
    """moe_combine_forward / moe_combine_backward / moe_slots_from_order reject operands the
    kernels would read out of bounds (wrong dtype, shape or device) with RuntimeError and
    never reach the library. Device checks are stubbed so that CPU tensors stand in."""
    import torch

    import pulsar_cuda as pc

    class NoLib:
        def __getattr__(self, name):
            raise AssertionError(f"library called: {name}")

    monkeypatch.setattr(pc, "_LIB", NoLib())
    monkeypatch.setattr(pc, "_cuda", lambda t, n: None)
    monkeypatch.setattr(pc, "_stream", lambda t: 0)
    E, C, D, N, K = 4, 8, 16, 5, 2
    eo = torch.zeros(E, C, D, dtype=torch.bfloat16)
    idx = torch.zeros(N, K, dtype=torch.int64)
    w = torch.zeros(N, K, dtype=torch.bfloat16)
    slots = torch.zeros(N, K, dtype=torch.int32)
    sh = torch.zeros(N, D, dtype=torch.bfloat16)
    cases = {
        "topk_idx must be int64": dict(topk_idx=idx.int()),
        "token_to_slot must be int32": dict(token_to_slot=slots.long()),
        "token_to_slot must be \\[N, K\\]": dict(token_to_slot=slots[:3]),
        "topk_weights must be \\[N, K\\]": dict(topk_weights=w[:, :1]),
        "shared_out must have the dtype": dict(shared_out=sh.float()),
        "shared_out must be \\[N, D\\]": dict(shared_out=sh[:2]),
    }
    for msg, over in cases.items():
        args = dict(expert_outputs=eo, topk_idx=idx, topk_weights=w, token_to_slot=slots,
                    shared_out=sh)
        args.update(over)
        with pytest.raises(RuntimeError, match=msg):
            pc.moe_combine_forward(**args)
    dro = torch.zeros(N, D, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="topk_idx must be int64"):
        pc.moe_combine_backward(dro, eo, idx.int(), w, slots)
    with pytest.raises(RuntimeError, match="token_to_slot must be int32"):
        pc.moe_combine_backward(dro, eo, idx, w, slots.long())
    with pytest.raises(RuntimeError, match="d_routed_out must be \\[N, D\\]"):
        pc.moe_combine_backward(dro[:2], eo, idx, w, slots)
    with pytest.raises(RuntimeError, match="flat_e must be int64"):
        pc.moe_slots_from_order(idx.view(-1).int(), idx.view(-1), E, C)


def test_kv_cache_bytes_against_the_reference_table():
    """The reference's published unified-cache table (src/infer.py:834-846):
    73.4 MB at 32k; the engine's footprint differs only by the ring's one-block slack, page
    rounding and the pool's spare page."""
    cfg = PulsarConfig()
    want = {1024: 8.4, 4096: 14.7, 8192: 23.1, 16384: 39.8, 32768: 73.4}
    for ctx, mb in want.items():
        assert round(traffic.reference_unified_kv_bytes(ctx) / 1e6, 1) == mb
        got = traffic.kv_cache_bytes(cfg, 1, ctx)["total"]
        ref = traffic.reference_unified_kv_bytes(ctx)
        slack = 6 * (traffic.ring_positions(cfg) - min(ctx, 1024)) * 4 * 64 * 2 * 2
        spare = 2 * 64 * 4 * 64 * 2 * 2
        assert got - ref == slack + 2 * (-ctx % 64) * 4 * 64 * 2 * 2 + spare
    assert traffic.ring_positions(cfg) == 1088
    # a pool sized in pages instead of max_ctx
    assert (traffic.kv_cache_bytes(cfg, 4, 1024, pool_pages=20)["global"]
            == 2 * 21 * 64 * 4 * 64 * 2 * 2)
