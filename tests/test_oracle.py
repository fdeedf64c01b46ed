"""Pins for the oracle (CPU restatement of the reference decode path).

Each closed-form piece is checked against an independent formula (float64 textbook maths,
brute force on tiny inputs, or an invariant) chosen so that a dropped term, a wrong sign or
index, or a transposed operand fails. The composition (prefill + pulse passes + generators)
is checked against golden vectors written by the reference itself (tests/golden).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import golden
from oracle import pulsar_ref as R


def test_rmsnorm_matches_float64_formula():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 96, generator=g)
    w = torch.rand(96, generator=g) + 0.5
    ref = (x.double() / torch.sqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-6)) * w.double()
    torch.testing.assert_close(R.rmsnorm(x, w, 1e-6).double(), ref, atol=1e-6, rtol=1e-6)


def test_rope_tables_and_rotation_closed_form():
    theta, d = 10000.0, 64
    freq = R.inv_freq(theta, d).double()
    expect = torch.tensor([theta ** (-2.0 * i / d) for i in range(d // 2)], dtype=torch.float64)
    torch.testing.assert_close(freq, expect, rtol=1e-6, atol=0)
    cos, sin = R.rope_tables(theta, d, 40)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 2, 40, d, generator=g)
    y = R.apply_rope(x, cos, sin).double()
    # complex multiplication (x1 + i x2) * exp(i t f)
    t = torch.arange(40, dtype=torch.float64).view(1, 1, 40, 1)
    ang = t * freq.view(1, 1, 1, -1)
    z = torch.complex(x[..., :32].double(), x[..., 32:].double()) * torch.exp(1j * ang)
    torch.testing.assert_close(y, torch.cat([z.real, z.imag], -1), atol=2e-5, rtol=1e-5)
    # norms preserved and dot products depend only on the position difference
    torch.testing.assert_close(y.norm(dim=-1), x.double().norm(dim=-1), atol=1e-4, rtol=1e-5)
    q = torch.randn(d, generator=g).view(1, 1, 1, d).expand(1, 1, 40, d)
    k = torch.randn(d, generator=g).view(1, 1, 1, d).expand(1, 1, 40, d)
    rq, rk = R.apply_rope(q, cos, sin)[0, 0].double(), R.apply_rope(k, cos, sin)[0, 0].double()
    assert abs((rq[10] @ rk[7]) - (rq[23] @ rk[20])) < 1e-3


def test_conv_k4_brute_force_and_decode_special_case():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 7, 16, generator=g)
    w = torch.randn(16, 4, generator=g)
    y = R.conv_k4(x, w).double()
    ref = x.double().clone()
    for b in range(2):
        for t in range(7):
            for k in range(4):
                if t - k >= 0:
                    ref[b, t] += w[:, k].double() * x[b, t - k].double()
    torch.testing.assert_close(y, ref, atol=1e-5, rtol=1e-5)
    # decode feeds one token: the stem reduces to (1 + w[:,0]) * x
    x1 = x[:, :1]
    torch.testing.assert_close(R.conv_k4(x1, w), x1 * (1 + w[:, 0]), atol=1e-6, rtol=1e-6)


def test_swiglu_closed_form():
    g = torch.Generator().manual_seed(3)
    gu = torch.randn(3, 2 * 12, generator=g)
    gate, up = gu[:, :12].double(), gu[:, 12:].double()
    torch.testing.assert_close(R.swiglu(gu, 12).double(), gate / (1 + torch.exp(-gate)) * up,
                               atol=1e-6, rtol=1e-6)


def test_lora_merge_equals_separate_adapter():
    """W_eff x == W x + (alpha/q) sum_j M[k,j] B_j (A_j x) (reference tests/test_model.py:563-669)."""
    g = torch.Generator().manual_seed(4)
    P, q, din, dout, K, alpha = 8, 8, 32, 24, 3, 16.0
    W = torch.randn(dout, din, generator=g)
    A = torch.randn(P, q, din, generator=g)
    B = torch.randn(P, dout, q, generator=g)
    M = torch.randn(P, P, generator=g)
    x = torch.randn(5, din, generator=g).double()
    for k in range(K):
        Weff = R.merged_weight(W, A, B, M, k, K, alpha).double()
        sep = x @ W.double().t()
        for j in range(K):
            sep = sep + (alpha / q) * M[k, j].double() * ((x @ A[j].double().t()) @ B[j].double().t())
        torch.testing.assert_close(x @ Weff.t(), sep, atol=5e-4, rtol=1e-5)


def test_softcap_and_yarn_closed_forms():
    x = torch.tensor([-1e4, -3.0, 0.0, 3.0, 1e4])
    y = R.softcap(x, 30.0)
    assert y.abs().max() <= 30.0 and y[2] == 0
    assert abs(y[3].item() - 30 * math.tanh(0.1)) < 1e-5
    assert R.yarn_scale(1023, 1024) == 1.0
    assert R.yarn_scale(100, 1024) == 1.0
    assert abs(R.yarn_scale(2047, 1024) - (1 + 0.1 * math.log(2))) < 1e-12


def _brute_router(x, w, bias, k):
    lg = (x.double() @ w.double().t())
    c = lg - lg.mean(-1, keepdim=True)
    s = 1 / (1 + torch.exp(-c))
    out_i, out_w = [], []
    for r in range(x.shape[0]):
        order = sorted(range(w.shape[0]), key=lambda e: (-(s[r, e] + bias[e].double()).item(), e))
        sel = order[:k]
        tot = sum(s[r, e].item() for e in sel) + 1e-6
        out_i.append(sel)
        out_w.append([s[r, e].item() / tot for e in sel])
    return torch.tensor(out_i), torch.tensor(out_w, dtype=torch.float64)


def test_router_decode_brute_force_and_shift_invariance():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 32, generator=g)
    w = torch.randn(16, 32, generator=g) * 0.3
    bias = torch.randn(16, generator=g) * 0.05
    idx, wts = R.router_decode(x, w, bias, 4, torch.float32)
    bi, bw = _brute_router(x, w, bias, 4)
    assert torch.equal(idx, bi)
    torch.testing.assert_close(wts.double(), bw, atol=1e-6, rtol=1e-5)
    assert (wts.sum(-1) - 1).abs().max() < 1e-5
    # adding a per-token constant to every logit leaves the choice unchanged
    lg = F.linear(x, w)
    shifted = lg + torch.randn(64, 1, generator=g) * 5
    i2, w2 = R.router_prefill(shifted, bias, 4, torch.float32)
    i1, w1 = R.router_prefill(lg, bias, 4, torch.float32)
    assert torch.equal(i1, i2)
    torch.testing.assert_close(w1, w2, atol=1e-5, rtol=1e-4)


def test_capacity_closed_form():
    from pulsar_engine.config import PulsarConfig

    cfg = PulsarConfig()
    assert R.moe_capacity(128, cfg) == 64
    assert R.moe_capacity(512, cfg) == 160
    assert R.moe_capacity(2048, cfg) == 640
    assert R.moe_capacity(32768, cfg) == 10240
    assert R.moe_capacity(3, cfg) == 32


def test_token_slots_brute_force_rank_and_lowest_weight_drop():
    g = torch.Generator().manual_seed(6)
    N, K, E, C = 50, 2, 4, 16
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(N)])
    idx[:30, 0] = 1  # overload expert 1 so drops happen
    w = torch.rand(N, K, generator=g).to(torch.bfloat16)
    slots = R.token_slots(idx, w, E, C)
    wf = w.float()
    for e in range(E):
        members = [(n, k) for n in range(N) for k in range(K) if idx[n, k] == e]
        # (weight desc, flat index asc)
        members.sort(key=lambda nk: (-wf[nk].item(), nk[0] * K + nk[1]))
        for rank, nk in enumerate(members):
            assert slots[nk].item() == (rank if rank < C else -1)
    kept = wf[slots >= 0][idx[slots >= 0] == 1]
    dropped = wf[slots < 0]
    assert dropped.numel() > 0 and kept.min() >= dropped.max()


def test_sdpa_causal_top_left_alignment_when_queries_exceed_keys():
    """Prefill local layers call SDPA is_causal with L=T > S=window (infer.py:433-435)."""
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 2, 6, 8, generator=g)
    k = torch.randn(1, 2, 4, 8, generator=g)
    v = torch.randn(1, 2, 4, 8, generator=g)
    out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    ref = torch.zeros_like(out)
    for i in range(6):
        hi = min(i, 3)
        s = (q[:, :, i:i + 1] @ k[:, :, :hi + 1].transpose(-1, -2)) / math.sqrt(8)
        ref[:, :, i] = (s.softmax(-1) @ v[:, :, :hi + 1])[:, :, 0]
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)


def test_kv_cache_algebra():
    from pulsar_engine.config import tiny_config

    cfg = tiny_config()
    c = R.RefKVCache(cfg)
    T = 20
    k = torch.arange(T, dtype=torch.float32).view(1, 1, T, 1).expand(1, 2, T, 16).clone()
    c.put_prefill(0, k, k)       # local: keeps last 16
    c.put_prefill(3, k, k)       # global: keeps all
    assert c.k[0].shape[2] == 16 and c.k[0][0, 0, 0, 0] == T - 16
    assert c.k[3].shape[2] == T
    new = torch.full((1, 2, 1, 16), 100.0)
    c.put_decode(0, new, new, pulse=0)
    assert c.k[0].shape[2] == 16 and c.k[0][0, 0, -1, 0] == 100 and c.k[0][0, 0, 0, 0] == T - 15
    c.put_decode(0, new + 1, new + 1, pulse=2)
    assert c.k[0].shape[2] == 16 and c.k[0][0, 0, -1, 0] == 101 and c.k[0][0, 0, -2, 0] == T - 1


def test_sampling_rules():
    l = torch.tensor([[2.0, 3.0, -1.0, 2.9]])
    # penalty divides positive and multiplies negative seen logits
    assert R.RefEngine.sample(l, [1], 0.0, 1.0, 1.15) == 3
    assert R.RefEngine.sample(l, [], 0.0, 1.0, 1.15) == 1
    # ties resolve to the first index
    assert R.RefEngine.sample(torch.tensor([[1.0, 5.0, 5.0]]), [], 0.0, 1.0, 1.0) == 1
    # top-p keeps the smallest prefix whose mass reaches p (rank 0 always kept)
    p = R.sampling_distribution(torch.log(torch.tensor([[0.5, 0.3, 0.15, 0.05]])), [], 1.0, 0.7, 1.0)
    torch.testing.assert_close(p, torch.tensor([0.625, 0.375, 0.0, 0.0], dtype=torch.float64))
    p = R.sampling_distribution(torch.log(torch.tensor([[0.9, 0.05, 0.05]])), [], 1.0, 0.5, 1.0)
    torch.testing.assert_close(p, torch.tensor([1.0, 0.0, 0.0], dtype=torch.float64))


def test_accept_probability_matches_monte_carlo():
    g = torch.Generator().manual_seed(8)
    d = torch.randn(1, 50, generator=g) * 2
    v = d + torch.randn(1, 50, generator=g)
    p = R.accept_probability(d, v, [3, 4], 0.8, 0.95, 1.15)
    hits = 0
    n = 4000
    for _ in range(n):
        a = R.RefEngine.sample(d, [3, 4], 0.8, 0.95, 1.15, generator=g)
        b = R.RefEngine.sample(v, [3, 4], 0.8, 0.95, 1.15, generator=g)
        hits += a == b
    assert abs(hits / n - p) < 4 * math.sqrt(p * (1 - p) / n)


@pytest.mark.parametrize("rp", [1.15, 10.0])
def test_greedy_speculative_equals_plain(tiny_state, rp):
    """a2 == a3: the greedy self-speculative stream is the plain greedy stream."""
    cfg, st = tiny_state
    from pulsar_engine import weights as W

    eng = R.load_ref(cfg, st, torch.float32, stop_ids={0, 2})
    for seed in range(3):
        prompt = W.uniform_ids(seed, "eq_prompt", 10 + 7 * seed, cfg.vocab_size)
        a = list(eng.stream_generate_ids(prompt, 15, 0.0, 1.0, rp))
        b = list(eng.self_speculative_ids(prompt, 15, 0.0, 1.0, rp))
        assert a == b


def test_prefill_moe_without_drops_equals_dropless_formula(tiny_state):
    cfg, st = tiny_state
    eng = R.load_ref(cfg, st, torch.float32)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 6, cfg.d_model, generator=g)
    out = eng.moe_prefill(1, x, 2)
    ref = torch.cat([eng.moe_decode(1, x[:, t:t + 1], 2) for t in range(6)], dim=1)
    # prefill routes with activation-dtype logits, folds routed_scale into the weights
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("tag,dtype", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_tiny_goldens_bit_exact(tiny_state, tag, dtype):
    cfg, st = tiny_state
    g = golden(f"tiny_{tag}.npz")
    mk = lambda: R.load_ref(cfg, st, dtype, stop_ids={0, 2})  # noqa: E731
    eng = mk()
    eng.trace = []
    ids = list(eng.stream_generate_ids(g["prompt"], 6, 0.0, 1.0, 1.15))
    assert ids == g["greedy_plain_ids"].tolist()
    passes = [t for t in eng.trace if t[0] == "pulse"]
    assert [t[2] for t in passes] == g["pass_pos"].tolist()
    np.testing.assert_array_equal(np.stack([t[4].float().numpy().reshape(-1) for t in passes]),
                                  g["pass_logits"])
    cache = R.RefKVCache(cfg)
    pl = mk().prefill(torch.as_tensor(g["prompt"]).view(1, -1), cache)
    np.testing.assert_array_equal(pl.float().numpy().reshape(-1), g["prefill_logits"])
    e = mk()
    assert list(e.self_speculative_ids(g["prompt"], 20, 0.0, 1.0, 1.15)) == g["greedy_spec_ids"].tolist()
    assert list(e.stream_generate_ids(g["prompt"], 20, 0.0, 1.0, 10.0)) == g["greedy_rp10_plain_ids"].tolist()
    assert list(e.self_speculative_ids(g["prompt"], 20, 0.0, 1.0, 10.0)) == g["greedy_rp10_spec_ids"].tolist()
    torch.manual_seed(1234)
    assert list(e.self_speculative_ids(g["prompt"], 20, 0.8, 0.95, 1.15)) == g["sampled_spec_ids"].tolist()
    torch.manual_seed(99)
    assert list(e.self_speculative_ids(g["prompt"], 20, 1.0, 0.9, 10.0)) == g["sampled_rp10_spec_ids"].tolist()


def test_full_size_fp32_goldens(full_state):
    cfg, st = full_state
    g = golden("full_fp32.npz")
    eng = R.load_ref(cfg, st, torch.float32, stop_ids={0, 2})
    eng.trace = []
    ids = list(eng.self_speculative_ids(g["prompt"], 64, 0.0, 1.0, 1.15))
    assert ids == g["greedy_spec_ids"].tolist()
    first = [t for t in eng.trace if t[0] == "pulse" and t[2] == len(g["prompt"])][:3]
    np.testing.assert_array_equal(np.stack([t[4].numpy().reshape(-1) for t in first]),
                                  g["step0_pass_logits"])
    eng.trace = None
    ids = list(eng.self_speculative_ids(g["prompt"], 32, 0.0, 1.0, 10.0))
    assert ids == g["greedy_rp10_spec_ids"].tolist()


# -- adaptive early exit (src/infer.py:198-232, :526-549) -------------------------------

@pytest.mark.parametrize("tag,dtype", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_early_exit_tiny_goldens(tag, dtype):
    """Streams and per-pulse exit counts equal the reference's at three thresholds (the
    last sends the first decoded token out after pulse 1), plain and self-speculative,
    greedy and seeded sampled."""
    from pulsar_engine import weights as W
    from pulsar_engine.config import tiny_config

    cfg = tiny_config()
    st = W.exit_probe_state(cfg)
    g = golden("early_exit.npz")
    prompt = g["tiny_prompt"]
    eng = R.load_ref(cfg, st, dtype, stop_ids={0, 2})
    cases = {
        "greedy_plain": (0.0, 1.0, 10.0, False, None),
        "greedy_spec": (0.0, 1.0, 10.0, True, None),
        "sampled_spec": (0.8, 0.95, 10.0, True, 1234),
        "sampled_plain": (0.8, 0.95, 10.0, False, 1234),
        "greedy_spec_rp115": (0.0, 1.0, 1.15, True, None),
    }
    seen_exit_pulses = set()
    for i, thr in enumerate(g[f"tiny_{tag}_thresholds"].tolist()):
        for name, (T, tp, rp, spec, seed) in cases.items():
            eng.set_early_exit_threshold(thr)
            if seed is not None:
                torch.manual_seed(seed)
            gen = eng.self_speculative_ids if spec else eng.stream_generate_ids
            ids = list(gen(prompt, 20, T, tp, rp))
            assert ids == g[f"tiny_{tag}_{name}_{i}_ids"].tolist(), (name, thr)
            assert eng.early_exit_counts == g[f"tiny_{tag}_{name}_{i}_counts"].tolist(), (name, thr)
            seen_exit_pulses |= {k for k, c in enumerate(eng.early_exit_counts) if c}
    assert seen_exit_pulses == {0, 1, 2}
    # set_early_exit_threshold clears the counts; None switches the exit off
    eng.set_early_exit_threshold(None)
    assert eng.early_exit_counts == [0, 0, 0] and eng.get_early_exit_stats() == {}
    assert list(eng.stream_generate_ids(prompt, 6, 0.0, 1.0, 10.0)) == \
        list(R.load_ref(cfg, st, dtype, stop_ids={0, 2}).stream_generate_ids(prompt, 6, 0.0, 1.0, 10.0))
    assert eng.early_exit_counts == [0, 0, 0]


def test_early_exit_stats_text_matches_reference():
    """generate()'s statistics block (src/infer.py:775-780) from the counts of the golden
    run, formatted by the host mirror, equals what the reference printed."""
    from pulsar_engine.engine import early_exit_stats, format_early_exit_stats

    g = golden("early_exit.npz")
    for tag in ("fp32", "bf16"):
        thr = float(g[f"tiny_{tag}_thresholds"][2])
        stats = early_exit_stats(g[f"tiny_{tag}_generate_counts"].tolist())
        assert format_early_exit_stats(thr, stats) == str(g[f"tiny_{tag}_generate_stdout"])
        # the oracle's statistics agree with the host mirror's
        eng = R.RefEngine.__new__(R.RefEngine)
        eng.early_exit_counts = g[f"tiny_{tag}_generate_counts"].tolist()
        assert R.RefEngine.get_early_exit_stats(eng) == stats
    assert early_exit_stats([0, 0, 0]) == {}
    s = early_exit_stats([1, 1, 2])
    # closed form: (8 + 16 + 2 * 24) / 4 = 18 layers, 24 / 18 speedup
    assert s["effective_layers"] == 18.0 and abs(s["compute_speedup"] - 24 / 18) < 1e-12
    assert s["pulse_pcts"] == [25.0, 25.0, 50.0]


def test_early_exit_full_fp32_golden(full_state):
    """Full-size fp32 model at threshold 0.9978: streams and exit counts of the reference."""
    cfg, st = full_state
    g = golden("early_exit.npz")
    eng = R.load_ref(cfg, st, torch.float32, stop_ids={0, 2})
    thr = float(g["full_threshold"])
    for name, spec in (("greedy_plain", False), ("greedy_spec", True)):
        eng.set_early_exit_threshold(thr)
        gen = eng.self_speculative_ids if spec else eng.stream_generate_ids
        assert list(gen(g["full_prompt"], 32, 0.0, 1.0, 10.0)) == g[f"full_{name}_ids"].tolist()
        assert eng.early_exit_counts == g[f"full_{name}_counts"].tolist()


def test_early_exit_rule_on_hand_built_passes():
    """decode_step's exit rule with stubbed pulse passes: after pulse k < 2 the token leaves
    when softmax's top-1 probability >= threshold, returns pulse k's logits and counts at
    k; a token running every pulse counts at pulse 2; no threshold, no counting."""
    V = 8

    def logits_with_top(p):
        # softmax of [a, 0, ..., 0] has top-1 probability e^a / (e^a + V - 1) = p
        lg = torch.zeros(1, V)
        lg[0, 5] = math.log(p * (V - 1) / (1.0 - p))
        return lg

    probs = {0: 0.50, 1: 0.80, 2: 0.30}
    eng = R.RefEngine.__new__(R.RefEngine)
    eng.cfg = type("C", (), {"default_pulses": 3})()
    eng.trace = None
    ran = []

    def fake_pass(token, pos, cache, pulse, h=None, e=None):
        ran.append(pulse)
        return logits_with_top(probs[pulse]), None, None

    eng.decode_pulse_pass = fake_pass
    cache = type("K", (), {})()
    for thr, want_pulses, want_counts in ((0.45, [0], [1, 0, 0]), (0.75, [0, 1], [0, 1, 0]),
                                          (0.85, [0, 1, 2], [0, 0, 1]), (None, [0, 1, 2], [0, 0, 0])):
        R.RefEngine.set_early_exit_threshold(eng, thr)
        ran.clear()
        out = R.RefEngine.decode_step(eng, 3, 10, cache)
        assert ran == want_pulses and eng.early_exit_counts == want_counts, thr
        top = F.softmax(out, dim=-1).max().item()
        assert abs(top - probs[want_pulses[-1]]) < 1e-6
        assert cache.seq_len == 11


def test_replay_acceptance_reproduces_the_generators_own_tests(tiny_state):
    """Driving the loop along the generator's own emitted stream gives back, test for test,
    the acceptance probabilities and outcomes the generator recorded."""
    cfg, st = tiny_state
    for dtype, T, rp, seed in ((torch.float32, 0.02, 10.0, 3), (torch.bfloat16, 0.05, 10.0, 3)):
        eng = R.load_ref(cfg, st, dtype, stop_ids=set())
        stats = {}
        torch.manual_seed(seed)
        ids = list(eng.self_speculative_ids(W_prompt(cfg), 30, T, 0.95, rp, stats=stats))
        assert len(ids) == 30 and stats["accepted"] > 0 and stats["tests"] > stats["accepted"]
        rep = R.replay_acceptance(R.load_ref(cfg, st, dtype, stop_ids=set()), W_prompt(cfg),
                                  ids, stats["kinds"], T, 0.95, rp)
        assert [p for p, _ in rep] == stats["p_accept"]
        assert sum(a for _, a in rep) == stats["accepted"] and len(rep) == stats["tests"]


def W_prompt(cfg):
    from pulsar_engine import weights as W

    return W.uniform_ids(0, "tiny_prompt", 24, cfg.vocab_size)


def test_spec_token_marginals_match_monte_carlo():
    """The exact first-three-token distributions of the self-speculative loop against 1500
    seeded runs of the generator itself (small config, temperature 0.05, penalty 10)."""
    import copy

    from conftest import chi_square_pvalue
    from pulsar_engine import weights as W
    from pulsar_engine.config import small_config

    cfg = small_config()
    st = W.synthetic_state(cfg, seed=0)
    prompt = W.uniform_ids(0, "dist_prompt", 24, cfg.vocab_size)
    m = R.spec_token_marginals(R.load_ref(cfg, st, torch.float32, stop_ids=set()), prompt,
                               0.05, 0.95, 10.0, prune=1e-4)
    assert abs(m[0].sum().item() - 1) < 1e-9 and abs(m[1].sum().item() - 1) < 1e-6
    assert m[2].sum().item() > 0.99
    eng = R.load_ref(cfg, st, torch.float32, stop_ids=set())
    # every run starts from the same prompt: keep one prefill and hand out copies of it
    saved = {}
    real_prefill = eng.prefill

    def prefill_once(ids, cache):
        if not saved:
            saved["logits"] = real_prefill(ids, cache)
            saved["cache"] = copy.deepcopy(cache)
        cache.__dict__.update(copy.deepcopy(saved["cache"]).__dict__)
        return saved["logits"].clone()

    eng.prefill = prefill_once
    g = torch.Generator().manual_seed(2024)
    draws = np.array([list(eng.self_speculative_ids(prompt, 3, 0.05, 0.95, 10.0, generator=g))
                      for _ in range(1500)])
    for k in range(3):
        pv = chi_square_pvalue(draws[:, k], m[k].numpy())
        assert pv > 1e-4, (k, pv)
    # a plausible mistake fails: token 2 drawn from the verify logits alone (no draft mix)
    ref2 = R.load_ref(cfg, st, torch.float32, stop_ids=set())
    cache = R.RefKVCache(cfg)
    lg = ref2.prefill(torch.as_tensor(prompt).view(1, -1), cache)[:, -1, :]
    p1 = R.sampling_distribution(lg, prompt.tolist(), 0.05, 0.95, 10.0)
    wrong = torch.zeros_like(m[1])
    for t1 in torch.nonzero(p1 > 1e-4).view(-1).tolist():
        c = copy.deepcopy(cache)
        _, h, e = ref2.decode_pulse_pass(t1, 24, c, 0)
        _, h, _ = ref2.decode_pulse_pass(t1, 24, c, 1, h, e)
        lv, _, _ = ref2.decode_pulse_pass(t1, 24, c, 2, h, e)
        wrong += p1[t1] * R.sampling_distribution(lv, prompt.tolist() + [t1], 0.05, 0.95, 10.0)
    assert (wrong - m[1]).abs().sum() > 0.05
