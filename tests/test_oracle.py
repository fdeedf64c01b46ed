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
