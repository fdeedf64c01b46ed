"""GPU parity of the HIP decode engine against the oracle (and the reference goldens).

* fp32: every pulse pass's logits match the oracle's to 1e-4 of max|logit|, and the greedy
  token stream of the full-size model (128-token prompt, 64 new tokens, self-speculative)
  is identical to the stream the reference produced (tests/golden/full_fp32.npz).
* bf16: every pulse pass's logits within max|diff| / max|ref| <= 2e-2 of the oracle.
* greedy self-speculative == plain greedy, and batched runs equal single-sequence runs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden, max_abs_rel

pytestmark = pytest.mark.gpu


def _oracle(full_state, dtype):
    from oracle import pulsar_ref as R

    cfg, st = full_state
    return R.load_ref(cfg, st, dtype, rope_tables_fp32=True, stop_ids=set())


def _compare_passes(models, full_state, dtype, prompt, n_new, tol, rp=1.15):
    """Run plain greedy with logits for every pass; compare each with the oracle's."""
    from pulsar_engine.engine import HipEngine

    eng_ref = _oracle(full_state, dtype)
    eng_ref.trace = []
    ref_ids = list(eng_ref.stream_generate_ids(prompt, n_new, 0.0, 1.0, rp))
    ref_passes = {(t[1], t[2], t[3]): t[4].float().numpy().reshape(-1)
                  for t in eng_ref.trace if t[0] == "pulse"}
    cache = __import__("oracle.pulsar_ref", fromlist=["RefKVCache"]).RefKVCache(full_state[0])
    ref_prefill = eng_ref.prefill(torch.as_tensor(prompt).view(1, -1), cache).float().numpy().reshape(-1)

    eng = HipEngine(models[dtype], batch=1, max_prompt=len(prompt), max_new=n_new,
                    speculative=False, temperature=0.0, repetition_penalty=rp, stop_ids=[],
                    all_logits=True)
    eng.prefill(np.asarray(prompt)[None])
    errs = [("prefill", max_abs_rel(eng.logits(1)[0], ref_prefill))]
    n_steps = 0
    while not eng.state()[0, 0] and n_steps < 3 * (n_new + 1):
        eng.step(1)
        n_steps += 1
        rows = eng.rows(last=True)
        lg = eng.logits(len(rows))
        for r in rows:
            key = (int(r[4]), int(r[3]), int(r[2]))
            if key in ref_passes:
                errs.append((key, max_abs_rel(lg[int(r[5])], ref_passes[key])))
    print(f"{dtype} passes compared: {len(errs)}; worst: {max(e for _, e in errs):.3e}")
    bad = [(k, e) for k, e in errs if e > tol]
    assert not bad, bad[:5]
    if dtype == torch.float32:
        # the reference also runs the passes of the last emitted token; the engine stops
        assert len(errs) == 1 + 3 * (n_new - 1), len(errs)
        assert eng.tokens()[0] == ref_ids
    else:
        # bf16 streams may part at a near-tie; passes are compared while they agree
        assert len(errs) >= 4, len(errs)
    eng.close()


def test_fp32_pass_logits_match_oracle(models, full_state):
    from pulsar_engine import weights as W

    prompt = W.uniform_ids(7, "gpu_prompt", 40, full_state[0].vocab_size).tolist()
    _compare_passes(models, full_state, torch.float32, prompt, 6, tol=1e-4, rp=10.0)


def test_bf16_pass_logits_within_2e2(models, full_state):
    from pulsar_engine import weights as W

    prompt = W.uniform_ids(8, "gpu_prompt", 40, full_state[0].vocab_size).tolist()
    _compare_passes(models, full_state, torch.bfloat16, prompt, 6, tol=2e-2, rp=10.0)


def test_fp32_greedy_stream_identical_to_reference_golden(models):
    from pulsar_engine.engine import PulsarInferenceEngine

    g = golden("full_fp32.npz")
    eng = PulsarInferenceEngine(models[torch.float32])
    ids = eng.generate_ids([g["prompt"].tolist()], max_new_tokens=64, temperature=0.0,
                           repetition_penalty=1.15, speculative=True, stop_ids=[0, 2])[0]
    assert ids == g["greedy_spec_ids"].tolist()
    ids = eng.generate_ids([g["prompt"].tolist()], max_new_tokens=32, temperature=0.0,
                           repetition_penalty=10.0, speculative=True, stop_ids=[0, 2])[0]
    assert ids == g["greedy_rp10_spec_ids"].tolist()


@pytest.mark.parametrize("dtype,plen", [(torch.float32, 33), (torch.bfloat16, 33),
                                         (torch.bfloat16, 160)])
def test_greedy_speculative_equals_plain_and_batch_equals_single(models, full_state, dtype, plen):
    """160-token prompts take the wide-tile prefill GEMMs, 33-token ones the row-tile ones;
    either way a sequence's arithmetic does not depend on the rest of the batch."""
    from pulsar_engine import weights as W
    from pulsar_engine.engine import PulsarInferenceEngine

    cfg = full_state[0]
    prompts = [W.uniform_ids(s, "batch_prompt", plen, cfg.vocab_size).tolist() for s in range(4)]
    eng = PulsarInferenceEngine(models[dtype])
    kw = dict(max_new_tokens=12, temperature=0.0, repetition_penalty=10.0, stop_ids=[0, 2])
    spec = eng.generate_ids(prompts, speculative=True, **kw)
    plain = eng.generate_ids(prompts, speculative=False, **kw)
    assert spec == plain
    for i, p in enumerate(prompts):
        assert eng.generate_ids([p], speculative=True, **kw)[0] == spec[i]


def test_bf16_sampled_acceptance_matches_draft_verify_overlap(models, full_state):
    """Sampled self-speculation: the number of accepted drafts is a sum of independent
    Bernoulli(p_i), p_i = sum_x p_draft(x) p_verify(x) from the engine's own pulse-0 and
    pulse-2 logits of the tested token (src/infer.py:688-725). The observed count must lie
    within 4 standard deviations of sum p_i (temperature 1.0 gives p_i ~ 0.6 here)."""
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    B, T_, N = 16, 24, 20
    temp, top_p, rp = 1.0, 0.95, 1.15
    prompts = np.stack([W.uniform_ids(40 + b, "acc_prompt", T_, cfg.vocab_size) for b in range(B)])
    eng = HipEngine(models[torch.bfloat16], batch=B, max_prompt=T_, max_new=N, speculative=True,
                    temperature=temp, top_p=top_p, repetition_penalty=rp, stop_ids=[],
                    all_logits=True, seed=1234)
    eng.prefill(prompts)
    P = cfg.default_pulses
    pulse0 = {}
    expected, var, observed, n_tests = 0.0, 0.0, 0, 0
    for _ in range(4 * (N + 2) * P):
        before = eng.state().copy()
        if before[:, 0].all():
            break
        eng.step(1)
        after = eng.state()
        rows = eng.rows(last=True)
        lg = eng.logits(len(rows))
        for r in rows:
            seq, pulse, pos, tok, lrow = int(r[0]), int(r[2]), int(r[3]), int(r[4]), int(r[5])
            if lrow < 0:
                continue
            if pulse == 0:
                pulse0[(seq, pos, tok)] = lg[lrow].copy()
        toks = eng.tokens()
        for b in range(B):
            dt = int(after[b, 11] - before[b, 11])
            if dt == 0:
                continue
            assert dt == 1
            c_tok, c_pos = int(before[b, 3]), int(before[b, 4])
            v_row = [r for r in rows if int(r[0]) == b and int(r[3]) == c_pos and int(r[2]) == P - 1]
            assert len(v_row) == 1
            d_logits = torch.from_numpy(pulse0[(b, c_pos, c_tok)]).view(1, -1)
            v_logits = torch.from_numpy(lg[int(v_row[0][5])].copy()).view(1, -1)
            seen = prompts[b].tolist() + toks[b][: c_pos - T_ + 1]
            p = R.accept_probability(d_logits, v_logits, seen, temp, top_p, rp)
            expected += p
            var += p * (1.0 - p)
            observed += int(after[b, 12] - before[b, 12])
            n_tests += 1
    st = eng.state()
    assert n_tests == int(st[:, 11].sum()) and observed == int(st[:, 12].sum())
    sigma = max(var, 1e-9) ** 0.5
    print(f"tests {n_tests}, accepted {observed}, expected {expected:.1f} +- {sigma:.1f}")
    assert n_tests >= 100 and 0.2 < expected / n_tests < 0.95
    assert abs(observed - expected) <= 4.0 * sigma + 1.0
    eng.close()


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_long_prompt_passes_cover_window_and_yarn(models, full_state, dtype, tol):
    """A 1100-token prompt: local layers keep the newest 1024 positions (prefill top-left
    SDPA alignment, decode ring), global layers span two pages past 1024 and apply YaRN."""
    from pulsar_engine import weights as W

    prompt = W.uniform_ids(9, "long_prompt", 1100, full_state[0].vocab_size).tolist()
    _compare_passes(models, full_state, dtype, prompt, 3, tol=tol, rp=10.0)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_prefill_capacity_drops_match_oracle(full_state, dtype, tol):
    """Expert biases that send every token to experts 0-3 put each of them far over the
    prefill capacity of a 200-token prompt (C = 64 slots for 200 assignments): the kept
    set, chosen by routing weight, decides every later hidden state. Two sequences in one
    batch (capacity is per sequence); prefill logits of each against the oracle."""
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine
    from pulsar_engine.model import DeviceModel

    cfg, st = full_state
    bias = np.zeros(cfg.n_routed_experts, np.float32)
    bias[:4] = 1.0
    st2 = dict(st)
    for i in range(cfg.n_core):
        st2[f"core.{i}.mlp.expert_bias"] = np.tile(bias, (cfg.max_pulses, 1))
    T_ = 200
    assert R.moe_capacity(T_, cfg) == 64
    prompts = np.stack([W.uniform_ids(70 + b, "cap_prompt", T_, cfg.vocab_size) for b in range(2)])
    model = DeviceModel(cfg, st2, dtype)
    eng = HipEngine(model, batch=2, max_prompt=T_, max_new=4, speculative=False,
                    temperature=0.0, repetition_penalty=1.0, stop_ids=[])
    eng.prefill(prompts)
    got = eng.logits(2)
    ref_eng = R.load_ref(cfg, st2, dtype, rope_tables_fp32=True, stop_ids=set())
    for b in range(2):
        cache = R.RefKVCache(cfg)
        ref = ref_eng.prefill(torch.as_tensor(prompts[b]).view(1, -1), cache).float().numpy().reshape(-1)
        err = max_abs_rel(got[b], ref)
        print(f"{dtype} sequence {b}: {err:.3e}")
        assert err <= tol, (b, err)
    eng.close()


@pytest.mark.parametrize("T_", [200, 1100])
def test_prefill_capacity_ties_rank_by_flat_index(full_state, T_):
    """Zero router weights give every token the same sigmoid scores, and the expert biases
    send all of them to experts 0-3 with equal routing weights: every assignment of an
    expert sits on one key, so the kept set is the first C assignments in flat-index order
    (C = 64 of 200 and 352 of 1100 per expert). fp32 prefill logits against the oracle."""
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine
    from pulsar_engine.model import DeviceModel

    cfg, st = full_state
    bias = np.zeros(cfg.n_routed_experts, np.float32)
    bias[:4] = 1.0
    st2 = dict(st)
    for i in range(cfg.n_core):
        st2[f"core.{i}.mlp.expert_bias"] = np.tile(bias, (cfg.max_pulses, 1))
        st2[f"core.{i}.mlp.router_weight"] = np.zeros_like(st[f"core.{i}.mlp.router_weight"])
    C = R.moe_capacity(T_, cfg)
    assert C < T_
    prompt = W.uniform_ids(90, "tie_prompt", T_, cfg.vocab_size)
    model = DeviceModel(cfg, st2, torch.float32)
    eng = HipEngine(model, batch=1, max_prompt=T_, max_new=4, speculative=False,
                    temperature=0.0, repetition_penalty=1.0, stop_ids=[])
    eng.prefill(prompt[None])
    got = eng.logits(1)[0]
    ref_eng = R.load_ref(cfg, st2, torch.float32, rope_tables_fp32=True, stop_ids=set())
    ref = ref_eng.prefill(torch.as_tensor(prompt).view(1, -1), R.RefKVCache(cfg))
    err = max_abs_rel(got, ref.float().numpy().reshape(-1))
    print(f"capacity ties T={T_} C={C}: {err:.3e}")
    assert err <= 1e-4
    eng.close()


@pytest.mark.parametrize("draft_len", [0, 4])
def test_multi_step_graphs_equal_single_steps_and_eager(models, full_state, draft_len):
    """Runs of steps launch four steps per graph: the same sampled decode stepped one graph
    step at a time, as one 26-step call (six four-step graphs and two single steps) and
    eagerly gives identical tokens and per-sequence state."""
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    B, T_, N, n = 4, 24, 12, 26
    prompts = np.stack([W.uniform_ids(60 + b, "graph_prompt", T_, cfg.vocab_size)
                        for b in range(B)])
    eng = HipEngine(models[torch.bfloat16], batch=B, max_prompt=T_, max_new=N, speculative=True,
                    temperature=0.8, top_p=0.95, repetition_penalty=1.15, stop_ids=[], seed=7,
                    draft_len=draft_len)
    eng.prefill(prompts)
    runs = []
    for mode in ("single", "multi", "eager"):
        eng.rewind(11)
        if mode == "single":
            for _ in range(n):
                eng.step(1, graph=True)
        else:
            eng.step(n, graph=mode == "multi")
        runs.append((eng.tokens(), eng.state().copy()))
    assert all(len(t) > 0 for t in runs[0][0])
    for toks, st in runs[1:]:
        assert toks == runs[0][0]
        np.testing.assert_array_equal(st, runs[0][1])
    eng.close()
