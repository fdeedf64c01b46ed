"""GPU: the headline workload itself — bf16 Pulsar-283M, 16 sequences of 2048 uniform-random
prompt tokens, sampled self-speculative decode (temperature 0.8, top-p 0.95, repetition
penalty 1.15, 256 new tokens, no stop ids), reference schedule (draft length 1).

* Sequence 0: prefill logits and the three pulse passes of its first decoded token within
  max|diff| / max|ref| <= 2e-2 of the oracle (bf16).
* Every sequence emits 256 tokens; sequences 0 and 15 of the batch equal the same prompts
  decoded alone with the same random stream (the engine's generator is keyed by the seed
  and the sequence's slot; a single run reproduces slot b with seed + b * 0x9E3779B97F4A7C15).
* Acceptance against the oracle, not the engine itself: the oracle re-runs the loop along
  the emitted stream of sequences 0 (all 256 tokens) and 15 (first 96), computing each
  test's acceptance probability sum_x p_draft(x) p_verify(x) from its own pulse-0 and
  pulse-2 logits; the engine's accepted count must not be an outlier of that
  Poisson-binomial law (two-sided p-value >= 1e-4).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_abs_rel, poisson_binomial_pvalue

pytestmark = pytest.mark.gpu

B, T, N_NEW = 16, 2048, 256
TEMP, TOP_P, RP = 0.8, 0.95, 1.15
SEED = 11
GOLDEN_RATIO64 = 0x9E3779B97F4A7C15


@pytest.fixture(scope="module")
def c2_prompts(full_state):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    return np.stack([W.uniform_ids(0, f"bench_prompt_{b}", T, cfg.vocab_size) for b in range(B)])


@pytest.mark.timeout(600)
def test_c2_headline_parity_and_acceptance(models, full_state, c2_prompts):
    from oracle import pulsar_ref as R
    from pulsar_engine.engine import HipEngine

    cfg, st = full_state
    model = models[torch.bfloat16]
    kw = dict(max_prompt=T, max_new=N_NEW, speculative=True, temperature=TEMP, top_p=TOP_P,
              repetition_penalty=RP, stop_ids=[])
    with HipEngine(model, batch=B, seed=SEED, all_logits=True, **kw) as eng:
        eng.prefill(c2_prompts)
        pre = eng.logits(B)
        first = eng.tokens()[0][0]
        passes = {}
        for _ in range(3):
            eng.step(1)
            rows = eng.rows(last=True)
            lg = eng.logits(len(rows))
            for r in rows:
                if int(r[0]) == 0 and int(r[3]) == T:
                    passes[int(r[2])] = lg[int(r[5])].copy()
        eng.run()
        toks, kinds = eng.tokens(), eng.token_kinds()
        tests, accepted = eng.acceptance()
    print(f"[c2] tests {tests} accepted {accepted}", flush=True)
    assert all(len(t) == N_NEW for t in toks)
    assert sorted(passes) == [0, 1, 2]

    ref = R.load_ref(cfg, st, torch.bfloat16, stop_ids=set())
    cache = R.RefKVCache(cfg)
    ref_pre = ref.prefill(torch.as_tensor(c2_prompts[0]).view(1, -1), cache)
    err = [max_abs_rel(pre[0], ref_pre.float().numpy().reshape(-1))]
    h = e = None
    for k in range(3):
        lg, h, e = ref.decode_pulse_pass(first, T, cache, k, h, e)
        err.append(max_abs_rel(passes[k], lg.float().numpy().reshape(-1)))
    print(f"[c2] sequence 0 prefill / pulse 0-2 errors {['%.2e' % x for x in err]}", flush=True)
    assert max(err) <= 2e-2

    # batch == single for slots 0 and 15 (same random stream through the seed shift)
    for b in (0, 15):
        seed_b = (SEED + b * GOLDEN_RATIO64) & 0xFFFFFFFFFFFFFFFF
        with HipEngine(model, batch=1, seed=seed_b, **kw) as one:
            one.prefill(c2_prompts[b:b + 1])
            one.run()
            assert one.tokens()[0] == toks[b], f"sequence {b}: batch != single"

    for b, n in ((0, N_NEW), (15, 96)):
        rep = R.replay_acceptance(ref, c2_prompts[b], toks[b][:n], kinds[b][:n], TEMP, TOP_P, RP)
        ps = [p for p, _ in rep]
        acc = sum(a for _, a in rep)
        pv = poisson_binomial_pvalue(ps, acc)
        print(f"[c2] sequence {b}: {len(rep)} tests, accepted {acc}, oracle expectation "
              f"{sum(ps):.2f}, p-value {pv:.3g}", flush=True)
        assert len(rep) > 0 and pv >= 1e-4
