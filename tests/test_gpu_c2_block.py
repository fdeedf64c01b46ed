"""GPU: the headline workload in the draft-length-4 schedule the benchmark times — bf16
Pulsar-283M, 16 sequences of 2048 uniform-random prompt tokens, sampled (temperature 0.8,
top-p 0.95, repetition penalty 1.15, no stop ids), 256 new tokens, draft length 4.

* Sequence 0's first round against the oracle's block restatement
  (RefEngine.block_verify over the engine's own block [t, d1..d4] at the prompt's end): the
  pulse-0 logits of the five rows (four draft steps, and the verify's pulse 0, which runs
  the last row alone: the draft steps ran the others' pulse 0 under the verify's rule) and
  the verify's pulse 1/2 logits of all five rows within max|diff| / max|ref| <= 2e-2.
* Every sequence emits 256 tokens; sequences 0 and 15 of the batch equal the same prompts
  decoded alone with the same random stream (a single run reproduces slot b with
  seed + b * 0x9E3779B97F4A7C15).
* Acceptance against the oracle, not the engine: replay_block_acceptance re-runs the
  oracle's rounds along the emitted streams of sequences 0 (all 256 tokens) and 15 (first
  96), each test's probability sum_x p_draft(x) p_verify(x) from the oracle's own pulse-0
  and last-pulse logits; the engine's accepted count must not be an outlier of that
  Poisson-binomial law (two-sided p-value >= 1e-4).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_abs_rel, poisson_binomial_pvalue

pytestmark = pytest.mark.gpu

B, T, N_NEW, G = 16, 2048, 256, 4
TEMP, TOP_P, RP = 0.8, 0.95, 1.15
SEED = 23
GOLDEN_RATIO64 = 0x9E3779B97F4A7C15


@pytest.fixture(scope="module")
def c2_prompts(full_state):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    return np.stack([W.uniform_ids(0, f"bench_prompt_{b}", T, cfg.vocab_size) for b in range(B)])


@pytest.mark.timeout(600)
def test_c2_draft_block_parity_and_acceptance(models, full_state, c2_prompts):
    from oracle import pulsar_ref as R
    from pulsar_engine.engine import HipEngine

    cfg, st = full_state
    P = cfg.default_pulses
    model = models[torch.bfloat16]
    kw = dict(max_prompt=T, max_new=N_NEW, speculative=True, temperature=TEMP, top_p=TOP_P,
              repetition_penalty=RP, stop_ids=[], draft_len=G)
    with HipEngine(model, batch=B, seed=SEED, all_logits=True, **kw) as eng:
        eng.prefill(c2_prompts)
        first = {}  # (pulse, block row) -> (token, logits) of the first round's rows
        for _ in range(2 * (G + P)):
            eng.step(1)
            rows = eng.rows(last=True)
            lg = eng.logits(len(rows))
            for r in rows:
                key = (int(r[2]), int(r[3]) - T)
                if int(r[0]) == 0 and 0 <= key[1] <= G and key not in first:
                    first[key] = (int(r[4]), lg[int(r[5])].copy())
            if len(first) == P * (G + 1):
                break
        eng.run()
        toks, kinds = eng.tokens(), eng.token_kinds()
        tests, accepted = eng.acceptance()
    print(f"[c2 draft 4] tests {tests} accepted {accepted}", flush=True)
    assert all(len(t) == N_NEW for t in toks)
    assert sorted(first) == [(k, i) for k in range(P) for i in range(G + 1)]
    blk = [first[(0, i)][0] for i in range(G + 1)]
    assert blk[0] == toks[0][0] and all(first[(k, i)][0] == blk[i] for k, i in first)

    ref = R.load_ref(cfg, st, torch.bfloat16, stop_ids=set())
    cache = R.RefKVCache(cfg)
    ref.prefill(torch.as_tensor(c2_prompts[0]).view(1, -1), cache)
    _, per_pulse, _ = ref.block_verify(blk, T, cache)
    err = {(k, i): max_abs_rel(got, per_pulse[k][i].float().numpy())
           for (k, i), (_, got) in first.items()}
    worst = max(err, key=err.get)
    print(f"[c2 draft 4] sequence 0 first round: worst {worst} {err[worst]:.2e}", flush=True)
    assert err[worst] <= 2e-2

    for b in (0, 15):
        seed_b = (SEED + b * GOLDEN_RATIO64) & 0xFFFFFFFFFFFFFFFF
        with HipEngine(model, batch=1, seed=seed_b, **kw) as one:
            one.prefill(c2_prompts[b:b + 1])
            one.run()
            assert one.tokens()[0] == toks[b], f"sequence {b}: batch != single"

    for b, n in ((0, N_NEW), (15, 96)):
        rep = R.replay_block_acceptance(ref, c2_prompts[b], toks[b][:n], kinds[b][:n], TEMP,
                                        TOP_P, RP, G, max_new=N_NEW)
        ps = [p for p, _ in rep]
        acc = sum(a for _, a in rep)
        pv = poisson_binomial_pvalue(ps, acc)
        print(f"[c2 draft 4] sequence {b}: {len(rep)} tests, accepted {acc}, oracle "
              f"expectation {sum(ps):.2f}, p-value {pv:.3g}", flush=True)
        assert len(rep) > 0 and pv >= 1e-4
