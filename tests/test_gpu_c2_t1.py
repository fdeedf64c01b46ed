"""GPU: the headline shape where drafts get rejected — bf16 Pulsar-283M, 16 sequences of 2048
uniform-random prompt tokens, sampled at temperature 1.0 (top-p 0.95, repetition penalty
1.15, no stop ids), 64 new tokens, in both schedules: the reference's (draft length 1) and
the draft-block mode at draft length 4.

At temperature 0.8 the random-init model accepts every draft, so the acceptance tests of
test_gpu_c2.py / test_gpu_c2_block.py hold only probabilities of 1. At 1.0 the oracle's
probabilities along the emitted streams are about 0.95: the engine's accepted count, pooled
over sequences 0, 5, 10 and 15, must not be an outlier of the Poisson-binomial law of the
oracle's probabilities (two-sided p-value >= 1e-4), and that law must expect rejections (the
sum of 1 - p over the pooled tests at least 2), so the check can see a wrong acceptance rule
and not only a spurious rejection. The probabilities come from the oracle's own logits,
re-run along each emitted stream (replay_acceptance for the reference schedule,
src/infer.py:688-731; replay_block_acceptance for the draft-block mode).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import poisson_binomial_pvalue

pytestmark = pytest.mark.gpu

B, T, N_NEW = 16, 2048, 64
TEMP, TOP_P, RP = 1.0, 0.95, 1.15
CHECK = (0, 5, 10, 15)


@pytest.fixture(scope="module")
def c2_prompts(full_state):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    return np.stack([W.uniform_ids(0, f"bench_prompt_{b}", T, cfg.vocab_size) for b in range(B)])


@pytest.fixture(scope="module")
def oracle_bf16(full_state):
    from oracle import pulsar_ref as R

    cfg, st = full_state
    return R.load_ref(cfg, st, torch.bfloat16, stop_ids=set())


@pytest.mark.timeout(900)
@pytest.mark.parametrize("draft_len", [0, 4])
def test_c2_shape_acceptance_at_temperature_one(models, full_state, c2_prompts, oracle_bf16,
                                                draft_len):
    from oracle import pulsar_ref as R
    from pulsar_engine.engine import HipEngine

    with HipEngine(models[torch.bfloat16], batch=B, max_prompt=T, max_new=N_NEW,
                   speculative=True, temperature=TEMP, top_p=TOP_P, repetition_penalty=RP,
                   stop_ids=[], seed=31 + draft_len, draft_len=draft_len) as eng:
        eng.prefill(c2_prompts)
        eng.run()
        toks, kinds = eng.tokens(), eng.token_kinds()
        tests, accepted = eng.acceptance()
    assert all(len(t) == N_NEW for t in toks)
    ps, acc = [], 0
    for b in CHECK:
        if draft_len:
            rep = R.replay_block_acceptance(oracle_bf16, c2_prompts[b], toks[b], kinds[b], TEMP,
                                            TOP_P, RP, draft_len, max_new=N_NEW)
        else:
            rep = R.replay_acceptance(oracle_bf16, c2_prompts[b], toks[b], kinds[b], TEMP,
                                      TOP_P, RP)
        ps += [p for p, _ in rep]
        acc += sum(a for _, a in rep)
    expected_rejections = sum(1.0 - p for p in ps)
    pv = poisson_binomial_pvalue(ps, acc)
    print(f"[c2 T=1.0 draft {draft_len}] batch: {accepted}/{tests} accepted; sequences "
          f"{CHECK}: {len(ps)} tests, accepted {acc}, oracle expectation {sum(ps):.2f} "
          f"(rejections {expected_rejections:.2f}), p-value {pv:.3g}", flush=True)
    assert tests > accepted  # drafts were rejected in the batch
    assert expected_rejections >= 2.0
    assert pv >= 1e-4
