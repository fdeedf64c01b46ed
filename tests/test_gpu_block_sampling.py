"""GPU: the draft-block mode's sampled acceptance and resample against the oracle, in a regime
where drafts are rejected about half the time.

The workload of tests/golden/block_marginals_small.npz (small configuration, fp32, seed-0
weights, a 24-token prompt, temperature 0.03, top-p 0.95, repetition penalty 10, draft
length 4, six emitted tokens, no stop ids): the oracle's tests there accept with probability
0.495 on average, and each of tokens 2-5 is an accepted draft with probability 0.44-0.58, so
most runs hold a rejection and its resample.

* 4096 runs (256 sequences x 16 seeds): the distribution of each of the six emitted tokens
  against the oracle's exact distributions (Pearson chi-square), and the share of runs in
  which token k is an accepted draft against the oracle's probability (binomial bound).
  The rule under test is the reference's, applied down the block (src/infer.py:704-725):
  a draft is accepted iff it equals an independent draw from the verify logits of the row
  before it; at the first rejection the next token is a second, independent draw from
  those logits.
* The draws of each verify row (v_i, tested against draft i + 1, and f_i, the resample at a
  rejection) are the sampler's two draws at the row's own counter, re-computed here by the
  standalone sampler on the row's logits: an accepted draft equals v_i, a rejected one
  differs from it, and the token emitted after a rejection is f_i, not v_i (checked on
  rows where the two differ).
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from conftest import chi_square_pvalue, golden

pytestmark = pytest.mark.gpu

# controller state words (SeqState in csrc/sample.h)
ST_CTR, ST_BLK_PHASE, ST_BLK_STEP = 17, 21, 22
MAX_BLOCK = 8  # rows of one sequence in a step (kMaxBlock)


@pytest.fixture(scope="module")
def workload():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pulsar_engine import weights as W
    from pulsar_engine.config import small_config
    from pulsar_engine.model import DeviceModel

    f = golden("block_marginals_small.npz")
    s = json.loads(str(f["settings"]))
    cfg = small_config()
    st = W.synthetic_state(cfg, seed=s["weight_seed"])
    assert str(f["weights_digest"]) == W.state_digest(st)
    prompt = W.uniform_ids(s["prompt_seed"], s["prompt_name"], s["prompt_len"], cfg.vocab_size)
    return f, s, cfg, DeviceModel(cfg, st, torch.float32), prompt


def _engine(model, s, batch, seed):
    from pulsar_engine.engine import HipEngine

    return HipEngine(model, batch=batch, max_prompt=s["prompt_len"], max_new=s["n_tokens"],
                     draft_len=s["draft_len"], temperature=s["temperature"], top_p=s["top_p"],
                     repetition_penalty=s["repetition_penalty"], stop_ids=[], seed=seed)


def test_block_sampled_tokens_follow_the_oracle_distribution(workload):
    f, s, cfg, model, prompt = workload
    n, B, reps = s["n_tokens"], 256, 16
    draws, kinds = [], []
    with _engine(model, s, B, 3000) as eng:
        eng.prefill(np.tile(prompt, (B, 1)))
        for rep in range(reps):
            if rep:
                eng.rewind(3000 + rep)
            eng.run()
            draws += eng.tokens()
            kinds += eng.token_kinds()
    draws, kinds = np.asarray(draws), np.asarray(kinds)
    N = B * reps
    assert draws.shape == (N, n) and kinds.shape == (N, n)
    pvals = []
    for k in range(n):
        p = np.zeros(cfg.vocab_size)
        p[f[f"idx_{k}"]] = f[f"p_{k}"]
        pvals.append(chi_square_pvalue(draws[:, k], p))
    acc = f["accepted_mass"]
    share = kinds.mean(axis=0)
    z = (share - acc) / np.sqrt(np.maximum(acc * (1 - acc), 1e-12) / N)
    print(f"[block sampling] {N} runs; chi-square p-values of tokens 1-{n}: "
          f"{[f'{x:.3g}' for x in pvals]}; accepted-draft share {np.round(share, 4).tolist()} "
          f"vs oracle {np.round(acc, 4).tolist()}", flush=True)
    # the regime: most runs hold a rejection and its resample
    assert 0.3 < share[1:n - 1].mean() < 0.7
    assert min(pvals) > 1e-4
    # shares with zero probability must be exactly zero (the first and last tokens are drawn)
    assert np.all(share[acc == 0] == 0)
    assert np.abs(z[acc > 0]).max() < 4.5


def test_block_resample_is_the_second_draw_of_the_rejecting_row(workload):
    from pulsar_engine.engine import sample_rows

    f, s, cfg, model, prompt = workload
    B, seed = 64, 4242
    checked = accepted = rejected = distinct = last_rows = 0
    with _engine(model, s, B, seed) as eng:
        eng.prefill(np.tile(prompt, (B, 1)))
        for _ in range(200):
            before = eng.state()
            if before[:, 0].all():
                break
            toks_before = eng.tokens()
            eng.step(1)
            rows = eng.rows(last=True)
            toks_after, kinds_after = eng.tokens(), eng.token_kinds()
            ending = [b for b in range(B) if not before[b, 0] and before[b, ST_BLK_PHASE] == 1
                      and before[b, ST_BLK_STEP] == cfg.default_pulses - 1]
            if not ending:
                continue
            lg = torch.from_numpy(eng.logits(int(eng.last_ctl()[1]))).cuda()
            for b in ending:
                blk_rows = sorted((r for r in rows if int(r[0]) == b and int(r[2]) == 2),
                                  key=lambda r: int(r[1]))
                blk = [int(r[4]) for r in blk_rows]
                new = toks_after[b][len(toks_before[b]):]
                new_kinds = kinds_after[b][len(toks_before[b]):]
                a = 0
                while a < len(new_kinds) and new_kinds[a] == 1:
                    a += 1
                if a >= len(new):
                    continue  # max_new reached on an accepted draft: no row ends the round
                assert new[:a] == blk[1:a + 1]
                ctr = int(np.uint32(before[b, ST_CTR]))
                seen0 = prompt.tolist() + toks_before[b]
                for i in range(min(a + 1, len(blk))):
                    r = blk_rows[i]
                    c = (ctr * 2 + 1) * MAX_BLOCK + int(r[1])
                    seen_i = seen0 + blk[1:i + 1]
                    # the standalone sampler's counter is ctr * 2 + (row has an extra seen
                    # token): an extra already in the seen set changes nothing else; the
                    # generator is keyed by the sequence index too, so the row names b
                    extra = seen_i[0] if c & 1 else -1
                    seen_all = [[] for _ in range(b)] + [seen_i]
                    _, dr = sample_rows(lg[int(r[5])][None], seen_all, [b], [extra],
                                        [0] * b + [c >> 1], seed, s["temperature"], s["top_p"],
                                        s["repetition_penalty"], dtype=torch.float32)
                    v, fr = int(dr[0, 0]), int(dr[0, 1])
                    checked += 1
                    if i < a:
                        assert v == blk[i + 1], (b, i, v, blk)
                        accepted += 1
                    elif i < len(blk) - 1:
                        # the rejection: v_i differs from the draft, the emitted token is f_i
                        assert v != blk[i + 1], (b, i, v, blk)
                        assert new[a] == fr, (b, i, new[a], v, fr)
                        rejected += 1
                        distinct += v != fr
                    else:
                        # every draft accepted: the last row's first draw is emitted
                        assert new[a] == v, (b, i, new[a], v)
                        last_rows += 1
    print(f"[block resample] {checked} verify rows re-drawn: {accepted} accepted drafts, "
          f"{rejected} rejections ({distinct} with f_i != v_i), {last_rows} last rows",
          flush=True)
    assert rejected >= 20 and distinct >= 10 and accepted >= 20
