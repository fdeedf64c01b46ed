"""GPU parity of the draft-block mode and the block-verify entry against the oracle.

The draft-block mode (HipEngine(draft_len=G)) has no reference counterpart; its oracle is
``RefEngine.block_speculative_ids`` / ``block_verify`` (pinned in tests/test_oracle_block.py
against the reference's goldens). Checks:

* fp32 greedy token streams identical to the oracle's, draft lengths 4 and 6;
* every pass's logits (drafts and the three verify pulses) within 2e-2 max-abs relative of
  the oracle in bf16 (1e-4 in fp32);
* the verify entry over a prefilled cache against ``block_verify`` (fp32 and bf16), equal
  under graph replay and on a second call;
* sampled mode: accepted drafts within 4 sigma of the sum of the per-test overlaps
  sum_x p_draft(x) p_verify(x) computed from the engine's own logits;
* at the verify-microbenchmark shape (64 sequences, 8192 cached N(0,1) positions, 5-token
  blocks): sequence 0 is identical in batches of 64 and 32 and within the bf16 bound of
  the same sequence alone, logits finite.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_abs_rel

pytestmark = pytest.mark.gpu


def _oracle(full_state, dtype):
    from oracle import pulsar_ref as R

    cfg, st = full_state
    return R.load_ref(cfg, st, dtype, rope_tables_fp32=True, stop_ids=set())


@pytest.mark.parametrize("G", [4, 6])
def test_fp32_block_greedy_streams_equal_oracle(models, full_state, G):
    from pulsar_engine import weights as W
    from pulsar_engine.engine import PulsarInferenceEngine

    cfg = full_state[0]
    prompts = [W.uniform_ids(60 + s, "block_prompt", 40, cfg.vocab_size).tolist() for s in range(2)]
    ref = _oracle(full_state, torch.float32)
    want = [list(ref.block_speculative_ids(p, 20, 0.0, 1.0, 10.0, G)) for p in prompts]
    eng = PulsarInferenceEngine(models[torch.float32])
    got = eng.generate_ids(prompts, max_new_tokens=20, temperature=0.0, repetition_penalty=10.0,
                           stop_ids=[], draft_len=G)
    print(f"G={G} gpu {got}\n      ref {want}")
    assert got == want


@pytest.mark.parametrize("k", [3, 6, 11])
def test_fp32_block_stop_id_drafted_mid_block(models, full_state, k):
    """A stop id among the drafts ends the block early; the verify then starts at pulse 1
    (every block row's pulse 0 ran in a draft step) and the stop id is never emitted. The
    stop is the k-th token of the stream without stop ids: greedy drafts are accepted here,
    so the run with that stop drafts it mid-block. Streams equal the oracle's."""
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import PulsarInferenceEngine

    cfg, st = full_state
    prompt = W.uniform_ids(64, "block_prompt", 40, cfg.vocab_size).tolist()
    free = list(_oracle(full_state, torch.float32).block_speculative_ids(prompt, 20, 0.0, 1.0,
                                                                        10.0, 4))
    stop = free[k]
    assert stop not in free[:k]
    ref = R.load_ref(cfg, st, torch.float32, rope_tables_fp32=True, stop_ids={stop})
    want = list(ref.block_speculative_ids(prompt, 20, 0.0, 1.0, 10.0, 4))
    eng = PulsarInferenceEngine(models[torch.float32])
    got = eng.generate_ids([prompt], max_new_tokens=20, temperature=0.0,
                           repetition_penalty=10.0, stop_ids=[stop], draft_len=4)[0]
    print(f"k={k} stop {stop}: gpu {got}\n                ref {want}")
    assert want == free[:k] and got == want


def _compare_block_passes(models, full_state, dtype, G, tol, prompt=None, n_new=12):
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    if prompt is None:
        prompt = W.uniform_ids(70, "block_pass_prompt", 40, cfg.vocab_size).tolist()
    ref = _oracle(full_state, dtype)
    ref.trace = []
    list(ref.block_speculative_ids(prompt, n_new, 0.0, 1.0, 10.0, G))
    table = {}
    for t in ref.trace:
        if t[0] == "block":
            table[(t[2], t[1], t[3])] = t[4].float().numpy()
    cache = R.RefKVCache(cfg)
    ref_prefill = ref.prefill(torch.as_tensor(prompt).view(1, -1), cache).float().numpy().reshape(-1)

    eng = HipEngine(models[dtype], batch=1, max_prompt=len(prompt), max_new=n_new,
                    temperature=0.0, repetition_penalty=10.0, stop_ids=[], all_logits=True,
                    draft_len=G)
    eng.prefill(np.asarray(prompt)[None])
    errs = [("prefill", max_abs_rel(eng.logits(1)[0], ref_prefill))]
    cur = []  # tokens of the current round's block, by slot, as the draft rows reveal them
    S = eng.slots
    for _ in range(200):
        if eng.state()[0, 0]:
            break
        eng.step(1)
        rows = eng.rows(last=True).tolist()
        lg = eng.logits(len(rows))
        groups = {}
        for r in rows:
            groups.setdefault(r[2], []).append(r)
        for pulse, grp in sorted(groups.items()):
            grp.sort(key=lambda r: r[1])
            for r in grp:
                slot, pos, tok, lrow = r[1], r[3], r[4], r[5]
                if lrow < 0:
                    continue
                if len(grp) == 1:
                    # a draft row, a one-row block, or (slot S - 1 beside a verify pass) the
                    # next round's first row
                    if slot == S - 1 and len(groups) > 1:
                        slot = 0
                    cur = cur[:slot] + [tok] if slot > 0 else [tok]
                    prefix = tuple(cur)
                else:
                    prefix = tuple(x[4] for x in grp[:slot + 1])
                # row `slot` of any oracle block at this position and pulse with the same
                # tokens up to it (rows do not depend on later block tokens)
                hit = [v for (p0, toks, k), v in table.items()
                       if p0 == pos - slot and k == pulse and toks[:slot + 1] == prefix]
                if hit:
                    errs.append(((pos, pulse, tok), max_abs_rel(lg[lrow], hit[0][slot])))
    print(f"{dtype} G={G} block passes compared: {len(errs)}; worst: {max(e for _, e in errs):.3e}")
    bad = [(k, e) for k, e in errs if e > tol]
    assert not bad, bad[:5]
    assert len(errs) >= 12, len(errs)
    eng.close()


def test_fp32_block_pass_logits_match_oracle(models, full_state):
    _compare_block_passes(models, full_state, torch.float32, 4, 1e-4)


def test_bf16_block_pass_logits_within_2e2(models, full_state):
    _compare_block_passes(models, full_state, torch.bfloat16, 4, 2e-2)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_verify_entry_matches_oracle_block_verify(models, full_state, dtype, tol):
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    B, T, n = 3, 36, 5
    prompts = np.stack([W.uniform_ids(80 + b, "verify_prompt", T, cfg.vocab_size) for b in range(B)])
    blocks = np.stack([W.uniform_ids(90 + b, "verify_block", n, cfg.vocab_size) for b in range(B)])
    eng = HipEngine(models[dtype], batch=B, max_prompt=T, max_new=8, temperature=0.0,
                    stop_ids=[], draft_len=n - 1)
    eng.prefill(prompts)
    eng.verify(blocks)
    got = eng.logits(B * n).reshape(B, n, -1).copy()
    eng.verify(blocks, graph=True)
    got_graph = eng.logits(B * n).reshape(B, n, -1).copy()
    eng.verify(None, graph=True)
    got_again = eng.logits(B * n).reshape(B, n, -1)
    np.testing.assert_array_equal(got, got_graph)
    np.testing.assert_array_equal(got, got_again)
    ref = _oracle(full_state, dtype)
    worst = 0.0
    for b in range(B):
        cache = R.RefKVCache(cfg)
        ref.prefill(torch.as_tensor(prompts[b]).view(1, -1), cache)
        lg, _, _ = ref.block_verify(blocks[b].tolist(), T, cache)
        for i in range(n):
            e = max_abs_rel(got[b, i], lg[i].float().numpy())
            worst = max(worst, e)
            assert e <= tol, (b, i, e)
    print(f"{dtype} verify entry worst {worst:.3e}")
    eng.close()


def test_bf16_block_sampled_acceptance_matches_draft_verify_overlap(models, full_state):
    """Accepted drafts minus the sum of p_i over the tests performed is a sum of
    martingale differences (each test accepts with probability p_i given the past), so the
    count lies within 4 sqrt(sum p_i (1 - p_i)) of sum p_i."""
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    B, T_, N, G = 16, 24, 24, 3
    temp, top_p, rp = 1.0, 0.95, 1.15
    prompts = np.stack([W.uniform_ids(140 + b, "blk_acc_prompt", T_, cfg.vocab_size)
                        for b in range(B)])
    eng = HipEngine(models[torch.bfloat16], batch=B, max_prompt=T_, max_new=N, temperature=temp,
                    top_p=top_p, repetition_penalty=rp, stop_ids=[], all_logits=True, seed=4321,
                    draft_len=G)
    eng.prefill(prompts)
    draft_lg = {}
    expected, var, n_tests = 0.0, 0.0, 0
    P = cfg.default_pulses
    for _ in range(40 * (N + 2)):
        before = eng.state().copy()
        if before[:, 0].all():
            break
        toks_before = eng.tokens()
        eng.step(1)
        after = eng.state()
        rows = eng.rows(last=True)
        lg = eng.logits(len(rows))
        by_seq = {}
        for r in rows:
            by_seq.setdefault(int(r[0]), []).append(r)
        for b, rs in by_seq.items():
            if len(rs) == 1 and int(rs[0][2]) == 0 and before[b, 21] == 0:
                # draft row of slot j: keep its logits for the verify's tests
                draft_lg[(b, int(rs[0][1]))] = lg[int(rs[0][5])].copy()
                continue
            blk_rows = sorted((r for r in rs if int(r[2]) == P - 1), key=lambda r: int(r[1]))
            # the next round's first row riding in the last verify step (pipelined rounds)
            spec = [r for r in rs if int(r[2]) == 0 and int(r[1]) == eng.slots - 1]
            if before[b, 21] != 1 or before[b, 22] != P - 1 or not blk_rows:
                continue
            rs = blk_rows
            blk = [int(r[4]) for r in rs]
            seen = [int(x) for x in prompts[b]] + toks_before[b]
            # tests 0 .. ran-1 of the block ran (each one only after every earlier draft of
            # the block was accepted)
            ran = int(after[b, 11] - before[b, 11])
            for i in range(ran):
                extra = blk[1:i + 1]
                pd = R.sampling_distribution(torch.from_numpy(draft_lg[(b, i)]).view(1, -1),
                                             seen + extra, temp, top_p, rp)
                pv = R.sampling_distribution(torch.from_numpy(lg[int(rs[i][5])]).view(1, -1),
                                             seen + extra, temp, top_p, rp)
                p = float((pd * pv).sum())
                expected += p
                var += p * (1 - p)
                n_tests += 1
            draft_lg = {k: v for k, v in draft_lg.items() if k[0] != b}
            if spec:
                # the next round's first draft, when the guess holds (else its own draft
                # step overwrites this)
                draft_lg[(b, 0)] = lg[int(spec[0][5])].copy()
    tests, accepted = eng.acceptance()
    sd = max(var, 1e-9) ** 0.5
    print(f"block tests {tests} (tracked {n_tests}), accepted {accepted}, "
          f"expected {expected:.1f} +- {sd:.1f}")
    assert tests == n_tests and tests >= 40
    assert abs(accepted - expected) <= 4 * sd + 1e-6
    eng.close()


def test_verify_microbench_shape_batch_consistent(models, full_state):
    """64 sequences over 8192 cached N(0,1) positions, 5-token blocks: sequence 0 gives the
    same logits in a batch of 64 as in a batch of 32 (both hold 128+ rows per step and run
    the output head in wide tiles: identical), and within the bf16 parity bound (2e-2 of
    max|logit|) of the same cache and block alone (row-tile head, another summation order);
    all logits finite."""
    from conftest import max_abs_rel
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    B, ctx, n = 64, 8192, 5
    blocks = np.stack([W.uniform_ids(300 + b, "c3_block", n, cfg.vocab_size) for b in range(B)])
    kw = dict(max_prompt=1, max_new=8, temperature=0.0, stop_ids=[], draft_len=n - 1,
              max_ctx=ctx + 16)
    first = {}
    for bsz in (B, B // 2, 1):
        eng = HipEngine(models[torch.bfloat16], batch=bsz, **kw)
        eng.fill_kv(ctx, seed=11)
        eng.verify(blocks[:bsz], graph=bsz > 1)
        lg = eng.logits(bsz * n).reshape(bsz, n, -1)
        assert np.isfinite(lg).all()
        first[bsz] = lg[0].copy()
        eng.close()
    assert np.array_equal(first[B], first[B // 2])
    err = max_abs_rel(torch.from_numpy(first[B]), torch.from_numpy(first[1]))
    print(f"[verify] batch 64 vs 32: identical; vs alone {err:.3e}", flush=True)
    assert err <= 2e-2
