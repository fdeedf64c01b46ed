"""GPU: the adaptive early exit of the HIP engine (reference src/infer.py:198-232, :526-549,
:775-780).

* Full-size fp32 model, threshold 0.9978: plain and self-speculative greedy streams and the
  per-pulse exit counts equal the reference's (tests/golden/early_exit.npz).
* Reduced fp32 model whose top-1 probability rises from pulse 0 to pulse 1
  (weights.exit_probe_state), three thresholds that send tokens out after every pulse,
  three prompts in one batch: streams and per-sequence counts equal the oracle's. The
  oracle's closest exit test sits >= 5e-4 (relative) from the threshold, far above the
  fp32 logits' difference.
* bf16: each exit decision of the engine equals the reference's rule (top-1 of a bf16
  softmax >= threshold) applied to the engine's own logits of that pass.
* generate() prints the reference's statistics block for the counts of its run.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def probe():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pulsar_engine import weights as W
    from pulsar_engine.config import small_config
    from pulsar_engine.model import DeviceModel

    cfg = small_config()
    st = W.exit_probe_state(cfg)
    return cfg, st, DeviceModel(cfg, st, torch.float32)


def test_full_fp32_streams_and_exit_counts_equal_reference(models):
    from pulsar_engine.engine import PulsarInferenceEngine

    g = golden("early_exit.npz")
    thr = float(g["full_threshold"])
    for name, spec in (("greedy_plain", False), ("greedy_spec", True)):
        eng = PulsarInferenceEngine(models[torch.float32])
        eng.set_early_exit_threshold(thr)
        ids = eng.generate_ids([g["full_prompt"].tolist()], max_new_tokens=32, temperature=0.0,
                               repetition_penalty=10.0, speculative=spec, stop_ids=[0, 2])[0]
        print(f"[early exit] full fp32 {name}: counts {eng.early_exit_counts}", flush=True)
        assert ids == g[f"full_{name}_ids"].tolist(), name
        assert eng.early_exit_counts == g[f"full_{name}_counts"].tolist(), name


@pytest.mark.parametrize("thr", [0.038, 0.040, 0.042])
@pytest.mark.parametrize("spec", [False, True])
def test_reduced_fp32_exits_at_every_pulse_match_oracle(probe, thr, spec):
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg, st, model = probe
    prompts = np.stack([W.uniform_ids(s, "exit_prompt", 24, cfg.vocab_size) for s in range(3)])
    ref = R.load_ref(cfg, st, torch.float32, stop_ids=set())
    want_ids, want_counts, margin = [], [], 1.0
    for p in prompts:
        ref.set_early_exit_threshold(thr)
        ref.trace = []
        gen = ref.self_speculative_ids if spec else ref.stream_generate_ids
        want_ids.append(list(gen(p, 24, 0.0, 1.0, 10.0)))
        want_counts.append(list(ref.early_exit_counts))
        mps = np.array([e[4] for e in ref.trace if e[0] == "exit_check"])
        margin = min(margin, float(np.min(np.abs(mps - thr) / thr)))
    assert margin > 1e-4, "threshold too close to an exit test for an fp32 comparison"
    with HipEngine(model, batch=3, max_prompt=24, max_new=24, speculative=spec,
                   temperature=0.0, repetition_penalty=10.0, stop_ids=[],
                   early_exit_threshold=thr) as eng:
        eng.prefill(prompts)
        eng.run()
        got_ids, got_counts = eng.tokens(), eng.exit_counts().tolist()
    print(f"[early exit] thr {thr} spec {spec}: counts {got_counts}", flush=True)
    assert got_ids == want_ids
    assert got_counts == want_counts
    if not spec:
        assert all(sum(c) == 24 for c in got_counts)  # one decode per emitted token
    assert np.asarray(got_counts).sum(axis=0).min() > 0  # exits after every pulse


def test_bf16_exit_decisions_follow_the_rule_on_the_engines_logits():
    """Step by step, with every pass's logits readable: a token at pulse k < 2 leaves
    (the sequence's next row is a new token) iff the top-1 probability of the bf16 softmax
    of its pulse-k logits is >= the threshold."""
    import torch.nn.functional as F

    from pulsar_engine import weights as W
    from pulsar_engine.config import small_config
    from pulsar_engine.engine import HipEngine
    from pulsar_engine.model import DeviceModel

    cfg = small_config(n_heads=16, n_kv_heads=4)
    model = DeviceModel(cfg, W.exit_probe_state(cfg), torch.bfloat16)
    prompts = np.stack([W.uniform_ids(s, "exit_prompt", 24, cfg.vocab_size) for s in range(4)])
    thr = 0.034
    checked = exits = 0
    with HipEngine(model, batch=4, max_prompt=24, max_new=16, speculative=False,
                   temperature=0.0, repetition_penalty=10.0, stop_ids=[], all_logits=True,
                   early_exit_threshold=thr) as eng:
        eng.prefill(prompts)
        for _ in range(200):
            if eng.state()[:, 0].all():
                break
            eng.step(1)
            rows = eng.rows(last=True)
            lg = eng.logits(len(rows))
            nxt = {int(r[0]): r for r in eng.rows(last=False)}
            for r in rows:
                b, pulse, pos = int(r[0]), int(r[2]), int(r[3])
                if pulse >= 2 or b not in nxt:
                    continue
                x = torch.from_numpy(lg[int(r[5])]).to(torch.bfloat16)
                p = F.softmax(x, dim=-1).max().item()
                # the exact probability; skip it when it lies within 1e-5 (relative) of a
                # midpoint between two bf16 values, where fp32 summation order decides
                p64 = (1.0 / torch.exp(x.double() - x.double().max()).sum()).item()
                ulp = 2.0 ** (np.floor(np.log2(p64)) - 7)
                if abs((p64 / ulp) % 1.0 - 0.5) * ulp < p64 * 1e-5:
                    continue
                left = int(nxt[b][3]) == pos + 1
                assert left == (p >= thr), (b, pos, pulse, p)
                checked += 1
                exits += int(left)
        counts = eng.exit_counts()
    print(f"[early exit] bf16 decisions checked {checked}, exits {exits}, counts {counts.tolist()}",
          flush=True)
    assert checked >= 20 and 0 < exits < checked
    assert counts[:, 0].sum() > 0 and counts[:, 2].sum() > 0


def test_generate_prints_the_exit_statistics(probe, capsys):
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import (PulsarInferenceEngine, early_exit_stats,
                                      format_early_exit_stats)

    cfg, st, model = probe

    class Tok:
        unk_token_id = None

        def __init__(self, ids):
            self.ids = ids

        def encode(self, prompt, return_tensors=None):
            return torch.tensor([self.ids])

        def decode(self, ids, skip_special_tokens=False):
            return "".join(f"<{int(i)}>" for i in ids)

        def convert_tokens_to_ids(self, tok):
            return None

    prompt = W.uniform_ids(0, "exit_prompt", 24, cfg.vocab_size).tolist()
    ref = R.load_ref(cfg, st, torch.float32, stop_ids={cfg.eos_token_id})
    ref.set_early_exit_threshold(0.040)
    want = list(ref.stream_generate_ids(prompt, 12, 0.0, 1.0, 10.0))
    eng = PulsarInferenceEngine(model)
    eng.set_early_exit_threshold(0.040)
    text = eng.generate(Tok(prompt), "p", max_new_tokens=12, temperature=0.0,
                        repetition_penalty=10.0, stream=False, speculative=False)
    assert text == "p" + "".join(f"<{i}>" for i in want)
    assert eng.early_exit_counts == ref.early_exit_counts
    out = capsys.readouterr().out
    assert out == format_early_exit_stats(0.040, early_exit_stats(ref.early_exit_counts))
    assert "[Adaptive Early-Exit Stats | Threshold: 0.04]" in out


def test_early_exit_is_rejected_in_the_draft_block_mode(probe):
    from pulsar_engine.engine import HipEngine

    cfg, st, model = probe
    with pytest.raises(RuntimeError, match="exact schedule"):
        HipEngine(model, batch=1, max_prompt=8, max_new=4, draft_len=4,
                  early_exit_threshold=0.5)
