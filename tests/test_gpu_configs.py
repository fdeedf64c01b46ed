"""GPU cases at the sizes of the reference's benchmark configurations.

* c4: 4 sequences of 32768-token prompts (global layers past 32 pages, YaRN in decode,
  the RoPE tables grown past max_seq_len as the reference grows its cache), 512 new tokens:
  greedy self-speculative == plain, and a sequence decodes the same alone as in the batch.
* c5: 256 sequences of 512-token Zipf(1.1) prompts with router weights x4 (skewed routing,
  capacity drops in prefill), 512 new tokens: every pass of one sequence against the oracle
  in bf16, greedy self-speculative == plain over the whole batch, sequences 0 and 255 the
  same in a batch of 64 (batches of 64+ compute the output head in 128-row tiles).
* The same two shapes in the draft-block mode at the configs' draft lengths (c4: 4, c5: 6,
  2048 rows per step at batch 256), 512 new tokens: sequences decode the same in a smaller
  batch; at c5 every pass of one sequence against the oracle's block restatement in bf16.
* Capacity with more assignments per (sequence, expert) than the kernel stages in LDS
  (4200 tokens all routed to experts 0-3): prefill logits against the oracle in fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_abs_rel

pytestmark = pytest.mark.gpu


def _alone(eng, prompts, i, sub, **kw):
    """Sequence i decoded in a sub-batch of `sub` prompts around it (sub = 1: alone)."""
    lo = min(i - i % sub, len(prompts) - sub)
    return eng.generate_ids(prompts[lo:lo + sub], **kw)[i - lo]


def _spec_plain_single(model, prompts, n_new, singles, sub=1):
    """Greedy self-speculative == plain over the batch, and sequences `singles` decode the same
    in a sub-batch of `sub` prompts (1: alone). Batches of 64+ sequences hold 128+ rows per
    step and run the output head in 128-row tiles (1024+ rows: the projections too), and
    those of 128+ sequences take 1024-key attention splits below the long-cache threshold,
    so they are compared with sub-batches on the same side of those thresholds."""
    from pulsar_engine.engine import PulsarInferenceEngine

    eng = PulsarInferenceEngine(model)
    kw = dict(max_new_tokens=n_new, temperature=0.0, repetition_penalty=10.0, stop_ids=[0, 2])
    spec = eng.generate_ids(prompts, speculative=True, **kw)
    plain = eng.generate_ids(prompts, speculative=False, **kw)
    assert spec == plain
    for i in singles:
        assert _alone(eng, prompts, i, sub, speculative=True, **kw) == spec[i], i
    return spec


def test_c4_long_context_spec_equals_plain_and_batch_equals_single(models, full_state):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    T_ = 32768
    prompts = [W.uniform_ids(90 + b, "c4_prompt", T_, cfg.vocab_size).tolist() for b in range(4)]
    spec = _spec_plain_single(models[torch.bfloat16], prompts, 512, singles=[0])
    assert models[torch.bfloat16].rope_len >= T_ + 512
    print("c4 lengths", [len(s) for s in spec])
    print("c4 first tokens", [s[:6] for s in spec])


@pytest.fixture(scope="module")
def c5_model(full_state):
    from pulsar_engine import weights as W
    from pulsar_engine.model import DeviceModel

    cfg = full_state[0]
    st = W.synthetic_state(cfg, seed=0, router_scale=4.0)
    return st, DeviceModel(cfg, st, torch.bfloat16)


def test_c5_skewed_routing_passes_match_oracle(full_state, c5_model):
    from test_gpu_engine import _compare_passes

    from pulsar_engine import weights as W

    cfg = full_state[0]
    st, model = c5_model
    prompt = W.zipf_ids(5, "c5_prompt_0", 512, cfg.vocab_size).tolist()
    _compare_passes({torch.bfloat16: model}, (cfg, st), torch.bfloat16, prompt, 3, tol=2e-2,
                    rp=10.0)


def test_c5_batch_256_spec_equals_plain_and_batch_equals_single(full_state, c5_model):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    prompts = [W.zipf_ids(5, f"c5_prompt_{b}", 512, cfg.vocab_size).tolist() for b in range(256)]
    spec = _spec_plain_single(c5_model[1], prompts, 512, singles=[0, 255], sub=128)
    print("c5 first tokens", [s[:4] for s in spec[:4]], "lengths", sorted({len(s) for s in spec}))


def _block_batch_single(model, prompts, n_new, G, singles, sub=1):
    from pulsar_engine.engine import PulsarInferenceEngine

    eng = PulsarInferenceEngine(model)
    kw = dict(max_new_tokens=n_new, temperature=0.0, repetition_penalty=10.0, stop_ids=[0, 2],
              draft_len=G)
    out = eng.generate_ids(prompts, **kw)
    for i in singles:
        assert _alone(eng, prompts, i, sub, **kw) == out[i], i
    return out


def test_c4_long_context_draft_block_batch_equals_single(models, full_state):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    prompts = [W.uniform_ids(90 + b, "c4_prompt", 32768, cfg.vocab_size).tolist() for b in range(4)]
    out = _block_batch_single(models[torch.bfloat16], prompts, 512, 4, singles=[0])
    print("c4 draft-block first tokens", [s[:6] for s in out])


def test_c5_draft6_block_passes_match_oracle(full_state, c5_model):
    from test_gpu_block import _compare_block_passes

    from pulsar_engine import weights as W

    cfg = full_state[0]
    st, model = c5_model
    prompt = W.zipf_ids(5, "c5_prompt_0", 512, cfg.vocab_size).tolist()
    _compare_block_passes({torch.bfloat16: model}, (cfg, st), torch.bfloat16, 6, 2e-2,
                          prompt=prompt, n_new=8)


def test_c5_batch_256_draft6_batch_equals_single(full_state, c5_model):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    prompts = [W.zipf_ids(5, f"c5_prompt_{b}", 512, cfg.vocab_size).tolist() for b in range(256)]
    # 256 x 7 rows per step run the projections in wide tiles from 1024 rows: a sub-batch
    # of 160 (1120 rows) is on the same side
    out = _block_batch_single(c5_model[1], prompts, 512, 6, singles=[0, 255], sub=160)
    print("c5 draft-block first tokens", [s[:4] for s in out[:4]])


def test_prefill_capacity_beyond_lds_staging_matches_oracle(full_state):
    """4200 assignments per (sequence, expert) against capacity 1344: the threshold is found
    by bisection over the key bits and ties on it are ranked by flat index."""
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
    T_ = 4200
    assert R.moe_capacity(T_, cfg) == 1344
    prompt = W.uniform_ids(80, "cap_big", T_, cfg.vocab_size)
    model = DeviceModel(cfg, st2, torch.float32)
    eng = HipEngine(model, batch=1, max_prompt=T_, max_new=4, speculative=False,
                    temperature=0.0, repetition_penalty=1.0, stop_ids=[])
    eng.prefill(prompt[None])
    got = eng.logits(1)[0]
    ref_eng = R.load_ref(cfg, st2, torch.float32, rope_tables_fp32=True, stop_ids=set())
    ref = ref_eng.prefill(torch.as_tensor(prompt).view(1, -1), R.RefKVCache(cfg))
    err = max_abs_rel(got, ref.float().numpy().reshape(-1))
    print(f"capacity beyond staging: {err:.3e}")
    assert err <= 1e-4
    eng.close()
