"""GPU: models loaded from reference checkpoints and kernel-format files, a second bf16
shape, and the tokenizer-level generate interface.

* A reduced bf16 model whose query width (16 heads x 64) exceeds d_model (256): every
  pulse pass within max|diff| / max|ref| <= 2e-2 of the oracle.
* The same weights reached three ways (a reference-format checkpoint with an old [E]
  expert_bias, its kernel-format export, and the state converted directly with the bias
  broadcast and centred by hand) give identical greedy and sampled streams.
* ``generate`` with a tokenizer returns the prompt plus the decoded id stream of
  ``generate_ids`` under the tokenizer's stop ids (src/infer.py:733-782, :649-656).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def reduced():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pulsar_engine import weights as W
    from pulsar_engine.config import small_config

    cfg = small_config(n_heads=16, n_kv_heads=4)
    return cfg, W.synthetic_state(cfg, seed=5)


@pytest.fixture(scope="module")
def reduced_model(reduced):
    from pulsar_engine.model import DeviceModel

    cfg, st = reduced
    return DeviceModel(cfg, st, torch.bfloat16)


def test_reduced_bf16_pass_logits_within_2e2(reduced, reduced_model):
    from test_gpu_engine import _compare_passes

    from pulsar_engine import weights as W

    cfg = reduced[0]
    prompt = W.uniform_ids(9, "gpu_prompt", 40, cfg.vocab_size).tolist()
    _compare_passes({torch.bfloat16: reduced_model}, reduced, torch.bfloat16, prompt, 6,
                    tol=2e-2, rp=10.0)


def test_checkpoint_kernel_format_and_direct_streams_agree(reduced, tmp_path):
    from pulsar_engine import checkpoint as C
    from pulsar_engine import weights as W
    from pulsar_engine.engine import PulsarInferenceEngine
    from pulsar_engine.model import DeviceModel

    cfg, st = reduced
    E, mp = cfg.n_routed_experts, cfg.max_pulses
    rng = np.random.default_rng(11)
    ck_model, direct = {}, dict(st)
    for k, v in st.items():
        if k.endswith("expert_bias"):
            b = torch.from_numpy(rng.normal(0, 0.5, E).astype(np.float32))  # old [E] buffer
            ck_model[k] = b
            full = b.unsqueeze(0).expand(mp, -1)
            direct[k] = (full - full.mean(dim=-1, keepdim=True)).numpy()
        else:
            ck_model[k] = torch.from_numpy(v)
    ck_model["core.0.mlp.expert_counts_accum"] = torch.zeros(E)
    path = str(tmp_path / "best.pt")
    torch.save({"config": cfg.to_dict(), "model": ck_model, "step": 100}, path)
    kdir = C.export_checkpoint(path, str(tmp_path / "kernel"), torch.bfloat16)

    engines = {
        "checkpoint": C.load_inference_model(path, dtype=torch.bfloat16)[0],
        "kernel_format": C.load_inference_model(kdir)[0],
        "direct": PulsarInferenceEngine(DeviceModel(cfg, direct, torch.bfloat16)),
    }
    prompts = [W.uniform_ids(60 + s, "ck_prompt", 29, cfg.vocab_size).tolist() for s in range(3)]
    out = {}
    for name, eng in engines.items():
        assert eng.dtype == torch.bfloat16
        greedy = eng.generate_ids(prompts, max_new_tokens=16, temperature=0.0,
                                  repetition_penalty=10.0, speculative=True, stop_ids=[])
        sampled = eng.generate_ids(prompts, max_new_tokens=16, temperature=0.8, top_p=0.9,
                                   repetition_penalty=1.15, speculative=True, stop_ids=[],
                                   seed=77)
        out[name] = (greedy, sampled)
        print(name, greedy[0][:8], sampled[0][:8])
    assert out["checkpoint"] == out["direct"]
    assert out["kernel_format"] == out["direct"]


class ByteTokenizer:
    """Bytes 0-255 as ids 3-258; three special tokens; ``encode`` like a Hugging Face
    tokenizer called with ``return_tensors="pt"``."""

    specials = {"<|im_end|>": 300, "<|endoftext|>": 301, "</s>": 302}
    unk_token_id = 1

    def encode(self, text, return_tensors=None):
        ids = [b + 3 for b in text.encode("utf-8")]
        return torch.tensor([ids]) if return_tensors == "pt" else ids

    def decode(self, ids, skip_special_tokens=False):
        return "".join(chr(i - 3) if 3 <= i < 259 else f"<{i}>" for i in ids)

    def convert_tokens_to_ids(self, tok):
        return self.specials.get(tok, self.unk_token_id)


@pytest.mark.parametrize("speculative", [True, False])
def test_tokenizer_generate_decodes_the_id_stream(reduced_model, speculative, capsys):
    from pulsar_engine.engine import PulsarInferenceEngine, stop_ids_for

    tok = ByteTokenizer()
    eng = PulsarInferenceEngine(reduced_model)
    prompt = "The pulse of a star, sampled on the GPU:"
    ids = tok.encode(prompt, return_tensors="pt")[0].tolist()
    stops = stop_ids_for(reduced_model.cfg, tok)
    assert stops == {reduced_model.cfg.eos_token_id, 300, 301, 302}
    want = eng.generate_ids([ids], max_new_tokens=24, temperature=0.0, repetition_penalty=1.15,
                            speculative=True, stop_ids=stops)[0]
    text = eng.generate(tok, prompt, max_new_tokens=24, temperature=0.0,
                        repetition_penalty=1.15, stream=True, speculative=speculative)
    assert text == prompt + tok.decode(want)
    assert capsys.readouterr().out == tok.decode(want) + "\n"
