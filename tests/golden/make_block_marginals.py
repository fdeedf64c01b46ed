"""Write the exact emitted-token distributions of the draft-block mode in a regime where
drafts are rejected about half the time, for the GPU chi-square test of the sampled
acceptance and resample (tests/test_gpu_block_sampling.py).

    python tests/golden/make_block_marginals.py [--jobs 8]

The distributions come from the oracle's enumerator (``block_token_marginals``), not from
the reference: the draft-block mode has no reference counterpart. Its first draft test of
every round is the reference's test (src/infer.py:704-725); the enumerator is pinned on
the CPU against a literal enumeration of every draw of ``block_speculative_ids``
(tests/test_oracle_block.py), and the stored file against a fresh enumeration of its first
tokens.

Workload: the small configuration (``pulsar_engine.config.small_config``) with synthetic
weights of seed 0 in fp32, the 24-token prompt ``uniform_ids(0, "dist_prompt", 24, 4096)``,
temperature 0.03, top-p 0.95, repetition penalty 10, draft length 4, the first 6 emitted
tokens, no stop ids. The enumeration's tests accept with probability 0.495 on average
(weighted by path probability; between 0.1 and 1 per test).

Output ``block_marginals_small.npz``: per emitted token k (0..5) the support ``idx_k`` and
probabilities ``p_k`` (fp64, paths below ``prune`` left out), ``accepted_mass`` [6] (the
probability that token k is an accepted draft), the settings, and the weight digest.
Roughly 2.5k verified prefixes, two minutes on one core; the subtrees of the first token's
values are split over worker processes.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from concurrent.futures import ProcessPoolExecutor

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for _p in (ROOT, os.path.join(ROOT, "pulsar-300m_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

SETTINGS = dict(temperature=0.03, top_p=0.95, repetition_penalty=10.0, draft_len=4,
                n_tokens=6, prune=1e-5, prompt_seed=0, prompt_name="dist_prompt",
                prompt_len=24, weight_seed=0)
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "block_marginals_small.npz")


def _setup():
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.config import small_config

    cfg = small_config()
    st = W.synthetic_state(cfg, seed=SETTINGS["weight_seed"])
    prompt = W.uniform_ids(SETTINGS["prompt_seed"], SETTINGS["prompt_name"],
                           SETTINGS["prompt_len"], cfg.vocab_size)
    return R, W, cfg, st, prompt


def marginals(n_tokens=None, first=None):
    """The enumerator's output for the stored workload (`first`: expand only these first
    tokens; see ``block_token_marginals``)."""
    R, W, cfg, st, prompt = _setup()
    torch.set_num_threads(1)
    s = SETTINGS
    eng = R.load_ref(cfg, st, torch.float32, stop_ids=set())
    stats = {}
    m = R.block_token_marginals(eng, prompt, s["temperature"], s["top_p"],
                                s["repetition_penalty"], s["draft_len"],
                                n_tokens or s["n_tokens"], prune=s["prune"], stats=stats,
                                first=first)
    return [x.numpy() for x in m], stats


def _first_support():
    R, W, cfg, st, prompt = _setup()
    eng = R.load_ref(cfg, st, torch.float32, stop_ids=set())
    s = SETTINGS
    cache = R.RefKVCache(cfg)
    lg = eng.prefill(torch.as_tensor(prompt).view(1, -1), cache)[:, -1, :]
    p = R.sampling_distribution(lg, list(prompt), s["temperature"], s["top_p"],
                                s["repetition_penalty"])
    return torch.nonzero(p > s["prune"]).view(-1).tolist()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    args = ap.parse_args()
    t0 = time.time()
    firsts = _first_support()
    with ProcessPoolExecutor(max(1, args.jobs)) as ex:
        parts = list(ex.map(marginals, [None] * len(firsts), [[t] for t in firsts]))
    n = SETTINGS["n_tokens"]
    # every part holds the whole first distribution; the later ones add up
    marg = [parts[0][0][0]] + [sum(p[0][k] for p in parts) for k in range(1, n)]
    acc = [sum(p[1]["accepted_mass"][k] for p in parts) for k in range(n)]
    nodes = sum(p[1]["nodes"] for p in parts)
    pa = np.concatenate([np.asarray(p[1]["p_accept"]) for p in parts])
    wa = np.concatenate([np.asarray(p[1]["w_accept"]) for p in parts])
    mean_acc = float((pa * wa).sum() / wa.sum())
    R, W, cfg, st, prompt = _setup()
    out = {"settings": np.asarray(json.dumps(SETTINGS)),
           "weights_digest": np.asarray(W.state_digest(st)),
           "prompt": np.asarray(prompt, dtype=np.int32),
           "accepted_mass": np.asarray(acc), "mean_p_accept": np.asarray(mean_acc)}
    for k in range(n):
        idx = np.nonzero(marg[k] > 0)[0]
        out[f"idx_{k}"] = idx.astype(np.int32)
        out[f"p_{k}"] = marg[k][idx]
    np.savez_compressed(OUT, **out)
    print(f"[block marginals] {nodes} verified prefixes in {time.time() - t0:.0f} s; mass per "
          f"token {[round(float(m.sum()), 6) for m in marg]}; accepted mass "
          f"{[round(a, 4) for a in acc]}; mean P(accept) {mean_acc:.3f} -> {OUT}")


if __name__ == "__main__":
    main()
