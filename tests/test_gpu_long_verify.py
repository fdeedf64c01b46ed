"""GPU: block verify over long pre-filled caches against the oracle, at the verify
microbenchmark's shape (64 sequences x 8192 cached positions), the long-context shape
(4 sequences x 32768 cached positions, YaRN in the global layers, 513 pages per sequence)
and a wide one (224 sequences x 1024 positions: 1120 rows per pass, so the projections
run in the 128 x 256 LDS tiles).

The engine's synthetic cache (pulsar_engine_fill_kv: every key/value element ~ N(0,1) from
a counter-based generator) is regenerated on the CPU for the compared sequences
(oracle.fill_kv_cache), and the oracle's block_verify of the same 5 tokens (4 drafts + 1)
over it gives the reference logits: every row of the last pulse within max|diff| / max|ref|
<= 2e-2 (bf16). A graph replay of the same verify gives identical logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import max_abs_rel

pytestmark = pytest.mark.gpu


@pytest.mark.timeout(900)
@pytest.mark.parametrize("B,ctx,check", [(64, 8192, [0, 63]), (4, 32768, [0, 3]),
                                         (224, 1024, [0, 223])])
def test_verify_over_prefilled_cache_matches_oracle(models, full_state, B, ctx, check):
    from oracle import pulsar_ref as R
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg, st = full_state
    n = 5
    tokens = np.stack([W.uniform_ids(7, f"verify_block_{b}", n, cfg.vocab_size) for b in range(B)])
    with HipEngine(models[torch.bfloat16], batch=B, max_prompt=1, max_new=8, draft_len=4,
                   max_ctx=ctx + 16, stop_ids=[]) as eng:
        eng.fill_kv(ctx, seed=5)
        layout = eng.kv_layout()
        eng.verify(tokens)
        got = eng.logits(B * n)
        eng.verify(None, graph=True)
        eng.verify(None, graph=True)
        again = eng.logits(B * n)
    np.testing.assert_array_equal(again, got)
    ref = R.load_ref(cfg, st, torch.bfloat16, stop_ids=set())
    for b in check:
        cache = R.fill_kv_cache(cfg, layout, ctx, 5, b, B)
        want, _, _ = ref.block_verify(tokens[b].tolist(), ctx, cache)
        err = max_abs_rel(got[b * n:(b + 1) * n], want.float().numpy())
        print(f"[verify] {B} x {ctx}: sequence {b} last-pulse logits error {err:.3e}", flush=True)
        assert err <= 2e-2
