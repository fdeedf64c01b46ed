"""GPU: the mid-size projection GEMMs (launch_gemm_mid: 128-row x 64-column tiles with the
weights staged through LDS) give results identical to the row-tile GEMMs (launch_gemm) on
every projection of a pass: qkv + gate (rows of a pulse), wo with the residual, the fused
shared + routed gate/up (SwiGLU, K0 = K) and down (K0 = 2K) launches.

The mid-size kernel cuts K into the row-tile kernel's 8 chunks and adds the chunk sums in
its order, so the two must agree bit for bit. The environment variable
PULSAR_GEMM_MID_ROWS (read when an engine is created) picks the kernel: 0 keeps the
row-tile GEMMs, 1 runs the mid-size ones at every step size. Cases: a block verify over a
filled cache (320 rows per pass, the verify microbenchmark's row count at a shorter
cache), sampled decoding in the reference's schedule at batch 64 (128 rows per step) and a
greedy draft-block run at batch 4 (a few rows per expert: most tile rows clamped).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _engine(models, mid_rows, **kw):
    from pulsar_engine.engine import HipEngine

    old = os.environ.get("PULSAR_GEMM_MID_ROWS")
    os.environ["PULSAR_GEMM_MID_ROWS"] = str(mid_rows)
    try:
        return HipEngine(models[torch.bfloat16], **kw)
    finally:
        if old is None:
            del os.environ["PULSAR_GEMM_MID_ROWS"]
        else:
            os.environ["PULSAR_GEMM_MID_ROWS"] = old


def test_mid_gemm_verify_identical(models, full_state):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    B, ctx, n = 64, 1024, 5
    blocks = np.stack([W.uniform_ids(500 + b, "mid_block", n, cfg.vocab_size) for b in range(B)])
    kw = dict(batch=B, max_prompt=1, max_new=8, temperature=0.0, stop_ids=[], draft_len=n - 1,
              max_ctx=ctx + 16)
    out = {}
    for mid in (0, 1):
        print(f"[mid gemm] verify B={B} ctx={ctx} block={n} mid_rows={mid}", flush=True)
        with _engine(models, mid, **kw) as eng:
            eng.fill_kv(ctx, seed=5)
            eng.verify(blocks)
            out[mid] = eng.logits(B * n).copy()
    assert np.isfinite(out[0]).all()
    diff = np.abs(out[0] - out[1]).max()
    print(f"[mid gemm] verify max |diff| {diff}", flush=True)
    assert np.array_equal(out[0], out[1])


@pytest.mark.parametrize("batch,draft_len,temperature", [(64, 0, 0.8), (4, 4, 0.0)])
def test_mid_gemm_decode_identical(models, full_state, batch, draft_len, temperature):
    from pulsar_engine import weights as W

    cfg = full_state[0]
    T, N_NEW = 96, 24
    prompts = np.stack([W.uniform_ids(700 + b, "mid_prompt", T, cfg.vocab_size)
                        for b in range(batch)])
    kw = dict(batch=batch, max_prompt=T, max_new=N_NEW, speculative=True,
              temperature=temperature, top_p=0.95, repetition_penalty=1.15, stop_ids=[],
              seed=77, draft_len=draft_len)
    toks, lg = {}, {}
    for mid in (0, 1):
        print(f"[mid gemm] decode batch={batch} draft_len={draft_len} T={temperature} "
              f"mid_rows={mid}", flush=True)
        with _engine(models, mid, **kw) as eng:
            eng.prefill(prompts)
            eng.run()
            toks[mid] = eng.tokens()
            n_l = int(eng.last_ctl()[1])
            lg[mid] = eng.logits(max(n_l, 1)).copy()
    assert all(len(t) == N_NEW for t in toks[0])
    assert toks[0] == toks[1]
    assert np.array_equal(lg[0], lg[1])
