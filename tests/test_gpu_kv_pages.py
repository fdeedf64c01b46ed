"""GPU: the global layers' KV page pool (pages of 64 positions handed out as sequences reach
them; PulsarEngineConfig.kv_pages).

* A pool of exactly the pages the batch needs gives the same streams as the default pool
  (every sequence up to max_ctx), and hands out exactly that many pages; rewind returns the
  decode pages, so a second generation from the same prefill fits again.
* A pool short of pages stops the sequences that find it spent (their streams are a prefix
  of the full run's), run() raises, and nothing else is disturbed; a prompt set larger than
  the pool fails prefill with a message.
* The block verify takes the page of its block positions: logits equal the default pool's.
* A verify block the pool cannot hold fails before any launch and takes no page.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

B, T, NEW = 4, 100, 200


def _prompts(cfg):
    from pulsar_engine import weights as W

    return np.stack([W.uniform_ids(40 + b, "kv_pages_prompt", T, cfg.vocab_size)
                     for b in range(B)])


def _engine(models, **kw):
    from pulsar_engine.engine import HipEngine

    return HipEngine(models[torch.bfloat16], batch=B, max_prompt=T, max_new=NEW,
                     temperature=0.0, repetition_penalty=1.15, stop_ids=[], max_ctx=1024, **kw)


def test_exact_pool_gives_the_full_pools_streams(models, full_state):
    prompts = _prompts(full_state[0])
    need = B * ((T + NEW + 1 + 63) // 64)  # positions 0 .. T + NEW (the last speculative row)
    with _engine(models) as full:
        full.prefill(prompts)
        full.run()
        want = full.tokens()
        assert full.kv_pages()["pool"] == B * (1024 // 64)
    with _engine(models, kv_pages=need) as eng:
        eng.prefill(prompts)
        assert eng.kv_pages() == {"pool": need, "used": B * 2, "spent": False}
        eng.run()
        pages = eng.kv_pages()
        print(f"[kv pages] pool {need}: {pages}", flush=True)
        assert eng.tokens() == want
        assert pages["used"] <= need and not pages["spent"]
        eng.rewind(0)
        assert eng.kv_pages()["used"] == B * 2
        eng.run()
        assert eng.tokens() == want


def test_short_pool_stops_sequences_and_raises(models, full_state):
    prompts = _prompts(full_state[0])
    with _engine(models) as full:
        full.prefill(prompts)
        full.run()
        want = full.tokens()
    with _engine(models, kv_pages=B * 2 + 5) as eng:
        eng.prefill(prompts)
        with pytest.raises(RuntimeError, match="KV page pool spent"):
            eng.run()
        got = eng.tokens()
        print(f"[kv pages] short pool: lengths {[len(g) for g in got]}", flush=True)
        assert all(g == w[: len(g)] for g, w in zip(got, want))
        assert min(len(g) for g in got) < NEW
        assert eng.kv_pages()["spent"]
    with _engine(models, kv_pages=B * 2 - 1) as eng:
        with pytest.raises(RuntimeError, match="KV page pool too small"):
            eng.prefill(prompts)


def test_verify_takes_its_block_page(models, full_state):
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    ctx, n = 128, 5  # the block's positions 128..132 start a third page
    blocks = np.stack([W.uniform_ids(60 + b, "kv_pages_block", n, cfg.vocab_size)
                       for b in range(B)])
    out = []
    for kv in (None, B * 3):
        with HipEngine(models[torch.bfloat16], batch=B, max_prompt=1, max_new=8,
                       temperature=0.0, stop_ids=[], draft_len=n - 1, max_ctx=512,
                       kv_pages=kv) as eng:
            eng.fill_kv(ctx, seed=3)
            eng.verify(blocks, graph=True)
            eng.verify(None, graph=True)
            out.append(eng.logits(B * n))
            pages = eng.kv_pages()
            assert pages["used"] == B * 3 and not pages["spent"], pages
    np.testing.assert_array_equal(out[0], out[1])


def test_verify_refuses_a_block_the_pool_cannot_hold(models, full_state):
    """A block whose positions need pages the pool no longer has fails before any launch
    (instead of reading and writing the spare page) and takes no page; a block on the cached
    pages runs."""
    from pulsar_engine import weights as W
    from pulsar_engine.engine import HipEngine

    cfg = full_state[0]
    ctx, n = 126, 5  # cached positions 0..125: two pages per sequence
    blocks = np.stack([W.uniform_ids(60 + b, "kv_pages_block", n, cfg.vocab_size)
                       for b in range(B)])
    with HipEngine(models[torch.bfloat16], batch=B, max_prompt=1, max_new=8, temperature=0.0,
                   stop_ids=[], draft_len=n - 1, max_ctx=512, kv_pages=B * 2 + 1) as eng:
        eng.fill_kv(ctx, seed=3)
        eng.verify(blocks[:, :2])  # positions 126, 127: the second page
        assert eng.kv_pages() == {"pool": B * 2 + 1, "used": B * 2, "spent": False}
        with pytest.raises(RuntimeError, match="KV page pool too small for the block"):
            eng.verify(blocks)  # positions 126..130: a third page for each of B sequences
        assert eng.kv_pages() == {"pool": B * 2 + 1, "used": B * 2, "spent": False}
        assert np.isfinite(eng.logits(B * 2)).all()
