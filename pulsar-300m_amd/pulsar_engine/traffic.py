"""Algorithmic HBM bytes of a decode step, per kernel class.

The figure the roofline fraction is quoted against: every weight byte a step must read once
(per-pulse projection variants once per pulse present in the step, routed experts once per
expert that received at least one row, the tied output head once when any row needs
logits), the KV entries each sequence's rows attend to (the union of their key ranges,
read once), and the activations each kernel reads and writes. Caches and re-reads are not counted; measured HBM traffic is reported beside it.
"""

from __future__ import annotations

from collections import defaultdict

from .config import PulsarConfig

CLASSES = (
    "pulse_input", "rmsnorm", "qkv_gate_gemm", "qk_post", "attention", "wo_gemm", "router",
    "shared_gate_up", "routed_gate_up", "shared_down", "routed_down", "moe_combine",
    "pulse_output", "lm_head", "sample", "controller",
)


def step_bytes(cfg: PulsarConfig, es: int, rows, expert_counts, n_lrows: int,
               fused_post: bool | None = None) -> dict:
    """rows: iterable of (seq, pulse, pos); expert_counts: [layers][E] rows per expert.

    fused_post (default: es == 2, the bf16 engine): the q/k/v post-processing runs inside
    the decode attention, which then also reads each row's raw keys and values and writes
    them to the cache (queries are finished in registers, not written back); no qk_post
    class."""
    if fused_post is None:
        fused_post = es == 2
    D, H, Hk, hd = cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    E, K, de, ds, V = cfg.n_routed_experts, cfg.top_k, cfg.d_expert, cfg.d_shared, cfg.vocab_size
    q_dim, qkv = cfg.q_dim, cfg.qkv_dim
    rows = list(rows)
    n = len(rows)
    out: dict[str, float] = defaultdict(float)
    if n == 0:
        return out
    pulses = {p for _, p, _ in rows}
    npul = len(pulses)
    r = cfg.reinject_gate_rank
    out["pulse_input"] = n * D * es * 4 + npul * (3 * r * D + 2 * D) * es
    # decode attention reads each sequence's cache once for all of its rows in the step
    # (the current token and the speculative token one position later share key blocks)
    by_seq: dict[int, list[int]] = defaultdict(list)
    for seq, _, pos in rows:
        by_seq[seq].append(pos)
    for L in range(cfg.n_core):
        local = cfg.is_local(L)
        W = cfg.sliding_window
        ctx = sum(max(ps) - (max(0, min(ps) - W + 1) if local else 0) + 1
                  for ps in by_seq.values())
        touched = int(sum(1 for c in expert_counts[L] if c > 0))
        assigned = int(sum(expert_counts[L]))
        out["rmsnorm"] += 2 * (n * D * es * 2 + npul * D * 4)
        out["qkv_gate_gemm"] += npul * (qkv + H) * D * es + n * (D + qkv + H) * es
        out["attention"] += ctx * Hk * hd * 2 * es + n * (q_dim + H + q_dim) * es
        if fused_post:
            out["attention"] += n * 4 * Hk * hd * es
        else:
            out["qk_post"] += n * (qkv * es * 2 + 2 * Hk * hd * es)
        out["wo_gemm"] += npul * D * q_dim * es + n * (q_dim + 2 * D) * es
        out["router"] += npul * E * D * 4 + n * D * es
        out["shared_gate_up"] += 2 * ds * D * es + n * (D + ds) * es
        out["routed_gate_up"] += touched * 2 * de * D * es + assigned * (D + de) * es
        out["shared_down"] += D * ds * es + n * (ds + D) * es
        out["routed_down"] += touched * D * de * es + assigned * (de + D) * es
        out["moe_combine"] += n * (K + 3) * D * es
    out["pulse_output"] = n * 3 * D * es + n_lrows * D * es
    if n_lrows:
        out["lm_head"] = V * D * es + n_lrows * (D * es + V * 4)
        out["sample"] = n_lrows * V * 4
    return out


def prefill_flops(cfg: PulsarConfig, batch: int, prompt_len: int) -> dict:
    """Algorithmic multiply-add FLOPs (2 per MAC) of one prefill of ``batch`` prompts of
    ``prompt_len`` tokens: every pulse of every layer over every token, each token at its
    top_k experts (capacity drops ignored), attention over the key range each query sees
    (local layers: the newest ``sliding_window`` positions, top-left aligned when the prompt
    is longer, as in the reference's prefill), and the output head for the last token."""
    D, H, hd = cfg.d_model, cfg.n_heads, cfg.head_dim
    E, K, de, ds = cfg.n_routed_experts, cfg.top_k, cfg.d_expert, cfg.d_shared
    P, T, W, r = cfg.default_pulses, prompt_len, cfg.sliding_window, cfg.reinject_gate_rank
    tok = batch * T
    per_layer = 2 * ((cfg.qkv_dim + H) * D + D * cfg.q_dim + E * D + 3 * ds * D
                     + K * 3 * de * D)
    keys_global = T * (T + 1) // 2
    if T > W:
        keys_local = W * (W + 1) // 2 + (T - W) * W
    else:
        keys_local = keys_global
    n_local = sum(1 for L in range(cfg.n_core) if cfg.is_local(L))
    attn_keys = n_local * keys_local + (cfg.n_core - n_local) * keys_global
    out = {
        "projections": P * cfg.n_core * tok * per_layer,
        "attention": P * batch * H * 4 * hd * attn_keys,
        "reinject": (P - 1) * tok * 2 * 3 * r * D,
        "lm_head": batch * 2 * cfg.vocab_size * D,
    }
    out["total"] = sum(out.values())
    return out


# Rows one sequence may hold in a step (a draft block plus the next round's first row), the
# positions per global page, and the ring of a sliding-window layer: the window plus one
# step's rows, rounded to whole pages (mirrors the engine's allocation in csrc/engine.hip).
MAX_BLOCK = 8
PAGE = 64


def ring_positions(cfg: PulsarConfig) -> int:
    return (cfg.sliding_window + MAX_BLOCK + PAGE - 1) // PAGE * PAGE


def kv_cache_bytes(cfg: PulsarConfig, batch: int, max_ctx: int, es: int = 2,
                   pool_pages: int = 0) -> dict:
    """Device bytes of the engine's KV cache for `batch` sequences of up to max_ctx positions:
    sliding-window layers hold a ring of ring_positions() positions per sequence, global
    layers a pool of pool_pages pages of PAGE positions (0: enough for every sequence to
    reach max_ctx) plus one spare page; K and V, kv heads x head_dim elements of es bytes
    each. The copy of the rings prefill leaves for rewind is reported apart."""
    per_pos = cfg.n_kv_heads * cfg.head_dim * 2 * es
    n_local = sum(1 for L in range(cfg.n_core) if cfg.is_local(L))
    n_global = cfg.n_core - n_local
    pages = pool_pages or batch * ((max_ctx + PAGE - 1) // PAGE)
    local = n_local * batch * ring_positions(cfg) * per_pos
    glob = n_global * (pages + 1) * PAGE * per_pos
    return {"local": local, "global": glob, "total": local + glob, "rewind_copy": local}


def reference_unified_kv_bytes(context: int) -> int:
    """The reference's analytic figure for its unified cache at batch 1 in bf16
    (src/infer.py:840-843): six sliding-window layers at min(context, 1024) positions and two
    global layers at `context`, 4 kv heads of 64, K and V, two bytes."""
    loc = min(context, 1024)
    return 6 * 2 * 4 * 64 * loc * 2 + 2 * 2 * 4 * 64 * context * 2
