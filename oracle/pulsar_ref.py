"""Oracle: CPU restatement of the reference's KV-cache self-speculative decode path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the checker
or the timed CPU baseline; the product path (``pulsar_cuda`` / ``pulsar_engine``) never
calls it.

Restates ``src/infer.py:64-731`` of the reference (PulsarInferenceEngine and
UnifiedKVCache) on PyTorch CPU tensors, reproducing the behaviours a faithful restatement
must keep (each cited where it is implemented):

* the unified cache: pulse 0 appends, pulses 1-2 overwrite the newest slot, local layers
  keep the newest ``sliding_window`` entries;
* no value residual on pulses >= 1; decode stem conv sees only the current token;
* prefill: pulse-k K/V replace the cache, no YaRN, SDPA ``is_causal`` with top-left
  alignment when a local layer's prompt exceeds the window, un-softcapped logits,
  capacity-limited MoE with lowest-weight drops;
* decode: fp32 router, dropless experts summed in top-k order, softcap every pulse;
* sampling: repetition penalty over the seen set, temperature, shifted top-p, nan_to_num,
  multinomial; acceptance = equality of two independent draws.

Tensor ops follow the reference's order so that, on the same torch build, fp32 results
match the reference bit for bit (pinned by ``tests/golden``).

Parity status of each part (what checks it):
* ``rmsnorm``/``rope``/``swiglu``/``conv_k4``/router/softcap/gate: closed forms, checked
  against textbook formulas and invariants in ``tests/test_oracle.py``.
* ``prefill``/``decode_pulse_pass``/``decode_step``/generators: golden vectors written by
  ``tests/golden/make_golden.py`` from the reference itself (tiny config, fp32 and bf16,
  greedy and seeded-sampled streams; full-size fp32 greedy stream).
* ``moe_prefill``: goldens above, plus slot-assignment invariants.
"""

from __future__ import annotations

import math
import os
import sys
from typing import Iterator, Optional

import numpy as np
import torch
import torch.nn.functional as F

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_PKG = os.path.join(_ROOT, "pulsar-300m_amd")
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

from pulsar_engine.config import PulsarConfig  # noqa: E402

# Substrings of parameters the reference keeps in fp32 when the model runs in bf16
# (src/model.py:1661-1677); every 1-D parameter stays fp32 as well (:1727-1728).
_FP32_SUBSTRINGS = (
    "norm", "bias", "router", "mix_logit", "reinject_gate", "lora_", "loop_M",
    "canon_weight", "res_scale", "routed_scale", "attn_gate", "pulse_step_emb",
    "v_resid_lambda", "q_norm_weight", "k_norm_weight",
)


def _stays_fp32(name: str, arr: np.ndarray) -> bool:
    return arr.ndim == 1 or any(s in name for s in _FP32_SUBSTRINGS) or name.endswith("expert_bias")


# ---------------------------------------------------------------------------
# Closed-form pieces
# ---------------------------------------------------------------------------

def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm fallback path, src/model.py:386-392: fp32 statistics, cast back."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (w.float() * (xf * inv)).to(x.dtype)


def inv_freq(theta: float, dim: int) -> torch.Tensor:
    """src/model.py:532, :536-543."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2).float() / dim))


def rope_tables(theta: float, dim: int, n: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables of positions 0..n-1, src/model.py:545-552."""
    t = torch.arange(n, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq(theta, dim))
    return freqs.cos(), freqs.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE with fp32 arithmetic, src/model.py:578-589 (CPU branch)."""
    half = x.shape[-1] // 2
    c = cos.unsqueeze(0).unsqueeze(0).float()
    s = sin.unsqueeze(0).unsqueeze(0).float()
    xf = x.float()
    lo, hi = xf[..., :half], xf[..., half:]
    return torch.cat([lo * c - hi * s, hi * c + lo * s], dim=-1).to(x.dtype)


def conv_k4(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Causal depthwise conv (k=4) plus residual, src/model.py:592-602."""
    xp = F.pad(x.float().transpose(1, 2), (3, 0))
    y = F.conv1d(xp, w.unsqueeze(1).flip(-1), groups=x.shape[2]).transpose(1, 2)
    return (x + y).to(x.dtype)


def swiglu(gu: torch.Tensor, d_ff: int) -> torch.Tensor:
    """silu(gate)*up in fp32, cast back, src/model.py:930-935."""
    return (F.silu(gu[..., :d_ff].float()) * gu[..., d_ff:].float()).to(gu.dtype)


def merged_weight(base: torch.Tensor, lora_A: torch.Tensor, lora_B: torch.Tensor,
                  loop_M: torch.Tensor, pulse: int, K: int, alpha: float) -> torch.Tensor:
    """W + (alpha/q) * sum_j M[pulse, j] B_j A_j, src/model.py:716-727."""
    q = lora_A.shape[1]
    d_in = lora_A.shape[2]
    d_out = lora_B.shape[1]
    A_all = lora_A[:K].to(base.dtype).reshape(K * q, d_in)
    B_perm = lora_B[:K].to(base.dtype).permute(1, 0, 2)
    coef = (loop_M[pulse, :K] * (alpha / q)).view(1, K, 1).to(base.dtype)
    return torch.addmm(base, (B_perm * coef).reshape(d_out, K * q), A_all)


def softcap(logits: torch.Tensor, cap: float) -> torch.Tensor:
    """src/infer.py:521-522."""
    return cap * torch.tanh(logits / cap)


def yarn_scale(pos: int, base: int) -> float:
    """Per-query temperature of global layers in decode, src/infer.py:288-291."""
    return 1.0 + 0.1 * math.log(max(pos + 1, base) / base)


def router_decode(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor, k: int,
                  out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 centred-sigmoid top-k router of the decode step, src/infer.py:324-333."""
    logits = F.linear(x.float(), w.float())
    logits = logits - logits.mean(dim=-1, keepdim=True)
    scores = torch.sigmoid(logits)
    _, idx = torch.topk(scores + bias.float(), k=k, dim=-1)
    raw = torch.gather(scores, -1, idx)
    return idx, (raw / (raw.sum(dim=-1, keepdim=True) + 1e-6)).to(out_dtype)


def router_prefill(logits: torch.Tensor, bias: torch.Tensor, k: int,
                   out_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """Router of PulsarMoEMLP.forward's torch branch, src/model.py:1312-1317."""
    c = logits.float() - logits.float().mean(dim=-1, keepdim=True)
    scores = torch.sigmoid(c)
    _, idx = torch.topk(scores + bias, k=k, dim=-1)
    raw = torch.gather(scores, -1, idx)
    return idx, (raw / (raw.sum(dim=-1, keepdim=True) + 1e-6)).to(out_dtype)


def moe_capacity(n_tokens: int, cfg: PulsarConfig) -> int:
    """Capacity of the prefill MoE, src/model.py:1339-1342."""
    avg = n_tokens * cfg.top_k / cfg.n_routed_experts
    raw = int(math.ceil(avg * cfg.moe_capacity_factor))
    align = max(1, int(cfg.moe_capacity_align))
    return max(align, ((raw + align - 1) // align) * align)


def token_slots(topk_idx: torch.Tensor, topk_w: torch.Tensor, n_experts: int,
                capacity: int) -> torch.Tensor:
    """Deterministic slot per (token, k); -1 when dropped. src/model.py:996-1054, :952-965.

    Assignments are ordered by (expert ascending, weight descending) through the float32
    key ``e - 0.5*w/(1+w)`` with a stable sort; the slot is the rank within the expert.
    """
    N, K = topk_idx.shape
    flat_e = topk_idx.reshape(-1).long()
    M = flat_e.numel()
    if M == 0:
        return torch.empty((N, K), dtype=torch.int32)
    w = topk_w.reshape(-1).float().clamp_min(0.0)
    key = flat_e.to(torch.float32) - (w / (1.0 + w)) * 0.5
    order = torch.argsort(key, stable=True)
    e_sorted = flat_e[order]
    counts = torch.zeros(n_experts, dtype=torch.long)
    counts.index_add_(0, e_sorted, torch.ones(M, dtype=torch.long))
    start = counts.cumsum(0) - counts
    rank = torch.arange(M) - start[e_sorted]
    slot_sorted = torch.where(rank < capacity, rank.to(torch.int32),
                              torch.full_like(rank, -1, dtype=torch.int32))
    slots = torch.empty(M, dtype=torch.int32)
    slots[order] = slot_sorted
    return slots.view(N, K)


# ---------------------------------------------------------------------------
# Model container
# ---------------------------------------------------------------------------

class RefModel:
    """Weights in the reference precision policy (src/model.py:1689-1728)."""

    def __init__(self, cfg: PulsarConfig, state: dict, dtype: torch.dtype = torch.float32,
                 rope_tables_fp32: bool = True):
        self.cfg = cfg
        self.dtype = dtype
        # With a pulsar_cuda module importable the reference hands fp32 cos/sin tables to
        # RoPE; without one it casts them to the activation dtype (src/model.py:557).
        self.rope_tables_fp32 = rope_tables_fp32
        self.p: dict[str, torch.Tensor] = {}
        for name, arr in state.items():
            t = torch.from_numpy(np.ascontiguousarray(arr)).float()
            if dtype != torch.float32:
                # The reference casts the whole model first and only then restores the
                # fp32 policy, so fp32-kept values carry the low-precision rounding too.
                t = t.to(dtype)
                if _stays_fp32(name, np.asarray(arr)):
                    t = t.float()
            self.p[name] = t
        n_tab = cfg.max_seq_len
        self._tables = {
            True: rope_tables(cfg.rope_theta_local, cfg.head_dim, n_tab),
            False: rope_tables(cfg.rope_theta_global, cfg.head_dim, n_tab),
        }

    def rope(self, local: bool, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        """First n rows of a table, grown on demand as src/model.py:554-561 does."""
        cos, sin = self._tables[local]
        if n > cos.shape[0]:
            theta = self.cfg.rope_theta_local if local else self.cfg.rope_theta_global
            cos, sin = rope_tables(theta, self.cfg.head_dim, n)
            self._tables[local] = (cos, sin)
        dt = torch.float32 if self.rope_tables_fp32 else self.dtype
        return cos[:n].to(dt), sin[:n].to(dt)

    def w(self, name: str) -> torch.Tensor:
        return self.p[name]

    def eff_weight(self, layer: int, which: str, pulse: int) -> torch.Tensor:
        """Per-pulse LoRA-merged projection (which = 'wqkv' or 'wo')."""
        cfg = self.cfg
        pre = f"core.{layer}.attn."
        base = self.p[pre + which + ".weight"]
        if cfg.loop_lora_rank <= 0:
            return base
        ad = pre + which + "_adapter."
        return merged_weight(base, self.p[ad + "lora_A"], self.p[ad + "lora_B"],
                             self.p[ad + "loop_M"], pulse, cfg.default_pulses,
                             cfg.loop_lora_alpha)


# ---------------------------------------------------------------------------
# Unified KV cache (src/infer.py:64-178)
# ---------------------------------------------------------------------------

class RefKVCache:
    def __init__(self, cfg: PulsarConfig):
        self.cfg = cfg
        self.k: list[Optional[torch.Tensor]] = [None] * cfg.n_core
        self.v: list[Optional[torch.Tensor]] = [None] * cfg.n_core
        self.seq_len = 0

    def put_prefill(self, layer: int, k: torch.Tensor, v: torch.Tensor):
        """Prefill replaces the layer's cache; local layers keep the last window (:128-137)."""
        W = self.cfg.sliding_window
        if self.cfg.is_local(layer) and k.shape[2] > W:
            k, v = k[:, :, -W:, :], v[:, :, -W:, :]
        self.k[layer], self.v[layer] = k.clone(), v.clone()
        return self.k[layer], self.v[layer]

    def put_decode(self, layer: int, k: torch.Tensor, v: torch.Tensor, pulse: int):
        """Pulse 0 appends (evicting beyond the window); later pulses overwrite (:139-157)."""
        if self.k[layer] is None:
            return self.put_prefill(layer, k, v)
        if pulse == 0:
            kk = torch.cat([self.k[layer], k], dim=2)
            vv = torch.cat([self.v[layer], v], dim=2)
            W = self.cfg.sliding_window
            if self.cfg.is_local(layer) and kk.shape[2] > W:
                kk, vv = kk[:, :, -W:, :].contiguous(), vv[:, :, -W:, :].contiguous()
            self.k[layer], self.v[layer] = kk, vv
        else:
            self.k[layer][:, :, -1:, :] = k
            self.v[layer][:, :, -1:, :] = v
        return self.k[layer], self.v[layer]

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.k + self.v if t is not None)


# ---------------------------------------------------------------------------
# Engine
# ---------------------------------------------------------------------------

class RefEngine:
    """Batch-1 decode engine with the reference's semantics (src/infer.py:181-731)."""

    def __init__(self, model: RefModel, stop_ids=None):
        self.m = model
        self.cfg = model.cfg
        self.dtype = model.dtype
        self.stop_ids = set(stop_ids) if stop_ids is not None else {self.cfg.eos_token_id}
        self.trace: Optional[list] = None  # optional per-pass record for tests
        # adaptive early exit (src/infer.py:198-200): off when the threshold is None
        self.early_exit_threshold: Optional[float] = None
        self.early_exit_counts = [0] * self.cfg.default_pulses

    def set_early_exit_threshold(self, threshold: Optional[float]) -> None:
        """src/infer.py:210-213: set the threshold and clear the per-pulse exit counts."""
        self.early_exit_threshold = threshold
        self.early_exit_counts = [0] * self.cfg.default_pulses

    # -- pulse input -------------------------------------------------------
    def _stem(self, ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """h_0 and the anchor (normed, conv'd) embedding, src/infer.py:359-365, :474-479."""
        m, cfg = self.m, self.cfg
        h0 = F.embedding(ids, m.w("tok_emb.weight"))
        e = rmsnorm(h0, m.w("anchor_norm.weight"), cfg.rms_eps)
        if cfg.use_canon_conv:
            e = conv_k4(e, m.w("stem_canon_weight"))
        return h0, e

    def _pulse_input(self, pulse: int, e: torch.Tensor, h_prev: Optional[torch.Tensor]):
        """h_in of a pulse, src/infer.py:369-387 and :480-501."""
        m, cfg = self.m, self.cfg
        step = m.w("pulse_step_emb.weight")[pulse].to(e.dtype).view(1, 1, -1)
        if pulse == 0:
            return e + step
        r = rmsnorm(h_prev, m.w("pulse_state_norm.weight"), cfg.rms_eps)
        wd = m.w("reinject_gate_down")[pulse].to(e.dtype)
        D = cfg.d_model
        g = F.linear(e, wd[:, :D]) + F.linear(r, wd[:, D:])
        mix = torch.sigmoid(F.linear(g, m.w("reinject_gate_up")[pulse].to(e.dtype),
                                     m.w("reinject_gate_bias")[pulse].to(e.dtype)))
        return torch.lerp(r, e, mix) + step

    def _pulse_output(self, pulse: int, h_in: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
        """Harmonic residual, src/infer.py:455-456, :516-517."""
        return h_in + (h - h_in) * self.m.w("pulse_res_scale")[pulse].to(h_in.dtype)

    # -- attention pieces --------------------------------------------------
    def _qkv(self, layer: int, x: torch.Tensor, pulse: int, v_first):
        """Merged projection, split, value residual and QK-RMSNorm (src/infer.py:249-276)."""
        m, cfg = self.m, self.cfg
        B, T, _ = x.shape
        qkv = F.linear(x, m.eff_weight(layer, "wqkv", pulse))
        q, k, v = qkv.split([cfg.q_dim, cfg.kv_dim, cfg.kv_dim], dim=-1)
        q = q.view(B, T, cfg.n_heads, cfg.head_dim).transpose(1, 2)
        k = k.view(B, T, cfg.n_kv_heads, cfg.head_dim).transpose(1, 2)
        v = v.view(B, T, cfg.n_kv_heads, cfg.head_dim).transpose(1, 2)
        pre = f"core.{layer}.attn."
        if layer == 0 and pulse == 0:
            v_first = v
        elif v_first is not None:
            lv = torch.sigmoid(m.w(pre + "v_resid_lambda")[pulse]).to(v.dtype)
            v = (1.0 - lv) * v + lv * v_first
        qn = m.w(pre + "q_norm_weight")[pulse].view(1, cfg.n_heads, 1, cfg.head_dim)
        kn = m.w(pre + "k_norm_weight")[pulse].view(1, cfg.n_kv_heads, 1, cfg.head_dim)
        q = (qn.float() * (q.float() * torch.rsqrt(q.float().pow(2).mean(-1, keepdim=True)
                                                   + cfg.rms_eps))).to(q.dtype)
        k = (kn.float() * (k.float() * torch.rsqrt(k.float().pow(2).mean(-1, keepdim=True)
                                                   + cfg.rms_eps))).to(k.dtype)
        return q, k, v, v_first

    def _gate_and_out(self, layer: int, x: torch.Tensor, attn: torch.Tensor, pulse: int):
        """Per-head sigmoid gate, head merge and merged wo (src/infer.py:301-313)."""
        m = self.m
        B, T, _ = x.shape
        pre = f"core.{layer}.attn."
        g = torch.sigmoid(F.linear(x, m.w(pre + "attn_gate")[pulse].to(x.dtype),
                                   m.w(pre + "attn_gate_bias")[pulse].to(x.dtype)))
        out = attn * g.transpose(1, 2).unsqueeze(-1)
        out = out.transpose(1, 2).contiguous().view(B, T, -1)
        return F.linear(out, m.eff_weight(layer, "wo", pulse))

    # -- MoE -----------------------------------------------------------------
    def _shared_expert(self, layer: int, x: torch.Tensor) -> torch.Tensor:
        m, cfg = self.m, self.cfg
        pre = f"core.{layer}.mlp.shared_expert."
        gu = F.linear(x, m.w(pre + "w_gate_up.weight"))
        return F.linear(swiglu(gu, cfg.d_shared), m.w(pre + "w_down.weight"))

    def _bias(self, layer: int, pulse: int) -> torch.Tensor:
        b = self.m.w(f"core.{layer}.mlp.expert_bias")
        return (b[pulse] if self.cfg.per_pulse_bias else b).float()

    def moe_decode(self, layer: int, x: torch.Tensor, pulse: int) -> torch.Tensor:
        """Dropless single-token MoE, src/infer.py:316-351."""
        m, cfg = self.m, self.cfg
        B, T, D = x.shape
        xf = x.view(-1, D)
        pre = f"core.{layer}.mlp."
        idx, wts = router_decode(xf, m.w(pre + "router_weight")[pulse], self._bias(layer, pulse),
                                 cfg.top_k, x.dtype)
        if self.trace is not None:
            # the biased scores ranked by top-k, for the size of each decision's margin
            biased = torch.sigmoid((lambda lg: lg - lg.mean(dim=-1, keepdim=True))(
                F.linear(xf.float(), m.w(pre + "router_weight")[pulse].float())))
            biased = biased + self._bias(layer, pulse)
            self.trace.append(("router", layer, pulse, idx.clone(), biased.clone()))
        shared = self._shared_expert(layer, xf)
        routed = torch.zeros_like(xf)
        for i in range(cfg.top_k):
            e = int(idx[0, i])
            gu = F.linear(xf, m.w(pre + "routed_gate_up")[e].t().to(x.dtype))
            act = swiglu(gu, cfg.d_expert)
            out_e = F.linear(act, m.w(pre + "routed_down")[e].t().to(act.dtype))
            routed = routed + out_e * wts[0, i]
        rs = m.w(pre + "routed_scale")[pulse].to(x.dtype)
        return (shared + routed * rs).view(B, T, D)

    def moe_prefill(self, layer: int, x: torch.Tensor, pulse: int) -> torch.Tensor:
        """Capacity-limited MoE of PulsarMoEMLP.forward's torch branch, src/model.py:1265-1483."""
        m, cfg = self.m, self.cfg
        B, T, D = x.shape
        N = B * T
        xf = x.view(N, D)
        pre = f"core.{layer}.mlp."
        logits = F.linear(xf, m.w(pre + "router_weight")[pulse].to(xf.dtype))
        idx, wts = router_prefill(logits, self._bias(layer, pulse), cfg.top_k, x.dtype)
        shared = self._shared_expert(layer, xf)
        E, C, K = cfg.n_routed_experts, moe_capacity(N, cfg), cfg.top_k
        slots = token_slots(idx, wts, E, C)
        if self.trace is not None:
            self.trace.append(("prefill_router", layer, pulse, idx.clone(), slots.clone()))
        tok = torch.arange(N).unsqueeze(1).expand(N, K).reshape(-1)
        fe = idx.reshape(-1)
        fw = wts.reshape(-1).to(x.dtype)
        fs = slots.reshape(-1)
        valid = (fs >= 0) & (fe >= 0) & (fe < E)
        dest = fe * C + fs.clamp(min=0).long()
        buf = torch.zeros(E * C, D, dtype=x.dtype)
        buf.index_add_(0, dest, xf[tok] * valid.unsqueeze(-1).to(x.dtype))
        gu_w = m.w(pre + "routed_gate_up")
        gu = torch.bmm(buf.view(E, C, D).to(gu_w.dtype), gu_w)
        act = swiglu(gu, cfg.d_expert)
        rs = m.w(pre + "routed_scale")[pulse].to(x.dtype)
        eo = torch.bmm(act, m.w(pre + "routed_down").to(act.dtype) * rs.view(1, 1, D))
        contrib = ((fw * valid.to(fw.dtype)).unsqueeze(-1) * eo.view(E * C, D)[dest]).to(x.dtype)
        routed = torch.zeros(N, D, dtype=x.dtype)
        routed.index_add_(0, tok, contrib)
        return (shared + routed).view(B, T, D)

    # -- passes ----------------------------------------------------------------
    def prefill(self, ids: torch.Tensor, cache: RefKVCache) -> torch.Tensor:
        """Parallel prompt ingestion; returns raw last-row logits [1,1,V] (src/infer.py:353-461)."""
        m, cfg = self.m, self.cfg
        B, T = ids.shape
        h0, e = self._stem(ids)
        h_pulse = h0
        for k in range(cfg.default_pulses):
            h_in = self._pulse_input(k, e, h_pulse)
            h = h_in
            v_first = None
            for L in range(cfg.n_core):
                x = rmsnorm(h, m.w(f"core.{L}.attn_norm.weight")[k], cfg.rms_eps)
                q, kk, v, v_first = self._qkv(L, x, k, v_first)
                cos, sin = m.rope(cfg.is_local(L), T)
                q = apply_rope(q, cos, sin)
                kk = apply_rope(kk, cos, sin)
                kc, vc = cache.put_prefill(L, kk, v)
                a = F.scaled_dot_product_attention(q, kc, vc, is_causal=True,
                                                   enable_gqa=cfg.n_heads > cfg.n_kv_heads)
                h = h + self._gate_and_out(L, x, a, k)
                y = rmsnorm(h, m.w(f"core.{L}.mlp_norm.weight")[k], cfg.rms_eps)
                h = h + self.moe_prefill(L, y, k)
            h_pulse = self._pulse_output(k, h_in, h)
            if self.trace is not None:
                self.trace.append(("prefill_pulse", k, h_pulse.clone()))
        cache.seq_len = T
        hf = rmsnorm(h_pulse[:, -1:, :], m.w("final_norm.weight"), cfg.rms_eps)
        return F.linear(hf, m.w("tok_emb.weight"))

    def decode_pulse_pass(self, token: int, pos: int, cache: RefKVCache, pulse: int,
                          h_prev=None, e_cached=None):
        """One pulse of one token through all layers (src/infer.py:463-524)."""
        m, cfg = self.m, self.cfg
        if pulse == 0:
            _, e = self._stem(torch.tensor([[token]], dtype=torch.long))
        else:
            e = e_cached
        h_in = self._pulse_input(pulse, e, h_prev)
        h = h_in
        v_first = None
        for L in range(cfg.n_core):
            x = rmsnorm(h, m.w(f"core.{L}.attn_norm.weight")[pulse], cfg.rms_eps)
            q, kk, v, v_first = self._qkv(L, x, pulse, v_first)
            local = cfg.is_local(L)
            cos, sin = m.rope(local, pos + 1)
            cos, sin = cos[-1:], sin[-1:]
            q = apply_rope(q, cos, sin)
            kk = apply_rope(kk, cos, sin)
            if not local and pos + 1 > cfg.base_seq_len:
                q = q * yarn_scale(pos, cfg.base_seq_len)
            kc, vc = cache.put_decode(L, kk, v, pulse)
            a = F.scaled_dot_product_attention(q, kc, vc, is_causal=False,
                                               enable_gqa=cfg.n_heads > cfg.n_kv_heads)
            h = h + self._gate_and_out(L, x, a, pulse)
            y = rmsnorm(h, m.w(f"core.{L}.mlp_norm.weight")[pulse], cfg.rms_eps)
            h = h + self.moe_decode(L, y, pulse)
        h_out = self._pulse_output(pulse, h_in, h)
        hf = rmsnorm(h_out, m.w("final_norm.weight"), cfg.rms_eps)
        logits = F.linear(hf, m.w("tok_emb.weight"))[:, -1, :]
        if cfg.logit_softcap > 0:
            logits = softcap(logits, cfg.logit_softcap)
        if self.trace is not None:
            self.trace.append(("pulse", token, pos, pulse, logits.clone()))
        return logits, h_out, e

    def decode_step(self, token: int, pos: int, cache: RefKVCache) -> torch.Tensor:
        """The pulses of one token with the optional adaptive early exit (src/infer.py:526-549).

        After pulse k < last, when a threshold is set, the top-1 probability of softmax(logits)
        (the softcapped logits in the model dtype, so rounded to bf16 in bf16 mode) is compared
        with it; at or above it the token stops at pulse k: its cache entry keeps pulse k's
        keys/values and pulse k's logits are returned. Exits are counted per pulse; a token that
        runs every pulse counts at the last one."""
        h, e, logits = None, None, None
        P = self.cfg.default_pulses
        thr = self.early_exit_threshold
        for k in range(P):
            logits, h, e = self.decode_pulse_pass(token, pos, cache, k, h, e)
            if thr is not None and k < P - 1:
                max_prob = F.softmax(logits, dim=-1).max(dim=-1).values.item()
                if self.trace is not None:
                    self.trace.append(("exit_check", token, pos, k, max_prob))
                if max_prob >= thr:
                    self.early_exit_counts[k] += 1
                    break
        else:
            if thr is not None:
                self.early_exit_counts[P - 1] += 1
        cache.seq_len = pos + 1
        return logits

    def get_early_exit_stats(self) -> dict:
        """Exit distribution over the counted tokens (src/infer.py:215-232); the reference
        weighs pulses 1-3 as 8, 16 and 24 layers."""
        c = self.early_exit_counts
        total = sum(c)
        if total == 0:
            return {}
        eff = (8 * c[0] + 16 * c[1] + 24 * c[2]) / total
        return {"total_tokens": total, "pulse_counts": list(c),
                "pulse_pcts": [c[0] / total * 100.0, c[1] / total * 100.0, c[2] / total * 100.0],
                "effective_layers": eff, "compute_speedup": 24.0 / eff}

    # -- sampling (src/infer.py:658-685) ----------------------------------------
    @staticmethod
    def sample(lgt: torch.Tensor, seen: list, temperature: float, top_p: float,
               repetition_penalty: float, generator=None) -> int:
        l = lgt.clone()
        if repetition_penalty != 1.0:
            for tid in set(seen):
                val = l[0, tid]
                if val > 0:
                    l[0, tid] = val / repetition_penalty
                else:
                    l[0, tid] = val * repetition_penalty
        if temperature <= 1e-4:
            return int(l.argmax(dim=-1).item())
        scaled = l / max(temperature, 1e-5)
        if top_p < 1.0:
            sl, si = torch.sort(scaled, descending=True)
            cum = torch.cumsum(F.softmax(sl, dim=-1), dim=-1)
            drop = cum > top_p
            drop[..., 1:] = drop[..., :-1].clone()
            drop[..., 0] = 0
            scaled[0, si[drop]] = float("-inf")
        probs = F.softmax(scaled, dim=-1).nan_to_num(0.0)
        if probs.sum() <= 0:
            return int(l.argmax(dim=-1).item())
        probs = probs / probs.sum()
        return int(torch.multinomial(probs, num_samples=1, generator=generator).item())

    # -- generators (id level) ---------------------------------------------------
    def stream_generate_ids(self, prompt_ids, max_new_tokens: int, temperature: float,
                            top_p: float, repetition_penalty: float,
                            generator=None) -> Iterator[int]:
        """Plain decode, src/infer.py:551-621."""
        ids = torch.as_tensor(prompt_ids, dtype=torch.long).view(1, -1)
        cache = RefKVCache(self.cfg)
        logits = self.prefill(ids, cache)[:, -1, :].clone()
        seen = ids[0].tolist()
        pos = len(seen) - 1
        for _ in range(max_new_tokens):
            tok = self.sample(logits, seen, temperature, top_p, repetition_penalty, generator)
            if tok in self.stop_ids:
                break
            seen.append(tok)
            pos += 1
            yield tok
            logits = self.decode_step(tok, pos, cache)

    def self_speculative_ids(self, prompt_ids, max_new_tokens: int, temperature: float,
                             top_p: float, repetition_penalty: float, generator=None,
                             stats: Optional[dict] = None) -> Iterator[int]:
        """Pulse-0 draft, pulse-2 verify, accept on equal draws (src/infer.py:623-731)."""
        ids = torch.as_tensor(prompt_ids, dtype=torch.long).view(1, -1)
        cache = RefKVCache(self.cfg)
        logits = self.prefill(ids, cache)[:, -1, :].clone()
        seen = ids[0].tolist()
        pos = len(seen) - 1
        produced = 0
        if stats is not None:
            stats.setdefault("tests", 0)
            stats.setdefault("accepted", 0)
            stats.setdefault("p_accept", [])
            stats.setdefault("kinds", [])
        smp = lambda lg: self.sample(lg, seen, temperature, top_p, repetition_penalty, generator)  # noqa: E731
        while produced < max_new_tokens:
            t = smp(logits)
            if t in self.stop_ids:
                break
            seen.append(t)
            pos += 1
            produced += 1
            if stats is not None:
                stats["kinds"].append(0)
            yield t
            if produced >= max_new_tokens:
                break
            d_logits, h, e = self.decode_pulse_pass(t, pos, cache, 0)
            draft = smp(d_logits)
            _, h, _ = self.decode_pulse_pass(t, pos, cache, 1, h, e)
            v_logits, h, _ = self.decode_pulse_pass(t, pos, cache, 2, h, e)
            cache.seq_len = pos + 1
            true = smp(v_logits)
            if stats is not None:
                stats["tests"] += 1
                stats["p_accept"].append(accept_probability(
                    d_logits, v_logits, seen, temperature, top_p, repetition_penalty))
            if draft == true and draft not in self.stop_ids:
                if stats is not None:
                    stats["accepted"] += 1
                    stats["kinds"].append(1)
                seen.append(draft)
                pos += 1
                produced += 1
                yield draft
                if produced >= max_new_tokens:
                    break
                logits = self.decode_step(draft, pos, cache)
            else:
                logits = v_logits

    # -- draft-block mode (this build's multi-token draft; no reference counterpart) -----
    #
    # The reference drafts one token (src/infer.py:688-725). The draft-block mode drafts up
    # to G tokens with pulse 0 only and verifies the block [t, d1..dG] with all pulses in
    # one pass per pulse. Its attention rule is the reference prefill's (src/infer.py:
    # 353-461, src/model.py:880-901): at pulse k a block row sees the committed cache plus
    # the block's own pulse-k keys at positions <= its own. Everything else in a row is the
    # decode pass (src/infer.py:463-524): stem of one token, fp32 router, dropless MoE,
    # YaRN, softcapped logits. Block row 0 is therefore exactly the reference's decode of t,
    # and the first draft test of every round is the reference's test.

    def block_pass(self, tokens, pos0: int, cache: RefKVCache, pulse: int, h_prev=None,
                   e_cached=None):
        """One pulse of the block `tokens` at positions pos0.. over a committed cache.

        The cache is not modified. Returns (logits [n, V], h_out list, e list, kv) where
        kv[L] = (k, v) [1, Hkv, n, hd] are the block's keys/values of this pulse."""
        m, cfg = self.m, self.cfg
        n = len(tokens)
        W = cfg.sliding_window
        if pulse == 0:
            es = [self._stem(torch.tensor([[int(t)]], dtype=torch.long))[1] for t in tokens]
        else:
            es = list(e_cached)
        h_in = [self._pulse_input(pulse, es[i], h_prev[i] if pulse else None) for i in range(n)]
        h = list(h_in)
        v_first = [None] * n
        kv = []
        gqa = cfg.n_heads > cfg.n_kv_heads
        for L in range(cfg.n_core):
            local = cfg.is_local(L)
            cos, sin = m.rope(local, pos0 + n)
            qs, ks, vs, xs = [], [], [], []
            for i in range(n):
                x = rmsnorm(h[i], m.w(f"core.{L}.attn_norm.weight")[pulse], cfg.rms_eps)
                q, kk, v, v_first[i] = self._qkv(L, x, pulse, v_first[i])
                p = pos0 + i
                c, s = cos[p:p + 1], sin[p:p + 1]
                q = apply_rope(q, c, s)
                kk = apply_rope(kk, c, s)
                if not local and p + 1 > cfg.base_seq_len:
                    q = q * yarn_scale(p, cfg.base_seq_len)
                qs.append(q)
                ks.append(kk)
                vs.append(v)
                xs.append(x)
            kb, vb = torch.cat(ks, dim=2), torch.cat(vs, dim=2)
            kv.append((kb, vb))
            ck, cv = cache.k[L], cache.v[L]
            for i in range(n):
                kk, vv = kb[:, :, :i + 1], vb[:, :, :i + 1]
                if ck is not None:
                    kk, vv = torch.cat([ck, kk], dim=2), torch.cat([cv, vv], dim=2)
                if local and kk.shape[2] > W:
                    kk, vv = kk[:, :, -W:], vv[:, :, -W:]
                a = F.scaled_dot_product_attention(qs[i], kk.contiguous(), vv.contiguous(),
                                                   is_causal=False, enable_gqa=gqa)
                h[i] = h[i] + self._gate_and_out(L, xs[i], a, pulse)
                y = rmsnorm(h[i], m.w(f"core.{L}.mlp_norm.weight")[pulse], cfg.rms_eps)
                h[i] = h[i] + self.moe_decode(L, y, pulse)
        h_out = [self._pulse_output(pulse, h_in[i], h[i]) for i in range(n)]
        rows = []
        for i in range(n):
            hf = rmsnorm(h_out[i], m.w("final_norm.weight"), cfg.rms_eps)
            lg = F.linear(hf, m.w("tok_emb.weight"))[:, -1, :]
            if cfg.logit_softcap > 0:
                lg = softcap(lg, cfg.logit_softcap)
            rows.append(lg)
        logits = torch.cat(rows, dim=0)
        if self.trace is not None:
            self.trace.append(("block", tuple(int(t) for t in tokens), pos0, pulse,
                               logits.clone()))
        return logits, h_out, es, kv

    def commit_block(self, cache: RefKVCache, kv, n_keep: int) -> None:
        """Append the first n_keep block rows' keys/values (the last pulse's) to the cache;
        local layers keep the newest `sliding_window` entries (src/infer.py:139-150)."""
        W = self.cfg.sliding_window
        for L, (kb, vb) in enumerate(kv):
            k, v = kb[:, :, :n_keep], vb[:, :, :n_keep]
            if cache.k[L] is not None:
                k, v = torch.cat([cache.k[L], k], dim=2), torch.cat([cache.v[L], v], dim=2)
            if self.cfg.is_local(L) and k.shape[2] > W:
                k, v = k[:, :, -W:], v[:, :, -W:]
            cache.k[L], cache.v[L] = k.contiguous(), v.contiguous()

    def block_verify(self, tokens, pos0: int, cache: RefKVCache):
        """All pulses of a block; returns (last-pulse logits [n, V], per-pulse logits, kv)."""
        h = e = None
        per_pulse = []
        kv = None
        for k in range(self.cfg.default_pulses):
            lg, h, e, kv = self.block_pass(tokens, pos0, cache, k, h, e)
            per_pulse.append(lg)
        return per_pulse[-1], per_pulse, kv

    def block_speculative_ids(self, prompt_ids, max_new_tokens: int, temperature: float,
                              top_p: float, repetition_penalty: float, draft_len: int,
                              generator=None, stats: Optional[dict] = None) -> Iterator[int]:
        """Draft up to `draft_len` tokens with pulse 0, verify the block with all pulses,
        accept drafts while each equals an independent draw from the verify logits of the
        row before it (the reference's rule, src/infer.py:704-725, applied down the block).

        A round starts from an emitted token t at position pos. Draft j (j < G, G =
        min(draft_len, tokens still wanted - 1)) is a draw from the pulse-0 logits of block
        row j; a stop id ends the block. Verify row i gives draw v_i (and a second draw
        f_i); the draft of row i+1 is accepted iff it equals v_i and is not a stop id. At
        the first rejection (row i) the next t is f_i; when no draft is left it is the
        draw from the last row. Accepted rows' last-pulse keys/values are committed; the
        rejected rows' are discarded. Row i samples with the seen set plus block tokens
        1..i. With draft_len = 0 every round is one decode step of t, so the stream is
        stream_generate_ids's, draw for draw."""
        cfg = self.cfg
        ids = torch.as_tensor(prompt_ids, dtype=torch.long).view(1, -1)
        cache = RefKVCache(cfg)
        logits = self.prefill(ids, cache)[:, -1, :].clone()
        seen = ids[0].tolist()
        pos = len(seen)
        produced = 0
        if stats is not None:
            stats.setdefault("tests", 0)
            stats.setdefault("accepted", 0)
            stats.setdefault("rounds", 0)
            stats.setdefault("p_accept", [])
            stats.setdefault("kinds", [])  # per emitted token: 1 accepted draft, 0 drawn
        stops = self.stop_ids

        def kind(k):
            if stats is not None:
                stats["kinds"].append(k)

        def smp(lg, extra):
            return self.sample(lg, seen + list(extra), temperature, top_p, repetition_penalty,
                               generator)

        if max_new_tokens <= 0:
            return
        t = smp(logits, [])
        if t in stops:
            return
        seen.append(t)
        produced += 1
        kind(0)
        yield t
        while produced < max_new_tokens:
            g = min(draft_len, max_new_tokens - produced - 1)
            blk = [t]
            draft_lg = []
            for j in range(g):
                lg0, _, _, _ = self.block_pass(blk, pos, cache, 0)
                draft_lg.append(lg0[j:j + 1].clone())
                d = smp(lg0[j:j + 1], blk[1:j + 1])
                if d in stops:
                    break
                blk.append(d)
            lg, _, kv = self.block_verify(blk, pos, cache)
            if stats is not None:
                stats["rounds"] += 1
            n = len(blk)
            acc = 0
            nxt = None
            done = False
            for i in range(n):
                extra = blk[1:i + 1]
                if i < n - 1:
                    v = smp(lg[i:i + 1], extra)
                    if stats is not None:
                        stats["tests"] += 1
                        stats["p_accept"].append(accept_probability(
                            draft_lg[i], lg[i:i + 1], seen + list(extra), temperature, top_p,
                            repetition_penalty))
                    if v == blk[i + 1] and blk[i + 1] not in stops:
                        if stats is not None:
                            stats["accepted"] += 1
                        acc = i + 1
                        seen.append(blk[i + 1])
                        produced += 1
                        kind(1)
                        yield blk[i + 1]
                        if produced >= max_new_tokens:
                            done = True
                            break
                        continue
                nxt = smp(lg[i:i + 1], extra)
                break
            self.commit_block(cache, kv, acc + 1)
            pos += acc + 1
            if done or nxt in stops:
                return
            seen.append(nxt)
            produced += 1
            kind(0)
            yield nxt
            t = nxt


def replay_block_acceptance(engine: "RefEngine", prompt_ids, emitted, kinds, temperature: float,
                            top_p: float, repetition_penalty: float, draft_len: int,
                            max_new: Optional[int] = None) -> list:
    """``RefEngine.block_speculative_ids`` driven along a given emitted stream instead of its
    own draws (no stop ids): emitted[i] is the i-th output token, kinds[i] is 1 for an
    accepted draft and 0 for a drawn token. A round starts at a drawn token t; the accepted
    drafts d1..da that follow it were tested and accepted, and the round ran
    min(a + 1, G) tests (G = min(draft_len, tokens still wanted - 1)): the last one
    failed unless a == G. Test i depends on block rows 0..i only (t, d1..di, all emitted),
    so the oracle's verify over those rows gives P(accept) = sum_x p_draft(x) p_verify(x)
    from its pulse-0 (the draft's logits: the draft pass of row i sees the block's pulse-0
    keys, as the verify's pulse 0 does) and last-pulse logits. `emitted` may be the start
    of a longer generation of max_new tokens (default: its own length); a round cut off by
    its end is left out. Returns (P(accept), accepted) per test."""
    cfg = engine.cfg
    ids = torch.as_tensor(prompt_ids, dtype=torch.long).view(1, -1)
    cache = RefKVCache(cfg)
    engine.prefill(ids, cache)
    seen = ids[0].tolist()
    pos = len(seen)
    n = len(emitted)
    total = n if max_new is None else max_new
    out = []
    i = 0
    while i < n:
        if kinds[i] != 0:
            raise ValueError(f"token {i} marked as an accepted draft at the start of a round")
        t = int(emitted[i])
        seen.append(t)
        produced = i + 1
        if produced >= total:
            break
        a = 0
        while i + 1 + a < n and kinds[i + 1 + a] == 1:
            a += 1
        if i + 1 + a >= n and produced + a < total:
            break  # the round's last test lies past the given stream
        g = min(draft_len, total - produced - 1)
        if a > g:
            raise ValueError(f"round at token {i}: {a} accepted drafts, at most {g} drafted")
        blk = [t] + [int(x) for x in emitted[i + 1:i + 1 + a]]
        _, per_pulse, kv = engine.block_verify(blk, pos, cache)
        tests = min(a + 1, g)
        for j in range(tests):
            extra = blk[1:j + 1]
            out.append((accept_probability(per_pulse[0][j:j + 1], per_pulse[-1][j:j + 1],
                                           seen + extra, temperature, top_p,
                                           repetition_penalty), j < a))
        seen.extend(blk[1:])
        engine.commit_block(cache, kv, a + 1)
        pos += a + 1
        i += 1 + a
    return out


def replay_acceptance(engine: "RefEngine", prompt_ids, emitted, kinds, temperature: float,
                      top_p: float, repetition_penalty: float) -> list:
    """The reference's self-speculative loop (src/infer.py:688-731) driven along a given
    emitted stream instead of its own draws: emitted[i] is the i-th output token, kinds[i]
    is 1 when it was an accepted draft (then emitted[i-1] was tested and accepted) and 0
    when it was drawn. Returns, for each draft test, (P(accept), accepted) with
    P(accept) = sum_x p_draft(x) p_verify(x) from the oracle's own pulse-0 and pulse-2
    logits of the tested token over the oracle's own cache."""
    ids = torch.as_tensor(prompt_ids, dtype=torch.long).view(1, -1)
    cache = RefKVCache(engine.cfg)
    engine.prefill(ids, cache)
    seen = ids[0].tolist()
    pos = len(seen) - 1
    n = len(emitted)
    out = []
    i = 0
    while i < n:
        if kinds[i] != 0:
            raise ValueError(f"token {i} marked as an accepted draft without a test before it")
        t = int(emitted[i])
        seen.append(t)
        pos += 1
        if i == n - 1:
            break
        d_logits, h, e = engine.decode_pulse_pass(t, pos, cache, 0)
        _, h, _ = engine.decode_pulse_pass(t, pos, cache, 1, h, e)
        v_logits, h, _ = engine.decode_pulse_pass(t, pos, cache, 2, h, e)
        cache.seq_len = pos + 1
        acc = kinds[i + 1] == 1
        out.append((accept_probability(d_logits, v_logits, seen, temperature, top_p,
                                       repetition_penalty), bool(acc)))
        if acc:
            d = int(emitted[i + 1])
            seen.append(d)
            pos += 1
            if i + 1 < n - 1:
                engine.decode_step(d, pos, cache)
            i += 2
        else:
            i += 1
    return out


def spec_token_marginals(engine: "RefEngine", prompt_ids, temperature: float, top_p: float,
                         repetition_penalty: float, prune: float = 1e-7) -> list:
    """Exact distributions (fp64 [V] each) of the first three tokens self_speculative_ids
    emits (src/infer.py:688-731), with no stop ids and max_new_tokens >= 3.

    Token 1 is a draw from the prefill logits and is tested: its draft d ~ p_d (pulse 0)
    and check v ~ p_v (pulse 2) are independent, so token 2 = x with probability
    p_d(x) p_v(x) (accepted draft) + (1 - sum_y p_d(y) p_v(y)) p_v(x) (fresh draw from the
    verify logits). An accepted token 2 runs decode_step and token 3 is a plain draw from
    its pulse-2 logits; a drawn token 2 is tested in turn, like token 1. Branches of
    probability below `prune` are not expanded; their mass is missing from the token-3
    (and, below prune at token 1, token-2) distributions."""
    import copy

    cfg = engine.cfg
    dist = lambda lg, seen: sampling_distribution(lg, seen, temperature, top_p,  # noqa: E731
                                                  repetition_penalty)
    ids = torch.as_tensor(prompt_ids, dtype=torch.long).view(1, -1)
    cache0 = RefKVCache(cfg)
    logits0 = engine.prefill(ids, cache0)[:, -1, :].clone()
    seen0 = ids[0].tolist()
    pos0 = len(seen0) - 1
    V = cfg.vocab_size
    m1 = dist(logits0, seen0)
    m2 = torch.zeros(V, dtype=torch.float64)
    m3 = torch.zeros(V, dtype=torch.float64)

    def tested(token, pos, cache, seen):
        ld, h, e = engine.decode_pulse_pass(token, pos, cache, 0)
        _, h, _ = engine.decode_pulse_pass(token, pos, cache, 1, h, e)
        lv, h, _ = engine.decode_pulse_pass(token, pos, cache, 2, h, e)
        cache.seq_len = pos + 1
        return dist(ld, seen), dist(lv, seen)

    for t1 in torch.nonzero(m1 > prune).view(-1).tolist():
        w1 = float(m1[t1])
        c1 = copy.deepcopy(cache0)
        seen1 = seen0 + [t1]
        pd, pv = tested(t1, pos0 + 1, c1, seen1)
        acc = pd * pv
        rej = (1.0 - float(acc.sum())) * pv
        m2 += w1 * (acc + rej)
        for t2 in torch.nonzero(w1 * (acc + rej) > prune).view(-1).tolist():
            c2 = copy.deepcopy(c1)
            seen2 = seen1 + [t2]
            pd2, pv2 = tested(t2, pos0 + 2, c2, seen2)
            # accepted token 2: decode_step's logits are its pulse-2 logits (no early exit)
            m3 += w1 * float(acc[t2]) * pv2
            acc2 = pd2 * pv2
            m3 += w1 * float(rej[t2]) * (acc2 + (1.0 - float(acc2.sum())) * pv2)
    return [m1, m2, m3]


def block_token_marginals(engine: "RefEngine", prompt_ids, temperature: float, top_p: float,
                          repetition_penalty: float, draft_len: int, n_tokens: int,
                          prune: float = 1e-6, stats: Optional[dict] = None,
                          first: Optional[list] = None, depth: Optional[int] = None) -> list:
    """Exact distributions (fp64 [V] each) of the first `depth` (default: all `n_tokens`)
    tokens that ``RefEngine.block_speculative_ids`` emits with max_new_tokens = n_tokens and
    no stop ids.

    The drafts after a round's first rejection never reach the output: the next round
    starts from the fresh draw f_i of the rejecting row i and keeps block rows 0..i, whose
    keys, values and logits depend on rows 0..i only (a row attends block rows at positions
    <= its own). So the emitted stream is the sequential process: at block row i (prefix
    blk[0..i] over the committed cache) with a draft still to test (i < g), the next token
    is x as the accepted draft with probability p_d(x) p_v(x) (draft draw x from the row's
    pulse-0 logits, verify draw v from its last-pulse logits, independent), and the round
    continues at row i + 1; otherwise (probability 1 - sum_y p_d(y) p_v(y)) it is a fresh
    draw y ~ p_v and a round starts at y one position after row i. At i == g (no draft
    left) the next token is y ~ p_v. p_d and p_v of row i come from ``block_verify`` of the
    prefix (its pulse 0 is the draft pass of that row: both attend the block's pulse-0 keys
    at positions <= the row's). Paths of probability below `prune` are not expanded; their
    mass is missing from the later distributions. `stats` (optional) receives the number of
    verified prefixes ("nodes"), the acceptance probability of every expanded test
    ("p_accept", with its path weight in "w_accept") and, per emitted token, the probability
    that it is an accepted draft ("accepted_mass", a list of `depth` floats). `first`
    (optional) expands only the paths whose first token is in it (the first distribution is
    still the whole one), so disjoint `first` sets split the enumeration into parts whose
    later distributions add up."""
    cfg = engine.cfg
    ids = torch.as_tensor(prompt_ids, dtype=torch.long).view(1, -1)
    cache0 = RefKVCache(cfg)
    logits0 = engine.prefill(ids, cache0)[:, -1, :].clone()
    seen0 = ids[0].tolist()
    V = cfg.vocab_size
    depth = n_tokens if depth is None else min(depth, n_tokens)
    marg = [torch.zeros(V, dtype=torch.float64) for _ in range(depth)]
    if depth <= 0:
        return marg
    if stats is not None:
        stats.setdefault("nodes", 0)
        stats.setdefault("p_accept", [])
        stats.setdefault("w_accept", [])
        stats["accepted_mass"] = [0.0] * depth
    dist = lambda lg, seen: sampling_distribution(lg, seen, temperature, top_p,  # noqa: E731
                                                  repetition_penalty)

    def commit(cache, kv, n_keep):
        import copy

        c = copy.deepcopy(cache)
        engine.commit_block(c, kv, n_keep)
        return c

    m1 = dist(logits0, seen0)
    marg[0] += m1
    # stack entries: (path weight, committed cache, seen through block row 0, position of
    # block row 0, block prefix, tokens produced, drafts of this round)
    stack = []
    if depth > 1:
        g1 = min(draft_len, n_tokens - 2)
        for t in torch.nonzero(m1 > prune).view(-1).tolist():
            if first is not None and t not in first:
                continue
            stack.append((float(m1[t]), cache0, seen0 + [t], len(seen0), [t], 1, g1))
    while stack:
        w, cache, seen, pos, blk, produced, g = stack.pop()
        i = len(blk) - 1
        _, per_pulse, kv = engine.block_verify(blk, pos, cache)
        if stats is not None:
            stats["nodes"] += 1
        s_row = seen + blk[1:]
        pv = dist(per_pulse[-1][i:i + 1], s_row)
        k = produced  # index of the next emitted token
        if i < g:
            pd = dist(per_pulse[0][i:i + 1], s_row)
            acc = pd * pv
            p_acc = float(acc.sum())
            if stats is not None:
                stats["p_accept"].append(p_acc)
                stats["w_accept"].append(w)
                stats["accepted_mass"][k] += w * p_acc
            marg[k] += w * acc
            if k + 1 < depth:
                for x in torch.nonzero(w * acc > prune).view(-1).tolist():
                    stack.append((w * float(acc[x]), cache, seen, pos, blk + [x], produced + 1, g))
            nxt = (1.0 - p_acc) * pv
        else:
            nxt = pv
        marg[k] += w * nxt
        if k + 1 < depth:
            live = torch.nonzero(w * nxt > prune).view(-1).tolist()
            if live:
                c = commit(cache, kv, i + 1)
                g2 = min(draft_len, n_tokens - (produced + 1) - 1)
                for y in live:
                    stack.append((w * float(nxt[y]), c, s_row + [y], pos + i + 1, [y],
                                  produced + 1, g2))
    return marg


def sampling_distribution(lgt: torch.Tensor, seen: list, temperature: float, top_p: float,
                          repetition_penalty: float) -> torch.Tensor:
    """The distribution ``RefEngine.sample`` draws from, as an fp64 vector of length V."""
    l = lgt.clone().double()
    if repetition_penalty != 1.0:
        for tid in set(seen):
            val = l[0, tid]
            l[0, tid] = val / repetition_penalty if val > 0 else val * repetition_penalty
    if temperature <= 1e-4:
        p = torch.zeros_like(l[0])
        p[int(l.argmax(dim=-1))] = 1.0
        return p
    scaled = l / max(temperature, 1e-5)
    if top_p < 1.0:
        sl, si = torch.sort(scaled, descending=True)
        cum = torch.cumsum(F.softmax(sl, dim=-1), dim=-1)
        drop = cum > top_p
        drop[..., 1:] = drop[..., :-1].clone()
        drop[..., 0] = False
        scaled[0, si[drop]] = float("-inf")
    return F.softmax(scaled, dim=-1)[0]


def accept_probability(d_logits, v_logits, seen, temperature, top_p, repetition_penalty) -> float:
    """P(draft draw == verify draw) = sum_x p_d(x) p_v(x) for two independent draws."""
    pd = sampling_distribution(d_logits, seen, temperature, top_p, repetition_penalty)
    pv = sampling_distribution(v_logits, seen, temperature, top_p, repetition_penalty)
    return float((pd * pv).sum())


def load_ref(cfg: PulsarConfig, state: dict, dtype=torch.float32, rope_tables_fp32=True,
             stop_ids=None) -> RefEngine:
    return RefEngine(RefModel(cfg, state, dtype, rope_tables_fp32), stop_ids=stop_ids)


# ---------------------------------------------------------------------------
# Synthetic caches of the HIP engine's pulsar_engine_fill_kv, restated on the CPU so that a
# verify over a long pre-filled cache can be compared with block_verify on the same keys
# and values. (This follows the engine's test generator, not the reference.)
# ---------------------------------------------------------------------------

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix64(z: np.ndarray) -> np.ndarray:
    """SplitMix64 finaliser on uint64 arrays (wrapping arithmetic)."""
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def _fill_values(seed: int, layer: int, kv: int, idx: np.ndarray) -> np.ndarray:
    """Element values of the engine's fill kernel for flat indices idx of one layer's K
    (kv = 0) or V (kv = 1) buffer: Box-Muller in fp32 of a counter-based uniform pair."""
    sd = _mix64(np.array([np.uint64(seed) ^ np.uint64(2 * layer + kv + 1)], dtype=np.uint64))[0]
    with np.errstate(over="ignore"):
        h = _mix64(sd + np.uint64(0x9E3779B97F4A7C15) * (idx.astype(np.uint64) + np.uint64(1)))
    u1 = ((h >> np.uint64(40)) + np.uint64(1)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    u2 = ((h >> np.uint64(16)) & np.uint64(0xFFFFFF)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    return (np.sqrt(np.float32(-2.0) * np.log(u1)) *
            np.cos(np.float32(6.28318530718) * u2)).astype(np.float32)


def fill_kv_cache(cfg: PulsarConfig, layout: dict, ctx: int, seed: int, b: int, batch: int,
                  dtype=torch.bfloat16) -> RefKVCache:
    """RefKVCache of sequence b holding positions [0, ctx) of an engine cache filled by
    pulsar_engine_fill_kv(ctx, seed): sliding-window layers keep the last window positions
    (ring slot = position mod lcap), global layers every position. Each element's value is
    keyed by its index in a per-sequence layout (rings: the ring buffer; global layers:
    page b * max_pages + position / page, whichever pool page the engine stores it in); K is
    position-major, V dimension-major."""
    Hkv, hd, lcap, mp, pg = layout["hkv"], cfg.head_dim, layout["lcap"], layout["max_pages"], layout["page"]
    cache = RefKVCache(cfg)
    g = np.arange(Hkv, dtype=np.int64)[:, None, None]
    d = np.arange(hd, dtype=np.int64)[None, None, :]
    for L in range(cfg.n_core):
        if cfg.is_local(L):
            pos = np.arange(max(0, ctx - cfg.sliding_window), ctx, dtype=np.int64)[None, :, None]
            slot = pos % lcap
            ik = ((b * Hkv + g) * lcap + slot) * hd + d
            iv = ((b * Hkv + g) * hd + d) * lcap + slot
        else:
            pos = np.arange(ctx, dtype=np.int64)[None, :, None]
            page = b * mp + pos // pg
            ik = ((page * Hkv + g) * pg + pos % pg) * hd + d
            iv = ((page * Hkv + g) * hd + d) * pg + pos % pg
        k = torch.from_numpy(_fill_values(seed, L, 0, ik)).to(dtype)
        v = torch.from_numpy(_fill_values(seed, L, 1, iv)).to(dtype)
        cache.k[L], cache.v[L] = k.unsqueeze(0).contiguous(), v.unsqueeze(0).contiguous()
    cache.seq_len = ctx
    return cache
