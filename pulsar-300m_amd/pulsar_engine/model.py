"""Kernel-format weights on the GPU.

Converts a reference-format state dict (names of ``PulsarForCausalLM``; see
``weights.param_shapes``) into the layout the HIP engine reads, applying the reference's
inference-time transformations once at load instead of on every pulse:

* precision policy of ``to_training_precision`` (src/model.py:1689-1728): every parameter is
  cast to the activation dtype, then the fp32-kept ones (norms, router, gates, LoRA, scales,
  ...) are restored to fp32 — so in bf16 they carry bf16-rounded values, as in the reference;
* per-pulse LoRA merge ``W + (alpha/q) sum_j M[k,j] B_j A_j`` computed with the reference's
  own op sequence (src/model.py:716-727), in the activation dtype, on the CPU;
* ``.to(x.dtype)`` casts the decode step applies to gates, re-injection, step embedding and
  scales (src/infer.py:302-303, :480-499, :516, :350);
* routed experts transposed from [E, in, out] to [E, out, in] so every projection streams
  k-contiguous rows; attention-gate rows appended to the merged qkv weight;
* fp32 RoPE tables built with the reference formula (src/model.py:545-552).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from .config import PulsarConfig

# Parameters kept in fp32 under the reference precision policy (src/model.py:1661-1677).
_FP32_SUBSTRINGS = (
    "norm", "bias", "router", "mix_logit", "reinject_gate", "lora_", "loop_M", "canon_weight",
    "res_scale", "routed_scale", "attn_gate", "pulse_step_emb", "v_resid_lambda",
    "q_norm_weight", "k_norm_weight",
)


def _policy(name: str, t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    t = t.float()
    if dtype == torch.float32:
        return t
    t = t.to(dtype)
    if t.dim() == 1 or any(s in name for s in _FP32_SUBSTRINGS):
        t = t.float()
    return t


def pack_mfma(w: torch.Tensor) -> torch.Tensor:
    """[..., N, K] -> [..., N/16, K/32, 64, 8]: 16x32 tiles in the lane order of the
    16x16x32 bf16 MFMA B operand (lane l: row l % 16, columns 8 * (l // 16) .. +8)."""
    *lead, n, k = w.shape
    if n % 16 or k % 32:
        raise ValueError(f"GEMM weight {tuple(w.shape)}: N must be a multiple of 16, K of 32")
    nl = len(lead)
    t = w.reshape(*lead, n // 16, 16, k // 32, 4, 8)
    return t.permute(*range(nl), nl, nl + 2, nl + 3, nl + 1, nl + 4).contiguous()


def rope_tables(theta: float, dim: int, n: int):
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2).float() / dim))
    t = torch.arange(n, dtype=torch.float32)
    f = torch.outer(t, inv)
    return f.cos().contiguous(), f.sin().contiguous()


def _merge(base, A, B, M, pulse, K, alpha):
    q = A.shape[1]
    A_all = A[:K].to(base.dtype).reshape(K * q, A.shape[2])
    B_perm = B[:K].to(base.dtype).permute(1, 0, 2)
    coef = (M[pulse, :K] * (alpha / q)).view(1, K, 1).to(base.dtype)
    return torch.addmm(base, (B_perm * coef).reshape(B.shape[1], K * q), A_all)


class DeviceModel:
    """Weights of one model in kernel format on a GPU, plus the C descriptor."""

    def __init__(self, cfg: PulsarConfig, state: dict, dtype: torch.dtype = torch.bfloat16,
                 device: str | torch.device = "cuda", rope_len: int | None = None):
        from pulsar_cuda import _lib

        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("dtype must be torch.float32 or torch.bfloat16")
        if cfg.head_dim != 64 or cfg.n_heads != 4 * cfg.n_kv_heads:
            raise ValueError("the HIP engine implements head_dim 64 with 4 query heads per kv head")
        self.cfg = cfg
        self.dtype = dtype
        self.device = torch.device(device)
        P = cfg.default_pulses
        self.n_pulses = P
        self._keep: list[torch.Tensor] = []
        p = {k: _policy(k, torch.as_tensor(np.asarray(v)), dtype) for k, v in state.items()}
        T = dtype

        def dev(t: torch.Tensor, dt=None) -> torch.Tensor:
            t = t.to(dt) if dt is not None else t
            t = t.contiguous().to(self.device)
            self._keep.append(t)
            return t

        d = _lib.PulsarModelDesc()
        d.vocab, d.d_model = cfg.vocab_size, cfg.d_model
        d.n_heads, d.n_kv_heads, d.head_dim = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        d.d_expert, d.d_shared, d.n_layers = cfg.d_expert, cfg.d_shared, cfg.n_core
        d.n_pulses, d.n_experts, d.top_k = P, cfg.n_routed_experts, cfg.top_k
        d.window, d.base_seq_len = cfg.sliding_window, cfg.base_seq_len
        d.reinject_rank = cfg.reinject_gate_rank
        d.dtype = _lib.PULSAR_BF16 if dtype == torch.bfloat16 else _lib.PULSAR_F32
        d.local_mask = sum(1 << i for i in range(cfg.n_core) if cfg.is_local(i))
        d.rms_eps, d.softcap = cfg.rms_eps, cfg.logit_softcap
        self.rope_len = int(rope_len or cfg.max_seq_len)
        d.rope_len = self.rope_len

        ptr = lambda t: t.data_ptr()  # noqa: E731
        # GEMM weights: matrix-core tile layout for bf16, row-major for fp32
        gw = (lambda t: pack_mfma(t)) if dtype == torch.bfloat16 else (lambda t: t)  # noqa: E731
        self.tok_emb = dev(p["tok_emb.weight"], T)
        d.tok_emb = ptr(self.tok_emb)
        d.lm_head = ptr(dev(gw(self.tok_emb))) if dtype == torch.bfloat16 else d.tok_emb
        d.anchor_norm = ptr(dev(p["anchor_norm.weight"], torch.float32))
        d.state_norm = ptr(dev(p["pulse_state_norm.weight"], torch.float32))
        d.final_norm = ptr(dev(p["final_norm.weight"], torch.float32))
        d.conv_w = ptr(dev(p["stem_canon_weight"], torch.float32)) if cfg.use_canon_conv else None
        d.step_emb = ptr(dev(p["pulse_step_emb.weight"][:P], T))
        d.reinject_down = ptr(dev(p["reinject_gate_down"][:P], T))
        d.reinject_up = ptr(dev(p["reinject_gate_up"][:P], T))
        d.reinject_bias = ptr(dev(p["reinject_gate_bias"][:P], T))
        d.res_scale = ptr(dev(p["pulse_res_scale"][:P], T))
        cl, sl = rope_tables(cfg.rope_theta_local, cfg.head_dim, self.rope_len)
        cg, sg = rope_tables(cfg.rope_theta_global, cfg.head_dim, self.rope_len)
        d.rope_cos_local, d.rope_sin_local = ptr(dev(cl)), ptr(dev(sl))
        d.rope_cos_global, d.rope_sin_global = ptr(dev(cg)), ptr(dev(sg))
        alpha = cfg.loop_lora_alpha
        for i in range(cfg.n_core):
            pre = f"core.{i}."
            a = pre + "attn."
            d.attn_norm[i] = ptr(dev(p[pre + "attn_norm.weight"][:P], torch.float32))
            d.mlp_norm[i] = ptr(dev(p[pre + "mlp_norm.weight"][:P], torch.float32))
            wqkv = p[a + "wqkv.weight"].to(T)
            wo = p[a + "wo.weight"].to(T)
            qkvg, wos = [], []
            for k in range(P):
                if cfg.loop_lora_rank > 0:
                    mq = _merge(wqkv, p[a + "wqkv_adapter.lora_A"], p[a + "wqkv_adapter.lora_B"],
                                p[a + "wqkv_adapter.loop_M"], k, P, alpha)
                    mo = _merge(wo, p[a + "wo_adapter.lora_A"], p[a + "wo_adapter.lora_B"],
                                p[a + "wo_adapter.loop_M"], k, P, alpha)
                else:
                    mq, mo = wqkv, wo
                qkvg.append(torch.cat([mq, p[a + "attn_gate"][k].to(T)], dim=0))
                wos.append(mo)
            d.wqkvg[i] = ptr(dev(gw(torch.stack(qkvg))))
            d.wo[i] = ptr(dev(gw(torch.stack(wos))))
            d.gate_bias[i] = ptr(dev(p[a + "attn_gate_bias"][:P], T))
            d.q_norm[i] = ptr(dev(p[a + "q_norm_weight"][:P], torch.float32))
            d.k_norm[i] = ptr(dev(p[a + "k_norm_weight"][:P], torch.float32))
            d.v_lambda[i] = ptr(dev(torch.sigmoid(p[a + "v_resid_lambda"][:P]).to(T).float()))
            m = pre + "mlp."
            d.shared_gu[i] = ptr(dev(gw(p[m + "shared_expert.w_gate_up.weight"].to(T))))
            d.shared_down[i] = ptr(dev(gw(p[m + "shared_expert.w_down.weight"].to(T))))
            d.routed_gu[i] = ptr(dev(gw(p[m + "routed_gate_up"].to(T).transpose(1, 2))))
            d.routed_down[i] = ptr(dev(gw(p[m + "routed_down"].to(T).transpose(1, 2))))
            d.router[i] = ptr(dev(p[m + "router_weight"][:P], torch.float32))
            eb = p[m + "expert_bias"]
            if eb.dim() == 1:
                eb = eb.unsqueeze(0).expand(cfg.max_pulses, -1)
            d.expert_bias[i] = ptr(dev(eb[:P], torch.float32))
            d.routed_scale[i] = ptr(dev(p[m + "routed_scale"][:P], T))
        self.desc = d
        torch.cuda.synchronize(self.device)

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._keep)

    def desc_ref(self):
        return ctypes.byref(self.desc)
