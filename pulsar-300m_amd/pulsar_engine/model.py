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


# Names of the kernel-format tensors of one layer (prefixed with "layers.<i>.").
LAYER_TENSORS = (
    "attn_norm", "mlp_norm", "wqkvg", "wo", "gate_bias", "q_norm", "k_norm", "v_lambda",
    "shared_gu", "shared_down", "routed_gu", "routed_down", "router", "expert_bias",
    "routed_scale",
)
GLOBAL_TENSORS = (
    "tok_emb", "lm_head", "anchor_norm", "state_norm", "final_norm", "conv_w", "step_emb",
    "reinject_down", "reinject_up", "reinject_bias", "res_scale",
)
# Tensors held in the activation dtype; every other one is fp32.
ACT_DTYPE_TENSORS = frozenset((
    "tok_emb", "lm_head", "step_emb", "reinject_down", "reinject_up", "reinject_bias",
    "res_scale", "wqkvg", "wo", "gate_bias", "shared_gu", "shared_down", "routed_gu",
    "routed_down", "routed_scale",
))


def tensor_dtype(name: str, dtype: torch.dtype) -> torch.dtype:
    """Storage dtype of kernel tensor ``name`` in a model computing in ``dtype``."""
    return dtype if name.split(".")[-1] in ACT_DTYPE_TENSORS else torch.float32


def expected_kernel_shapes(cfg: PulsarConfig, dtype: torch.dtype) -> dict[str, tuple]:
    """Name -> shape of every tensor ``kernel_tensors`` produces for ``cfg`` and ``dtype``."""
    P, D, V = cfg.default_pulses, cfg.d_model, cfg.vocab_size
    H, Hk, hd, E = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.n_routed_experts
    de, ds, r = cfg.d_expert, cfg.d_shared, cfg.reinject_gate_rank

    def g(*s):  # GEMM weight [..., N, K]
        *lead, n, k = s
        return (*lead, n // 16, k // 32, 4, 16, 8) if dtype == torch.bfloat16 else tuple(s)

    out = {"tok_emb": (V, D), "lm_head": g(V, D), "anchor_norm": (D,), "state_norm": (D,),
           "final_norm": (D,), "step_emb": (P, D), "reinject_down": (P, r, 2 * D),
           "reinject_up": (P, D, r), "reinject_bias": (P, D), "res_scale": (P, D)}
    if cfg.use_canon_conv:
        out["conv_w"] = (D, cfg.canon_kernel_size)
    layer = {"attn_norm": (P, D), "mlp_norm": (P, D), "wqkvg": g(P, cfg.qkv_dim + H, D),
             "wo": g(P, D, cfg.q_dim), "gate_bias": (P, H), "q_norm": (P, H, hd),
             "k_norm": (P, Hk, hd), "v_lambda": (P,), "shared_gu": g(2 * ds, D),
             "shared_down": g(D, ds), "routed_gu": g(E, 2 * de, D), "routed_down": g(E, D, de),
             "router": (P, E, D), "expert_bias": (P, E), "routed_scale": (P, D)}
    for i in range(cfg.n_core):
        out.update({f"layers.{i}.{k}": v for k, v in layer.items()})
    return out


def kernel_tensors(cfg: PulsarConfig, state: dict, dtype: torch.dtype = torch.bfloat16) -> dict:
    """Reference-format state dict -> named CPU tensors in the layout the HIP engine reads.

    Applies, once, what the reference applies at load or on every pulse: the precision
    policy, the per-pulse LoRA merge, the attention-gate rows appended to the merged qkv
    weight, the decode-time ``.to(x.dtype)`` casts, expert transposition to [E][out][in],
    and (bf16) the matrix-core tile layout of every GEMM weight plus a packed copy of the
    tied output head.
    """
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("dtype must be torch.float32 or torch.bfloat16")
    if cfg.head_dim != 64 or cfg.n_heads != 4 * cfg.n_kv_heads:
        raise ValueError("the HIP engine implements head_dim 64 with 4 query heads per kv head")
    P = cfg.default_pulses
    T = dtype
    f32 = torch.float32
    p = {k: _policy(k, torch.as_tensor(np.asarray(v)), dtype) for k, v in state.items()}
    gw = (lambda t: pack_mfma(t)) if dtype == torch.bfloat16 else (lambda t: t)  # noqa: E731
    out = {}
    out["tok_emb"] = p["tok_emb.weight"].to(T)
    out["lm_head"] = gw(out["tok_emb"])
    out["anchor_norm"] = p["anchor_norm.weight"].to(f32)
    out["state_norm"] = p["pulse_state_norm.weight"].to(f32)
    out["final_norm"] = p["final_norm.weight"].to(f32)
    if cfg.use_canon_conv:
        out["conv_w"] = p["stem_canon_weight"].to(f32)
    out["step_emb"] = p["pulse_step_emb.weight"][:P].to(T)
    out["reinject_down"] = p["reinject_gate_down"][:P].to(T)
    out["reinject_up"] = p["reinject_gate_up"][:P].to(T)
    out["reinject_bias"] = p["reinject_gate_bias"][:P].to(T)
    out["res_scale"] = p["pulse_res_scale"][:P].to(T)
    alpha = cfg.loop_lora_alpha
    for i in range(cfg.n_core):
        pre, L = f"core.{i}.", f"layers.{i}."
        a, m = pre + "attn.", pre + "mlp."
        out[L + "attn_norm"] = p[pre + "attn_norm.weight"][:P].to(f32)
        out[L + "mlp_norm"] = p[pre + "mlp_norm.weight"][:P].to(f32)
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
        out[L + "wqkvg"] = gw(torch.stack(qkvg))
        out[L + "wo"] = gw(torch.stack(wos))
        out[L + "gate_bias"] = p[a + "attn_gate_bias"][:P].to(T)
        out[L + "q_norm"] = p[a + "q_norm_weight"][:P].to(f32)
        out[L + "k_norm"] = p[a + "k_norm_weight"][:P].to(f32)
        out[L + "v_lambda"] = torch.sigmoid(p[a + "v_resid_lambda"][:P]).to(T).float()
        out[L + "shared_gu"] = gw(p[m + "shared_expert.w_gate_up.weight"].to(T))
        out[L + "shared_down"] = gw(p[m + "shared_expert.w_down.weight"].to(T))
        out[L + "routed_gu"] = gw(p[m + "routed_gate_up"].to(T).transpose(1, 2))
        out[L + "routed_down"] = gw(p[m + "routed_down"].to(T).transpose(1, 2))
        out[L + "router"] = p[m + "router_weight"][:P].to(f32)
        eb = p[m + "expert_bias"]
        if eb.dim() == 1:
            eb = eb.unsqueeze(0).expand(cfg.max_pulses, -1)
        out[L + "expert_bias"] = eb[:P].to(f32)
        out[L + "routed_scale"] = p[m + "routed_scale"][:P].to(T)
    return {k: v.contiguous() for k, v in out.items()}


class DeviceModel:
    """Weights of one model in kernel format on a GPU, plus the C descriptor.

    ``state`` is either a reference-format state dict (converted by ``kernel_tensors``) or,
    with ``kernel_format=True``, the named kernel-format tensors themselves (as read by
    ``checkpoint.load_kernel_format``). Names, shapes and dtypes are checked before upload."""

    def __init__(self, cfg: PulsarConfig, state: dict, dtype: torch.dtype = torch.bfloat16,
                 device: str | torch.device = "cuda", rope_len: int | None = None,
                 kernel_format: bool = False):
        from pulsar_cuda import _lib

        self.cfg = cfg
        self.dtype = dtype
        self.device = torch.device(device)
        P = cfg.default_pulses
        self.n_pulses = P
        tensors = state if kernel_format else kernel_tensors(cfg, state, dtype)
        want = expected_kernel_shapes(cfg, dtype)
        if set(tensors) != set(want):
            raise ValueError(f"kernel tensors: missing {sorted(set(want) - set(tensors))}, "
                             f"unexpected {sorted(set(tensors) - set(want))}")
        for k, shape in want.items():
            if tuple(tensors[k].shape) != shape:
                raise ValueError(f"{k}: shape {tuple(tensors[k].shape)}, expected {shape}")
            if tensors[k].dtype != tensor_dtype(k, dtype):
                raise ValueError(f"{k}: dtype {tensors[k].dtype}, expected {tensor_dtype(k, dtype)}")
        self.tensors = {k: v.to(self.device) for k, v in tensors.items()}
        t = self.tensors
        T = dtype

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
        ptr = lambda x: x.data_ptr()  # noqa: E731
        self.tok_emb = t["tok_emb"]
        d.tok_emb = ptr(t["tok_emb"])
        d.lm_head = ptr(t["lm_head"])
        d.anchor_norm = ptr(t["anchor_norm"])
        d.state_norm = ptr(t["state_norm"])
        d.final_norm = ptr(t["final_norm"])
        d.conv_w = ptr(t["conv_w"]) if "conv_w" in t else None
        d.step_emb = ptr(t["step_emb"])
        d.reinject_down = ptr(t["reinject_down"])
        d.reinject_up = ptr(t["reinject_up"])
        d.reinject_bias = ptr(t["reinject_bias"])
        d.res_scale = ptr(t["res_scale"])
        self.desc = d
        self._rope_retired: list = []
        self._set_rope(self.rope_len)
        for i in range(cfg.n_core):
            L = f"layers.{i}."
            for name in LAYER_TENSORS:
                getattr(d, name)[i] = ptr(t[L + name])
        torch.cuda.synchronize(self.device)

    def _set_rope(self, n: int) -> None:
        cfg, d = self.cfg, self.desc
        cl, sl = rope_tables(cfg.rope_theta_local, cfg.head_dim, n)
        cg, sg = rope_tables(cfg.rope_theta_global, cfg.head_dim, n)
        self._rope = [x.to(self.device) for x in (cl, sl, cg, sg)]
        d.rope_cos_local, d.rope_sin_local = self._rope[0].data_ptr(), self._rope[1].data_ptr()
        d.rope_cos_global, d.rope_sin_global = self._rope[2].data_ptr(), self._rope[3].data_ptr()
        d.rope_len = n
        self.rope_len = n

    def ensure_rope(self, n: int) -> None:
        """Grow the RoPE tables to ``n`` positions, as the reference's rotary cache grows
        when a sequence outruns it (src/model.py:553-556; entries of a position do not
        depend on the table length). Engines created earlier keep the tables they were
        given: the old tensors stay alive with the model."""
        if n <= self.rope_len:
            return
        self._rope_retired.append(self._rope)
        self._set_rope(int(n))
        torch.cuda.synchronize(self.device)

    @property
    def nbytes(self) -> int:
        return sum(x.numel() * x.element_size() for x in self.tensors.values())

    def desc_ref(self):
        return ctypes.byref(self.desc)
