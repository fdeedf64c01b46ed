"""Parameter inventory and the deterministic synthetic-weight generator.

Names and shapes follow the reference state dict of ``PulsarForCausalLM``
(``src/model.py:762-815``, ``:1204-1263``, ``:1582-1589``, ``:1730-1775``), so a real
checkpoint's ``ck["model"]`` maps onto the same dict.

Synthetic weights come from a counter-based generator (splitmix64 + Box-Muller in
float64) keyed by ``(seed, parameter name)``. Every element depends only on its own
index, so the values are identical across machines, thread counts and frameworks, and
any slice can be regenerated on its own.

Init rule for random-init benchmark models (no checkpoint exists offline):

* N(0, 0.02) — every matrix-valued weight: ``tok_emb.weight`` (tied ``lm_head``),
  ``wqkv``/``wo`` and their LoRA ``lora_A``/``lora_B``, ``attn_gate``, shared and routed
  experts, ``router_weight``, ``reinject_gate_down``/``_up``, ``stem_canon_weight``,
  ``pulse_step_emb.weight``.
* Reference constant init for the rest: norm weights 1, ``loop_M`` = I,
  ``v_resid_lambda`` = -2.2, ``attn_gate_bias`` = 2.0, ``routed_scale`` = 1,
  ``pulse_res_scale`` = 1, ``reinject_gate_bias`` = 0, ``expert_bias`` = 0.
* ``router_scale`` multiplies ``router_weight`` (the skewed-load workload uses 4).
"""

from __future__ import annotations

import hashlib
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .config import PulsarConfig

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_TWO_PI = 2.0 * np.pi


def _mix64(z: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser on a uint64 array (wrapping arithmetic)."""
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for b in text.encode("utf-8"):
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_key(seed: int, name: str) -> np.uint64:
    """64-bit key of the stream (seed, name)."""
    k = np.array([((seed * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) ^ _fnv1a64(name)],
                 dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(k + _GOLDEN)[0]


def _uniform53(key: np.uint64, counters: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = _mix64(key + (counters + np.uint64(1)) * _GOLDEN)
    return (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def _normal_chunk(key: np.uint64, start: int, count: int) -> np.ndarray:
    idx = np.arange(start, start + count, dtype=np.uint64)
    u1 = _uniform53(key, idx * np.uint64(2))
    u2 = _uniform53(key, idx * np.uint64(2) + np.uint64(1))
    return np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(_TWO_PI * u2)


_CHUNK = 1 << 22


def _workers() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def normal(seed: int, name: str, shape, std: float = 1.0, dtype=np.float32) -> np.ndarray:
    """Deterministic N(0, std^2) array; element i depends only on (seed, name, i)."""
    n = int(np.prod(shape)) if len(shape) else 1
    key = stream_key(seed, name)
    out = np.empty(n, dtype=dtype)

    def fill(start: int) -> None:
        cnt = min(_CHUNK, n - start)
        out[start:start + cnt] = (_normal_chunk(key, start, cnt) * std).astype(dtype)

    starts = list(range(0, n, _CHUNK))
    if len(starts) <= 1:
        for s in starts:
            fill(s)
    else:
        with ThreadPoolExecutor(_workers()) as ex:
            list(ex.map(fill, starts))
    return out.reshape(shape)


def uniform_ids(seed: int, name: str, count: int, vocab: int) -> np.ndarray:
    """Deterministic token ids uniform over [0, vocab)."""
    key = stream_key(seed, name)
    with np.errstate(over="ignore"):
        z = _mix64(key + (np.arange(count, dtype=np.uint64) + np.uint64(1)) * _GOLDEN)
    return (z % np.uint64(vocab)).astype(np.int64)


def zipf_ids(seed: int, name: str, count: int, vocab: int, a: float = 1.1) -> np.ndarray:
    """Deterministic ids with P(rank r) proportional to r^-a over [0, vocab), by inverse CDF."""
    key = stream_key(seed, name)
    u = _uniform53(key, np.arange(count, dtype=np.uint64))
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-a)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.int64)


def param_shapes(cfg: PulsarConfig) -> dict[str, tuple]:
    """State-dict names and shapes used by the decode path (sorted by name)."""
    D, mp = cfg.d_model, cfg.max_pulses
    H, Hk, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    q = cfg.loop_lora_rank
    E, de, ds = cfg.n_routed_experts, cfg.d_expert, cfg.d_shared
    r = cfg.reinject_gate_rank
    s: dict[str, tuple] = {
        "tok_emb.weight": (cfg.vocab_size, D),
        "pulse_step_emb.weight": (mp, D),
        "pulse_state_norm.weight": (D,),
        "anchor_norm.weight": (D,),
        "final_norm.weight": (D,),
        "reinject_gate_down": (mp, r, 2 * D),
        "reinject_gate_up": (mp, D, r),
        "reinject_gate_bias": (mp, D),
        "pulse_res_scale": (mp, D),
    }
    if cfg.use_canon_conv:
        s["stem_canon_weight"] = (D, cfg.canon_kernel_size)
    for i in range(cfg.n_core):
        p = f"core.{i}."
        s[p + "attn_norm.weight"] = (mp, D)
        s[p + "mlp_norm.weight"] = (mp, D)
        s[p + "attn.wqkv.weight"] = (cfg.qkv_dim, D)
        s[p + "attn.wo.weight"] = (D, cfg.q_dim)
        if q > 0:
            s[p + "attn.wqkv_adapter.lora_A"] = (mp, q, D)
            s[p + "attn.wqkv_adapter.lora_B"] = (mp, cfg.qkv_dim, q)
            s[p + "attn.wqkv_adapter.loop_M"] = (mp, mp)
            s[p + "attn.wo_adapter.lora_A"] = (mp, q, cfg.q_dim)
            s[p + "attn.wo_adapter.lora_B"] = (mp, D, q)
            s[p + "attn.wo_adapter.loop_M"] = (mp, mp)
        s[p + "attn.q_norm_weight"] = (mp, H, hd)
        s[p + "attn.k_norm_weight"] = (mp, Hk, hd)
        s[p + "attn.v_resid_lambda"] = (mp,)
        s[p + "attn.attn_gate"] = (mp, H, D)
        s[p + "attn.attn_gate_bias"] = (mp, H)
        s[p + "mlp.shared_expert.w_gate_up.weight"] = (2 * ds, D)
        s[p + "mlp.shared_expert.w_down.weight"] = (D, ds)
        s[p + "mlp.routed_gate_up"] = (E, D, 2 * de)
        s[p + "mlp.routed_down"] = (E, de, D)
        s[p + "mlp.router_weight"] = (mp, E, D)
        s[p + "mlp.routed_scale"] = (mp, D)
        s[p + "mlp.expert_bias"] = (mp, E) if cfg.per_pulse_bias else (E,)
    return dict(sorted(s.items()))


_RANDOM_SUFFIXES = (
    "tok_emb.weight", "pulse_step_emb.weight", "reinject_gate_down", "reinject_gate_up",
    "stem_canon_weight", "wqkv.weight", "wo.weight", "lora_A", "lora_B", "attn_gate",
    "w_gate_up.weight", "w_down.weight", "routed_gate_up", "routed_down", "router_weight",
)


def _init_kind(name: str) -> str:
    if any(name.endswith(s) for s in _RANDOM_SUFFIXES):
        return "normal"
    return "const"


def _const_value(name: str, shape) -> np.ndarray:
    if name.endswith("loop_M"):
        return np.eye(shape[0], shape[1], dtype=np.float32)
    if name.endswith("v_resid_lambda"):
        return np.full(shape, -2.2, dtype=np.float32)
    if name.endswith("attn_gate_bias"):
        return np.full(shape, 2.0, dtype=np.float32)
    if name.endswith(("reinject_gate_bias", "expert_bias")):
        return np.zeros(shape, dtype=np.float32)
    # norm weights, routed_scale, pulse_res_scale
    return np.ones(shape, dtype=np.float32)


def synthetic_state(cfg: PulsarConfig, seed: int = 0, std: float = 0.02,
                    router_scale: float = 1.0) -> dict[str, np.ndarray]:
    """Random-init fp32 weights by the init rule in the module docstring."""
    out: dict[str, np.ndarray] = {}
    for name, shape in param_shapes(cfg).items():
        if _init_kind(name) == "normal":
            arr = normal(seed, name, shape, std=std)
            if name.endswith("router_weight") and router_scale != 1.0:
                arr = (arr * np.float32(router_scale)).astype(np.float32)
        else:
            arr = _const_value(name, shape)
        out[name] = arr
    return out


def exit_probe_state(cfg: PulsarConfig, seed: int = 0) -> dict[str, np.ndarray]:
    """synthetic_state with pulse 0's harmonic residual scale x3 and pulse 1's x0.

    With the plain init the top-1 probability falls from pulse to pulse, so an early-exit
    threshold never sends a token out after pulse 1; with these scales it rises from pulse
    0 to pulse 1 and every exit pulse can be exercised."""
    st = synthetic_state(cfg, seed=seed)
    rs = st["pulse_res_scale"].copy()
    rs[0] *= np.float32(3.0)
    rs[1] *= np.float32(0.0)
    st["pulse_res_scale"] = rs
    return st


def state_digest(state: dict[str, np.ndarray]) -> str:
    """SHA-256 over names, shapes and fp32 bytes in sorted-name order."""
    h = hashlib.sha256()
    for name in sorted(state):
        a = np.ascontiguousarray(state[name], dtype=np.float32)
        h.update(name.encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()
