"""Architecture constants of the Pulsar recurrent MoE decoder.

Mirrors the inference-relevant fields of ``PulsarConfig`` (reference ``src/model.py:13-107``)
with the same names and defaults, so a checkpoint's ``config`` dict loads unchanged
(``from_dict`` ignores training-only keys with a warning, as the reference does at
``src/model.py:77-97``).
"""

from __future__ import annotations

import json
import warnings
from dataclasses import asdict, dataclass, fields


@dataclass
class PulsarConfig:
    vocab_size: int = 32768
    d_model: int = 1024
    n_heads: int = 16
    n_kv_heads: int = 4
    head_dim: int = 64
    d_expert: int = 512
    d_shared: int | None = None
    n_core: int = 8
    max_pulses: int = 8
    default_pulses: int = 3
    reinject_gate_rank: int = 8
    loop_lora_rank: int = 8
    loop_lora_alpha: float = 16.0
    use_canon_conv: bool = True
    canon_kernel_size: int = 4
    base_seq_len: int = 1024
    max_seq_len: int = 32768
    rope_theta_local: float = 10000.0
    rope_theta_global: float = 1000000.0
    sliding_window: int = 1024
    n_routed_experts: int = 16
    top_k: int = 4
    eos_token_id: int = 0
    rms_eps: float = 1e-6
    logit_softcap: float = 30.0
    moe_capacity_factor: float = 1.25
    moe_capacity_align: int = 32
    per_pulse_bias: bool = True

    def __post_init__(self):
        # src/model.py:70-72
        if self.d_shared is None:
            self.d_shared = 1024 if self.d_model >= 1024 else self.d_expert

    # Layers 0,1,2,4,5,6 are sliding-window layers; every other index is global.
    # The reference hard-codes this set (src/infer.py:93, src/model.py:771).
    LOCAL_LAYER_SET = frozenset({0, 1, 2, 4, 5, 6})

    def is_local(self, layer: int) -> bool:
        return layer in self.LOCAL_LAYER_SET

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def qkv_dim(self) -> int:
        return self.q_dim + 2 * self.kv_dim

    def to_dict(self) -> dict:
        return asdict(self)

    @classmethod
    def from_dict(cls, d: dict, *, strict: bool = False) -> "PulsarConfig":
        names = {f.name for f in fields(cls)}
        unknown = sorted(set(d) - names)
        if unknown:
            msg = f"PulsarConfig keys not used by the decode engine: {', '.join(unknown)}"
            if strict:
                raise ValueError(msg)
            warnings.warn(msg, RuntimeWarning, stacklevel=2)
        return cls(**{k: v for k, v in d.items() if k in names})

    def to_json(self, path: str) -> None:
        with open(path, "w", encoding="utf-8") as f:
            json.dump(self.to_dict(), f, indent=2)

    @classmethod
    def from_json(cls, path: str) -> "PulsarConfig":
        with open(path, "r", encoding="utf-8") as f:
            return cls.from_dict(json.load(f))


def tiny_config(**overrides) -> PulsarConfig:
    """Small configuration for fast CPU tests.

    Follows the reference's test config (tests/conftest.py:30-51) but with four core
    layers so that layer 3 is a global layer, and a 16-token window so prompts of a
    few dozen tokens exercise window truncation and the YaRN query scale.
    """
    base = dict(
        vocab_size=256,
        d_model=64,
        n_heads=4,
        n_kv_heads=2,
        head_dim=16,
        d_expert=32,
        d_shared=64,
        n_core=4,
        n_routed_experts=4,
        top_k=2,
        max_pulses=4,
        default_pulses=3,
        base_seq_len=32,
        max_seq_len=128,
        sliding_window=16,
    )
    base.update(overrides)
    return PulsarConfig(**base)


def small_config(**overrides) -> PulsarConfig:
    """Reduced configuration that satisfies the HIP engine's shape rules (head_dim 64, four
    query heads per kv head, widths multiples of 256, vocab a multiple of 4096); layer 3 is
    global and the 16-token window is exceeded by short prompts. For fast GPU checks in
    fp32; bf16 also needs qkv_dim + n_heads to be a multiple of 16 (the matrix-core tile
    height), e.g. ``n_heads=16, n_kv_heads=4``."""
    base = dict(
        vocab_size=4096,
        d_model=256,
        n_heads=4,
        n_kv_heads=1,
        head_dim=64,
        d_expert=256,
        d_shared=256,
        n_core=4,
        n_routed_experts=8,
        top_k=2,
        max_pulses=4,
        default_pulses=3,
        base_seq_len=32,
        max_seq_len=512,
        sliding_window=16,
    )
    base.update(overrides)
    return PulsarConfig(**base)
