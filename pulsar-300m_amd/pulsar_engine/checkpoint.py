"""Checkpoints: reference training checkpoints in, kernel-format weight files out and back.

Reference side (src/infer.py:785-817): ``torch.load(path)`` of a dict holding ``"config"``
(a ``PulsarConfig`` dict, possibly empty) and ``"model"`` (a ``PulsarForCausalLM`` state
dict), ``PulsarConfig.from_dict``, ``load_state_dict(..., strict=False)`` through the
checkpoint migrations of src/model.py:1796-1849, then ``to_training_precision(dtype)``.

Here the file is opened with ``torch.load(..., weights_only=True)``, which executes nothing
from the file; a checkpoint that holds pickled objects other than tensors and plain
containers is refused with an error instead of being unpickled. ``strict=False`` keeps its
meaning: keys the decode path does not read (optimizer state, MoE counters, training
buffers) are ignored, and a parameter the checkpoint lacks keeps the value the reference's
constructor gives it. That value is a constant for norms, scales, biases, ``loop_M`` and
``v_resid_lambda``; for a randomly initialised matrix the reference would decode with
fresh random weights, which has no deterministic equivalent, so that case raises. A shape
that differs from the configuration raises, as ``load_state_dict`` does.

Kernel format: the named tensors of ``model.kernel_tensors`` (merged LoRA, casts and, for
bf16, the matrix-core tile order already applied) in one safetensors file, next to a
``manifest.json`` with the layout version, dtype, configuration and a SHA-256 per tensor.
Loading checks every name, shape, dtype and hash before anything reaches the GPU.
"""

from __future__ import annotations

import hashlib
import json
import os
from typing import Optional

import numpy as np
import torch

from .config import PulsarConfig
from . import weights as W

KERNEL_FORMAT = "pulsar-hip-kernel-weights"
LAYOUT_VERSION = 1
WEIGHTS_FILE = "weights.safetensors"
MANIFEST_FILE = "manifest.json"

_DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16}
_DTYPE_NAMES = {v: k for k, v in _DTYPES.items()}


class CheckpointError(ValueError):
    """A checkpoint or kernel-format file that cannot be loaded as asked."""


# ---------------------------------------------------------------- reference checkpoints


def migrate_state(cfg: PulsarConfig, model_state: dict) -> dict[str, np.ndarray]:
    """Reference state dict -> the fp32 arrays the decode path reads, under ``strict=False``.

    expert_bias follows ``_migrate_checkpoint_bias`` (src/model.py:1803-1827): with
    ``per_pulse_bias`` an [E] bias is broadcast to [max_pulses, E], a missing one becomes
    zeros, and every bias is zero-centred across experts. ``_migrate_counters``
    (src/model.py:1829-1849) only fills training counters, which decode never reads.
    """
    shapes = W.param_shapes(cfg)
    E, mp = cfg.n_routed_experts, cfg.max_pulses
    out: dict[str, np.ndarray] = {}
    for name, shape in shapes.items():
        v = model_state.get(name)
        is_bias = name.endswith("expert_bias")
        if v is None:
            if is_bias:
                v = np.zeros(shape, np.float32)
            elif W._init_kind(name) == "const":
                v = W._const_value(name, shape)
            else:
                raise CheckpointError(
                    f"checkpoint lacks {name} {shape}: the reference would decode with a fresh "
                    "random initialisation of it, which cannot be reproduced")
        a = (v.detach().to("cpu", torch.float32).numpy() if isinstance(v, torch.Tensor)
             else np.asarray(v, dtype=np.float32))
        if is_bias and cfg.per_pulse_bias:
            b = torch.from_numpy(np.array(a, dtype=np.float32))
            if tuple(b.shape) == (E,):
                b = b.unsqueeze(0).expand(mp, -1).clone()
            a = (b - b.mean(dim=-1, keepdim=True)).numpy()
        if tuple(a.shape) != tuple(shape):
            raise CheckpointError(f"{name}: checkpoint shape {tuple(a.shape)}, model {tuple(shape)}")
        out[name] = np.ascontiguousarray(a, dtype=np.float32)
    return out


def load_reference_checkpoint(path: str) -> tuple[PulsarConfig, dict[str, np.ndarray]]:
    """(config, migrated fp32 state) of a reference training checkpoint."""
    if not os.path.exists(path):
        raise FileNotFoundError(f"Checkpoint not found at: {path}")
    try:
        ck = torch.load(path, map_location="cpu", weights_only=True)
    except Exception as e:  # the safe unpickler names the type it refused
        raise CheckpointError(
            f"{path}: not loadable without executing code from the file ({e})") from e
    if not isinstance(ck, dict) or "model" not in ck:
        raise CheckpointError(f"{path}: expected a dict with a 'model' state dict")
    cfg_dict = ck.get("config") or {}
    cfg = PulsarConfig.from_dict(cfg_dict) if cfg_dict else PulsarConfig()
    return cfg, migrate_state(cfg, ck["model"])


# ---------------------------------------------------------------- kernel format


def _tensor_sha256(t: torch.Tensor) -> str:
    b = t.detach().contiguous().reshape(-1).view(torch.uint8).numpy()
    return hashlib.sha256(b.tobytes()).hexdigest()


def save_kernel_format(out_dir: str, cfg: PulsarConfig, tensors: dict[str, torch.Tensor],
                       dtype: torch.dtype, source: Optional[str] = None) -> str:
    """Write ``tensors`` (from ``model.kernel_tensors``) and their manifest; returns out_dir."""
    from safetensors.torch import save_file

    os.makedirs(out_dir, exist_ok=True)
    cpu = {k: v.detach().to("cpu").contiguous() for k, v in sorted(tensors.items())}
    manifest = {
        "format": KERNEL_FORMAT,
        "layout_version": LAYOUT_VERSION,
        "dtype": _DTYPE_NAMES[dtype],
        "n_pulses": cfg.default_pulses,
        "config": cfg.to_dict(),
        "source": source,
        "tensors": {k: {"shape": list(v.shape), "dtype": str(v.dtype).replace("torch.", ""),
                        "sha256": _tensor_sha256(v)} for k, v in cpu.items()},
    }
    save_file(cpu, os.path.join(out_dir, WEIGHTS_FILE))
    with open(os.path.join(out_dir, MANIFEST_FILE), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    return out_dir


def load_kernel_format(in_dir: str) -> tuple[PulsarConfig, torch.dtype, dict[str, torch.Tensor]]:
    """Read and verify a kernel-format directory: (config, dtype, CPU tensors)."""
    from safetensors.torch import load_file

    from .model import expected_kernel_shapes

    with open(os.path.join(in_dir, MANIFEST_FILE)) as f:
        man = json.load(f)
    if man.get("format") != KERNEL_FORMAT:
        raise CheckpointError(f"{in_dir}: not a kernel-format directory ({man.get('format')!r})")
    if man.get("layout_version") != LAYOUT_VERSION:
        raise CheckpointError(f"{in_dir}: layout version {man.get('layout_version')}, "
                              f"this library reads {LAYOUT_VERSION}")
    if man.get("dtype") not in _DTYPES:
        raise CheckpointError(f"{in_dir}: unknown dtype {man.get('dtype')!r}")
    dtype = _DTYPES[man["dtype"]]
    cfg = PulsarConfig.from_dict(man["config"])
    tensors = load_file(os.path.join(in_dir, WEIGHTS_FILE))
    want = expected_kernel_shapes(cfg, dtype)
    listed = man.get("tensors", {})
    if set(tensors) != set(want) or set(listed) != set(want):
        missing = sorted(set(want) - set(tensors))
        extra = sorted(set(tensors) - set(want))
        raise CheckpointError(f"{in_dir}: tensor set differs (missing {missing}, extra {extra})")
    for name, shape in want.items():
        t = tensors[name]
        if tuple(t.shape) != shape or list(shape) != listed[name]["shape"]:
            raise CheckpointError(f"{name}: shape {tuple(t.shape)}, expected {shape}")
        if str(t.dtype).replace("torch.", "") != listed[name]["dtype"]:
            raise CheckpointError(f"{name}: dtype {t.dtype}, manifest {listed[name]['dtype']}")
        if _tensor_sha256(t) != listed[name]["sha256"]:
            raise CheckpointError(f"{name}: SHA-256 differs from the manifest")
    return cfg, dtype, tensors


def export_checkpoint(checkpoint_path: str, out_dir: str,
                      dtype: torch.dtype = torch.bfloat16) -> str:
    """Reference checkpoint -> kernel-format directory (CPU only)."""
    from .model import kernel_tensors

    cfg, state = load_reference_checkpoint(checkpoint_path)
    return save_kernel_format(out_dir, cfg, kernel_tensors(cfg, state, dtype), dtype,
                              source=os.path.basename(checkpoint_path))


def load_inference_model(checkpoint_path: str, device: str = "cuda",
                         dtype: torch.dtype = torch.bfloat16, tokenizer=None):
    """(engine, tokenizer) like src/infer.py:785-817, on the HIP path.

    ``checkpoint_path`` is a reference checkpoint file or a kernel-format directory (whose
    own dtype then applies). The reference loads its tokenizer from a local directory with
    ``transformers``; pass ``tokenizer`` (any object with ``encode``/``decode``/
    ``convert_tokens_to_ids``) or a path to load with ``AutoTokenizer``. Unlike the
    reference there is no CPU fallback: the HIP library and a GPU are required.
    """
    from .engine import PulsarInferenceEngine
    from .model import DeviceModel

    if os.path.isdir(checkpoint_path):
        cfg, dtype, tensors = load_kernel_format(checkpoint_path)
        model = DeviceModel(cfg, tensors, dtype, device=device, kernel_format=True)
    else:
        cfg, state = load_reference_checkpoint(checkpoint_path)
        model = DeviceModel(cfg, state, dtype, device=device)
    if isinstance(tokenizer, str):
        from transformers import AutoTokenizer

        tokenizer = AutoTokenizer.from_pretrained(tokenizer)
    return PulsarInferenceEngine(model, device=device, dtype=dtype), tokenizer
