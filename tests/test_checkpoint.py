"""Checkpoint loading and the kernel weight format, on the CPU.

* The expert_bias migration of the reference loader (src/model.py:1803-1827) on hand-worked
  values; ``strict=False`` handling of missing and unexpected keys; refusal of files that
  only an unpickler that executes code could open.
* The matrix-core tile order, checked element by element against the operand layout of
  ``v_mfma_f32_16x16x32_bf16`` (lane l holds row l % 16 and columns 8 * (l // 16) .. +8 of
  a 16x32 tile), and the declared kernel shapes against the conversion.
* Kernel-format export/import: a bit-exact round trip, and errors for a changed byte, a
  missing tensor and a different layout version.
"""

from __future__ import annotations

import argparse
import json
import os

import numpy as np
import pytest
import torch

from pulsar_engine import checkpoint as C
from pulsar_engine import weights as W
from pulsar_engine.config import small_config, tiny_config
from pulsar_engine.model import expected_kernel_shapes, kernel_tensors, pack_mfma, tensor_dtype


def _packable():
    # 16 query heads over 4 kv heads: qkv (1536) + gate rows (16) is a multiple of 16
    return small_config(n_heads=16, n_kv_heads=4)


def test_pack_mfma_places_each_element_in_its_lane():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(3, 48, 96, generator=g).to(torch.bfloat16)
    p = pack_mfma(w)
    assert p.shape == (3, 3, 3, 4, 16, 8)
    flat = p.reshape(3, 3, 3, 64, 8)  # [.., n tile, k tile, lane, element]
    for b, n, k in [(0, 0, 0), (1, 17, 40), (2, 47, 95), (0, 31, 63), (2, 5, 88)]:
        lane = (k % 32) // 8 * 16 + n % 16
        assert flat[b, n // 16, k // 32, lane, k % 8] == w[b, n, k]
    # a permutation: every element lands exactly once
    assert torch.equal(p.float().flatten().sort()[0], w.float().flatten().sort()[0])
    with pytest.raises(ValueError):
        pack_mfma(torch.zeros(20, 64))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kernel_shapes_match_the_conversion(dtype):
    cfg = _packable()
    t = kernel_tensors(cfg, W.synthetic_state(cfg, seed=1), dtype)
    want = expected_kernel_shapes(cfg, dtype)
    assert {k: tuple(v.shape) for k, v in t.items()} == want
    fp32 = {"anchor_norm", "state_norm", "final_norm", "conv_w", "attn_norm", "mlp_norm",
            "q_norm", "k_norm", "v_lambda", "router", "expert_bias"}
    for k, v in t.items():
        assert v.dtype == (torch.float32 if k.split(".")[-1] in fp32 else dtype), k
        assert v.dtype == tensor_dtype(k, dtype), k


def test_expert_bias_migration_broadcasts_and_centres():
    cfg = tiny_config()
    E, mp = cfg.n_routed_experts, cfg.max_pulses
    st = {k: torch.from_numpy(v) for k, v in W.synthetic_state(cfg, seed=0).items()}
    st["core.0.mlp.expert_bias"] = torch.tensor([1.0, 2.0, 3.0, 6.0])         # old [E]
    st["core.1.mlp.expert_bias"] = torch.arange(mp * E, dtype=torch.float32).view(mp, E)
    del st["core.2.mlp.expert_bias"]                                           # missing
    out = C.migrate_state(cfg, st)
    np.testing.assert_array_equal(out["core.0.mlp.expert_bias"],
                                  np.tile([-2.0, -1.0, 0.0, 3.0], (mp, 1)))
    np.testing.assert_array_equal(out["core.1.mlp.expert_bias"],
                                  np.tile([-1.5, -0.5, 0.5, 1.5], (mp, 1)))
    np.testing.assert_array_equal(out["core.2.mlp.expert_bias"], np.zeros((mp, E)))
    # without per-pulse biases the [E] buffer is loaded as it is
    cfg1 = tiny_config(per_pulse_bias=False)
    st1 = {k: torch.from_numpy(v) for k, v in W.synthetic_state(cfg1, seed=0).items()}
    st1["core.0.mlp.expert_bias"] = torch.tensor([1.0, 2.0, 3.0, 6.0])
    np.testing.assert_array_equal(C.migrate_state(cfg1, st1)["core.0.mlp.expert_bias"],
                                  [1.0, 2.0, 3.0, 6.0])


def test_missing_and_unexpected_keys_follow_strict_false():
    cfg = tiny_config()
    st = {k: torch.from_numpy(v) for k, v in W.synthetic_state(cfg, seed=0).items()}
    st["core.0.mlp.expert_counts_accum"] = torch.zeros(4)   # training buffer: ignored
    st["optimizer_step"] = torch.tensor(7)
    gone = st.pop("core.1.attn.attn_gate_bias")             # constant init: 2.0
    st.pop("final_norm.weight")                             # constant init: 1.0
    out = C.migrate_state(cfg, st)
    assert set(out) == set(W.param_shapes(cfg))
    np.testing.assert_array_equal(out["core.1.attn.attn_gate_bias"], np.full(gone.shape, 2.0))
    np.testing.assert_array_equal(out["final_norm.weight"], np.ones(cfg.d_model))
    st.pop("core.0.attn.wqkv.weight")
    with pytest.raises(C.CheckpointError, match="random initialisation"):
        C.migrate_state(cfg, st)
    st = {k: torch.from_numpy(v) for k, v in W.synthetic_state(cfg, seed=0).items()}
    st["core.0.attn.wo.weight"] = torch.zeros(3, 3)
    with pytest.raises(C.CheckpointError, match="shape"):
        C.migrate_state(cfg, st)


def test_reference_checkpoint_file(tmp_path):
    cfg = tiny_config()
    st = W.synthetic_state(cfg, seed=3)
    path = str(tmp_path / "best.pt")
    torch.save({"config": cfg.to_dict(), "step": 12,
                "model": {k: torch.from_numpy(v).to(torch.bfloat16) for k, v in st.items()}}, path)
    cfg2, st2 = C.load_reference_checkpoint(path)
    assert cfg2 == cfg
    for k, v in st.items():
        want = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
        if k.endswith("expert_bias"):
            want = want - want.mean(axis=-1, keepdims=True)
        np.testing.assert_array_equal(st2[k], want, err_msg=k)
    bad = str(tmp_path / "objects.pt")
    torch.save({"config": {}, "model": {}, "args": argparse.Namespace(lr=1.0)}, bad)
    with pytest.raises(C.CheckpointError, match="without executing code"):
        C.load_reference_checkpoint(bad)
    with pytest.raises(FileNotFoundError):
        C.load_reference_checkpoint(str(tmp_path / "absent.pt"))


def test_kernel_format_round_trip_and_integrity(tmp_path):
    cfg = _packable()
    t = kernel_tensors(cfg, W.synthetic_state(cfg, seed=2), torch.bfloat16)
    d = C.save_kernel_format(str(tmp_path / "kf"), cfg, t, torch.bfloat16, source="synthetic")
    cfg2, dt2, t2 = C.load_kernel_format(d)
    assert cfg2 == cfg and dt2 == torch.bfloat16 and set(t2) == set(t)
    for k in t:
        assert torch.equal(t2[k].view(torch.int16) if t2[k].dtype == torch.bfloat16 else t2[k],
                           t[k].view(torch.int16) if t[k].dtype == torch.bfloat16 else t[k]), k

    wpath = os.path.join(d, C.WEIGHTS_FILE)
    raw = bytearray(open(wpath, "rb").read())
    raw[-3] ^= 0x40
    open(wpath, "wb").write(bytes(raw))
    with pytest.raises(C.CheckpointError, match="SHA-256"):
        C.load_kernel_format(d)

    d2 = C.save_kernel_format(str(tmp_path / "kf2"), cfg,
                              {k: v for k, v in t.items() if k != "layers.1.wo"}, torch.bfloat16)
    with pytest.raises(C.CheckpointError, match="layers.1.wo"):
        C.load_kernel_format(d2)

    d3 = C.save_kernel_format(str(tmp_path / "kf3"), cfg, t, torch.bfloat16)
    mpath = os.path.join(d3, C.MANIFEST_FILE)
    man = json.load(open(mpath))
    man["layout_version"] = C.LAYOUT_VERSION + 1
    json.dump(man, open(mpath, "w"))
    with pytest.raises(C.CheckpointError, match="layout version"):
        C.load_kernel_format(d3)


def test_export_checkpoint_equals_direct_conversion(tmp_path):
    cfg = _packable()
    st = W.synthetic_state(cfg, seed=4)
    path = str(tmp_path / "ck.pt")
    torch.save({"config": cfg.to_dict(), "model": {k: torch.from_numpy(v) for k, v in st.items()}},
               path)
    d = C.export_checkpoint(path, str(tmp_path / "kf"), torch.bfloat16)
    _, _, t = C.load_kernel_format(d)
    direct = kernel_tensors(cfg, st, torch.bfloat16)
    for k in direct:
        assert torch.equal(t[k].float(), direct[k].float()), k
