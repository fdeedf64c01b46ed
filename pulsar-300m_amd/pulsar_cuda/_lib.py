"""ctypes binding of libpulsar_hip.so (declarations mirror include/pulsar_hip.h)."""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpulsar_hip.so")

PULSAR_OK = 0
PULSAR_F32 = 0
PULSAR_BF16 = 1
MAX_LAYERS = 16

BUF_TOKENS = 0
BUF_SEQSTATE = 1
BUF_LOGITS = 2
BUF_ROWS = 3
BUF_CTL = 4
BUF_LAST_ROWS = 5
BUF_LAST_CTL = 6
BUF_EXPERT_COUNTS = 7
BUF_EXIT_COUNTS = 8
BUF_TOPK_IDX = 9
BUF_TOKEN_KINDS = 10
BUF_KV_LAYOUT = 11
BUF_KV_PAGES = 12
ABI_VERSION = 5
SEQSTATE_INTS = 32
ROW_INTS = 8
CTL_INTS = 16
PROF_CLASSES = 17
PROF_NAMES = (
    "pulse_input", "rmsnorm", "qkv_gate_gemm", "qk_post", "attention", "wo_gemm", "router",
    "shared_gate_up", "routed_gate_up", "shared_down", "routed_down", "moe_combine",
    "pulse_output", "lm_head", "sample", "controller", "event_pair",
)

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_vp = ctypes.c_void_p


class PulsarModelDesc(ctypes.Structure):
    _fields_ = [
        ("vocab", _c_i32), ("d_model", _c_i32), ("n_heads", _c_i32), ("n_kv_heads", _c_i32),
        ("head_dim", _c_i32), ("d_expert", _c_i32), ("d_shared", _c_i32), ("n_layers", _c_i32),
        ("n_pulses", _c_i32), ("n_experts", _c_i32), ("top_k", _c_i32), ("window", _c_i32),
        ("base_seq_len", _c_i32), ("reinject_rank", _c_i32), ("dtype", _c_i32),
        ("local_mask", ctypes.c_uint32), ("rms_eps", _c_f32), ("softcap", _c_f32),
        ("rope_len", _c_i32),
        ("tok_emb", _vp), ("anchor_norm", _vp), ("state_norm", _vp), ("final_norm", _vp),
        ("conv_w", _vp), ("step_emb", _vp), ("reinject_down", _vp), ("reinject_up", _vp),
        ("reinject_bias", _vp), ("res_scale", _vp),
        ("rope_cos_local", _vp), ("rope_sin_local", _vp),
        ("rope_cos_global", _vp), ("rope_sin_global", _vp),
        ("attn_norm", _vp * MAX_LAYERS), ("mlp_norm", _vp * MAX_LAYERS),
        ("wqkvg", _vp * MAX_LAYERS), ("gate_bias", _vp * MAX_LAYERS), ("wo", _vp * MAX_LAYERS),
        ("q_norm", _vp * MAX_LAYERS), ("k_norm", _vp * MAX_LAYERS),
        ("v_lambda", _vp * MAX_LAYERS), ("shared_gu", _vp * MAX_LAYERS),
        ("shared_down", _vp * MAX_LAYERS), ("routed_gu", _vp * MAX_LAYERS),
        ("routed_down", _vp * MAX_LAYERS), ("router", _vp * MAX_LAYERS),
        ("expert_bias", _vp * MAX_LAYERS), ("routed_scale", _vp * MAX_LAYERS),
        ("lm_head", _vp),
    ]


class PulsarEngineConfig(ctypes.Structure):
    _fields_ = [
        ("max_batch", _c_i32), ("max_prompt", _c_i32), ("max_new", _c_i32), ("max_ctx", _c_i32),
        ("speculative", _c_i32), ("all_logits", _c_i32),
        ("temperature", _c_f32), ("top_p", _c_f32), ("repetition_penalty", _c_f32),
        ("n_stop", _c_i32), ("stop_ids", _c_i32 * 8), ("seed", ctypes.c_uint64),
        ("draft_len", _c_i32), ("early_exit", _c_i32), ("early_exit_threshold", ctypes.c_double),
        ("kv_pages", _c_i32),
    ]


# name -> argument types (restype is int for every entry except pulsar_last_error)
_PROTOS = {
    "pulsar_abi_version": [],
    "pulsar_rmsnorm_forward": [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_f32, ctypes.c_int, _vp],
    "pulsar_rope_forward": [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int, _vp],
    "pulsar_qk_rmsnorm_rope_forward": [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _vp, _vp, _vp, _vp, _vp, _c_f32, ctypes.c_int, _vp],
    "pulsar_fused_attn_gate_forward": [_vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                       ctypes.c_int, _vp],
    "pulsar_causal_conv1d_k4_forward": [_vp, _vp, _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int, _vp],
    "pulsar_fused_swiglu_forward": [_vp, _vp, _c_i64, _c_i64, ctypes.c_int, _vp],
    "pulsar_moe_router_topk_forward": [_vp, ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64,
                                       _c_i64, _c_f32, _vp],
    "pulsar_moe_router_workspace_bytes": [_c_i64, _c_i64],
    "pulsar_moe_router_topk_forward_ws": [_vp, ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _c_i64,
                                          _c_i64, _c_i64, _c_f32, _vp, _vp],
    "pulsar_moe_dispatch_forward": [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                    _c_i64, ctypes.c_int, _vp],
    "pulsar_moe_combine_forward": [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                   _c_i64, ctypes.c_int, _vp],
    "pulsar_moe_slots_from_order": [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp],
    "pulsar_rmsnorm_backward": [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, ctypes.c_int, _vp],
    "pulsar_qk_rmsnorm_rope_backward": [_vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64,
                                        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp,
                                        _vp, _vp, ctypes.c_int, _vp],
    "pulsar_fused_attn_gate_backward": [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                        ctypes.c_int, _vp],
    "pulsar_fused_swiglu_backward": [_vp, _vp, _vp, _c_i64, _c_i64, ctypes.c_int, _vp],
    "pulsar_moe_dispatch_backward": [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                     ctypes.c_int, _vp],
    "pulsar_moe_combine_backward": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                    _c_i64, _c_i64, ctypes.c_int, _vp],
    "pulsar_moe_router_topk_backward": [_vp, _vp, ctypes.c_int, _vp, _c_f32, _vp, _vp, _vp,
                                        _c_i64, _c_i64, _c_i64, _vp],
    "pulsar_causal_conv1d_k4_backward": [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                         ctypes.c_int, _vp],
    "pulsar_engine_create": [ctypes.POINTER(PulsarModelDesc), ctypes.POINTER(PulsarEngineConfig),
                             ctypes.POINTER(_vp)],
    "pulsar_engine_destroy": [_vp],
    "pulsar_engine_prefill": [_vp, _vp, _c_i32, _c_i32, _vp],
    "pulsar_engine_step": [_vp, _c_i32, _c_i32, _vp],
    "pulsar_engine_generate": [_vp, _c_i32, _c_i32, _vp, ctypes.POINTER(_c_i32)],
    "pulsar_engine_read": [_vp, _c_i32, _vp, _c_i64, _vp],
    "pulsar_engine_rewind": [_vp, ctypes.c_uint64, _vp],
    "pulsar_engine_verify": [_vp, _vp, _c_i32, _c_i32, _vp],
    "pulsar_engine_fill_kv": [_vp, _c_i32, ctypes.c_uint64, _vp],
    "pulsar_engine_profile": [_vp, _c_i32],
    "pulsar_engine_profile_read": [_vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_i64)],
    "pulsar_sample_workspace_bytes": [_c_i32],
    "pulsar_sample_rows": [_vp, _c_i32, _c_i32, _c_i32, _vp, _vp, _vp, _vp, _c_i32,
                           ctypes.c_uint64, _c_f32, _c_f32, _c_f32, _c_i32, _vp, _vp, _vp, _vp],
    "pulsar_sample_rows_static": [_vp, _c_i32, _c_i32, _c_i32, _vp, _vp, _vp, _vp, _c_i32,
                                  ctypes.c_uint64, _c_f32, _c_f32, _c_f32, _c_i32, _vp, _vp,
                                  _vp],
}
# entries whose result is not an int status
_RESTYPES = {"pulsar_sample_workspace_bytes": _c_i64, "pulsar_moe_router_workspace_bytes": _c_i64}

EXPORTED = tuple(["pulsar_last_error", *_PROTOS])

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library once; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"libpulsar_hip.so not found at {path}; build it with "
            "`python pulsar-300m_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    lib.pulsar_last_error.restype = ctypes.c_char_p
    lib.pulsar_last_error.argtypes = []
    for name, args in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != PULSAR_OK:
        msg = load().pulsar_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg or f"pulsar_hip error {rc}")
