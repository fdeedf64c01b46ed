"""CPU checks of the C-ABI library: it loads, exports every declared entry point, and the
ctypes descriptors match the C struct layouts."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "pulsar_hip.h")


def _declared() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pulsar_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_op_surface():
    names = _declared()
    for op in ("rmsnorm_forward", "rope_forward", "qk_rmsnorm_rope_forward",
               "fused_attn_gate_forward", "causal_conv1d_k4_forward", "fused_swiglu_forward",
               "moe_router_topk_forward", "moe_dispatch_forward", "moe_combine_forward",
               "moe_slots_from_order", "engine_create", "engine_prefill", "engine_step"):
        assert f"pulsar_{op}" in names


def test_library_exports_every_declared_symbol():
    from pulsar_cuda import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libpulsar_hip.so not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_declared()) == set(_lib.EXPORTED)
    lib.pulsar_abi_version.restype = ctypes.c_int
    assert lib.pulsar_abi_version() == _lib.ABI_VERSION == 5


def test_struct_layouts_match_the_c_header(tmp_path):
    """Compile a tiny C++ program with the header and compare sizeof/offsetof."""
    from pulsar_cuda import _lib

    src = tmp_path / "layout.cpp"
    fields_m = ["vocab", "dtype", "local_mask", "rms_eps", "rope_len", "tok_emb", "rope_sin_global",
                "attn_norm", "wqkvg", "routed_scale"]
    fields_c = ["max_batch", "temperature", "n_stop", "stop_ids", "seed", "draft_len",
                "early_exit", "early_exit_threshold"]
    lines = ["#include <cstdio>", "#include <cstddef>", f'#include "{HEADER}"', "int main() {",
             'printf("%zu %zu\\n", sizeof(PulsarModelDesc), sizeof(PulsarEngineConfig));']
    lines += [f'printf("%zu\\n", offsetof(PulsarModelDesc, {f}));' for f in fields_m]
    lines += [f'printf("%zu\\n", offsetof(PulsarEngineConfig, {f}));' for f in fields_c]
    lines += ["return 0; }"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    r = subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                        str(src), "-o", str(exe)], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("host compiler cannot build against hip_runtime_api.h: " + r.stderr[-300:])
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    vals = [int(v) for v in out]
    assert vals[0] == ctypes.sizeof(_lib.PulsarModelDesc)
    assert vals[1] == ctypes.sizeof(_lib.PulsarEngineConfig)
    for f, v in zip(fields_m, vals[2:2 + len(fields_m)]):
        assert getattr(_lib.PulsarModelDesc, f).offset == v, f
    for f, v in zip(fields_c, vals[2 + len(fields_m):]):
        assert getattr(_lib.PulsarEngineConfig, f).offset == v, f


def test_missing_library_fails_loudly(tmp_path):
    from pulsar_cuda import _lib

    saved = _lib._lib
    try:
        _lib._lib = None
        with pytest.raises(RuntimeError, match="not found"):
            _lib.load(str(tmp_path / "nope.so"))
    finally:
        _lib._lib = saved


def test_sample_rows_validates_before_touching_the_device():
    """The sampler entry rejects bad arguments with a message, without a GPU."""
    from pulsar_cuda import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libpulsar_hip.so not built")
    lib = _lib.load()
    assert lib.pulsar_sample_workspace_bytes(4) >= 512 + 4 * 64
    assert lib.pulsar_sample_workspace_bytes(-1) == -1
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    args = [p, 2, 32768, _lib.PULSAR_BF16, p, p, p, p, 1, 0, 0.8, 0.9, 1.1, 0, p, p, p, None]
    bad = dict(null=(0, None), temperature=(10, 0.0), top_p=(11, 1.5), n_seq=(8, 0),
               dtype=(3, 7))
    for name, (i, v) in bad.items():
        a = list(args)
        a[i] = v
        rc = lib.pulsar_sample_rows(*a)
        assert rc != 0, name
        assert b"sample_rows" in lib.pulsar_last_error(), name


def test_router_workspace_entry_validates_without_a_device():
    """The router's workspace size for 128-token workgroups, and the workspace entry's refusal
    to compute statistics without one (checked before any launch)."""
    from pulsar_cuda import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libpulsar_hip.so not built")
    lib = _lib.load()
    assert lib.pulsar_moe_router_workspace_bytes(16384, 16) == 128 * 17 * 4
    assert lib.pulsar_moe_router_workspace_bytes(129, 32) == 2 * 33 * 4
    assert lib.pulsar_moe_router_workspace_bytes(10, 33) == -1
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    rc = lib.pulsar_moe_router_topk_forward_ws(p, _lib.PULSAR_BF16, p, p, p, p, p, 8, 16, 4,
                                               1e-3, None, None)
    assert rc != 0 and b"workspace" in lib.pulsar_last_error()
