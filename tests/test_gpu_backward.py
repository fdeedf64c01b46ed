"""GPU parity of the pulsar_cuda backward ops against the oracle's float64 adjoints
(oracle/backward_ref.py, pinned against torch autograd) on the same dtype-rounded inputs.

Tolerances, per output element e (want) with s = max|want| over the tensor:
* outputs in bf16: |got - want| <= 2^-8 |want| + 1e-4 s (one bf16 rounding of an fp32
  result whose own error is far below it);
* outputs in fp32 (fp32 activations, norm / conv weight gradients, gate-logit gradients):
  |got - want| <= 1e-5 s (fp32 sums in another order; atomics for the weight sums).
Shapes are the model's (d_model 1024, 16 heads of 64, 16 experts top-4) plus ragged and
degenerate ones: rows not a multiple of the workgroup, d_ff not a multiple of 8, sequences
shorter than the conv kernel, dropped MoE assignments, empty batches.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import backward_ref as BW

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float32]


@pytest.fixture(scope="module")
def pc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import pulsar_cuda

    return pulsar_cuda


def _rand(*shape, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(device="cuda", dtype=dtype)


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _check(got, want, dtype, what):
    got = _np(got)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    s = max(float(np.abs(want).max(initial=0.0)), 1e-30)
    if dtype == torch.bfloat16:
        bound = 2.0 ** -8 * np.abs(want) + 1e-4 * s
    else:
        bound = np.full_like(want, 1e-5 * s)
    err = np.abs(got - want)
    bad = err > bound
    assert not bad.any(), f"{what}: {bad.sum()} elements out of bound, max err {err.max():.3e}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,dim", [(300, 1024), (7, 96), (1, 8192)])
def test_rmsnorm_backward(pc, rows, dim, dtype):
    x = _rand(rows, dim, seed=dim, dtype=dtype)
    w = torch.rand(dim, device="cuda") + 0.5
    _, rs = pc.rmsnorm_forward(x, w, 1e-6)
    dy = _rand(rows, dim, seed=dim + 1, dtype=dtype)
    dx, dw = pc.rmsnorm_backward(dy, x, w, rs)
    ox, ow = BW.rmsnorm_bwd(_np(dy), _np(x), _np(w), _np(rs))
    _check(dx, ox, dtype, "rmsnorm dx")
    _check(dw, ow, torch.float32, "rmsnorm dw")
    assert dx.dtype == dtype and dw.dtype == torch.float32


def test_rmsnorm_backward_empty_and_limits(pc):
    x = torch.empty(0, 64, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(64, device="cuda")
    dx, dw = pc.rmsnorm_backward(x, x, w, torch.empty(0, device="cuda"))
    assert dx.shape == (0, 64) and float(dw.abs().sum()) == 0.0
    big = torch.zeros(1, 8200, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="8192"):
        pc.rmsnorm_backward(big, big, torch.ones(8200, device="cuda"),
                            torch.ones(1, device="cuda"))


def _tables(T, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, 64, 2).float() / 64))
    f = torch.outer(torch.arange(T, dtype=torch.float32), inv)
    return f.cos().cuda(), f.sin().cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["contiguous", "bthd_view"])
def test_qk_rmsnorm_rope_backward(pc, dtype, layout):
    B, H, T = 2, 16, 37
    if layout == "contiguous":
        x = _rand(B, H, T, 64, seed=11, dtype=dtype)
    else:  # [B,T,H,64] storage seen as [B,H,T,64], as a fused qkv projection leaves it
        x = _rand(B, T, H, 64, seed=11, dtype=dtype).transpose(1, 2)
    w = torch.rand(H, 64, device="cuda") + 0.5
    cos, sin = _tables(T)
    y, rs = pc.qk_rmsnorm_rope_forward(x, w, cos, sin, T)
    dy = _rand(*y.shape, seed=12, dtype=dtype)
    dx, dw = pc.qk_rmsnorm_rope_backward(dy, x, w, rs, cos, sin, T)
    if layout == "bthd_view":
        assert dx.stride(1) < dx.stride(2), dx.stride()
    else:
        assert dx.is_contiguous()
    ox, ow = BW.qk_rmsnorm_rope_bwd(_np(dy), _np(x), _np(w), _np(rs), _np(cos), _np(sin))
    _check(dx, ox, dtype, "qk dx")
    _check(dw, ow, torch.float32, "qk dw")


def test_qk_rmsnorm_rope_backward_long_sequence(pc):
    """Training-sized sequence: 2 x 2048 vectors per head summed into each weight row."""
    B, H, T = 2, 16, 2048
    x = _rand(B, T, H, 64, seed=13).transpose(1, 2)
    w = torch.rand(H, 64, device="cuda") + 0.5
    cos, sin = _tables(T)
    y, rs = pc.qk_rmsnorm_rope_forward(x, w, cos, sin, T)
    dy = _rand(*y.shape, seed=14)
    dx, dw = pc.qk_rmsnorm_rope_backward(dy, x, w, rs, cos, sin, T)
    ox, ow = BW.qk_rmsnorm_rope_bwd(_np(dy), _np(x), _np(w), _np(rs), _np(cos), _np(sin))
    _check(dx, ox, torch.bfloat16, "qk dx (T=2048)")
    _check(dw, ow, torch.float32, "qk dw (T=2048)")


def test_qk_rmsnorm_rope_backward_rejects_head_dim(pc):
    x = torch.zeros(1, 2, 3, 32, device="cuda", dtype=torch.bfloat16)
    cos, sin = _tables(3)
    with pytest.raises(RuntimeError, match="head_dim == 64"):
        pc.qk_rmsnorm_rope_backward(x, x, torch.ones(2, 32, device="cuda"),
                                    torch.ones(6, device="cuda"), cos, sin, 3)


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_attn_gate_backward(pc, dtype):
    B, H, T = 2, 16, 37
    a = _rand(B, H, T, 64, seed=21, dtype=dtype)
    gl = _rand(B, T, H, seed=22, dtype=torch.float32, scale=2.0)
    go = _rand(B, T, H * 64, seed=23, dtype=dtype)
    da, dl = pc.fused_attn_gate_backward(go, a, gl)
    oa, ol = BW.attn_gate_bwd(_np(go), _np(a), _np(gl))
    _check(da, oa, dtype, "gate d_attn")
    _check(dl, ol, torch.float32, "gate d_logits")
    assert dl.dtype == torch.float32 and dl.shape == (B, T, H)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,d_ff", [(300, 768), (5, 24), (3, 13)])
def test_fused_swiglu_backward(pc, rows, d_ff, dtype):
    gu = _rand(rows, 2 * d_ff, seed=d_ff, dtype=dtype, scale=3.0)
    dout = _rand(rows, d_ff, seed=d_ff + 1, dtype=dtype)
    dgu = pc.fused_swiglu_backward(dout, gu, d_ff)
    _check(dgu, BW.swiglu_bwd(_np(dout), _np(gu), d_ff), dtype, "swiglu dgu")


def _routing(N, K, E, C, seed):
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(N)]).astype(np.int64)
    slots = np.full((N, K), -1, np.int32)
    fill = np.zeros(E, np.int64)
    for t in range(N):
        for k in range(K):
            e = idx[t, k]
            if fill[e] < C:
                slots[t, k] = fill[e]
            fill[e] += 1
    slots[rng.random((N, K)) < 0.05] = -1
    return idx, slots


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("N,D", [(300, 1024), (9, 96)])
def test_moe_dispatch_and_combine_backward(pc, N, D, dtype):
    K, E = 4, 16
    C = max(8, int(np.ceil(N * K / E * 0.9)))  # below the mean load: drops at capacity
    idx, slots = _routing(N, K, E, C, N)
    assert (slots < 0).any()
    ti = torch.as_tensor(idx, device="cuda")
    ts = torch.as_tensor(slots, device="cuda")
    dei = _rand(E, C, D, seed=31, dtype=dtype)
    dx = pc.moe_dispatch_backward(dei, ti, ts, N, D)
    _check(dx, BW.dispatch_bwd(_np(dei), idx, slots, N, D), dtype, "dispatch dx")

    eo = _rand(E, C, D, seed=32, dtype=dtype)
    w = torch.rand(N, K, device="cuda").to(torch.bfloat16)
    dout = _rand(N, D, seed=33, dtype=dtype)
    deo, dw = pc.moe_combine_backward(dout, eo, ti, w, ts)
    oe, ow = BW.combine_bwd(_np(dout), _np(eo), idx, _np(w), slots)
    _check(deo, oe, dtype, "combine d_eo")
    _check(dw, ow, torch.bfloat16, "combine d_w")
    assert dw.dtype == torch.bfloat16
    assert float(dw[torch.as_tensor(slots < 0, device="cuda")].abs().sum()) == 0.0


def test_moe_backward_empty_batch(pc):
    E, C, D = 4, 8, 64
    ti = torch.empty(0, 2, dtype=torch.int64, device="cuda")
    ts = torch.empty(0, 2, dtype=torch.int32, device="cuda")
    dei = _rand(E, C, D, seed=1)
    assert pc.moe_dispatch_backward(dei, ti, ts, 0, D).shape == (0, D)
    deo, dw = pc.moe_combine_backward(torch.empty(0, D, device="cuda", dtype=torch.bfloat16),
                                      dei, ti, torch.empty(0, 2, device="cuda",
                                                           dtype=torch.bfloat16), ts)
    assert float(deo.float().abs().sum()) == 0.0 and dw.shape == (0, 2)


@pytest.mark.parametrize("ldtype", DTYPES)
@pytest.mark.parametrize("zw,dz,with_pm", [(1e-2, 0.5, True), (0.0, None, False),
                                           (1e-4, None, True)])
def test_moe_router_topk_backward(pc, ldtype, zw, dz, with_pm):
    N, E, K = 300, 16, 4
    logits = _rand(N, E, seed=41, dtype=ldtype, scale=2.0)
    bias = 0.1 * torch.randn(E, device="cuda")
    idx, _, _, _ = pc.moe_router_topk_forward(logits, bias, K, zw)
    dtw = _rand(N, K, seed=42, dtype=torch.bfloat16)
    dzt = None if dz is None else torch.tensor(dz, device="cuda", dtype=torch.float32)
    dpm = _rand(E, seed=43, dtype=torch.float32) if with_pm else None
    dl = pc.moe_router_topk_backward(dtw, logits, idx, zw, dzt, dpm)
    want = BW.router_bwd(_np(dtw), _np(logits), idx.cpu().numpy(), zw,
                         None if dz is None else np.float64(dz),
                         _np(dpm) if with_pm else None)
    assert dl.dtype == ldtype
    _check(dl, want, ldtype, "router d_logits")


def test_moe_router_topk_backward_rejects_wide(pc):
    l = torch.zeros(2, 40, device="cuda")
    with pytest.raises(RuntimeError, match="E <= 32"):
        pc.moe_router_topk_backward(torch.zeros(2, 2, device="cuda", dtype=torch.bfloat16), l,
                                    torch.zeros(2, 2, device="cuda", dtype=torch.int64))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,T,D", [(2, 300, 1024), (3, 2, 40), (1, 1, 8)])
def test_causal_conv1d_k4_backward(pc, B, T, D, dtype):
    x = _rand(B, T, D, seed=T, dtype=dtype)
    w = _rand(D, 4, seed=T + 1, dtype=torch.float32, scale=0.5)
    dout = _rand(B, T, D, seed=T + 2, dtype=dtype)
    dx, dw = pc.causal_depthwise_conv1d_k4_backward(dout, x, w)
    ox, ow = BW.conv_k4_bwd(_np(dout), _np(x), _np(w))
    _check(dx, ox, dtype, "conv dx")
    _check(dw, ow, torch.float32, "conv dw")
