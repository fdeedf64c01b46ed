"""GPU parity of the pulsar_cuda op surface against fp32 torch references of the same op.

Shapes mirror the reference's tests/test_kernels.py; tolerances are stated per test
(bf16 outputs: one bf16 rounding of an fp32-exact value; integer outputs: exact).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from conftest import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pc():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import pulsar_cuda

    return pulsar_cuda


def _rand(*shape, seed=0, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(device="cuda", dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dim", [96, 768, 1024, 2048])
def test_rmsnorm(pc, dim, dtype):
    x = _rand(16, dim, seed=dim, dtype=dtype)
    w = torch.rand(dim, device="cuda") + 0.5
    y, rs = pc.rmsnorm_forward(x, w, 1e-6)
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = (w * xf * inv)
    tol = 8e-3 if dtype == torch.bfloat16 else 1e-5
    assert_close(y, ref, atol=tol, rtol=tol, msg=f"rmsnorm {dim}")
    assert_close(rs, inv.view(-1), atol=1e-5, rtol=1e-5)


def _tables(T, theta=10000.0, dim=64):
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2).float() / dim))
    f = torch.outer(torch.arange(T, dtype=torch.float32), inv)
    return f.cos().cuda(), f.sin().cuda()


def _rope_ref(x, cos, sin):
    d = x.shape[-1] // 2
    xf = x.float()
    c, s = cos.view(1, 1, *cos.shape), sin.view(1, 1, *sin.shape)
    return torch.cat([xf[..., :d] * c - xf[..., d:] * s, xf[..., d:] * c + xf[..., :d] * s], -1)


def test_rope(pc):
    x = _rand(2, 4, 37, 64, seed=1)
    cos, sin = _tables(37)
    assert_close(pc.rope_forward(x, cos, sin), _rope_ref(x, cos, sin), atol=2e-2, rtol=8e-3)
    assert pc.rope_forward(x[:, :, :0].contiguous(), cos, sin).numel() == 0


@pytest.mark.parametrize("H", [4, 16])
def test_qk_rmsnorm_rope_strided(pc, H):
    # strided input: q view of a fused qkv projection, as PulsarAttention passes it
    B, T = 2, 9
    qkv = _rand(B, T, H * 64 * 3, seed=H)
    x = qkv[..., : H * 64].view(B, T, H, 64).transpose(1, 2)
    w = torch.rand(H, 64, device="cuda") + 0.5
    cos, sin = _tables(T)
    y, rs = pc.qk_rmsnorm_rope_forward(x, w, cos, sin, T, 1e-6)
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = _rope_ref(xf * inv * w.view(1, H, 1, 64), cos, sin)
    assert y.is_contiguous()
    assert_close(y, ref, atol=2e-2, rtol=8e-3)
    assert_close(rs, inv.reshape(-1), atol=1e-5, rtol=1e-5)


def test_qk_rmsnorm_rope_rejects_wrong_head_dim(pc):
    x = _rand(1, 2, 3, 32)
    with pytest.raises(RuntimeError, match="head_dim == 64"):
        pc.qk_rmsnorm_rope_forward(x, torch.ones(2, 32, device="cuda"), *_tables(3, dim=32), 3)


def test_fused_attn_gate(pc):
    a = _rand(2, 16, 5, 64, seed=3)
    gl = _rand(2, 5, 16, seed=4, dtype=torch.float32)
    out = pc.fused_attn_gate_forward(a, gl)
    ref = (a.float().transpose(1, 2) * torch.sigmoid(gl).unsqueeze(-1)).reshape(2, 5, 1024)
    assert_close(out, ref, atol=1e-2, rtol=8e-3)


def test_causal_conv1d_k4(pc):
    x = _rand(2, 11, 1024, seed=5)
    w = _rand(1024, 4, seed=6, dtype=torch.float32, scale=0.3)
    y = pc.causal_depthwise_conv1d_k4_forward(x, w)
    xp = F.pad(x.float().transpose(1, 2), (3, 0))
    ref = x.float() + F.conv1d(xp, w.unsqueeze(1).flip(-1), groups=1024).transpose(1, 2)
    assert_close(y, ref, atol=2e-2, rtol=8e-3)


@pytest.mark.parametrize("d_ff", [512, 1024, 513])
def test_swiglu(pc, d_ff):
    gu = _rand(7, 2 * d_ff, seed=d_ff)
    ref = F.silu(gu[:, :d_ff].float()) * gu[:, d_ff:].float()
    assert_close(pc.fused_swiglu_forward(gu, d_ff), ref, atol=2e-2, rtol=8e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N", [1, 16, 320, 4096])
def test_router_topk_bit_exact_indices(pc, N, dtype):
    E, K = 16, 4
    logits = _rand(N, E, seed=N, dtype=dtype, scale=2.0)
    bias = (torch.rand(E, device="cuda") - 0.5) * 0.1
    idx, w, z, pm = pc.moe_router_topk_forward(logits, bias, K, 1e-3)
    lf = logits.float()
    c = lf - lf.mean(-1, keepdim=True)
    s = torch.sigmoid(c)
    _, ref_idx = torch.topk(s + bias, K, dim=-1)
    assert torch.equal(idx, ref_idx), "router indices must be bit-exact"
    raw = torch.gather(s, -1, ref_idx)
    ref_w = raw / (raw.sum(-1, keepdim=True) + 1e-6)
    assert w.dtype == torch.bfloat16
    assert (w.float() - ref_w).abs().max().item() <= 2 ** -8
    assert_close(pm, s.mean(0), atol=1e-5, rtol=1e-4)
    lse = torch.logsumexp(c, -1)
    assert_close(z, 1e-3 * lse.pow(2).mean(), atol=1e-6, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,E", [(4096, 16), (1000, 24), (300, 7)])
def test_router_statistics_with_and_without_workspace(pc, N, E, dtype):
    """The workspace entry (per-workgroup partials) and the plain entry (one workgroup over
    every token): identical indices and weights, statistics equal up to summation order."""
    from pulsar_cuda import _lib

    lib = _lib.load()
    K = 4
    logits = _rand(N, E, seed=N + E, dtype=dtype, scale=2.0)
    bias = (torch.rand(E, device="cuda") - 0.5) * 0.1
    outs = []
    for ws in (True, False):
        idx = torch.empty(N, K, dtype=torch.int64, device="cuda")
        w = torch.empty(N, K, dtype=torch.bfloat16, device="cuda")
        z = torch.zeros((), device="cuda")
        pm = torch.zeros(E, device="cuda")
        code = 1 if dtype == torch.bfloat16 else 0
        stream = torch.cuda.current_stream().cuda_stream
        if ws:
            buf = torch.empty(lib.pulsar_moe_router_workspace_bytes(N, E) // 4, device="cuda")
            rc = lib.pulsar_moe_router_topk_forward_ws(
                logits.data_ptr(), code, bias.data_ptr(), idx.data_ptr(), w.data_ptr(),
                z.data_ptr(), pm.data_ptr(), N, E, K, 1e-3, buf.data_ptr(), stream)
        else:
            rc = lib.pulsar_moe_router_topk_forward(
                logits.data_ptr(), code, bias.data_ptr(), idx.data_ptr(), w.data_ptr(),
                z.data_ptr(), pm.data_ptr(), N, E, K, 1e-3, stream)
        assert rc == 0, lib.pulsar_last_error()
        outs.append((idx, w, z, pm))
    (i1, w1, z1, p1), (i2, w2, z2, p2) = outs
    assert torch.equal(i1, i2) and torch.equal(w1, w2)
    assert_close(p1, p2, atol=0, rtol=1e-5)
    assert_close(z1, z2, atol=0, rtol=1e-5)


def test_router_three_argument_overload(pc):
    logits = _rand(8, 8, seed=9, dtype=torch.float32)
    idx, w, z, pm = pc.moe_router_topk_forward(logits, torch.zeros(8, device="cuda"), 0.0)
    assert idx.shape == (8, 2) and float(z) == 0.0


def test_slots_dispatch_combine(pc):
    N, K, E, D = 64, 4, 16, 1024
    g = torch.Generator().manual_seed(11)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(N)]).cuda()
    w = torch.rand(N, K, generator=g).cuda().to(torch.bfloat16)
    flat_e = idx.reshape(-1).contiguous()
    key = flat_e.float() - 0.5 * (w.reshape(-1).float() / (1 + w.reshape(-1).float()))
    order = torch.argsort(key, stable=True)
    C = 12
    slots, counts = pc.moe_slots_from_order(flat_e, order, E, C)
    # brute-force rank within expert in `order`
    ref = torch.full((N * K,), -1, dtype=torch.int32)
    seen = {}
    for pos in order.cpu().tolist():
        e = int(flat_e[pos])
        r = seen.get(e, 0)
        seen[e] = r + 1
        ref[pos] = r if r < C else -1
    assert torch.equal(slots.cpu(), ref)
    assert torch.equal(counts.cpu(), torch.bincount(flat_e.cpu(), minlength=E))
    x = _rand(N, D, seed=12)
    slots2 = slots.view(N, K).contiguous()
    (buf,) = pc.moe_dispatch_forward(x, idx, slots2, E, C, counts)
    # every kept assignment's row landed in its slot; unused slots are zero
    for n in range(N):
        for k in range(K):
            s = int(slots2[n, k])
            if s >= 0:
                assert torch.equal(buf[idx[n, k], s], x[n])
    used = torch.zeros(E, C, dtype=torch.bool)
    for n in range(N):
        for k in range(K):
            if int(slots2[n, k]) >= 0:
                used[int(idx[n, k]), int(slots2[n, k])] = True
    assert buf[~used.cuda()].abs().max().item() == 0.0
    eo = _rand(E, C, D, seed=13)
    sh = _rand(N, D, seed=14)
    out = pc.moe_combine_forward(eo, idx, w, slots2, sh)
    ref = sh.float().clone()
    for n in range(N):
        for k in range(K):
            s = int(slots2[n, k])
            if s >= 0:
                ref[n] += w[n, k].float() * eo[idx[n, k], s].float()
    assert_close(out, ref, atol=3e-2, rtol=8e-3)


def _misaligned(t: torch.Tensor) -> torch.Tensor:
    """The same values in a contiguous view one element past a 16-byte boundary, which sends
    an op to its scalar kernel instead of the 16-byte one."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = buf[1:].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0 and v.is_contiguous()
    return v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_vector_and_scalar_kernels_agree(pc, dtype):
    """Each elementwise op's 16-byte kernel (aligned inputs) and scalar kernel (misaligned
    copy) compute every element by the same expression: equal outputs. RMSNorm's sum of
    squares runs in another order: within one rounding of the output dtype."""
    # bf16: one rounding step; fp32: a few ulp from the reordered 768-term sum
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -20
    x = _rand(8, 768, seed=21, dtype=dtype)
    w = torch.rand(768, device="cuda") + 0.5
    (ya, ra), (yb, rb) = pc.rmsnorm_forward(x, w, 1e-6), pc.rmsnorm_forward(_misaligned(x), w, 1e-6)
    assert ((ya.float() - yb.float()).abs() <= ulp * yb.float().abs() + 1e-30).all()
    assert_close(ra, rb, atol=0, rtol=1e-6)

    q = _rand(2, 4, 13, 64, seed=22, dtype=dtype)
    cos, sin = _tables(13)
    assert torch.equal(pc.rope_forward(q, cos, sin), pc.rope_forward(_misaligned(q), cos, sin))

    B, T, H = 2, 7, 4
    qkv = _rand(B, T, H * 64 * 3, seed=23, dtype=dtype)
    xs = qkv[..., : H * 64].view(B, T, H, 64).transpose(1, 2)
    xm = _misaligned(qkv)[..., : H * 64].view(B, T, H, 64).transpose(1, 2)
    wq = torch.rand(H, 64, device="cuda") + 0.5
    cq, sq = _tables(T)
    (y1, r1), (y2, r2) = (pc.qk_rmsnorm_rope_forward(xs, wq, cq, sq, T, 1e-6),
                          pc.qk_rmsnorm_rope_forward(xm, wq, cq, sq, T, 1e-6))
    # the rotation's differences may cancel: bound by the head's largest output
    assert ((y1.float() - y2.float()).abs()
            <= 2 * ulp * y2.float().abs().amax(-1, keepdim=True)).all()
    assert_close(r1, r2, atol=0, rtol=1e-6)

    a = _rand(2, 16, 5, 64, seed=24, dtype=dtype)
    gl = _rand(2, 5, 16, seed=25, dtype=torch.float32)
    assert torch.equal(pc.fused_attn_gate_forward(a, gl),
                       pc.fused_attn_gate_forward(_misaligned(a), gl))

    xc = _rand(2, 11, 256, seed=26, dtype=dtype)
    wc = _rand(256, 4, seed=27, dtype=torch.float32, scale=0.3)
    assert torch.equal(pc.causal_depthwise_conv1d_k4_forward(xc, wc),
                       pc.causal_depthwise_conv1d_k4_forward(_misaligned(xc), wc))

    gu = _rand(7, 1024, seed=28, dtype=dtype)
    assert torch.equal(pc.fused_swiglu_forward(gu, 512),
                       pc.fused_swiglu_forward(_misaligned(gu), 512))

    N, K, E, C, D = 32, 2, 8, 10, 256
    g = torch.Generator().manual_seed(29)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(N)]).cuda()
    wt = torch.rand(N, K, generator=g).cuda().to(torch.bfloat16)
    flat_e = idx.reshape(-1).contiguous()
    slots, counts = pc.moe_slots_from_order(flat_e, torch.argsort(flat_e, stable=True), E, C)
    slots = slots.view(N, K).contiguous()
    xd = _rand(N, D, seed=30, dtype=dtype)
    (b1,) = pc.moe_dispatch_forward(xd, idx, slots, E, C, counts)
    (b2,) = pc.moe_dispatch_forward(_misaligned(xd), idx, slots, E, C, counts)
    assert torch.equal(b1, b2)
    eo = _rand(E, C, D, seed=31, dtype=dtype)
    sh = _rand(N, D, seed=32, dtype=dtype)
    assert torch.equal(pc.moe_combine_forward(eo, idx, wt, slots, sh),
                       pc.moe_combine_forward(_misaligned(eo), idx, wt, slots, sh))
