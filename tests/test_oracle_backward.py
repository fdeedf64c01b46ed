"""Pins for the oracle's backward restatement (oracle/backward_ref.py).

Each adjoint is checked against torch autograd in float64 through the forward definition
of the same op, written here from the forward's semantics (not from the adjoint), so a
dropped term, a wrong sign in the rotation's transpose, a missed centring or a transposed
layout fails. The cases include what the kernels treat on their own: dropped MoE
assignments (slot -1 and slot >= capacity), the first positions of the causal conv and
sequences shorter than the kernel, z-loss switched off, and d_probs_mean absent.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import backward_ref as BW
from oracle import pulsar_ref as R


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _close(got, want, tol=1e-10):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want.detach().numpy() if isinstance(want, torch.Tensor) else want,
                      dtype=np.float64)
    assert got.shape == want.shape
    scale = max(1.0, float(np.abs(want).max(initial=0.0)))
    np.testing.assert_allclose(got, want, atol=tol * scale, rtol=0)


def test_rmsnorm_bwd_matches_autograd():
    g = _gen(0)
    x = torch.randn(6, 40, dtype=torch.float64, generator=g, requires_grad=True)
    w = (torch.rand(40, dtype=torch.float64, generator=g) + 0.5).requires_grad_(True)
    eps = 1e-6
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    y = x * r * w
    dy = torch.randn(6, 40, dtype=torch.float64, generator=g)
    dx, dw = torch.autograd.grad(y, (x, w), dy)
    ox, ow = BW.rmsnorm_bwd(dy.numpy(), x.detach().numpy(), w.detach().numpy(),
                            r.detach().numpy().reshape(-1))
    _close(ox, dx)
    _close(ow, dw)


@pytest.mark.parametrize("B,H,T", [(2, 3, 5), (1, 4, 1)])
def test_qk_rmsnorm_rope_bwd_matches_autograd(B, H, T):
    g = _gen(1)
    x = torch.randn(B, H, T, 64, dtype=torch.float64, generator=g, requires_grad=True)
    w = (torch.rand(H, 64, dtype=torch.float64, generator=g) + 0.5).requires_grad_(True)
    cos, sin = R.rope_tables(10000.0, 64, T)
    cos, sin = cos.double(), sin.double()
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    n = x * r * w[None, :, None, :]
    lo, hi = n[..., :32], n[..., 32:]
    y = torch.cat([lo * cos - hi * sin, hi * cos + lo * sin], dim=-1)
    dy = torch.randn(B, H, T, 64, dtype=torch.float64, generator=g)
    dx, dw = torch.autograd.grad(y, (x, w), dy)
    ox, ow = BW.qk_rmsnorm_rope_bwd(dy.numpy(), x.detach().numpy(), w.detach().numpy(),
                                    r.detach().numpy().reshape(-1), cos.numpy(), sin.numpy())
    _close(ox, dx)
    _close(ow, dw)


def test_attn_gate_bwd_matches_autograd():
    g = _gen(2)
    B, H, T = 2, 3, 4
    a = torch.randn(B, H, T, 64, dtype=torch.float64, generator=g, requires_grad=True)
    lg = torch.randn(B, T, H, dtype=torch.float64, generator=g, requires_grad=True)
    out = (a.transpose(1, 2) * torch.sigmoid(lg)[..., None]).reshape(B, T, H * 64)
    go = torch.randn(B, T, H * 64, dtype=torch.float64, generator=g)
    da, dl = torch.autograd.grad(out, (a, lg), go)
    oa, ol = BW.attn_gate_bwd(go.numpy(), a.detach().numpy(), lg.detach().numpy())
    _close(oa, da)
    _close(ol, dl)


def test_swiglu_bwd_matches_autograd():
    g = _gen(3)
    gu = (3 * torch.randn(5, 2 * 24, dtype=torch.float64, generator=g)).requires_grad_(True)
    out = F.silu(gu[:, :24]) * gu[:, 24:]
    dout = torch.randn(5, 24, dtype=torch.float64, generator=g)
    (dgu,) = torch.autograd.grad(out, (gu,), dout)
    _close(BW.swiglu_bwd(dout.numpy(), gu.detach().numpy(), 24), dgu)


def _routing(N, K, E, C, seed):
    """Distinct experts per token, slots by arrival order, with drops at capacity C and
    a few assignments forced to slot -1."""
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
    slots[rng.random((N, K)) < 0.1] = -1
    return idx, slots


def test_dispatch_and_combine_bwd_match_autograd():
    N, K, E, C, D = 12, 3, 5, 6, 16
    idx, slots = _routing(N, K, E, C, 4)
    assert (slots < 0).any()
    g = _gen(4)
    x = torch.randn(N, D, dtype=torch.float64, generator=g, requires_grad=True)
    eo = torch.randn(E, C, D, dtype=torch.float64, generator=g, requires_grad=True)
    w = torch.rand(N, K, dtype=torch.float64, generator=g, requires_grad=True)
    ei = torch.zeros(E, C, D, dtype=torch.float64)
    out = torch.zeros(N, D, dtype=torch.float64)
    for t in range(N):
        for k in range(K):
            e, sl = int(idx[t, k]), int(slots[t, k])
            if 0 <= sl < C:
                ei = ei.index_put((torch.tensor(e), torch.tensor(sl)), x[t])
                out = out.index_put((torch.tensor(t),), out[t] + w[t, k] * eo[e, sl])
    dei = torch.randn(E, C, D, dtype=torch.float64, generator=g)
    (dx,) = torch.autograd.grad(ei, (x,), dei)
    _close(BW.dispatch_bwd(dei.numpy(), idx, slots, N, D), dx)
    dout = torch.randn(N, D, dtype=torch.float64, generator=g)
    deo, dw = torch.autograd.grad(out, (eo, w), dout)
    oe, ow = BW.combine_bwd(dout.numpy(), eo.detach().numpy(), idx, w.detach().numpy(), slots)
    _close(oe, deo)
    _close(ow, dw)


@pytest.mark.parametrize("zw,dz,with_pm", [(1e-2, 0.7, True), (0.0, None, False),
                                           (1e-4, None, True)])
def test_router_bwd_matches_autograd(zw, dz, with_pm):
    N, E, K = 9, 16, 4
    g = _gen(5)
    l = (2 * torch.randn(N, E, dtype=torch.float64, generator=g)).requires_grad_(True)
    bias = 0.1 * torch.randn(E, dtype=torch.float64, generator=g)
    c = l - l.mean(-1, keepdim=True)
    s = torch.sigmoid(c)
    idx = torch.topk((s + bias).detach(), K, dim=-1).indices
    raw = s.gather(-1, idx)
    w = raw / (raw.sum(-1, keepdim=True) + 1e-6)
    z = zw * torch.logsumexp(c, -1).pow(2).mean()
    pm = s.mean(0)
    dtw = torch.randn(N, K, dtype=torch.float64, generator=g)
    dpm = torch.randn(E, dtype=torch.float64, generator=g)
    loss = (dtw * w).sum() + (1.0 if dz is None else dz) * z
    if with_pm:
        loss = loss + (dpm * pm).sum()
    (dl,) = torch.autograd.grad(loss, (l,))
    got = BW.router_bwd(dtw.numpy(), l.detach().numpy(), idx.numpy(), zw,
                        None if dz is None else np.float64(dz),
                        dpm.numpy() if with_pm else None)
    _close(got, dl)
    np.testing.assert_allclose(got.sum(-1), 0.0, atol=1e-12)


@pytest.mark.parametrize("B,T,D", [(2, 9, 6), (3, 2, 5)])
def test_conv_k4_bwd_matches_autograd(B, T, D):
    g = _gen(6)
    x = torch.randn(B, T, D, dtype=torch.float64, generator=g, requires_grad=True)
    w = torch.randn(D, 4, dtype=torch.float64, generator=g, requires_grad=True)
    y = x.clone()
    for k in range(4):
        if k < T:
            shifted = torch.cat([torch.zeros(B, k, D, dtype=torch.float64), x[:, : T - k]], 1)
            y = y + w[:, k] * shifted
    dout = torch.randn(B, T, D, dtype=torch.float64, generator=g)
    dx, dw = torch.autograd.grad(y, (x, w), dout)
    ox, ow = BW.conv_k4_bwd(dout.numpy(), x.detach().numpy(), w.detach().numpy())
    _close(ox, dx)
    _close(ow, dw)


def test_conv_forward_definition_matches_oracle_forward():
    """The conv forward used above is the oracle's conv_k4 (y = x + causal conv)."""
    g = _gen(7)
    x = torch.randn(2, 7, 5, generator=g)
    w = torch.randn(5, 4, generator=g)
    y = x.double().clone()
    for k in range(4):
        y[:, k:] += w[:, k].double() * x[:, : 7 - k].double()
    torch.testing.assert_close(R.conv_k4(x, w).double(), y, atol=1e-5, rtol=1e-5)
