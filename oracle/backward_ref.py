"""Oracle: CPU restatement of the backward ops of the reference's pulsar_cuda surface.

TEST INFRASTRUCTURE ONLY. Only ``tests/`` may import this module, as the checker of the
HIP backward ops; the product path (``pulsar_cuda``) never calls it.

Each function is the closed-form adjoint of one forward op, in float64 numpy on the given
(already dtype-rounded) inputs, and follows the reference kernel cited in its docstring.

Parity status: every function is pinned by ``tests/test_oracle_backward.py`` against
torch autograd (float64) through the forward definitions of the same ops, including the
special cases the kernels treat on their own (dropped MoE assignments, the first three
positions of the causal conv, z-loss off, absent d_probs_mean).
"""

from __future__ import annotations

import numpy as np


def _f64(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64)


def rmsnorm_bwd(dy, x, w, rsq):
    """csrc/kernels.cu:138-222 (rmsnorm_backward_vec8_kernel): with r the saved rsqrt,
    dx = r w dy - x r^3 mean(dy x w), dw = sum_rows dy x r."""
    dy, x, w = _f64(dy), _f64(x), _f64(w)
    r = _f64(rsq).reshape(-1, 1)
    dim = x.shape[-1]
    dy2, x2 = dy.reshape(-1, dim), x.reshape(-1, dim)
    tot = (dy2 * x2 * w).sum(-1, keepdims=True)
    dx = r * w * dy2 - x2 * r ** 3 * tot / dim
    dw = (dy2 * x2 * r).sum(0)
    return dx.reshape(x.shape), dw


def qk_rmsnorm_rope_bwd(dy, x, w, rsq, cos, sin):
    """csrc/kernels.cu:2638-2714 (qk_rmsnorm_rope_backward_kernel). dy, x: [B,H,T,64];
    w: [H,64]; rsq: [B*H*T]; cos, sin: [T,32]. The rotation's transpose takes dy back to
    the normed vector n = x r w, then the RMSNorm adjoint per (b, h, t)."""
    dy, x, w = _f64(dy), _f64(x), _f64(w)
    B, H, T, _ = x.shape
    r = _f64(rsq).reshape(B, H, T, 1)
    c = _f64(cos)[None, None]
    s = _f64(sin)[None, None]
    lo, hi = dy[..., :32], dy[..., 32:]
    dn = np.concatenate([lo * c + hi * s, hi * c - lo * s], axis=-1)
    wb = w[None, :, None, :]
    tot = (dn * x * wb).sum(-1, keepdims=True)
    dx = r * wb * dn - x * r ** 3 * tot / 64.0
    dw = (dn * x * r).sum(axis=(0, 2))
    return dx, dw


def attn_gate_bwd(grad_out, attn, gate_logits):
    """csrc/kernels.cu:2879-2928: out[b,t,h] = attn[b,h,t] sigmoid(l[b,t,h]);
    d_attn = grad g, d_l = <grad, attn> g (1 - g)."""
    a = _f64(attn)
    B, H, T, D = a.shape
    go = _f64(grad_out).reshape(B, T, H, D).transpose(0, 2, 1, 3)
    g = 1.0 / (1.0 + np.exp(-_f64(gate_logits)))  # [B,T,H]
    gh = g.transpose(0, 2, 1)[..., None]
    d_attn = go * gh
    dot = (go * a).sum(-1).transpose(0, 2, 1)
    return d_attn, dot * g * (1.0 - g)


def swiglu_bwd(dout, gu, d_ff):
    """csrc/kernels.cu:747-823: out = silu(gate) up; d_gate = dout up s (1 + gate (1 - s)),
    d_up = dout silu(gate)."""
    gu = _f64(gu)
    d = _f64(dout)
    gt, up = gu[..., :d_ff], gu[..., d_ff:]
    s = 1.0 / (1.0 + np.exp(-gt))
    return np.concatenate([d * up * s * (1.0 + gt * (1.0 - s)), d * gt * s], axis=-1)


def _kept(e, sl, E, C):
    return 0 <= e < E and 0 <= sl < C


def dispatch_bwd(dei, idx, slots, N, D):
    """csrc/kernels.cu:1357-1397: dx[t] = sum over t's kept assignments of
    d_expert_inputs[e, slot], in top-k order."""
    dei = _f64(dei)
    E, C, _ = dei.shape
    idx, slots = np.asarray(idx), np.asarray(slots)
    dx = np.zeros((N, D))
    for t in range(N):
        for k in range(idx.shape[1]):
            e, sl = int(idx[t, k]), int(slots[t, k])
            if _kept(e, sl, E, C):
                dx[t] += dei[e, sl]
    return dx


def combine_bwd(dout, eo, idx, w, slots):
    """csrc/kernels.cu:1454-1546: d_eo[e_k, slot_k] = w[t,k] dout[t],
    d_w[t,k] = <dout[t], eo[e_k, slot_k]>; dropped assignments: d_w = 0, no d_eo write;
    rows no assignment names stay 0."""
    dout, eo, w = _f64(dout), _f64(eo), _f64(w)
    E, C, _ = eo.shape
    idx, slots = np.asarray(idx), np.asarray(slots)
    N, K = idx.shape
    deo = np.zeros_like(eo)
    dw = np.zeros((N, K))
    for t in range(N):
        for k in range(K):
            e, sl = int(idx[t, k]), int(slots[t, k])
            if _kept(e, sl, E, C):
                deo[e, sl] = w[t, k] * dout[t]
                dw[t, k] = dout[t] @ eo[e, sl]
    return deo, dw


def router_bwd(dtw, logits, idx, z_loss_weight, d_z_loss=None, d_probs_mean=None):
    """csrc/kernels.cu:2274-2415 (moe_router_topk_backward_kernel), the forward's selection
    held fixed. c = l - mean(l), s = sigmoid(c), w_k = s_k / (sum_top s + 1e-6),
    z = zw mean_t lse(c)^2, pm = mean_t s. Per token:
    g = 2 zw dz lse softmax(c) / N + sum_k [e = e_k] (d_k - sum_j d_j w_j) s_k (1 - s_k) / den
        + dpm s (1 - s) / N ; d_l = g - mean(g)."""
    l = _f64(logits)
    d = _f64(dtw)
    idx = np.asarray(idx)
    N, E = l.shape
    c = l - l.mean(-1, keepdims=True)
    s = 1.0 / (1.0 + np.exp(-c))
    g = np.zeros_like(c)
    zeff = float(z_loss_weight) * (1.0 if d_z_loss is None else float(np.asarray(d_z_loss)))
    if zeff > 0:
        m = c.max(-1, keepdims=True)
        ex = np.exp(c - m)
        se = ex.sum(-1, keepdims=True)
        lse = m + np.log(se)
        g += 2.0 * zeff * lse / N * ex / se
    u = np.take_along_axis(s, idx, axis=-1)
    den = u.sum(-1, keepdims=True) + 1e-6
    dbar = (d * u).sum(-1, keepdims=True) / den
    du = (d - dbar) / den * u * (1.0 - u)
    for k in range(idx.shape[1]):
        np.add.at(g, (np.arange(N), idx[:, k]), du[:, k])
    if d_probs_mean is not None:
        g += _f64(d_probs_mean)[None] / N * s * (1.0 - s)
    return g - g.mean(-1, keepdims=True)


def conv_k4_bwd(dout, x, w):
    """csrc/kernels.cu:3508-3651: y_t = x_t + sum_k w[d,k] x_{t-k} (k = 0..3, within each
    batch row); dx_t = dout_t + sum_k w[d,k] dout_{t+k}, dw[d,k] = sum_{b,t} dout_t x_{t-k}."""
    dout, x, w = _f64(dout), _f64(x), _f64(w)
    B, T, D = x.shape
    dx = dout.copy()
    dw = np.zeros((D, 4))
    for k in range(4):
        if k < T:
            dx[:, : T - k] += w[:, k] * dout[:, k:]
            dw[:, k] = (dout[:, k:] * x[:, : T - k]).sum(axis=(0, 1))
    return dx, dw
