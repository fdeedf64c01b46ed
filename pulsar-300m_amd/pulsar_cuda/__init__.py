"""Drop-in ``pulsar_cuda`` module backed by libpulsar_hip.so (gfx950 HIP kernels).

Function names, argument order, defaults, return structures and error behaviour follow the
reference's pybind module (csrc/pulsar_cuda.cpp:201-280): inputs are torch tensors on the
GPU, outputs are new tensors allocated on the input's device, invalid arguments raise
RuntimeError (the reference's TORCH_CHECK). Work is enqueued on torch's current stream.
Beyond the reference, every op also accepts fp32 activations.

The forward ops of the decode path and the backward ops of the training path through
model.forward are provided; the loss (softcapped cross-entropy) and optimizer ops are not
part of this module.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import PULSAR_BF16, PULSAR_F32

__all__ = [
    "rmsnorm_forward", "rope_forward", "qk_rmsnorm_rope_forward", "fused_attn_gate_forward",
    "causal_depthwise_conv1d_k4_forward", "fused_swiglu_forward", "moe_router_topk_forward",
    "moe_dispatch_forward", "moe_combine_forward", "moe_slots_from_order",
    "rmsnorm_backward", "qk_rmsnorm_rope_backward", "fused_attn_gate_backward",
    "causal_depthwise_conv1d_k4_backward", "fused_swiglu_backward", "moe_router_topk_backward",
    "moe_dispatch_backward", "moe_combine_backward",
]

_LIB = _lib.load()


def _stream(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def _dtype_code(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.bfloat16:
        return PULSAR_BF16
    if t.dtype == torch.float32:
        return PULSAR_F32
    raise RuntimeError(f"{what} must be bfloat16 or float32, got {t.dtype}")


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _cuda(t: torch.Tensor, name: str) -> None:
    _req(isinstance(t, torch.Tensor) and t.is_cuda, f"{name} must be a CUDA tensor")


def _p(t):
    return None if t is None else t.data_ptr()


def rmsnorm_forward(x: torch.Tensor, weight: torch.Tensor, eps: float):
    """(y, rsqrt) with y = x * rsqrt(mean(x^2) + eps) * w (csrc/kernels.cu:224-266)."""
    _cuda(x, "x")
    _req(x.is_contiguous(), "x must be a contiguous CUDA tensor")
    _req(weight.dtype == torch.float32, "weight must be float32")
    code = _dtype_code(x, "x")
    dim = x.shape[-1]
    rows = x.numel() // dim if dim else 0
    y = torch.empty_like(x)
    rs = torch.empty(rows, dtype=torch.float32, device=x.device)
    wc = weight.contiguous()
    if rows:
        _lib.check(_LIB.pulsar_rmsnorm_forward(_p(x), _p(wc), _p(y), _p(rs), rows,
                                               dim, float(eps), code, _stream(x)))
    return y, rs


def rope_forward(qk: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of a contiguous [B, H, T, hd] tensor (csrc/kernels.cu:935-965)."""
    _cuda(qk, "qk")
    _req(qk.is_contiguous(), "qk must be a contiguous CUDA tensor")
    code = _dtype_code(qk, "qk")
    out = torch.empty_like(qk)
    if qk.numel() == 0:
        return out
    B, H, T, hd = qk.shape
    cf = cos.float().contiguous()
    sf = sin.float().contiguous()
    _lib.check(_LIB.pulsar_rope_forward(_p(qk), _p(out), _p(cf), _p(sf), B * H * T, T, hd, code,
                                        _stream(qk)))
    return out


def qk_rmsnorm_rope_forward(x: torch.Tensor, weight: torch.Tensor, cos: torch.Tensor,
                            sin: torch.Tensor, T: int, eps: float = 1e-6):
    """Per-head RMSNorm then RoPE; stride-aware input, contiguous output
    (csrc/kernels.cu:2716-2765). Returns (y, rsqrt)."""
    head_dim = x.shape[-1]
    _req(head_dim == 64, f"qk_rmsnorm_rope requires head_dim == 64, got {head_dim}")
    _req(x.stride(-1) == 1, f"qk_rmsnorm_rope requires stride(-1) == 1, got {x.stride(-1)}")
    _cuda(x, "x")
    code = _dtype_code(x, "x")
    _req(weight.dtype == torch.float32 and weight.is_contiguous(), "weight must be contiguous float32")
    H = weight.shape[0]
    n = x.numel() // head_dim
    if x.dim() == 4:
        sB, sH, sT = x.stride(0), x.stride(1), x.stride(2)
    else:
        sB, sH, sT = H * T * 64, T * 64, 64
    B = n // (H * T) if H * T else 0
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rs = torch.empty(n, dtype=torch.float32, device=x.device)
    if n:
        cf = cos.float().contiguous()
        sf = sin.float().contiguous()
        _lib.check(_LIB.pulsar_qk_rmsnorm_rope_forward(
            _p(x), sB, sH, sT, B, H, T, head_dim, _p(weight), _p(cf), _p(sf), _p(y), _p(rs),
            float(eps), code, _stream(x)))
    return y, rs


def fused_attn_gate_forward(attn_out: torch.Tensor, gate_logits: torch.Tensor) -> torch.Tensor:
    """out[b,t,h,:] = attn[b,h,t,:] * sigmoid(gate[b,t,h]) as [B, T, H*64]
    (csrc/kernels.cu:2930-2958)."""
    B, H, T, D = attn_out.shape
    _req(D == 64, f"fused_attn_gate requires head_dim == 64, got {D}")
    _cuda(attn_out, "attn_out")
    _req(attn_out.is_contiguous(), "attn_out must be contiguous CUDA")
    code = _dtype_code(attn_out, "attn_out")
    gl = gate_logits.float().contiguous()
    out = torch.empty((B, T, H * D), dtype=attn_out.dtype, device=attn_out.device)
    if out.numel():
        _lib.check(_LIB.pulsar_fused_attn_gate_forward(_p(attn_out), _p(gl), _p(out), B, H, T, D,
                                                       code, _stream(attn_out)))
    return out


def causal_depthwise_conv1d_k4_forward(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """y = x + sum_k w[:,k] * x[t-k] within each batch row (csrc/kernels.cu:3653-3691)."""
    _cuda(x, "x")
    _req(x.is_contiguous(), "x must be contiguous")
    _req(weight.is_contiguous(), "weight must be contiguous")
    _req(weight.dtype == torch.float32, "weight must be float32")
    _req(x.dim() == 3, "x must be [B, T, D]")
    _req(weight.dim() == 2 and weight.shape[1] == 4, "weight must be [D, 4]")
    B, T, D = x.shape
    _req(weight.shape[0] == D, "weight dim 0 must match D")
    code = _dtype_code(x, "x")
    y = torch.empty_like(x)
    if y.numel():
        _lib.check(_LIB.pulsar_causal_conv1d_k4_forward(_p(x), _p(weight), _p(y), B, T, D, code,
                                                         _stream(x)))
    return y


def fused_swiglu_forward(gu: torch.Tensor, d_ff: int) -> torch.Tensor:
    """silu(gu[..., :d_ff]) * gu[..., d_ff:] in fp32 (csrc/kernels.cu:825-863)."""
    _cuda(gu, "gu")
    _req(gu.is_contiguous(), "gu must be a contiguous CUDA tensor")
    code = _dtype_code(gu, "gu")
    out = torch.empty(*gu.shape[:-1], d_ff, dtype=gu.dtype, device=gu.device)
    rows = gu.numel() // (2 * d_ff) if d_ff else 0
    if rows:
        _lib.check(_LIB.pulsar_fused_swiglu_forward(_p(gu), _p(out), rows, d_ff, code, _stream(gu)))
    return out


def moe_router_topk_forward(logits: torch.Tensor, expert_bias: torch.Tensor, top_k=2,
                            z_loss_weight: float = 1e-4):
    """(topk_idx int64, topk_weights bf16, z_loss, probs_mean); also the reference's 3-argument
    overload (logits, expert_bias, z_loss_weight) with top_k = 2 (csrc/pulsar_cuda.cpp:255-266)."""
    if isinstance(top_k, float):
        z_loss_weight, top_k = top_k, 2
    _cuda(logits, "logits")
    _cuda(expert_bias, "expert_bias")
    _req(logits.is_contiguous(), "logits must be contiguous")
    _req(expert_bias.is_contiguous(), "expert_bias must be contiguous")
    _req(logits.dim() == 2, "logits must be 2D [N, E]")
    N, E = logits.shape
    _req(E <= 32, f"moe_router_topk_forward_cuda supports E <= 32, got {E}")
    _req(0 < top_k <= 8 and top_k <= E, f"top_k must be in [1, min(8, E)], got {top_k}")
    _req(expert_bias.shape[0] == E, "expert_bias size must match E")
    _req(logits.dtype in (torch.float32, torch.bfloat16), "logits must be float32 or bfloat16")
    _req(expert_bias.dtype == torch.float32, "expert_bias must be float32")
    dev = logits.device
    idx = torch.empty((N, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((N, top_k), dtype=torch.bfloat16, device=dev)
    z = torch.zeros((), dtype=torch.float32, device=dev)
    pm = torch.zeros(E, dtype=torch.float32, device=dev)
    # per-workgroup partial statistics (merged in a fixed order inside the library)
    ws = torch.empty(max(1, _LIB.pulsar_moe_router_workspace_bytes(N, E) // 4),
                     dtype=torch.float32, device=dev)
    _lib.check(_LIB.pulsar_moe_router_topk_forward_ws(
        _p(logits), _dtype_code(logits, "logits"), _p(expert_bias), _p(idx), _p(w), _p(z), _p(pm),
        N, E, top_k, float(z_loss_weight), _p(ws), _stream(logits)))
    return idx, w, z, pm


def moe_dispatch_forward(x: torch.Tensor, topk_idx: torch.Tensor, token_to_slot: torch.Tensor,
                         num_experts: int, capacity: int, expert_counts=None):
    """Scatter token rows into [E, C, D] slots; returns a one-element list
    (csrc/kernels.cu:1548-1605)."""
    for t, n in ((x, "x"), (topk_idx, "topk_idx"), (token_to_slot, "token_to_slot")):
        _cuda(t, n)
        _req(t.is_contiguous(), f"{n} must be contiguous")
    _req(topk_idx.dtype == torch.int64, "topk_idx must be int64")
    _req(token_to_slot.dtype == torch.int32, "token_to_slot must be int32")
    N, D = x.shape
    K = topk_idx.shape[1]
    _req(tuple(token_to_slot.shape) == (N, K), "token_to_slot must be [N, K]")
    _req(D % 8 == 0, f"D must be a multiple of 8 for vectorised dispatch, got {D}")
    if expert_counts is not None:
        _cuda(expert_counts, "expert_counts")
        _req(expert_counts.dtype == torch.int64, "expert_counts must be int64")
        _req(expert_counts.numel() >= num_experts, "expert_counts must have at least E elements")
    code = _dtype_code(x, "x")
    out = torch.empty((num_experts, capacity, D), dtype=x.dtype, device=x.device)
    _lib.check(_LIB.pulsar_moe_dispatch_forward(
        _p(x), _p(topk_idx), _p(token_to_slot), _p(expert_counts), _p(out), N, D, K, num_experts,
        capacity, code, _stream(x)))
    return [out]


def moe_combine_forward(expert_outputs: torch.Tensor, topk_idx: torch.Tensor,
                        topk_weights: torch.Tensor, token_to_slot: torch.Tensor, shared_out=None):
    """out[t] = shared[t] + sum_k w[t,k] * expert_out[e, slot] (csrc/kernels.cu:1633-1664).

    The reference reads these through typed data_ptr calls, which raise on a wrong dtype;
    here every operand the kernel dereferences is checked before the launch."""
    for t, n in ((expert_outputs, "expert_outputs"), (topk_idx, "topk_idx"),
                 (topk_weights, "topk_weights"), (token_to_slot, "token_to_slot")):
        _cuda(t, n)
        _req(t.device == expert_outputs.device, f"{n} must be on the device of expert_outputs")
    _req(expert_outputs.dim() == 3, "expert_outputs must be [E, C, D]")
    _req(topk_idx.dim() == 2, "topk_idx must be [N, K]")
    _req(topk_idx.dtype == torch.int64, "topk_idx must be int64")
    _req(token_to_slot.dtype == torch.int32, "token_to_slot must be int32")
    E, C, D = expert_outputs.shape
    N, K = topk_idx.shape
    _req(tuple(token_to_slot.shape) == (N, K), "token_to_slot must be [N, K]")
    _req(tuple(topk_weights.shape) == (N, K), "topk_weights must be [N, K]")
    code = _dtype_code(expert_outputs, "expert_outputs")
    if shared_out is not None and shared_out.numel():
        _cuda(shared_out, "shared_out")
        _req(shared_out.device == expert_outputs.device,
             "shared_out must be on the device of expert_outputs")
        _req(shared_out.dtype == expert_outputs.dtype,
             "shared_out must have the dtype of expert_outputs")
        _req(shared_out.numel() == N * D and shared_out.shape[-1] == D,
             "shared_out must be [N, D]")
    w = topk_weights.to(torch.bfloat16).contiguous()
    sh = shared_out.contiguous() if shared_out is not None and shared_out.numel() else None
    out = torch.empty((N, D), dtype=expert_outputs.dtype, device=expert_outputs.device)
    eo = expert_outputs.contiguous()
    ti = topk_idx.contiguous()
    ts = token_to_slot.contiguous()
    if N:
        _lib.check(_LIB.pulsar_moe_combine_forward(
            _p(eo), _p(ti), _p(w), _p(ts), _p(sh), _p(out), N, D, K, E, C, code,
            _stream(expert_outputs)))
    return out


def moe_slots_from_order(flat_e: torch.Tensor, order: torch.Tensor, num_experts: int,
                         capacity: int):
    """(slots int32 [M], counts int64 [E]): rank within expert in `order`, -1 when >= capacity
    (csrc/kernels.cu:3058-3095)."""
    _cuda(flat_e, "flat_e")
    _req(flat_e.is_contiguous(), "flat_e must be contiguous CUDA")
    _req(flat_e.dtype == torch.int64, "flat_e must be int64")
    _req(order.is_cuda and order.is_contiguous(), "order must be contiguous CUDA")
    _req(order.device == flat_e.device, "order must be on the device of flat_e")
    _req(order.numel() == flat_e.numel(), "order must have as many elements as flat_e")
    M = flat_e.numel()
    slots = torch.empty(M, dtype=torch.int32, device=flat_e.device)
    counts = torch.zeros(num_experts, dtype=torch.int64, device=flat_e.device)
    order64 = order.to(torch.int64)
    _lib.check(_LIB.pulsar_moe_slots_from_order(_p(flat_e), _p(order64), _p(slots),
                                                _p(counts), M, num_experts, capacity,
                                                _stream(flat_e)))
    return slots, counts


# ---------------------------------------------------------------------------
# Backward ops (training path)
# ---------------------------------------------------------------------------

def _same_code(a: torch.Tensor, b: torch.Tensor, na: str, nb: str) -> int:
    code = _dtype_code(a, na)
    _req(b.dtype == a.dtype, f"{nb} must have the dtype of {na}")
    return code


def rmsnorm_backward(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                     rsqrt: torch.Tensor):
    """[dx, dweight] of rmsnorm_forward given its saved rsqrt (csrc/kernels.cu:268-310)."""
    _cuda(x, "x")
    _cuda(dy, "dy")
    _req(x.is_contiguous(), "x must be a contiguous CUDA tensor")
    _req(weight.dtype == torch.float32, "weight must be float32")
    code = _same_code(x, dy, "x", "dy")
    dim = x.shape[-1]
    rows = x.numel() // dim if dim else 0
    dx = torch.empty_like(x)
    dw = torch.zeros_like(weight)
    if rows == 0:
        return [dx, dw]
    _req(dim <= 8192, f"rmsnorm backward supports dim <= 8192, got dim {dim}")
    dyc = dy.contiguous()
    rs = rsqrt.float().contiguous()
    _lib.check(_LIB.pulsar_rmsnorm_backward(_p(dyc), _p(x), _p(weight.contiguous()), _p(rs),
                                            _p(dx), _p(dw), rows, dim, code, _stream(x)))
    return [dx, dw]


def qk_rmsnorm_rope_backward(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                             rsqrt_in: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                             T: int):
    """[dx, dweight] of qk_rmsnorm_rope_forward (csrc/kernels.cu:2767-2835). dx takes the
    layout of a [B,T,H,64] buffer seen as [B,H,T,64] when x is such a view (head stride
    below time stride), else x's shape, contiguous."""
    head_dim = x.shape[-1]
    _req(head_dim == 64, f"qk_rmsnorm_rope requires head_dim == 64, got {head_dim}")
    _cuda(dy, "dy")
    _req(dy.is_contiguous(), "dy must be contiguous CUDA")
    _cuda(x, "x")
    _req(x.stride(-1) == 1, "x must have stride(-1) == 1")
    code = _same_code(x, dy, "x", "dy")
    _req(weight.is_cuda and weight.is_contiguous(), "weight must be contiguous CUDA")
    _req(weight.dtype == torch.float32, "weight must be float32")
    H = weight.shape[0]
    n = x.numel() // head_dim
    if x.dim() == 4:
        sB, sH, sT = x.stride(0), x.stride(1), x.stride(2)
    else:
        sB, sH, sT = H * T * 64, T * 64, 64
    B = n // (H * T) if H * T else 0
    if sH < sT and T > 1:
        dx = torch.empty((B, T, H, 64), dtype=x.dtype, device=x.device).transpose(1, 2)
        dB, dH, dT = dx.stride(0), dx.stride(1), dx.stride(2)
    else:
        dx = torch.empty_like(x, memory_format=torch.contiguous_format)
        if dx.dim() == 4:
            dB, dH, dT = dx.stride(0), dx.stride(1), dx.stride(2)
        else:
            dB, dH, dT = H * T * 64, T * 64, 64
    dw = torch.zeros_like(weight)
    if n:
        cf = cos.float().contiguous()
        sf = sin.float().contiguous()
        rs = rsqrt_in.float().contiguous()
        _lib.check(_LIB.pulsar_qk_rmsnorm_rope_backward(
            _p(dy), _p(x), sB, sH, sT, _p(dx), dB, dH, dT, B, H, T, head_dim, _p(weight), _p(rs),
            _p(cf), _p(sf), _p(dw), code, _stream(x)))
    return [dx, dw]


def fused_attn_gate_backward(grad_out: torch.Tensor, attn_out: torch.Tensor,
                             gate_logits: torch.Tensor):
    """[d_attn_out, d_gate_logits] of fused_attn_gate_forward (csrc/kernels.cu:2960-2992);
    d_gate_logits in gate_logits' dtype."""
    B, H, T, D = attn_out.shape
    _req(D == 64, f"fused_attn_gate requires head_dim == 64, got {D}")
    _cuda(grad_out, "grad_out")
    _req(grad_out.is_contiguous(), "grad_out must be contiguous CUDA")
    _cuda(attn_out, "attn_out")
    _req(attn_out.is_contiguous(), "attn_out must be contiguous CUDA")
    code = _same_code(attn_out, grad_out, "attn_out", "grad_out")
    gl = gate_logits.float().contiguous()
    d_attn = torch.empty_like(attn_out)
    d_gate = torch.empty((B, T, H), dtype=torch.float32, device=attn_out.device)
    if d_attn.numel():
        _lib.check(_LIB.pulsar_fused_attn_gate_backward(_p(grad_out), _p(attn_out), _p(gl),
                                                        _p(d_attn), _p(d_gate), B, H, T, D, code,
                                                        _stream(attn_out)))
    return [d_attn, d_gate.to(gate_logits.dtype)]


def causal_depthwise_conv1d_k4_backward(dout: torch.Tensor, x: torch.Tensor,
                                        weight: torch.Tensor):
    """[dx, dweight] of causal_depthwise_conv1d_k4_forward (csrc/kernels.cu:3693-3732)."""
    _req(dout.is_cuda and x.is_cuda and weight.is_cuda, "Inputs must be CUDA tensors")
    _req(dout.is_contiguous() and x.is_contiguous() and weight.is_contiguous(),
         "Inputs must be contiguous")
    code = _same_code(x, dout, "x", "dout")
    _req(weight.dtype == torch.float32, "weight must be float32")
    B, T, D = x.shape
    dx = torch.empty_like(x)
    dw = torch.zeros_like(weight)
    if B * T == 0:
        return [dx, dw]
    _lib.check(_LIB.pulsar_causal_conv1d_k4_backward(_p(dout), _p(x), _p(weight), _p(dx), _p(dw),
                                                      B, T, D, code, _stream(x)))
    return [dx, dw]


def fused_swiglu_backward(dout: torch.Tensor, gu: torch.Tensor, d_ff: int) -> torch.Tensor:
    """dgu = [d_gate | d_up] of fused_swiglu_forward (csrc/kernels.cu:865-900)."""
    _cuda(gu, "gu")
    _req(gu.is_contiguous(), "gu must be a contiguous CUDA tensor")
    _req(dout.is_contiguous(), "dout must be contiguous")
    code = _same_code(gu, dout, "gu", "dout")
    dgu = torch.empty_like(gu)
    rows = gu.numel() // (2 * d_ff) if d_ff else 0
    if rows:
        _lib.check(_LIB.pulsar_fused_swiglu_backward(_p(dout), _p(gu), _p(dgu), rows, d_ff, code,
                                                     _stream(gu)))
    return dgu


def moe_router_topk_backward(d_topk_weights: torch.Tensor, logits: torch.Tensor,
                             topk_idx: torch.Tensor, z_loss_weight: float = 1e-4,
                             d_z_loss=None, d_probs_mean=None) -> torch.Tensor:
    """d_logits of moe_router_topk_forward with the selection held fixed
    (csrc/kernels.cu:2493-2578)."""
    for t, n in ((d_topk_weights, "d_topk_weights"), (logits, "logits"), (topk_idx, "topk_idx")):
        _cuda(t, n)
        _req(t.is_contiguous(), f"{n} must be contiguous")
    _req(d_topk_weights.dtype == torch.bfloat16, "d_topk_weights must be bfloat16")
    _req(topk_idx.dtype == torch.int64, "topk_idx must be int64")
    _req(logits.dtype in (torch.float32, torch.bfloat16), "logits must be float32 or bfloat16")
    N, E = logits.shape
    K = topk_idx.shape[1]
    _req(E <= 32, f"moe_router_topk_backward_cuda supports E <= 32, got {E}")
    _req(0 < K <= 8 and K <= E, f"top_k must be in [1, min(8, E)], got {K}")
    _req(tuple(d_topk_weights.shape) == (N, K), "d_topk_weights shape mismatch")
    if d_z_loss is not None:
        _cuda(d_z_loss, "d_z_loss")
        _req(d_z_loss.dtype == torch.float32, "d_z_loss must be float32")
    if d_probs_mean is not None:
        _cuda(d_probs_mean, "d_probs_mean")
        _req(d_probs_mean.dtype == torch.float32, "d_probs_mean must be float32")
        _req(d_probs_mean.numel() == E, "d_probs_mean numel must match E")
        d_probs_mean = d_probs_mean.contiguous()
    d_logits = torch.empty_like(logits)
    if N:
        _lib.check(_LIB.pulsar_moe_router_topk_backward(
            _p(d_topk_weights), _p(logits), _dtype_code(logits, "logits"), _p(topk_idx),
            float(z_loss_weight), _p(d_z_loss), _p(d_probs_mean), _p(d_logits), N, E, K,
            _stream(logits)))
    return d_logits


def moe_dispatch_backward(d_expert_inputs: torch.Tensor, topk_idx: torch.Tensor,
                          token_to_slot: torch.Tensor, N: int, D: int) -> torch.Tensor:
    """dx [N, D]: per token, the sum of its kept slots' gradients (csrc/kernels.cu:1607-1631)."""
    for t, n in ((d_expert_inputs, "d_expert_inputs"), (topk_idx, "topk_idx"),
                 (token_to_slot, "token_to_slot")):
        _cuda(t, n)
        _req(t.is_contiguous(), f"{n} must be contiguous")
    _req(topk_idx.dtype == torch.int64, "topk_idx must be int64")
    _req(token_to_slot.dtype == torch.int32, "token_to_slot must be int32")
    E, C, D_ = d_expert_inputs.shape
    _req(D_ == D, "d_expert_inputs last dimension must be D")
    K = topk_idx.shape[1]
    code = _dtype_code(d_expert_inputs, "d_expert_inputs")
    dx = torch.empty((N, D), dtype=d_expert_inputs.dtype, device=d_expert_inputs.device)
    if N:
        _lib.check(_LIB.pulsar_moe_dispatch_backward(
            _p(d_expert_inputs), _p(topk_idx), _p(token_to_slot), _p(dx), N, D, K, E, C, code,
            _stream(d_expert_inputs)))
    return dx


def moe_combine_backward(d_routed_out: torch.Tensor, expert_outputs: torch.Tensor,
                         topk_idx: torch.Tensor, topk_weights: torch.Tensor,
                         token_to_slot: torch.Tensor, expert_counts=None):
    """[d_expert_outputs, d_topk_weights] of moe_combine_forward (csrc/kernels.cu:1666-1711).
    expert_counts is accepted for signature parity: every slot a kept assignment does not
    name is zeroed either way."""
    E, C, D = expert_outputs.shape
    N, K = topk_idx.shape
    for t, n in ((d_routed_out, "d_routed_out"), (expert_outputs, "expert_outputs"),
                 (topk_idx, "topk_idx"), (token_to_slot, "token_to_slot")):
        _cuda(t, n)
        _req(t.is_contiguous(), f"{n} must be contiguous")
    _req(topk_idx.dtype == torch.int64, "topk_idx must be int64")
    _req(token_to_slot.dtype == torch.int32, "token_to_slot must be int32")
    _req(tuple(token_to_slot.shape) == (N, K), "token_to_slot must be [N, K]")
    _req(tuple(topk_weights.shape) == (N, K), "topk_weights must be [N, K]")
    _req(d_routed_out.numel() == N * D, "d_routed_out must be [N, D]")
    if expert_counts is not None:
        _cuda(expert_counts, "expert_counts")
        _req(expert_counts.dtype == torch.int64, "expert_counts must be int64")
        _req(expert_counts.numel() >= E, "expert_counts must have at least E elements")
    code = _same_code(expert_outputs, d_routed_out, "expert_outputs", "d_routed_out")
    w = topk_weights.to(torch.bfloat16).contiguous()
    d_eo = torch.empty_like(expert_outputs)
    d_w = torch.empty((N, K), dtype=torch.bfloat16, device=expert_outputs.device)
    _lib.check(_LIB.pulsar_moe_combine_backward(
        _p(d_routed_out), _p(expert_outputs), _p(topk_idx), _p(w), _p(token_to_slot), _p(d_eo),
        _p(d_w), N, D, K, E, C, code, _stream(expert_outputs)))
    return [d_eo, d_w.to(topk_weights.dtype)]
