// Backward ops of the pulsar_cuda surface (the reference's training path through
// model.forward), written for gfx950 (wave64). Each is the exact gradient of the matching
// forward op, in fp32 arithmetic with outputs in the reference's dtypes: activations in the
// activation dtype, norm / conv weights in fp32. Weight gradients are summed with fp32
// atomics (one per element per workgroup), so their rounding depends on scheduling order,
// as the reference's does.
#include <algorithm>
#include <string>

#include "common.h"

namespace pulsar {

namespace {

__global__ void fill_f32_kernel(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

template <typename T>
__global__ void fill_zero_kernel(T* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = from_f<T>(0.f);
}

#define PULSAR_TRY_STATUS(expr)     \
  do {                              \
    const int _st = (expr);         \
    if (_st != PULSAR_OK) return _st; \
  } while (0)

int zero_f32(float* p, int64_t n, hipStream_t s) {
  if (n <= 0) return PULSAR_OK;
  fill_f32_kernel<<<blocks_for(n, 256), 256, 0, s>>>(p, n);
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

// ---------------------------------------------------------------------------
// RMSNorm: y = w * x * r, r = rsqrt(mean(x^2) + eps) (saved by the forward).
//   dx = r * w * dy - x * r^3 * sum(dy * x * w) / D ;  dw = sum_rows dy * x * r
// Workgroups stride over rows; a thread keeps its columns' dw partials in registers
// (D <= 256 * kNormCols) and adds them once.
// ---------------------------------------------------------------------------
constexpr int kNormCols = 32;

template <typename T>
__global__ void __launch_bounds__(256) rmsnorm_bwd_kernel(const T* __restrict__ dy,
                                                          const T* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ rsq,
                                                          T* __restrict__ dx,
                                                          float* __restrict__ dw, int64_t rows,
                                                          int dim) {
  __shared__ float red[16];
  float acc[kNormCols];
#pragma unroll
  for (int j = 0; j < kNormCols; ++j) acc[j] = 0.f;
  const float inv_dim = 1.0f / (float)dim;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* dyr = dy + row * dim;
    const T* xr = x + row * dim;
    const float r = rsq[row];
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < kNormCols; ++j) {
      const int i = threadIdx.x + j * 256;
      if (i < dim) {
        const float g = to_f(dyr[i]), xv = to_f(xr[i]);
        part += g * xv * w[i];
        acc[j] += g * xv * r;
      }
    }
    const float tot = block_sum(part, red);
    const float c = r * r * r * tot * inv_dim;
#pragma unroll
    for (int j = 0; j < kNormCols; ++j) {
      const int i = threadIdx.x + j * 256;
      if (i < dim) dx[row * dim + i] = from_f<T>(r * w[i] * to_f(dyr[i]) - to_f(xr[i]) * c);
    }
    __syncthreads();  // red is reused by the next row's sum
  }
#pragma unroll
  for (int j = 0; j < kNormCols; ++j) {
    const int i = threadIdx.x + j * 256;
    if (i < dim) atomicAdd(&dw[i], acc[j]);
  }
}

// ---------------------------------------------------------------------------
// QK RMSNorm + RoPE (head_dim 64): y = rope(n), n = x * r * w[h]. One wave per vector.
//   dn = rope^T(dy) (rotation by -theta: dn_i = dy_i c + dy_{i+32} s,
//        dn_{i+32} = dy_{i+32} c - dy_i s)
//   dx = r * w * dn - x * r^3 * sum(dn * x * w) / 64 ;  dw[h] = sum dn * x * r
// Grid (workgroups per head, H): the waves of head h stride over its B*T vectors, keep
// their dw partial in a register and add it once.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) qk_norm_rope_bwd_kernel(
    const T* __restrict__ dy, const T* __restrict__ x, int64_t sB, int64_t sH, int64_t sT,
    int64_t dB, int64_t dH, int64_t dT, int H, int T_, int64_t per_head,
    const float* __restrict__ w, const float* __restrict__ rsq, const float* __restrict__ cs,
    const float* __restrict__ sn, T* __restrict__ dx, float* __restrict__ dw) {
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x / 64);
  const int j = lane & 31;
  const float wv = w[h * 64 + lane];
  float dwacc = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); i < per_head;
       i += nwaves) {
    const int64_t b = i / T_;
    const int t = (int)(i % T_);
    const int64_t v = (b * H + h) * T_ + t;  // vector index in [B, H, T] order
    const float g = to_f(dy[v * 64 + lane]);
    const float gp = __shfl_xor(g, 32, 64);
    const float c = cs[t * 32 + j], s = sn[t * 32 + j];
    const float dn = lane < 32 ? g * c + gp * s : g * c - gp * s;
    const float xv = to_f(x[b * sB + h * sH + (int64_t)t * sT + lane]);
    const float r = rsq[v];
    const float tot = wave_sum(dn * xv * wv);
    dx[b * dB + h * dH + (int64_t)t * dT + lane] =
        from_f<T>(r * wv * dn - xv * r * r * r * tot * (1.0f / 64.0f));
    dwacc += dn * xv * r;
  }
  atomicAdd(&dw[h * 64 + lane], dwacc);
}

// ---------------------------------------------------------------------------
// Attention gate + transpose: out[b,t,h,d] = a[b,h,t,d] * sigmoid(l[b,t,h]). One wave per
// (b, t, h): d_a = grad * g ; d_l = sum_d(grad * a) * g * (1 - g).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) attn_gate_bwd_kernel(const T* __restrict__ go,
                                                            const T* __restrict__ a,
                                                            const float* __restrict__ gl,
                                                            T* __restrict__ da,
                                                            float* __restrict__ dl, int H,
                                                            int T_, int64_t nvec) {
  const int64_t hv = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (hv >= nvec) return;
  const int lane = threadIdx.x & 63;
  const int h = (int)(hv % H);
  const int t = (int)((hv / H) % T_);
  const int64_t b = hv / ((int64_t)H * T_);
  const int64_t ai = ((b * H + h) * T_ + t) * 64 + lane;
  const float g = sigmoidf_(gl[hv]);
  const float gv = to_f(go[hv * 64 + lane]);
  const float dot = wave_sum(gv * to_f(a[ai]));
  da[ai] = from_f<T>(gv * g);
  if (lane == 0) dl[hv] = dot * g * (1.0f - g);
}

// ---------------------------------------------------------------------------
// SwiGLU: out = silu(gate) * up with gu = [gate | up] per row.
//   d_gate = dout * up * s * (1 + gate * (1 - s)), s = sigmoid(gate) ; d_up = dout * silu(gate)
// ---------------------------------------------------------------------------
template <typename T>
__global__ void swiglu_bwd_kernel(const T* __restrict__ dout, const T* __restrict__ gu,
                                  T* __restrict__ dgu, int64_t d_ff, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t r = i / d_ff, c = i % d_ff;
  const float gt = to_f(gu[r * 2 * d_ff + c]), up = to_f(gu[r * 2 * d_ff + d_ff + c]);
  const float d = to_f(dout[i]);
  const float sg = sigmoidf_(gt);
  dgu[r * 2 * d_ff + c] = from_f<T>(d * up * sg * (1.0f + gt * (1.0f - sg)));
  dgu[r * 2 * d_ff + d_ff + c] = from_f<T>(d * gt * sg);
}

// ---------------------------------------------------------------------------
// MoE dispatch: expert_inputs[e, slot] = x[t] for every kept assignment (e, slot) of t.
//   dx[t] = sum over t's kept assignments, in top-k order, of d_expert_inputs[e, slot]
// ---------------------------------------------------------------------------
template <typename T>
__global__ void dispatch_bwd_kernel(const T* __restrict__ dei, const int64_t* __restrict__ idx,
                                    const int32_t* __restrict__ slots, T* __restrict__ dx,
                                    int64_t D, int K, int64_t E, int64_t C) {
  const int64_t t = blockIdx.x;
  for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f;
    for (int k = 0; k < K; ++k) {
      const int64_t e = idx[t * K + k];
      const int32_t sl = slots[t * K + k];
      if (e >= 0 && e < E && sl >= 0 && sl < C) acc += to_f(dei[(e * C + sl) * D + d]);
    }
    dx[t * D + d] = from_f<T>(acc);
  }
}

// ---------------------------------------------------------------------------
// MoE combine: out[t] = shared[t] + sum_k w[t,k] * eo[e_k, slot_k] (kept assignments).
//   d_eo[e_k, slot_k] = w[t,k] * dout[t] ; d_w[t,k] = sum_d dout[t] * eo[e_k, slot_k]
//   (0 for dropped assignments; rows of d_eo no assignment names stay 0)
// One workgroup per token; the K dot products are reduced over the workgroup.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) combine_bwd_kernel(
    const T* __restrict__ dout, const T* __restrict__ eo, const int64_t* __restrict__ idx,
    const uint16_t* __restrict__ w_bf16, const int32_t* __restrict__ slots, T* __restrict__ deo,
    uint16_t* __restrict__ dw_bf16, int64_t D, int K, int64_t E, int64_t C) {
  __shared__ float red[16];
  const int64_t t = blockIdx.x;
  for (int k = 0; k < K; ++k) {
    const int64_t e = idx[t * K + k];
    const int32_t sl = slots[t * K + k];
    const bool kept = e >= 0 && e < E && sl >= 0 && sl < C;
    float part = 0.f;
    if (kept) {
      const float wk = bf2f(bf16{w_bf16[t * K + k]});
      const int64_t base = (e * C + sl) * D;
      for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
        const float g = to_f(dout[t * D + d]);
        part += g * to_f(eo[base + d]);
        deo[base + d] = from_f<T>(wk * g);
      }
    }
    const float dot = block_sum(part, red);
    if (threadIdx.x == 0) dw_bf16[t * K + k] = f2bf(kept ? dot : 0.f).u;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Router top-k. Forward: c = l - mean(l), s = sigmoid(c), top-k of s + bias (indices given),
// w_k = s_k / (sum_top s + 1e-6); z_loss = zw * mean_tokens(lse(c)^2); probs_mean =
// mean_tokens(s). Backward per token (one thread):
//   g_e = 2 zw dz lse(c) softmax(c)_e / N                      (z-loss)
//       + sum_k [e = e_k] (dw_k - sum_j dw_j w_j) s_k (1 - s_k) / (sum_top s + 1e-6)
//       + dpm_e s_e (1 - s_e) / N                               (probs_mean)
//   d_l = g - mean(g)                                           (centring)
// ---------------------------------------------------------------------------
// EM (16 or 32) >= E register slots in unrolled loops: every register-array index is a
// compile-time constant (runtime indices would move the arrays to scratch memory).
template <typename L, int EM>
__global__ void router_bwd_kernel(const uint16_t* __restrict__ dtw, const L* __restrict__ logits,
                                  const int64_t* __restrict__ idx, L* __restrict__ dl,
                                  float zw, const float* __restrict__ dz,
                                  const float* __restrict__ dpm, int64_t N, int E, int K) {
  const int64_t tok = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tok >= N) return;
  float c[EM], s[EM], g[EM];
  float mean = 0.f;
#pragma unroll
  for (int e = 0; e < EM; ++e) {
    c[e] = e < E ? to_f(logits[tok * E + e]) : 0.f;
    if (e < E) mean += c[e];
  }
  mean /= (float)E;
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < EM; ++e) {
    c[e] -= mean;
    s[e] = sigmoidf_(c[e]);
    if (e < E) mx = fmaxf(mx, c[e]);
    g[e] = 0.f;
  }
  const float zeff = zw * (dz ? dz[0] : 1.0f);
  if (zeff > 0.f) {
    float se = 0.f;
#pragma unroll
    for (int e = 0; e < EM; ++e)
      if (e < E) se += expf(c[e] - mx);
    se = fmaxf(se, 1e-20f);
    const float lse = mx + logf(se);
    const float f = 2.0f * zeff * lse / (float)N;
#pragma unroll
    for (int e = 0; e < EM; ++e) g[e] = f * expf(c[e] - mx) / se;
  }
  float den = 1e-6f, sdu = 0.f;
  int ek[8];
  float d[8], us[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    ek[k] = -1;
    d[k] = us[k] = 0.f;
    if (k >= K) continue;
    ek[k] = (int)idx[tok * K + k];
    d[k] = bf2f(bf16{dtw[tok * K + k]});
    float u = 0.f;
#pragma unroll
    for (int e = 0; e < EM; ++e)
      if (e < E && e == ek[k]) u = s[e];
    us[k] = u;
    den += u;
    sdu += d[k] * u;
  }
  const float dbar = sdu / den;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k >= K) continue;
    const float u = us[k];
    const float add = (d[k] - dbar) / den * u * (1.0f - u);
#pragma unroll
    for (int e = 0; e < EM; ++e)
      if (e < E && e == ek[k]) g[e] += add;
  }
  if (dpm) {
#pragma unroll
    for (int e = 0; e < EM; ++e)
      if (e < E) g[e] += dpm[e] / (float)N * s[e] * (1.0f - s[e]);
  }
  float gm = 0.f;
#pragma unroll
  for (int e = 0; e < EM; ++e)
    if (e < E) gm += g[e];
  gm /= (float)E;
#pragma unroll
  for (int e = 0; e < EM; ++e)
    if (e < E) dl[tok * E + e] = from_f<L>(g[e] - gm);
}

// ---------------------------------------------------------------------------
// Causal depthwise conv k=4 with residual: y_t = x_t + sum_k w[d,k] x_{t-k}.
//   dx_t = dout_t + sum_k w[d,k] dout_{t+k} (t + k < T) ;  dw[d,k] = sum_{b,t} dout_t x_{t-k}
// dw: a thread owns one channel of a chunk of tokens and adds its 4 sums once.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void conv_k4_bwd_dx_kernel(const T* __restrict__ dout, const float* __restrict__ w,
                                      T* __restrict__ dx, int64_t T_, int64_t D,
                                      int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t d = i % D;
  const int64_t t = (i / D) % T_;
  float acc = to_f(dout[i]);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (t + k < T_) acc += w[d * 4 + k] * to_f(dout[i + k * D]);
  dx[i] = from_f<T>(acc);
}

constexpr int kConvChunk = 256;  // tokens per workgroup row of the dw pass

template <typename T>
__global__ void conv_k4_bwd_dw_kernel(const T* __restrict__ dout, const T* __restrict__ x,
                                      float* __restrict__ dw, int64_t T_, int64_t D,
                                      int64_t ntok) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= D) return;
  const int64_t t0 = (int64_t)blockIdx.y * kConvChunk;
  const int64_t t1 = t0 + kConvChunk < ntok ? t0 + kConvChunk : ntok;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t n = t0; n < t1; ++n) {
    const int64_t t = n % T_;  // position within its sequence
    const float g = to_f(dout[n * D + d]);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (t >= k) a[k] += g * to_f(x[(n - k) * D + d]);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) atomicAdd(&dw[d * 4 + k], a[k]);
}

}  // namespace

}  // namespace pulsar

using namespace pulsar;

extern "C" {

int pulsar_rmsnorm_backward(const void* dy, const void* x, const float* w, const float* rsqrt,
                            void* dx, float* dw, int64_t rows, int64_t dim, int dtype,
                            hipStream_t stream) {
  PULSAR_REQUIRE(rows >= 0 && dim > 0, "rmsnorm backward: rows >= 0 and dim > 0 required");
  PULSAR_REQUIRE(dim <= 256 * kNormCols, "rmsnorm backward supports dim <= 8192");
  PULSAR_TRY_STATUS(zero_f32(dw, dim, stream));
  if (rows == 0) return PULSAR_OK;
  PULSAR_REQUIRE(dy && x && w && rsqrt && dx && dw, "rmsnorm backward: null pointer");
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    const unsigned grid = (unsigned)(rows < 1024 ? rows : 1024);
    rmsnorm_bwd_kernel<T><<<grid, 256, 0, stream>>>((const T*)dy, (const T*)x, w, rsqrt, (T*)dx,
                                                    dw, rows, (int)dim);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_qk_rmsnorm_rope_backward(const void* dy, const void* x, int64_t sB, int64_t sH,
                                    int64_t sT, void* dx, int64_t dB, int64_t dH, int64_t dT,
                                    int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                    const float* w, const float* rsqrt, const float* cos,
                                    const float* sin, float* dw, int dtype,
                                    hipStream_t stream) {
  if (head_dim != 64)
    return fail(PULSAR_ERR_INVALID,
                "qk_rmsnorm_rope requires head_dim == 64, got " + std::to_string(head_dim));
  PULSAR_REQUIRE(B >= 0 && H > 0 && T > 0, "qk_rmsnorm_rope backward: bad shape");
  PULSAR_REQUIRE(H <= 65535, "qk_rmsnorm_rope backward: at most 65535 heads");
  PULSAR_TRY_STATUS(zero_f32(dw, H * 64, stream));
  const int64_t per_head = B * T;
  if (per_head == 0) return PULSAR_OK;
  // up to 64 workgroups (256 waves) per head; each wave adds its dw partial once
  const unsigned gx = (unsigned)std::min<int64_t>(64, (per_head + 3) / 4);
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    qk_norm_rope_bwd_kernel<T_><<<dim3(gx, (unsigned)H), 256, 0, stream>>>(
        (const T_*)dy, (const T_*)x, sB, sH, sT, dB, dH, dT, (int)H, (int)T, per_head, w, rsqrt,
        cos, sin, (T_*)dx, dw);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_fused_attn_gate_backward(const void* grad_out, const void* attn,
                                    const float* gate_logits, void* d_attn, float* d_gate,
                                    int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                    int dtype, hipStream_t stream) {
  if (head_dim != 64)
    return fail(PULSAR_ERR_INVALID,
                "fused_attn_gate requires head_dim == 64, got " + std::to_string(head_dim));
  const int64_t nvec = B * H * T;
  if (nvec == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    attn_gate_bwd_kernel<T_><<<blocks_for(nvec, 4), 256, 0, stream>>>(
        (const T_*)grad_out, (const T_*)attn, gate_logits, (T_*)d_attn, d_gate, (int)H, (int)T,
        nvec);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_fused_swiglu_backward(const void* dout, const void* gu, void* dgu, int64_t rows,
                                 int64_t d_ff, int dtype, hipStream_t stream) {
  PULSAR_REQUIRE(rows >= 0 && d_ff > 0, "swiglu backward: bad shape");
  const int64_t total = rows * d_ff;
  if (total == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    swiglu_bwd_kernel<T_><<<blocks_for(total, 256), 256, 0, stream>>>(
        (const T_*)dout, (const T_*)gu, (T_*)dgu, d_ff, total);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_moe_dispatch_backward(const void* d_expert_inputs, const int64_t* topk_idx,
                                 const int32_t* slots, void* dx, int64_t N, int64_t D,
                                 int64_t K, int64_t E, int64_t C, int dtype,
                                 hipStream_t stream) {
  PULSAR_REQUIRE(N >= 0 && D > 0 && K >= 0 && E > 0 && C >= 0, "dispatch backward: bad shape");
  if (N == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    dispatch_bwd_kernel<T_><<<(unsigned)N, 128, 0, stream>>>(
        (const T_*)d_expert_inputs, topk_idx, slots, (T_*)dx, D, (int)K, E, C);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_moe_combine_backward(const void* d_routed_out, const void* expert_outputs,
                                const int64_t* topk_idx, const uint16_t* topk_w_bf16,
                                const int32_t* slots, void* d_expert_outputs,
                                uint16_t* d_topk_w_bf16, int64_t N, int64_t D, int64_t K,
                                int64_t E, int64_t C, int dtype, hipStream_t stream) {
  PULSAR_REQUIRE(N >= 0 && D > 0 && K >= 0 && E > 0 && C >= 0, "combine backward: bad shape");
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    const int64_t n_eo = E * C * D;
    if (n_eo > 0) {
      fill_zero_kernel<T_><<<blocks_for(n_eo, 256), 256, 0, stream>>>((T_*)d_expert_outputs, n_eo);
      PULSAR_LAUNCH_CHECK();
    }
    if (N > 0 && K > 0) {
      combine_bwd_kernel<T_><<<(unsigned)N, 256, 0, stream>>>(
          (const T_*)d_routed_out, (const T_*)expert_outputs, topk_idx, topk_w_bf16, slots,
          (T_*)d_expert_outputs, d_topk_w_bf16, D, (int)K, E, C);
      PULSAR_LAUNCH_CHECK();
    }
    return PULSAR_OK;
  });
}

int pulsar_moe_router_topk_backward(const uint16_t* d_topk_w_bf16, const void* logits,
                                    int logits_dtype, const int64_t* topk_idx,
                                    float z_loss_weight, const float* d_z_loss,
                                    const float* d_probs_mean, void* d_logits, int64_t N,
                                    int64_t E, int64_t K, hipStream_t stream) {
  if (E < 1 || E > 32)
    return fail(PULSAR_ERR_INVALID,
                "moe_router_topk_backward supports E <= 32, got " + std::to_string(E));
  if (K < 1 || K > 8 || K > E)
    return fail(PULSAR_ERR_INVALID, "top_k must be in [1, min(8, E)], got " + std::to_string(K));
  PULSAR_REQUIRE(N >= 0, "router backward: N must be >= 0");
  if (N == 0) return PULSAR_OK;
  return dispatch_dtype(logits_dtype, [&](auto tag) {
    using L = decltype(tag);
    if (E <= 16)
      router_bwd_kernel<L, 16><<<blocks_for(N, 128), 128, 0, stream>>>(
          d_topk_w_bf16, (const L*)logits, topk_idx, (L*)d_logits, z_loss_weight, d_z_loss,
          d_probs_mean, N, (int)E, (int)K);
    else
      router_bwd_kernel<L, 32><<<blocks_for(N, 128), 128, 0, stream>>>(
          d_topk_w_bf16, (const L*)logits, topk_idx, (L*)d_logits, z_loss_weight, d_z_loss,
          d_probs_mean, N, (int)E, (int)K);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_causal_conv1d_k4_backward(const void* dout, const void* x, const float* w, void* dx,
                                     float* dw, int64_t B, int64_t T, int64_t D, int dtype,
                                     hipStream_t stream) {
  PULSAR_REQUIRE(B >= 0 && T >= 0 && D > 0, "conv1d_k4 backward: bad shape");
  PULSAR_TRY_STATUS(zero_f32(dw, D * 4, stream));
  const int64_t ntok = B * T, total = ntok * D;
  if (total == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    conv_k4_bwd_dx_kernel<T_><<<blocks_for(total, 256), 256, 0, stream>>>(
        (const T_*)dout, w, (T_*)dx, T, D, total);
    PULSAR_LAUNCH_CHECK();
    const dim3 g(blocks_for(D, 256), blocks_for(ntok, kConvChunk));
    conv_k4_bwd_dw_kernel<T_><<<g, 256, 0, stream>>>((const T_*)dout, (const T_*)x, dw, T, D,
                                                      ntok);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

}  // extern "C"
