// Op surface of the reference's pulsar_cuda module, written for gfx950 (wave64).
//
// Each kernel is one pass over its tensors with 128-bit loads where the row length
// allows; reductions are wave64 shuffles. Every entry validates shapes on the host and
// returns a status code instead of throwing.
#include <algorithm>
#include <string>
#include <type_traits>

#include "common.h"


namespace pulsar {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// ---------------------------------------------------------------------------
// RMSNorm over rows: one block per row, fp32 statistics.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const T* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      T* __restrict__ y,
                                                      float* __restrict__ rsq, int dim,
                                                      float eps) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * dim;
  T* yr = y + row * dim;
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) {
    float v = to_f(xr[i]);
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
  if (threadIdx.x == 0 && rsq) rsq[row] = inv;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) yr[i] = from_f<T>(to_f(xr[i]) * inv * w[i]);
}

// ---------------------------------------------------------------------------
// RoPE (rotate-half) on contiguous rows of head_dim; table row = row % T.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void rope_kernel(const T* __restrict__ x, T* __restrict__ y,
                            const float* __restrict__ cs, const float* __restrict__ sn,
                            int64_t rows, int64_t T_, int hd) {
  const int half = hd / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = idx / half;
  const int i = (int)(idx % half);
  if (row >= rows) return;
  const int64_t t = row % T_;
  const float c = cs[t * half + i], s = sn[t * half + i];
  const float a = to_f(x[row * hd + i]), b = to_f(x[row * hd + i + half]);
  y[row * hd + i] = from_f<T>(fmaf(a, c, -(b * s)));
  y[row * hd + i + half] = from_f<T>(fmaf(b, c, a * s));
}

// ---------------------------------------------------------------------------
// QK RMSNorm + RoPE: one wave per 64-element head vector; lane i pairs with lane i^32.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(
    const T* __restrict__ x, int64_t sB, int64_t sH, int64_t sT, int H, int T_,
    int64_t nvec, const float* __restrict__ w, const float* __restrict__ cs,
    const float* __restrict__ sn, T* __restrict__ y, float* __restrict__ rsq, float eps) {
  const int64_t v = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (v >= nvec) return;
  const int lane = threadIdx.x & 63;
  const int t = (int)(v % T_);
  const int h = (int)((v / T_) % H);
  const int64_t b = v / ((int64_t)T_ * H);
  const float xv = to_f(x[b * sB + h * sH + (int64_t)t * sT + lane]);
  const float ss = wave_sum(xv * xv);
  const float inv = 1.0f / sqrtf(ss / 64.0f + eps);
  if (lane == 0 && rsq) rsq[v] = inv;
  const float n = xv * inv * w[h * 64 + lane];
  const float partner = __shfl_xor(n, 32, 64);
  const int j = lane & 31;
  const float c = cs[t * 32 + j], s = sn[t * 32 + j];
  const float out = (lane < 32) ? fmaf(n, c, -(partner * s)) : fmaf(n, c, partner * s);
  y[v * 64 + lane] = from_f<T>(out);
}

// ---------------------------------------------------------------------------
// Attention gate + [B,H,T,D] -> [B,T,H*D] transpose.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void attn_gate_kernel(const T* __restrict__ a, const float* __restrict__ gl,
                                 T* __restrict__ out, int H, int T_, int hd, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int d = (int)(idx % hd);
  const int64_t hv = idx / hd;  // (b, t, h) in output order
  const int h = (int)(hv % H);
  const int t = (int)((hv / H) % T_);
  const int64_t b = hv / ((int64_t)H * T_);
  const float g = sigmoidf_(gl[hv]);
  out[idx] = from_f<T>(to_f(a[((b * H + h) * T_ + t) * hd + d]) * g);
}

// ---------------------------------------------------------------------------
// Causal depthwise conv k=4 with residual, fp32 arithmetic.
// ---------------------------------------------------------------------------
// The elementwise ops spell their multiply-adds as fmaf so that the scalar and 16-byte
// kernels round identically whatever the compiler would contract.
__device__ __forceinline__ float conv4(const float* w, float x0, float x1, float x2, float x3) {
  return fmaf(w[3], x3, fmaf(w[2], x2, fmaf(w[1], x1, w[0] * x0)));
}

template <typename T>
__global__ void conv_k4_kernel(const T* __restrict__ x, const float* __restrict__ w,
                               T* __restrict__ y, int64_t T_, int64_t D, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t d = idx % D;
  const int64_t t = (idx / D) % T_;
  const float x0 = to_f(x[idx]);
  const float x1 = t >= 1 ? to_f(x[idx - D]) : 0.f;
  const float x2 = t >= 2 ? to_f(x[idx - 2 * D]) : 0.f;
  const float x3 = t >= 3 ? to_f(x[idx - 3 * D]) : 0.f;
  const float* wd = w + d * 4;
  y[idx] = from_f<T>(x0 + conv4(wd, x0, x1, x2, x3));
}

// ---------------------------------------------------------------------------
// SwiGLU: silu(gate) * up in fp32.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void swiglu_kernel(const T* __restrict__ gu, T* __restrict__ out, int64_t dff,
                              int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t r = idx / dff, c = idx % dff;
  const float g = to_f(gu[r * 2 * dff + c]);
  const float u = to_f(gu[r * 2 * dff + dff + c]);
  out[idx] = from_f<T>(g * sigmoidf_(g) * u);
}


// ---------------------------------------------------------------------------
// 16-byte forms of the elementwise ops (kVec<T> elements per thread and access), used when
// the row lengths are multiples of kVec<T> and the tensors 16-byte aligned; the arithmetic
// per element is the scalar kernels'.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) rmsnorm_vec_kernel(const T* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          T* __restrict__ y,
                                                          float* __restrict__ rsq, int dim,
                                                          float eps) {
  constexpr int V = kVec<T>;
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * dim;
  T* yr = y + row * dim;
  const int nc = dim / V;
  float ss = 0.f;
  for (int c = threadIdx.x; c < nc; c += blockDim.x) {
    float v[V];
    ldv<V>(xr + c * V, v);
#pragma unroll
    for (int j = 0; j < V; ++j) ss += v[j] * v[j];
  }
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
  if (threadIdx.x == 0 && rsq) rsq[row] = inv;
  for (int c = threadIdx.x; c < nc; c += blockDim.x) {
    float v[V], wv[V], o[V];
    ldv<V>(xr + c * V, v);
    ldv<V>(w + c * V, wv);
#pragma unroll
    for (int j = 0; j < V; ++j) o[j] = rnd<T>(v[j] * inv * wv[j]);
    stv<V>(yr + c * V, o);
  }
}

// Thread = 8 consecutive pairs (i, i + half) of one row.
template <typename T>
__global__ void rope_vec_kernel(const T* __restrict__ x, T* __restrict__ y,
                                const float* __restrict__ cs, const float* __restrict__ sn,
                                int64_t rows, int64_t T_, int hd) {
  const int half = hd / 2, per_row = half / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = idx / per_row;
  if (row >= rows) return;
  const int i = (int)(idx % per_row) * 8;
  const int64_t t = row % T_;
  float a[8], b[8], c[8], s[8], o1[8], o2[8];
  ldv<8>(x + row * hd + i, a);
  ldv<8>(x + row * hd + half + i, b);
  ldv<8>(cs + t * half + i, c);
  ldv<8>(sn + t * half + i, s);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    o1[j] = rnd<T>(fmaf(a[j], c[j], -(b[j] * s[j])));
    o2[j] = rnd<T>(fmaf(b[j], c[j], a[j] * s[j]));
  }
  stv<8>(y + row * hd + i, o1);
  stv<8>(y + row * hd + half + i, o2);
}

// 8 lanes per 64-element head vector, 8 elements per lane: lanes 0-3 of a group hold the
// first half, lanes 4-7 the second, so a lane's rotate-half partners sit in lane ^ 4.
template <typename T>
__global__ void __launch_bounds__(256) qk_norm_rope_vec_kernel(
    const T* __restrict__ x, int64_t sB, int64_t sH, int64_t sT, int H, int T_, int64_t nvec,
    const float* __restrict__ w, const float* __restrict__ cs, const float* __restrict__ sn,
    T* __restrict__ y, float* __restrict__ rsq, float eps) {
  const int64_t v = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
  const int j = threadIdx.x & 7;
  const bool ok = v < nvec;
  const int64_t vv = ok ? v : 0;
  const int t = (int)(vv % T_);
  const int h = (int)((vv / T_) % H);
  const int64_t b = vv / ((int64_t)T_ * H);
  float xv[8];
  ldv<8>(x + b * sB + h * sH + (int64_t)t * sT + j * 8, xv);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += xv[e] * xv[e];
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  ss += __shfl_xor(ss, 4, 64);
  const float inv = 1.0f / sqrtf(ss / 64.0f + eps);
  float wv[8], n[8], p[8], c[8], s[8], o[8];
  ldv<8>(w + h * 64 + j * 8, wv);
  ldv<8>(cs + t * 32 + (j & 3) * 8, c);
  ldv<8>(sn + t * 32 + (j & 3) * 8, s);
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = xv[e] * inv * wv[e];
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = __shfl_xor(n[e], 4, 64);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    o[e] = rnd<T>(j < 4 ? fmaf(n[e], c[e], -(p[e] * s[e])) : fmaf(n[e], c[e], p[e] * s[e]));
  if (!ok) return;
  if (j == 0 && rsq) rsq[v] = inv;
  stv<8>(y + v * 64 + j * 8, o);
}

// Thread = kVec<T> consecutive dims of one (b, t, h) output head.
template <typename T>
__global__ void attn_gate_vec_kernel(const T* __restrict__ a, const float* __restrict__ gl,
                                     T* __restrict__ out, int H, int T_, int hd, int64_t total) {
  constexpr int V = kVec<T>;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx * V >= total) return;
  const int d = (int)((idx * V) % hd);
  const int64_t hv = (idx * V) / hd;
  const int h = (int)(hv % H);
  const int t = (int)((hv / H) % T_);
  const int64_t b = hv / ((int64_t)H * T_);
  const float g = sigmoidf_(gl[hv]);
  float v[V];
  ldv<V>(a + ((b * H + h) * T_ + t) * hd + d, v);
#pragma unroll
  for (int j = 0; j < V; ++j) v[j] = rnd<T>(v[j] * g);
  stv<V>(out + idx * V, v);
}

// Thread = kVec<T> channels of one sequence over kConvTokens consecutive tokens: the three
// previous rows ride along in registers, so each row of x is read once and the channels'
// weights once per thread.
constexpr int kConvTokens = 16;
template <typename T>
__global__ void __launch_bounds__(256) conv_k4_vec_kernel(const T* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          T* __restrict__ y, int64_t B,
                                                          int64_t T_, int64_t D) {
  constexpr int V = kVec<T>;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nc = D / V, ntc = (T_ + kConvTokens - 1) / kConvTokens;
  const int64_t cv = idx % nc, rest = idx / nc;
  const int64_t tc = rest % ntc, b = rest / ntc;
  if (b >= B) return;
  const int64_t d0 = cv * V, t0 = tc * kConvTokens;
  const T* xb = x + b * T_ * D + d0;
  T* yb = y + b * T_ * D + d0;
  float wd[4 * V], h1[V], h2[V], h3[V], x0[kConvTokens][V], o[V];
  ldv<4 * V>(w + d0 * 4, wd);
#pragma unroll
  for (int j = 0; j < V; ++j) h1[j] = h2[j] = h3[j] = 0.f;
  if (t0 >= 1) ldv<V>(xb + (t0 - 1) * D, h1);
  if (t0 >= 2) ldv<V>(xb + (t0 - 2) * D, h2);
  if (t0 >= 3) ldv<V>(xb + (t0 - 3) * D, h3);
#pragma unroll
  for (int i = 0; i < kConvTokens; ++i)
    if (t0 + i < T_) ldv<V>(xb + (t0 + i) * D, x0[i]);
#pragma unroll
  for (int i = 0; i < kConvTokens; ++i) {
    if (t0 + i >= T_) break;
#pragma unroll
    for (int j = 0; j < V; ++j)
      o[j] = rnd<T>(x0[i][j] + conv4(wd + 4 * j, x0[i][j], h1[j], h2[j], h3[j]));
    stv<V>(yb + (t0 + i) * D, o);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      h3[j] = h2[j];
      h2[j] = h1[j];
      h1[j] = x0[i][j];
    }
  }
}

template <typename T>
__global__ void swiglu_vec_kernel(const T* __restrict__ gu, T* __restrict__ out, int64_t dff,
                                  int64_t total) {
  constexpr int V = kVec<T>;
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (i0 >= total) return;
  const int64_t r = i0 / dff, c = i0 % dff;
  float g[V], u[V], o[V];
  ldv<V>(gu + r * 2 * dff + c, g);
  ldv<V>(gu + r * 2 * dff + dff + c, u);
#pragma unroll
  for (int j = 0; j < V; ++j) o[j] = rnd<T>(g[j] * sigmoidf_(g[j]) * u[j]);
  stv<V>(out + i0, o);
}

// ---------------------------------------------------------------------------
// Router top-k: one lane per token. Scores in registers: EM (16 or 32) >= E slots in
// unrolled loops, so every register-array index is a compile-time constant (a runtime index
// would move the arrays to scratch memory).
// ---------------------------------------------------------------------------
// One token's logits into c[0..EM) (zero past E): 16-byte loads when VEC (rows a multiple
// of 16 bytes, 16-byte aligned), element loads otherwise.
template <typename L, int EM, bool VEC>
__device__ __forceinline__ void router_row(const L* lt, int E, float* c) {
  if constexpr (VEC) {
    constexpr int V = kVec<L>;
#pragma unroll
    for (int q = 0; q < EM / V; ++q) {
      if (q * V < E) {
        ldv<V>(lt + q * V, c + q * V);
      } else {
#pragma unroll
        for (int j = 0; j < V; ++j) c[q * V + j] = 0.f;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < EM; ++e) c[e] = e < E ? to_f(lt[e]) : 0.f;
  }
}

// Centred logits c[e] = l[e] - mean (mean summed in expert order, as the reference kernel).
template <typename L, int EM, bool VEC>
__device__ __forceinline__ void router_centred(const L* lt, int E, float* c) {
  router_row<L, EM, VEC>(lt, E, c);
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < EM; ++e)
    if (e < E) sum += c[e];
  const float mean = sum / (float)E;
#pragma unroll
  for (int e = 0; e < EM; ++e) c[e] -= mean;
}

// PART: the workgroup also sums its tokens' E + 1 statistics (each expert's score, the
// squared logsumexp) in a fixed order and writes them to part[blockIdx.x][0..E].
constexpr int kRouterTopkThreads = 128;
template <typename L, int EM, bool VEC, bool PART>
__global__ void __launch_bounds__(kRouterTopkThreads) router_topk_kernel(
    const L* __restrict__ logits, const float* __restrict__ bias, int64_t* __restrict__ idx_out,
    uint16_t* __restrict__ w_out, float* __restrict__ part, int64_t N, int E, int K) {
  const int64_t tok = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = tok < N;
  if (!PART && !valid) return;
  float c[EM], s[EM], b[EM];
  router_centred<L, EM, VEC>(logits + (valid ? tok : N - 1) * E, E, c);
#pragma unroll
  for (int e = 0; e < EM; ++e) {
    s[e] = e < E ? sigmoidf_(c[e]) : 0.f;
    b[e] = e < E ? s[e] + bias[e] : -INFINITY;
  }
  if constexpr (PART) {
    __shared__ float red[kRouterTopkThreads / 64][EM + 1];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < EM; ++e)
      if (e < E) mx = fmaxf(mx, c[e]);
    float se = 0.f;
#pragma unroll
    for (int e = 0; e < EM; ++e)
      if (e < E) se += expf(c[e] - mx);
    const float lse = mx + logf(se);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int e = 0; e <= EM; ++e) {
      const float v = wave_sum(valid ? (e < EM ? s[e] : lse * lse) : 0.f);
      if (lane == 0) red[w][e] = v;
    }
    __syncthreads();
    const int i = threadIdx.x;
    if (i < E || i == EM) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < kRouterTopkThreads / 64; ++k) v += red[k][i];
      part[(int64_t)blockIdx.x * (EM + 1) + i] = v;
    }
    if (!valid) return;
  }
  // K rounds of argmax over the experts not taken yet, ties to the lower index: the order
  // and tie rule of the reference's insertion top-k with strict '>' (csrc/kernels.cu:2181-2200)
  int sel[8];
  float sv[8];
  uint32_t taken = 0u;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sel[k] = 0;
    sv[k] = 0.f;
    if (k >= K) continue;
    int bi = -1;
    float best = -INFINITY, bs = 0.f;
#pragma unroll
    for (int e = 0; e < EM; ++e) {
      const bool free = e < E && !((taken >> e) & 1u);
      if (free && (bi < 0 || b[e] > best)) {
        bi = e;
        best = b[e];
        bs = s[e];
      }
    }
    taken |= 1u << bi;
    sel[k] = bi;
    sv[k] = bs;
  }
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < K) tot += sv[k];
  tot += 1e-6f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k >= K) continue;
    idx_out[tok * K + k] = sel[k];
    w_out[tok * K + k] = f2bf(sv[k] / tot).u;
  }
}

// The workgroups' partial statistics summed in workgroup order (one thread per statistic).
template <int EM>
__global__ void router_stats_merge_kernel(const float* __restrict__ part, int nblk,
                                          float* __restrict__ z_loss,
                                          float* __restrict__ probs_mean, int64_t N, int E,
                                          float zw) {
  const int i = threadIdx.x;
  if (i > EM || (i < EM && i >= E)) return;
  float v = 0.f;
  for (int k = 0; k < nblk; ++k) v += part[(int64_t)k * (EM + 1) + i];
  const float inv_n = N > 0 ? 1.0f / (float)N : 0.f;
  if (i < EM)
    probs_mean[i] = v * inv_n;
  else
    z_loss[0] = zw > 0.f ? zw * v * inv_n : 0.f;
}

// Deterministic z-loss and probs_mean in one workgroup: a thread takes tokens tid,
// tid + 1024, ... in increasing order and keeps E + 1 sums (each expert's score, the
// squared logsumexp); waves then reduce each sum in a fixed order, so the statistics do
// not depend on scheduling. U tokens per thread are loaded before any is used (one memory
// round trip per U tokens).
constexpr int kRouterStatThreads = 1024;
template <typename L, int EM, int U, bool VEC>
__global__ void __launch_bounds__(kRouterStatThreads) router_stats_kernel(
    const L* __restrict__ logits, float* __restrict__ z_loss, float* __restrict__ probs_mean,
    int64_t N, int E, float zw) {
  __shared__ float red[kRouterStatThreads / 64][EM + 1];
  float acc[EM + 1];
#pragma unroll
  for (int e = 0; e <= EM; ++e) acc[e] = 0.f;
  for (int64_t t0 = threadIdx.x; t0 < N; t0 += (int64_t)U * kRouterStatThreads) {
    float c[U][EM];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = min(t0 + (int64_t)u * kRouterStatThreads, N - 1);
      router_centred<L, EM, VEC>(logits + t * E, E, c[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t0 + (int64_t)u * kRouterStatThreads >= N) break;
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < EM; ++e)
        if (e < E) {
          acc[e] += sigmoidf_(c[u][e]);
          mx = fmaxf(mx, c[u][e]);
        }
      float se = 0.f;
#pragma unroll
      for (int e = 0; e < EM; ++e)
        if (e < E) se += expf(c[u][e] - mx);
      const float lse = mx + logf(se);
      acc[EM] += lse * lse;
    }
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int e = 0; e <= EM; ++e) {
    const float v = wave_sum(acc[e]);
    if (lane == 0) red[w][e] = v;
  }
  __syncthreads();
  const int i = threadIdx.x;
  if (i > EM || (i < EM && i >= E)) return;
  float v = 0.f;
  for (int k = 0; k < kRouterStatThreads / 64; ++k) v += red[k][i];
  const float inv_n = N > 0 ? 1.0f / (float)N : 0.f;
  if (i < EM)
    probs_mean[i] = v * inv_n;
  else
    z_loss[0] = zw > 0.f ? zw * v * inv_n : 0.f;
}

// ---------------------------------------------------------------------------
// MoE dispatch / combine / slots.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void moe_zero_kernel(T* __restrict__ buf, const int64_t* __restrict__ counts, int C,
                                int64_t D) {
  const int e = blockIdx.y;
  int64_t start = 0;
  if (counts) {
    const int64_t n = counts[e];
    start = n < 0 ? 0 : (n > C ? C : n);
  }
  const int64_t len = (C - start) * D;
  T* base = buf + ((int64_t)e * C + start) * D;
  T zero = from_f<T>(0.f);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
       i += (int64_t)gridDim.x * blockDim.x)
    base[i] = zero;
}

template <typename T>
__global__ void moe_dispatch_kernel(const T* __restrict__ x, const int64_t* __restrict__ idx,
                                    const int32_t* __restrict__ slots, T* __restrict__ dst,
                                    int64_t D, int K, int E, int C) {
  const int64_t tok = blockIdx.x;
  for (int k = 0; k < K; ++k) {
    const int slot = slots[tok * K + k];
    const int64_t e = idx[tok * K + k];
    if (slot < 0 || slot >= C || e < 0 || e >= E) continue;
    T* d = dst + (e * C + slot) * D;
    for (int64_t i = threadIdx.x; i < D; i += blockDim.x) d[i] = x[tok * D + i];
  }
}

template <typename T>
__global__ void moe_combine_kernel(const T* __restrict__ eo, const int64_t* __restrict__ idx,
                                   const uint16_t* __restrict__ wts,
                                   const int32_t* __restrict__ slots,
                                   const T* __restrict__ shared, T* __restrict__ out,
                                   int64_t D, int K, int E, int C) {
  const int64_t tok = blockIdx.x;
  for (int64_t i = threadIdx.x; i < D; i += blockDim.x) {
    float acc = shared ? to_f(shared[tok * D + i]) : 0.f;
    for (int k = 0; k < K; ++k) {
      const int slot = slots[tok * K + k];
      const int64_t e = idx[tok * K + k];
      if (slot < 0 || slot >= C || e < 0 || e >= E) continue;
      bf16 wb;
      wb.u = wts[tok * K + k];
      acc = fmaf(bf2f(wb), to_f(eo[(e * C + slot) * D + i]), acc);
    }
    out[tok * D + i] = from_f<T>(acc);
  }
}

// 16-byte forms of zero / dispatch / combine for 16-byte-aligned tensors whose rows are a
// multiple of 16 bytes (dispatch and zero move bytes; combine keeps the scalar kernel's
// per-element order: shared output first, then the k terms in order).
__global__ void moe_zero_vec_kernel(uint4* __restrict__ buf, const int64_t* __restrict__ counts,
                                    int C, int64_t row_q) {
  const int e = blockIdx.y;
  int64_t start = 0;
  if (counts) {
    const int64_t n = counts[e];
    start = n < 0 ? 0 : (n > C ? C : n);
  }
  const int64_t len = (C - start) * row_q;
  uint4* base = buf + ((int64_t)e * C + start) * row_q;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < len;
       i += (int64_t)gridDim.x * blockDim.x)
    base[i] = make_uint4(0u, 0u, 0u, 0u);
}

__global__ void moe_dispatch_vec_kernel(const uint4* __restrict__ x,
                                        const int64_t* __restrict__ idx,
                                        const int32_t* __restrict__ slots,
                                        uint4* __restrict__ dst, int64_t row_q, int K, int E,
                                        int C) {
  const int64_t tok = blockIdx.x;
  for (int k = 0; k < K; ++k) {
    const int slot = slots[tok * K + k];
    const int64_t e = idx[tok * K + k];
    if (slot < 0 || slot >= C || e < 0 || e >= E) continue;
    uint4* d = dst + (e * C + slot) * row_q;
    for (int64_t i = threadIdx.x; i < row_q; i += blockDim.x) d[i] = x[tok * row_q + i];
  }
}

template <typename T>
__global__ void moe_combine_vec_kernel(const T* __restrict__ eo, const int64_t* __restrict__ idx,
                                       const uint16_t* __restrict__ wts,
                                       const int32_t* __restrict__ slots,
                                       const T* __restrict__ shared, T* __restrict__ out,
                                       int64_t D, int K, int E, int C) {
  constexpr int V = kVec<T>;
  const int64_t tok = blockIdx.x;
  for (int64_t i = (int64_t)threadIdx.x * V; i < D; i += (int64_t)blockDim.x * V) {
    float acc[V], v[V];
    if (shared) {
      ldv<V>(shared + tok * D + i, acc);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = 0.f;
    }
    for (int k = 0; k < K; ++k) {
      const int slot = slots[tok * K + k];
      const int64_t e = idx[tok * K + k];
      if (slot < 0 || slot >= C || e < 0 || e >= E) continue;
      bf16 wb;
      wb.u = wts[tok * K + k];
      const float w = bf2f(wb);
      ldv<V>(eo + (e * C + slot) * D + i, v);
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = fmaf(w, v[j], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] = rnd<T>(acc[j]);
    stv<V>(out + tok * D + i, acc);
  }
}

__global__ void slots_count_kernel(const int64_t* __restrict__ flat_e, int64_t* __restrict__ counts,
                                   int64_t M, int E) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  const int64_t e = flat_e[i];
  if (e >= 0 && e < E) atomicAdd(reinterpret_cast<unsigned long long*>(&counts[e]), 1ull);
}

__global__ void slots_assign_kernel(const int64_t* __restrict__ flat_e,
                                    const int64_t* __restrict__ order,
                                    const int64_t* __restrict__ counts, int32_t* __restrict__ slots,
                                    int64_t M, int E, int C) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  const int64_t orig = order[i];
  const int64_t e = flat_e[orig];
  int64_t start = 0;
  for (int j = 0; j < E && j < e; ++j) start += counts[j];
  const int64_t rank = i - start;
  slots[orig] = (e >= 0 && e < E && rank >= 0 && rank < C) ? (int32_t)rank : -1;
}

__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}


// Router entry: top-k, and the statistics either through per-workgroup partials in a
// caller workspace or (no workspace) one workgroup over all tokens.
int router_topk_forward(const void* logits, int logits_dtype, const float* bias,
                        int64_t* topk_idx, uint16_t* topk_w_bf16, float* z_loss,
                        float* probs_mean, int64_t N, int64_t E, int64_t K,
                        float z_loss_weight, float* workspace, hipStream_t stream) {
  if (E < 1 || E > 32)
    return fail(PULSAR_ERR_INVALID,
                "moe_router_topk_forward supports E <= 32, got " + std::to_string(E));
  if (K < 1 || K > 8 || K > E)
    return fail(PULSAR_ERR_INVALID,
                "top_k must be in [1, min(8, E)], got " + std::to_string(K));
  PULSAR_REQUIRE(N >= 0, "router: N must be >= 0");
  return dispatch_dtype(logits_dtype, [&](auto tag) {
    using L = decltype(tag);
    const bool vec = E % kVec<L> == 0 && aligned16(logits);
    const bool stats = z_loss && probs_mean;
    const unsigned nblk = blocks_for(N, kRouterTopkThreads);
    auto run = [&](auto em, auto v) {
      constexpr int EM = decltype(em)::value;
      constexpr bool VEC = decltype(v)::value;
      if (stats && workspace && N > 0) {
        // per-workgroup partials, then their fixed-order sum
        router_topk_kernel<L, EM, VEC, true><<<nblk, kRouterTopkThreads, 0, stream>>>(
            (const L*)logits, bias, topk_idx, topk_w_bf16, workspace, N, (int)E, (int)K);
        router_stats_merge_kernel<EM><<<1, 64, 0, stream>>>(workspace, (int)nblk, z_loss,
                                                            probs_mean, N, (int)E,
                                                            z_loss_weight);
        return;
      }
      if (N > 0)
        router_topk_kernel<L, EM, VEC, false><<<nblk, kRouterTopkThreads, 0, stream>>>(
            (const L*)logits, bias, topk_idx, topk_w_bf16, nullptr, N, (int)E, (int)K);
      if (stats)
        router_stats_kernel<L, EM, EM == 16 ? 4 : 2, VEC><<<1, kRouterStatThreads, 0, stream>>>(
            (const L*)logits, z_loss, probs_mean, N, (int)E, z_loss_weight);
    };
    using T16 = std::integral_constant<int, 16>;
    using T32 = std::integral_constant<int, 32>;
    if (E <= 16)
      vec ? run(T16{}, std::true_type{}) : run(T16{}, std::false_type{});
    else
      vec ? run(T32{}, std::true_type{}) : run(T32{}, std::false_type{});
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

}  // namespace pulsar

using namespace pulsar;

extern "C" {

const char* pulsar_last_error(void) { return g_last_error.c_str(); }

int pulsar_abi_version(void) { return 5; }

int pulsar_rmsnorm_forward(const void* x, const float* w, void* y, float* rsqrt_out,
                           int64_t rows, int64_t dim, float eps, int dtype,
                           hipStream_t stream) {
  PULSAR_REQUIRE(rows >= 0 && dim > 0, "rmsnorm: rows >= 0 and dim > 0 required");
  if (rows == 0) return PULSAR_OK;
  PULSAR_REQUIRE(x && w && y, "rmsnorm: null pointer");
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (dim % kVec<T> == 0 && aligned16(x) && aligned16(w) && aligned16(y)) {
      // one 16-byte chunk per thread where the row allows (a multiple of 64 threads, <= 256)
      const int64_t nc = dim / kVec<T>;
      const int threads = (int)std::min<int64_t>(256, std::max<int64_t>(64, (nc + 63) / 64 * 64));
      rmsnorm_vec_kernel<T><<<(unsigned)rows, threads, 0, stream>>>((const T*)x, w, (T*)y,
                                                                    rsqrt_out, (int)dim, eps);
    }
    else
      rmsnorm_kernel<T><<<(unsigned)rows, 256, 0, stream>>>((const T*)x, w, (T*)y, rsqrt_out,
                                                            (int)dim, eps);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_rope_forward(const void* x, void* y, const float* cos, const float* sin,
                        int64_t rows, int64_t T, int64_t head_dim, int dtype,
                        hipStream_t stream) {
  PULSAR_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "rope: head_dim must be even");
  PULSAR_REQUIRE(T > 0 || rows == 0, "rope: T must be positive");
  if (rows == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    if ((head_dim / 2) % 8 == 0 && aligned16(x) && aligned16(y) && aligned16(cos) &&
        aligned16(sin)) {
      const int64_t n = rows * (head_dim / 16);
      rope_vec_kernel<T_><<<blocks_for(n, 256), 256, 0, stream>>>(
          (const T_*)x, (T_*)y, cos, sin, rows, T, (int)head_dim);
    } else {
      const int64_t n = rows * (head_dim / 2);
      rope_kernel<T_><<<blocks_for(n, 256), 256, 0, stream>>>((const T_*)x, (T_*)y, cos, sin,
                                                              rows, T, (int)head_dim);
    }
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_qk_rmsnorm_rope_forward(const void* x, int64_t sB, int64_t sH, int64_t sT,
                                   int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                   const float* w, const float* cos, const float* sin,
                                   void* y, float* rsqrt_out, float eps, int dtype,
                                   hipStream_t stream) {
  if (head_dim != 64)
    return fail(PULSAR_ERR_INVALID,
                "qk_rmsnorm_rope requires head_dim == 64, got " + std::to_string(head_dim));
  const int64_t nvec = B * H * T;
  if (nvec == 0) return PULSAR_OK;
  PULSAR_REQUIRE(T > 0 && H > 0, "qk_rmsnorm_rope: H and T must be positive");
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    constexpr int V = kVec<T_>;
    if (sB % V == 0 && sH % V == 0 && sT % V == 0 && aligned16(x) && aligned16(w) &&
        aligned16(cos) && aligned16(sin) && aligned16(y))
      qk_norm_rope_vec_kernel<T_><<<blocks_for(nvec * 8, 256), 256, 0, stream>>>(
          (const T_*)x, sB, sH, sT, (int)H, (int)T, nvec, w, cos, sin, (T_*)y, rsqrt_out, eps);
    else
      qk_norm_rope_kernel<T_><<<blocks_for(nvec, 4), 256, 0, stream>>>(
          (const T_*)x, sB, sH, sT, (int)H, (int)T, nvec, w, cos, sin, (T_*)y, rsqrt_out, eps);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_fused_attn_gate_forward(const void* attn, const float* gate_logits, void* out,
                                   int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                   int dtype, hipStream_t stream) {
  if (head_dim != 64)
    return fail(PULSAR_ERR_INVALID,
                "fused_attn_gate requires head_dim == 64, got " + std::to_string(head_dim));
  const int64_t total = B * H * T * head_dim;
  if (total == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    if (aligned16(attn) && aligned16(out))  // head_dim 64 is a multiple of kVec
      attn_gate_vec_kernel<T_><<<blocks_for(total / kVec<T_>, 256), 256, 0, stream>>>(
          (const T_*)attn, gate_logits, (T_*)out, (int)H, (int)T, (int)head_dim, total);
    else
      attn_gate_kernel<T_><<<blocks_for(total, 256), 256, 0, stream>>>(
          (const T_*)attn, gate_logits, (T_*)out, (int)H, (int)T, (int)head_dim, total);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_causal_conv1d_k4_forward(const void* x, const float* w, void* y, int64_t B,
                                    int64_t T, int64_t D, int dtype, hipStream_t stream) {
  PULSAR_REQUIRE(B >= 0 && T >= 0 && D > 0, "conv1d_k4: bad shape");
  const int64_t total = B * T * D;
  if (total == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    if (D % kVec<T_> == 0 && aligned16(x) && aligned16(w) && aligned16(y))
      conv_k4_vec_kernel<T_><<<blocks_for(B * ((T + kConvTokens - 1) / kConvTokens) *
                                              (D / kVec<T_>), 256), 256, 0, stream>>>(
          (const T_*)x, w, (T_*)y, B, T, D);
    else
      conv_k4_kernel<T_><<<blocks_for(total, 256), 256, 0, stream>>>((const T_*)x, w, (T_*)y,
                                                                     T, D, total);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_fused_swiglu_forward(const void* gu, void* out, int64_t rows, int64_t d_ff,
                                int dtype, hipStream_t stream) {
  PULSAR_REQUIRE(rows >= 0 && d_ff > 0, "swiglu: bad shape");
  const int64_t total = rows * d_ff;
  if (total == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T_ = decltype(tag);
    if (d_ff % kVec<T_> == 0 && aligned16(gu) && aligned16(out))
      swiglu_vec_kernel<T_><<<blocks_for(total / kVec<T_>, 256), 256, 0, stream>>>(
          (const T_*)gu, (T_*)out, d_ff, total);
    else
      swiglu_kernel<T_><<<blocks_for(total, 256), 256, 0, stream>>>((const T_*)gu, (T_*)out,
                                                                    d_ff, total);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_moe_router_topk_forward(const void* logits, int logits_dtype, const float* bias,
                                   int64_t* topk_idx, uint16_t* topk_w_bf16, float* z_loss,
                                   float* probs_mean, int64_t N, int64_t E, int64_t K,
                                   float z_loss_weight, hipStream_t stream) {
  return router_topk_forward(logits, logits_dtype, bias, topk_idx, topk_w_bf16, z_loss,
                             probs_mean, N, E, K, z_loss_weight, nullptr, stream);
}

int64_t pulsar_moe_router_workspace_bytes(int64_t N, int64_t E) {
  if (N < 0 || E < 1 || E > 32) return -1;
  const int64_t em = E <= 16 ? 16 : 32;
  return (int64_t)blocks_for(N, kRouterTopkThreads) * (em + 1) * (int64_t)sizeof(float);
}

int pulsar_moe_router_topk_forward_ws(const void* logits, int logits_dtype, const float* bias,
                                      int64_t* topk_idx, uint16_t* topk_w_bf16, float* z_loss,
                                      float* probs_mean, int64_t N, int64_t E, int64_t K,
                                      float z_loss_weight, float* workspace,
                                      hipStream_t stream) {
  PULSAR_REQUIRE(workspace || !(z_loss && probs_mean) || N == 0,
                 "moe_router_topk_forward_ws: workspace required for the statistics");
  return router_topk_forward(logits, logits_dtype, bias, topk_idx, topk_w_bf16, z_loss,
                             probs_mean, N, E, K, z_loss_weight, workspace, stream);
}

int pulsar_moe_dispatch_forward(const void* x, const int64_t* topk_idx, const int32_t* slots,
                                const int64_t* expert_counts, void* expert_inputs, int64_t N,
                                int64_t D, int64_t K, int64_t E, int64_t C, int dtype,
                                hipStream_t stream) {
  if (D % 8 != 0)
    return fail(PULSAR_ERR_INVALID,
                "D must be a multiple of 8 for vectorised dispatch, got " + std::to_string(D));
  PULSAR_REQUIRE(N >= 0 && K >= 0 && E > 0 && C >= 0, "dispatch: bad shape");
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    const bool vec = aligned16(x) && aligned16(expert_inputs);  // rows: D % 8 == 0
    const int64_t row_q = D * (int64_t)sizeof(T) / 16;
    if (C > 0) {
      dim3 g(64, (unsigned)E);
      if (vec)
        moe_zero_vec_kernel<<<g, 256, 0, stream>>>((uint4*)expert_inputs, expert_counts,
                                                   (int)C, row_q);
      else
        moe_zero_kernel<T><<<g, 256, 0, stream>>>((T*)expert_inputs, expert_counts, (int)C, D);
      PULSAR_LAUNCH_CHECK();
    }
    if (N > 0 && K > 0 && C > 0) {
      if (vec)
        moe_dispatch_vec_kernel<<<(unsigned)N, 128, 0, stream>>>(
            (const uint4*)x, topk_idx, slots, (uint4*)expert_inputs, row_q, (int)K, (int)E,
            (int)C);
      else
        moe_dispatch_kernel<T><<<(unsigned)N, 128, 0, stream>>>(
            (const T*)x, topk_idx, slots, (T*)expert_inputs, D, (int)K, (int)E, (int)C);
      PULSAR_LAUNCH_CHECK();
    }
    return PULSAR_OK;
  });
}

int pulsar_moe_combine_forward(const void* expert_outputs, const int64_t* topk_idx,
                               const uint16_t* topk_w_bf16, const int32_t* slots,
                               const void* shared_out, void* out, int64_t N, int64_t D,
                               int64_t K, int64_t E, int64_t C, int dtype, hipStream_t stream) {
  PULSAR_REQUIRE(N >= 0 && D > 0 && K >= 0, "combine: bad shape");
  if (N == 0) return PULSAR_OK;
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (D % kVec<T> == 0 && aligned16(expert_outputs) && aligned16(out) &&
        (!shared_out || aligned16(shared_out)))
      moe_combine_vec_kernel<T><<<(unsigned)N, 128, 0, stream>>>(
          (const T*)expert_outputs, topk_idx, topk_w_bf16, slots, (const T*)shared_out,
          (T*)out, D, (int)K, (int)E, (int)C);
    else
      moe_combine_kernel<T><<<(unsigned)N, 128, 0, stream>>>(
          (const T*)expert_outputs, topk_idx, topk_w_bf16, slots, (const T*)shared_out,
          (T*)out, D, (int)K, (int)E, (int)C);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  });
}

int pulsar_moe_slots_from_order(const int64_t* flat_e, const int64_t* order, int32_t* slots,
                                int64_t* counts, int64_t M, int64_t E, int64_t C,
                                hipStream_t stream) {
  PULSAR_REQUIRE(E > 0 && E <= 1024 && M >= 0, "slots_from_order: bad shape");
  fill_i64_kernel<<<blocks_for(E, 64), 64, 0, stream>>>(counts, E, 0);
  PULSAR_LAUNCH_CHECK();
  if (M == 0) return PULSAR_OK;
  slots_count_kernel<<<blocks_for(M, 256), 256, 0, stream>>>(flat_e, counts, M, (int)E);
  PULSAR_LAUNCH_CHECK();
  slots_assign_kernel<<<blocks_for(M, 256), 256, 0, stream>>>(flat_e, order, counts, slots, M,
                                                              (int)E, (int)C);
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

}  // extern "C"
