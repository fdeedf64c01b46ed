// Per-row kernels of a decode/prefill pulse: pulse input (stem / re-injection), RMSNorm,
// QK-norm + RoPE + YaRN + KV write, attention (split-K decode, tiled prefill), router,
// MoE combine, pulse output. Every kernel reads its row set from the step control block,
// so a captured graph serves any mix of rows; rows past n_rows exit immediately.
//
// Rounding follows the reference op by op: every intermediate the reference materialises
// in the activation dtype T is rounded through T here (rnd<T>), so fp32 runs differ from
// the reference only by summation order and bf16 runs see the same quantisation points.
#include "rows.h"

namespace pulsar {

namespace {

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f(p[i]); }

// 8 consecutive elements with 128-bit loads.
__device__ __forceinline__ void load8(const bf16* p, float* o) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(w[i] << 16);
    o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load8(const float* p, float* o) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// Row-wise sum of squares of a D-vector held by the block (256 threads).
template <typename T>
__device__ float row_inv_rms(const T* x, int D, float eps, float* red) {
  float ss = 0.f;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const float v = ld(x, i);
    ss += v * v;
  }
  ss = block_sum(ss, red);
  return 1.0f / sqrtf(ss / (float)D + eps);
}

// Store a row held as hv[c] (element threadIdx.x + 256c) into h_in and h, and, when w is
// given, its RMSNorm T(w * (h * inv)) into xn.
template <typename T, int NPER>
__device__ void store_and_norm(const float* hv, T* h_in, T* h, const float* w, T* xn, int D,
                               float eps, float* red) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NPER; ++c) {
    const int i = threadIdx.x + c * 256;
    if (h_in) h_in[i] = from_f<T>(hv[c]);
    h[i] = from_f<T>(hv[c]);
    ss += hv[c] * hv[c];
  }
  if (!w) return;
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int c = 0; c < NPER; ++c) {
    const int i = threadIdx.x + c * 256;
    xn[i] = from_f<T>(w[i] * (hv[c] * inv));
  }
}

__device__ __forceinline__ float lerp_ref(float s, float e, float w) {
  // torch.lerp: start + w*(end-start) for |w| < 0.5, else end - (end-start)*(1-w)
  return fabsf(w) < 0.5f ? s + w * (e - s) : e - (e - s) * (1.0f - w);
}

}  // namespace

// ---------------------------------------------------------------------------
// Pulse input. pulse 0: stem (decode: embed, anchor norm, conv over one token) + step
// embedding. pulse >= 1: rank-r re-injection gate on (anchor, state-normed previous pulse).
// ---------------------------------------------------------------------------
template <typename T, int NPER>
__global__ void __launch_bounds__(256) pulse_input_kernel(PulseInputArgs a) {
  __shared__ float red[16];
  __shared__ float gh[16];
  if (blockIdx.x == 0 && a.zero_counts) {
    for (int i = threadIdx.x; i < a.n_zero; i += blockDim.x) a.zero_counts[i] = 0;
  }
  const int r = blockIdx.x;
  if (r >= a.ctl->n_rows) return;
  const RowDesc rd = a.rows[r];
  const int D = a.D;
  const int st = a.prefill ? rd.pos + rd.seq * a.prefill_T : rd.seq * 2 + rd.slot;
  T* e = reinterpret_cast<T*>(a.e_state) + (int64_t)st * D;
  T* h_in = reinterpret_cast<T*>(a.h_in) + (int64_t)r * D;
  T* h = reinterpret_cast<T*>(a.h) + (int64_t)r * D;
  const T* step = reinterpret_cast<const T*>(a.step_emb) + (int64_t)rd.pulse * D;
  float hv[NPER];
  if (rd.pulse == 0) {
    if (!a.prefill) {
      const T* x0 = reinterpret_cast<const T*>(a.tok_emb) + (int64_t)rd.token * D;
      const float inv = row_inv_rms(x0, D, a.eps, red);
#pragma unroll
      for (int c = 0; c < NPER; ++c) {
        const int i = threadIdx.x + c * 256;
        float v = rnd<T>(ld(x0, i) * inv * a.anchor_norm[i]);
        if (a.conv_w) v = rnd<T>(v + a.conv_w[i * 4] * v);
        e[i] = from_f<T>(v);
        hv[c] = rnd<T>(v + ld(step, i));
      }
    } else {
#pragma unroll
      for (int c = 0; c < NPER; ++c) {
        const int i = threadIdx.x + c * 256;
        hv[c] = rnd<T>(ld(e, i) + ld(step, i));
      }
    }
    store_and_norm<T, NPER>(hv, h_in, h, a.norm_w ? a.norm_w + (int64_t)rd.pulse * D : nullptr,
                      reinterpret_cast<T*>(a.xn) + (int64_t)r * D, D, a.eps, red);
    return;
  }
  // pulse >= 1
  const T* hp = reinterpret_cast<const T*>(a.hout_state) + (int64_t)st * D;
  const float inv = row_inv_rms(hp, D, a.eps, red);
  const int R = a.rank;
  const T* wd = reinterpret_cast<const T*>(a.reinject_down) + (int64_t)rd.pulse * R * 2 * D;
  // g_hidden[j] = T(T(e . wd[j][:D]) + T(r . wd[j][D:])), all 2R partial sums in one pass
  float pe[kMaxRank], pr[kMaxRank];
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j) pe[j] = pr[j] = 0.f;
#pragma unroll
  for (int c = 0; c < NPER; ++c) {
    const int i = threadIdx.x + c * 256;
    const float ev = ld(e, i);
    const float rv = rnd<T>(ld(hp, i) * inv * a.state_norm[i]);
#pragma unroll
    for (int j = 0; j < kMaxRank; ++j) {
      if (j < R) {
        pe[j] += ev * ld(wd, (int64_t)j * 2 * D + i);
        pr[j] += rv * ld(wd, (int64_t)j * 2 * D + D + i);
      }
    }
  }
  __shared__ float gred[4][2 * kMaxRank];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < kMaxRank; ++j) {
    if (j < R) {
      const float x = wave_sum(pe[j]), y = wave_sum(pr[j]);
      if (lane == 0) {
        gred[wv][j] = x;
        gred[wv][kMaxRank + j] = y;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < R) {
    const int j = threadIdx.x;
    const float se = gred[0][j] + gred[1][j] + gred[2][j] + gred[3][j];
    const float sr = gred[0][kMaxRank + j] + gred[1][kMaxRank + j] + gred[2][kMaxRank + j] +
                     gred[3][kMaxRank + j];
    gh[j] = rnd<T>(rnd<T>(se) + rnd<T>(sr));
  }
  __syncthreads();
  const T* wu = reinterpret_cast<const T*>(a.reinject_up) + (int64_t)rd.pulse * D * R;
  const T* bu = reinterpret_cast<const T*>(a.reinject_bias) + (int64_t)rd.pulse * D;
#pragma unroll
  for (int c = 0; c < NPER; ++c) {
    const int i = threadIdx.x + c * 256;
    float acc = 0.f;
    for (int j = 0; j < R; ++j) acc += gh[j] * ld(wu, (int64_t)i * R + j);
    const float mix = rnd<T>(sigmoidf_(rnd<T>(acc + ld(bu, i))));
    const float rv = rnd<T>(ld(hp, i) * inv * a.state_norm[i]);
    hv[c] = rnd<T>(rnd<T>(lerp_ref(rv, ld(e, i), mix)) + ld(step, i));
  }
  store_and_norm<T, NPER>(hv, h_in, h, a.norm_w ? a.norm_w + (int64_t)rd.pulse * D : nullptr,
                    reinterpret_cast<T*>(a.xn) + (int64_t)r * D, D, a.eps, red);
}

// ---------------------------------------------------------------------------
// Prefill stem: anchor norm of every prompt token, then the causal k=4 conv.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) prefill_embed_kernel(const int32_t* __restrict__ ids,
                                                            const T* __restrict__ emb,
                                                            const float* __restrict__ w, T* out,
                                                            int D, int n, float eps) {
  __shared__ float red[16];
  const int t = blockIdx.x;
  if (t >= n) return;
  const T* x = emb + (int64_t)ids[t] * D;
  const float inv = row_inv_rms(x, D, eps, red);
  for (int i = threadIdx.x; i < D; i += blockDim.x)
    out[(int64_t)t * D + i] = from_f<T>(ld(x, i) * inv * w[i]);
}

template <typename T>
__global__ void prefill_conv_kernel(const T* __restrict__ a, const float* __restrict__ w,
                                    T* __restrict__ e, int T_, int D, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int d = (int)(idx % D);
  const int t = (int)((idx / D) % T_);
  const float x0 = ld(a, idx);
  if (!w) {
    e[idx] = from_f<T>(x0);
    return;
  }
  float y = w[d * 4] * x0;
  if (t >= 1) y += w[d * 4 + 1] * ld(a, idx - D);
  if (t >= 2) y += w[d * 4 + 2] * ld(a, idx - 2 * D);
  if (t >= 3) y += w[d * 4 + 3] * ld(a, idx - 3 * D);
  e[idx] = from_f<T>(x0 + y);
}

// ---------------------------------------------------------------------------
// RMSNorm of step rows with per-pulse weights: out[r] = T(w[pulse] * (x * inv)).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) norm_rows_kernel(NormArgs a) {
  __shared__ float red[16];
  const int r = blockIdx.x;
  const int n = a.use_lrows ? a.ctl->n_lrows : a.ctl->n_rows;
  if (r >= n) return;
  int src = r, pulse = 0;
  if (a.use_lrows) {
    src = a.lrow_src[r];
  } else {
    pulse = a.rows[r].pulse;
  }
  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)src * a.ldx;
  const float* w = a.w + (int64_t)pulse * a.w_pulse_stride;
  const float inv = row_inv_rms(x, a.D, a.eps, red);
  T* y = reinterpret_cast<T*>(a.y) + (int64_t)r * a.D;
  for (int i = threadIdx.x; i < a.D; i += blockDim.x) y[i] = from_f<T>(w[i] * (ld(x, i) * inv));
}

// ---------------------------------------------------------------------------
// QK-norm + RoPE (+YaRN) on q heads, value residual + K-norm + RoPE on kv heads and the
// cache write. One wave per head vector (lane = element, rotate-half partner = lane^32).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) qk_post_kernel(QKPostArgs a) {
  const int r = blockIdx.x;
  if (r >= a.ctl->n_rows) return;
  const int hh = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int H = a.H, Hk = a.Hkv;
  if (hh >= H + Hk) return;
  const int lane = threadIdx.x & 63;
  const RowDesc rd = a.rows[r];
  const int pulse = rd.pulse, pos = rd.pos;
  T* q = reinterpret_cast<T*>(a.qkv) + (int64_t)r * a.ldq;
  const float* cs = a.cos + (int64_t)pos * 32;
  const float* sn = a.sin + (int64_t)pos * 32;
  const int j = lane & 31;
  auto norm_rope = [&](float x, const float* w) {
    const float ss = wave_sum(x * x);
    const float inv = 1.0f / sqrtf(ss / 64.0f + a.eps);
    const float y = rnd<T>(w[lane] * (x * inv));
    const float p = __shfl_xor(y, 32, 64);
    const float c = cs[j], s = sn[j];
    return rnd<T>(lane < 32 ? y * c - p * s : y * c + p * s);
  };
  if (hh < H) {
    float y = norm_rope(ld(q, hh * 64 + lane), a.q_norm + ((int64_t)pulse * H + hh) * 64);
    if (!a.prefill && !a.is_local && pos + 1 > a.base_seq_len) {
      const double base = (double)a.base_seq_len;
      const double pp = (double)(pos + 1) > base ? (double)(pos + 1) : base;
      const float scale = (float)(1.0 + 0.1 * log(pp / base));
      y = rnd<T>(y * scale);
    }
    q[hh * 64 + lane] = from_f<T>(y);
    return;
  }
  const int g = hh - H;
  float v = ld(q, H * 64 + Hk * 64 + g * 64 + lane);
  if (pulse == 0) {
    T* vf = reinterpret_cast<T*>(a.v_first) + (int64_t)r * Hk * 64 + g * 64 + lane;
    if (a.layer == 0) {
      *vf = from_f<T>(v);
    } else {
      const float lv = a.v_lambda[pulse];
      v = rnd<T>(rnd<T>(rnd<T>(1.0f - lv) * v) + rnd<T>(lv * to_f(*vf)));
    }
  }
  const float k = norm_rope(ld(q, H * 64 + g * 64 + lane), a.k_norm + ((int64_t)pulse * Hk + g) * 64);
  if (a.prefill && a.is_local && pos < a.prefill_T - a.window) return;
  const int64_t off = kv_offset(a.kv, a.layer, rd.seq, g, pos) + lane;
  reinterpret_cast<T*>(a.kv.k[a.layer])[off] = from_f<T>(k);
  reinterpret_cast<T*>(a.kv.v[a.layer])[off] = from_f<T>(v);
}

// ---------------------------------------------------------------------------
// Decode attention, split over keys: block (row, kv head, split) serves the 4 query heads
// of the group over up to 256 keys, 64 per wave. Lane l owns key group (l >> 3), i.e. keys
// kbeg + (l >> 3) + 8i for i < 8, and dims 8*(l & 7) .. +8, so each K and V load is 128
// contiguous bits and every 8 lanes read one 128-byte key row: the wave reads 1 KB of
// contiguous cache per load instruction. Scores are reduced over the 8 lanes of a key
// group, softmax statistics over the wave; partials (max, sum, acc[64]) per query head go
// to `part` and the combine kernel merges the splits.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void load8v(const T* p, float* o, bool valid) {
  if (valid) {
    load8(p, o);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0.f;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) attn_decode_kernel(AttnArgs a) {
  __shared__ float wm[4][4], wl[4][4];
  __shared__ float wacc[4][4][64];
  const int r = blockIdx.x;
  if (r >= a.ctl->n_rows) return;
  const int g = blockIdx.y, s = blockIdx.z;
  const RowDesc rd = a.rows[r];
  const int pos = rd.pos;
  const int lo = a.is_local ? max(0, pos - a.window + 1) : 0;
  const int nkeys = pos - lo + 1;
  const int nsplit = (nkeys + kSplitLen - 1) / kSplitLen;
  if (s >= nsplit) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int kg = lane >> 3, dc = lane & 7;
  // q of the 4 heads, this lane's 8 dims
  const T* q = reinterpret_cast<const T*>(a.qkv) + (int64_t)r * a.ldq + (g * 4) * 64 + dc * 8;
  float qv[4][8];
#pragma unroll
  for (int h = 0; h < 4; ++h) load8(q + h * 64, qv[h]);
  const int kbeg = lo + s * kSplitLen + wv * 64;
  const T* Kc = reinterpret_cast<const T*>(a.kv.k[a.layer]);
  const T* Vc = reinterpret_cast<const T*>(a.kv.v[a.layer]);
  float kf[8][8], vf[8][8];
  bool valid[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = kbeg + kg + 8 * i;
    valid[i] = key <= pos;
    const int64_t off = valid[i] ? kv_offset(a.kv, a.layer, rd.seq, g, key) + dc * 8 : 0;
    load8v(Kc + off, kf[i], valid[i]);
    load8v(Vc + off, vf[i], valid[i]);
  }
  float sc[4][8];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc += qv[h][d] * kf[i][d];
      // sum the 8 dim chunks of this key
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      acc += __shfl_xor(acc, 4, 64);
      sc[h][i] = valid[i] ? acc * a.scale : -INFINITY;
    }
  }
  float m[4], l[4], o[4][8];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, sc[h][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    m[h] = mx;
    float ls = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) o[h][d] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = valid[i] ? expf(sc[h][i] - mx) : 0.f;
      ls += p;
#pragma unroll
      for (int d = 0; d < 8; ++d) o[h][d] += p * vf[i][d];
    }
    // the 8 lanes of a key group hold the same scores: sum over key groups only
    ls += __shfl_xor(ls, 8, 64);
    ls += __shfl_xor(ls, 16, 64);
    ls += __shfl_xor(ls, 32, 64);
    l[h] = ls;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float v = o[h][d];
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      o[h][d] = v;
    }
  }
  if (lane < 8) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int d = 0; d < 8; ++d) wacc[wv][h][dc * 8 + d] = o[h][d];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      wm[wv][h] = m[h];
      wl[wv][h] = l[h];
    }
  }
  __syncthreads();
  // combine the 4 waves: thread (h = tid/64, d = tid%64)
  const int h = wv, d = lane;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) M = fmaxf(M, wm[w][h]);
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (wm[w][h] == -INFINITY) continue;
    const float f = expf(wm[w][h] - M);
    L += wl[w][h] * f;
    O += wacc[w][h][d] * f;
  }
  float* out = a.part + ((((int64_t)r * a.Hkv + g) * a.max_splits + s) * 4 + h) * 66;
  out[2 + d] = O;
  if (d == 0) {
    out[0] = M;
    out[1] = L;
  }
}

// Merge split partials, normalise, round as SDPA output, apply the head gate.
template <typename T>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a) {
  const int r = blockIdx.x;
  if (r >= a.ctl->n_rows) return;
  const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = head / 4, h = head % 4;
  const RowDesc rd = a.rows[r];
  const int pos = rd.pos;
  const int lo = a.is_local ? max(0, pos - a.window + 1) : 0;
  const int nsplit = (pos - lo + 1 + kSplitLen - 1) / kSplitLen;
  const float* base = a.part + (((int64_t)r * a.Hkv + g) * a.max_splits * 4 + h) * 66;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, base[(int64_t)s * 4 * 66]);
  float L = 0.f, O = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float* p = base + (int64_t)s * 4 * 66;
    const float f = expf(p[0] - M);
    L += p[1] * f;
    O += p[2 + lane] * f;
  }
  const float o = rnd<T>(O / L);
  const float gate = to_f(reinterpret_cast<const T*>(a.gate)[(int64_t)r * a.H + head]);
  reinterpret_cast<T*>(a.out)[(int64_t)r * a.H * 64 + head * 64 + lane] = from_f<T>(o * gate);
}

// ---------------------------------------------------------------------------
// Prefill attention: block (sequence, 64-query tile, kv head); wave = query head of the
// group, lane = query. K/V tiles of 64 keys are staged in LDS (fp32). Key range per query:
// global or short prompt: [0, t]; local with T > window (reference SDPA is_causal with
// L=T > S=window, top-left aligned): [T-W, T-W+min(t, W-1)].
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) attn_prefill_kernel(AttnArgs a) {
  __shared__ float Ks[64][65];
  __shared__ float Vs[64][64];
  const int T_ = a.prefill_T;
  const int ntile = (T_ + 63) / 64;
  const int b = blockIdx.x / ntile, qt = blockIdx.x % ntile;
  const int g = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int head = g * 4 + wv;
  const int t = qt * 64 + lane;
  const bool qvalid = t < T_;
  const bool quirk = a.is_local && T_ > a.window;
  auto range = [&](int tq, int& lo, int& hi) {
    if (quirk) {
      lo = T_ - a.window;
      hi = T_ - a.window + min(tq, a.window - 1);
    } else {
      lo = 0;
      hi = tq;
    }
  };
  int qlo, qhi;
  range(min(t, T_ - 1), qlo, qhi);
  // key span of the whole tile
  int tlo, thi, dummy;
  range(qt * 64, tlo, dummy);
  range(min(qt * 64 + 63, T_ - 1), dummy, thi);
  const int64_t row = (int64_t)b * T_ + (qvalid ? t : T_ - 1);
  const T* qp = reinterpret_cast<const T*>(a.qkv) + row * a.ldq + head * 64;
  float q[64], acc[64];
#pragma unroll
  for (int d = 0; d < 64; ++d) {
    q[d] = ld(qp, d);
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const T* Kc = reinterpret_cast<const T*>(a.kv.k[a.layer]);
  const T* Vc = reinterpret_cast<const T*>(a.kv.v[a.layer]);
  for (int k0 = tlo; k0 <= thi; k0 += 64) {
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
      const int kk = i >> 6, d = i & 63;
      const int key = k0 + kk;
      float kv = 0.f, vv = 0.f;
      if (key <= thi) {
        const int64_t off = kv_offset(a.kv, a.layer, b, g, key) + d;
        kv = ld(Kc, off);
        vv = ld(Vc, off);
      }
      Ks[kk][d] = kv;
      Vs[kk][d] = vv;
    }
    __syncthreads();
    float sc[64];
    float tmax = -INFINITY;
#pragma unroll
    for (int kk = 0; kk < 64; ++kk) {
      const int key = k0 + kk;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < 64; ++d) s += q[d] * Ks[kk][d];
      s *= a.scale;
      const bool ok = qvalid && key >= qlo && key <= qhi;
      sc[kk] = ok ? s : -INFINITY;
      tmax = fmaxf(tmax, sc[kk]);
    }
    if (tmax != -INFINITY) {
      const float mn = fmaxf(m, tmax);
      const float f = (m == -INFINITY) ? 0.f : expf(m - mn);
      l *= f;
#pragma unroll
      for (int d = 0; d < 64; ++d) acc[d] *= f;
#pragma unroll
      for (int kk = 0; kk < 64; ++kk) {
        const float p = sc[kk] == -INFINITY ? 0.f : expf(sc[kk] - mn);
        l += p;
#pragma unroll
        for (int d = 0; d < 64; ++d) acc[d] += p * Vs[kk][d];
      }
      m = mn;
    }
  }
  if (!qvalid) return;
  const float gate = to_f(reinterpret_cast<const T*>(a.gate)[row * a.H + head]);
  T* op = reinterpret_cast<T*>(a.out) + row * a.H * 64 + head * 64;
  const float inv = 1.0f / l;
#pragma unroll
  for (int d = 0; d < 64; ++d) op[d] = from_f<T>(rnd<T>(acc[d] * inv) * gate);
}

// ---------------------------------------------------------------------------
// Decode router: fp32 logits of the normed row, centred sigmoid + bias, top-k, and the
// per-expert assignment lists of this layer.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) router_decode_kernel(RouterArgs a) {
  __shared__ float part[4][32];
  __shared__ float lg[32];
  const int r = blockIdx.x;
  if (r >= a.ctl->n_rows) return;
  const int pulse = a.rows[r].pulse;
  const int E = a.E, D = a.D;
  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)r * D;
  const float* W = a.w + (int64_t)pulse * E * D;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int e = 0; e < E; ++e) {
    float s = 0.f;
    for (int i = threadIdx.x; i < D; i += blockDim.x) s += ld(x, i) * W[(int64_t)e * D + i];
    s = wave_sum(s);
    if (lane == 0) part[wv][e] = s;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int e = 0; e < E; ++e) lg[e] = part[0][e] + part[1][e] + part[2][e] + part[3][e];
  route_topk<T>(lg, E, a.K, a.bias + (int64_t)pulse * E, r, a);
}

// mlp_norm + decode router in one pass over the residual row.
template <typename T, int E, int NPER>
__global__ void __launch_bounds__(256) norm_router_kernel(RouterArgs a) {
  __shared__ float red[16];
  __shared__ float part[4][E];
  __shared__ float lg[32];
  const int r = blockIdx.x;
  if (r >= a.ctl->n_rows) return;
  const int pulse = a.rows[r].pulse;
  const int D = a.D;
  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)r * D;
  const float* nw = a.norm_w + (int64_t)pulse * D;
  const float* W = a.w + (int64_t)pulse * E * D;
  float xv[NPER];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NPER; ++c) {
    const int i = threadIdx.x + c * 256;
    xv[c] = ld(x, i);
    ss += xv[c] * xv[c];
  }
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  T* xn = reinterpret_cast<T*>(a.xn) + (int64_t)r * D;
#pragma unroll
  for (int c = 0; c < NPER; ++c) {
    const int i = threadIdx.x + c * 256;
    const float y = rnd<T>(nw[i] * (xv[c] * inv));
    xn[i] = from_f<T>(y);
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] += y * W[(int64_t)e * D + i];
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float v = wave_sum(acc[e]);
    if (lane == 0) part[wv][e] = v;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int e = 0; e < E; ++e) lg[e] = part[0][e] + part[1][e] + part[2][e] + part[3][e];
  route_topk<T>(lg, E, a.K, a.bias + (int64_t)pulse * E, r, a);
}

// Prefill router: logits in the activation dtype with T-rounded weights.
template <typename T>
__global__ void __launch_bounds__(256) router_prefill_kernel(RouterArgs a) {
  __shared__ float part[4][32];
  __shared__ float lg[32];
  const int r = blockIdx.x;
  if (r >= a.m_fixed) return;
  const int E = a.E, D = a.D;
  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)r * D;
  const float* W = a.w + (int64_t)a.pulse * E * D;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int e = 0; e < E; ++e) {
    float s = 0.f;
    for (int i = threadIdx.x; i < D; i += blockDim.x)
      s += ld(x, i) * rnd<T>(W[(int64_t)e * D + i]);
    s = wave_sum(s);
    if (lane == 0) part[wv][e] = s;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int e = 0; e < E; ++e) lg[e] = rnd<T>(part[0][e] + part[1][e] + part[2][e] + part[3][e]);
  route_topk<T>(lg, E, a.K, a.bias + (int64_t)a.pulse * E, r, a);
}

// ---------------------------------------------------------------------------
// Prefill capacity: per (sequence, expert) count, then the rank of each assignment in
// (weight desc, flat index asc) order via the float key e - 0.5*w/(1+w); assignments
// ranked >= capacity are dropped. Kept assignments are appended to the expert lists.
// ---------------------------------------------------------------------------
__global__ void prefill_count_kernel(const int32_t* __restrict__ idx, int32_t* __restrict__ cnt,
                                     int T_, int K, int E, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int b = (int)(i / ((int64_t)T_ * K));
  atomicAdd(&cnt[b * E + idx[i]], 1);
}

__global__ void prefill_slots_kernel(const int32_t* __restrict__ idx, const float* __restrict__ w,
                                     const int32_t* __restrict__ cnt, int32_t* __restrict__ keep,
                                     int32_t* __restrict__ lists, int32_t* __restrict__ lcount,
                                     int64_t list_stride, int T_, int K, int E, int C,
                                     int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t per = (int64_t)T_ * K;
  const int b = (int)(i / per);
  const int e = idx[i];
  bool kept = true;
  if (cnt[b * E + e] > C) {
    const float wi = fmaxf(w[i], 0.f);
    const float ki = (float)e - (wi / (1.0f + wi)) * 0.5f;
    int rank = 0;
    const int64_t s0 = (int64_t)b * per;
    for (int64_t j = s0; j < s0 + per; ++j) {
      if (idx[j] != e || j == i) continue;
      const float wj = fmaxf(w[j], 0.f);
      const float kj = (float)e - (wj / (1.0f + wj)) * 0.5f;
      if (kj < ki || (kj == ki && j < i)) ++rank;
    }
    kept = rank < C;
  }
  keep[i] = kept ? 1 : 0;
  if (kept) {
    const int p = atomicAdd(&lcount[e], 1);
    lists[(int64_t)e * list_stride + p] = (int32_t)i;
  }
}

// ---------------------------------------------------------------------------
// MoE combine + residual.
// decode: routed = sum_k T(out_k * w_k) in T, mlp = T(shared + T(routed * rs)), h += mlp.
// prefill: routed = index_add of T(w_k * out_k) in T (dropped = 0), mlp = T(shared + routed).
// ---------------------------------------------------------------------------
template <typename T, int NPER>
__global__ void __launch_bounds__(256) moe_combine_rows_kernel(CombineArgs a) {
  const int r = blockIdx.x;
  const int n = a.ctl ? a.ctl->n_rows : a.m_fixed;
  if (r >= n) return;
  const int K = a.K, D = a.D;
  const T* sh = reinterpret_cast<const T*>(a.shared) + (int64_t)r * D;
  const T* ro = reinterpret_cast<const T*>(a.routed) + (int64_t)r * K * D;
  T* h = reinterpret_cast<T*>(a.h) + (int64_t)r * D;
  float w[8];
  bool kept[8];
  for (int k = 0; k < K; ++k) {
    w[k] = a.topk_w[(int64_t)r * K + k];
    kept[k] = a.keep ? a.keep[(int64_t)r * K + k] != 0 : true;
  }
  const int pulse = a.ctl ? a.rows[r].pulse : a.pulse;
  const T* rs = reinterpret_cast<const T*>(a.routed_scale) + (int64_t)pulse * D;
  float hv[NPER];
#pragma unroll
  for (int c = 0; c < NPER; ++c) {
    const int i = threadIdx.x + c * 256;
    float routed = 0.f, mlp;
    if (!a.prefill) {
      for (int k = 0; k < K; ++k) routed = rnd<T>(routed + rnd<T>(ld(ro, (int64_t)k * D + i) * w[k]));
      mlp = rnd<T>(ld(sh, i) + rnd<T>(routed * ld(rs, i)));
    } else {
      for (int k = 0; k < K; ++k) {
        const float cv = kept[k] ? rnd<T>(w[k] * ld(ro, (int64_t)k * D + i)) : 0.f;
        routed = rnd<T>(routed + cv);
      }
      mlp = rnd<T>(ld(sh, i) + routed);
    }
    hv[c] = rnd<T>(ld(h, i) + mlp);
  }
  __shared__ float red[16];
  store_and_norm<T, NPER>(hv, (T*)nullptr, h, a.next_norm ? a.next_norm + (int64_t)pulse * D : nullptr,
                    reinterpret_cast<T*>(a.xn) + (int64_t)r * D, D, a.eps, red);
}

// ---------------------------------------------------------------------------
// Pulse output (harmonic residual) and, for rows that need logits, the final RMSNorm.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) pulse_output_kernel(PulseOutputArgs a) {
  __shared__ float red[16];
  const int r = blockIdx.x;
  if (r >= a.ctl->n_rows) return;
  const RowDesc rd = a.rows[r];
  const int D = a.D;
  const int st = a.prefill ? rd.pos + rd.seq * a.prefill_T : rd.seq * 2 + rd.slot;
  const T* hi = reinterpret_cast<const T*>(a.h_in) + (int64_t)r * D;
  const T* h = reinterpret_cast<const T*>(a.h) + (int64_t)r * D;
  const T* rs = reinterpret_cast<const T*>(a.res_scale) + (int64_t)rd.pulse * D;
  T* out = reinterpret_cast<T*>(a.hout_state) + (int64_t)st * D;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const float x = ld(hi, i);
    out[i] = from_f<T>(x + rnd<T>(rnd<T>(ld(h, i) - x) * ld(rs, i)));
  }
  if (rd.lrow < 0) return;
  __syncthreads();
  const float inv = row_inv_rms(out, D, a.eps, red);
  T* y = reinterpret_cast<T*>(a.xn_final) + (int64_t)rd.lrow * D;
  for (int i = threadIdx.x; i < D; i += blockDim.x) y[i] = from_f<T>(a.final_norm[i] * (ld(out, i) * inv));
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
#define PULSAR_DISPATCH(dtype, KERNEL, grid, block, arg)                      \
  do {                                                                        \
    if ((dtype) == PULSAR_BF16)                                               \
      KERNEL<bf16><<<(grid), (block), 0, s>>>(arg);                           \
    else                                                                      \
      KERNEL<float><<<(grid), (block), 0, s>>>(arg);                          \
    PULSAR_LAUNCH_CHECK();                                                    \
    return PULSAR_OK;                                                         \
  } while (0)

// Row kernels hold D/256 elements per thread in registers (D a multiple of 256, <= 2048).
#define PULSAR_NPER_DISPATCH(D, KERNEL_T, grid, arg)                                         \
  do {                                                                                       \
    const int _nper = (D) / 256;                                                             \
    if ((D) % 256 != 0 || _nper < 1 || _nper > kMaxPer)                                      \
      return fail(PULSAR_ERR_UNSUPPORTED, "d_model must be a multiple of 256 up to 2048");   \
    switch (_nper) {                                                                         \
      case 1: KERNEL_T(1)<<<(grid), 256, 0, s>>>(arg); break;                                \
      case 2: KERNEL_T(2)<<<(grid), 256, 0, s>>>(arg); break;                                \
      case 4: KERNEL_T(4)<<<(grid), 256, 0, s>>>(arg); break;                                \
      case 8: KERNEL_T(8)<<<(grid), 256, 0, s>>>(arg); break;                                \
      default: return fail(PULSAR_ERR_UNSUPPORTED, "d_model/256 must be 1, 2, 4 or 8");      \
    }                                                                                        \
    PULSAR_LAUNCH_CHECK();                                                                   \
    return PULSAR_OK;                                                                        \
  } while (0)

int launch_pulse_input(const PulseInputArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (dtype == PULSAR_BF16) {
#define K_(N) pulse_input_kernel<bf16, N>
    PULSAR_NPER_DISPATCH(a.D, K_, dim3(max_rows), a);
#undef K_
  }
#define K_(N) pulse_input_kernel<float, N>
  PULSAR_NPER_DISPATCH(a.D, K_, dim3(max_rows), a);
#undef K_
}
int launch_norm_rows(const NormArgs& a, int dtype, int max_rows, hipStream_t s) {
  PULSAR_DISPATCH(dtype, norm_rows_kernel, dim3(max_rows), 256, a);
}
int launch_qk_post(const QKPostArgs& a, int dtype, int max_rows, hipStream_t s) {
  PULSAR_DISPATCH(dtype, qk_post_kernel, dim3(max_rows, (a.H + a.Hkv + 3) / 4), 256, a);
}
int launch_attn_decode(const AttnArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (dtype == PULSAR_BF16)
    attn_decode_kernel<bf16><<<dim3(max_rows, a.Hkv, a.max_splits), 256, 0, s>>>(a);
  else
    attn_decode_kernel<float><<<dim3(max_rows, a.Hkv, a.max_splits), 256, 0, s>>>(a);
  PULSAR_LAUNCH_CHECK();
  PULSAR_DISPATCH(dtype, attn_combine_kernel, dim3(max_rows, a.H / 4), 256, a);
}
int launch_attn_prefill(const AttnArgs& a, int dtype, int B, hipStream_t s) {
  const int ntile = (a.prefill_T + 63) / 64;
  PULSAR_DISPATCH(dtype, attn_prefill_kernel, dim3(B * ntile, a.Hkv), 256, a);
}
int launch_router_decode(const RouterArgs& a, int dtype, int max_rows, hipStream_t s) {
  PULSAR_DISPATCH(dtype, router_decode_kernel, dim3(max_rows), 256, a);
}
int launch_norm_router(const RouterArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (a.D > 256 * kMaxPer) return fail(PULSAR_ERR_UNSUPPORTED, "norm_router: d_model > 2048");
#define PULSAR_NR_CASE(EV)                                                  \
  if (a.E == EV) {                                                          \
    if (dtype == PULSAR_BF16) {                                             \
      PULSAR_NPER_DISPATCH(a.D, K_BF16_##EV, dim3(max_rows), a);            \
    }                                                                       \
    PULSAR_NPER_DISPATCH(a.D, K_F32_##EV, dim3(max_rows), a);               \
  }
#define K_BF16_16(N) norm_router_kernel<bf16, 16, N>
#define K_F32_16(N) norm_router_kernel<float, 16, N>
#define K_BF16_8(N) norm_router_kernel<bf16, 8, N>
#define K_F32_8(N) norm_router_kernel<float, 8, N>
  PULSAR_NR_CASE(16)
  PULSAR_NR_CASE(8)
#undef K_BF16_16
#undef K_F32_16
#undef K_BF16_8
#undef K_F32_8
#undef PULSAR_NR_CASE
  return fail(PULSAR_ERR_UNSUPPORTED, "norm_router: n_experts must be 8 or 16");
}
int launch_router_prefill(const RouterArgs& a, int dtype, hipStream_t s) {
  PULSAR_DISPATCH(dtype, router_prefill_kernel, dim3(a.m_fixed), 256, a);
}
int launch_prefill_capacity(const int32_t* idx, const float* w, int32_t* cnt, int32_t* keep,
                            int32_t* lists, int32_t* lcount, int64_t list_stride, int B, int T_,
                            int K, int E, int C, hipStream_t s) {
  const int64_t total = (int64_t)B * T_ * K;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  prefill_count_kernel<<<blocks, 256, 0, s>>>(idx, cnt, T_, K, E, total);
  PULSAR_LAUNCH_CHECK();
  prefill_slots_kernel<<<blocks, 256, 0, s>>>(idx, w, cnt, keep, lists, lcount, list_stride, T_,
                                              K, E, C, total);
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}
int launch_moe_combine(const CombineArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (dtype == PULSAR_BF16) {
#define K_(N) moe_combine_rows_kernel<bf16, N>
    PULSAR_NPER_DISPATCH(a.D, K_, dim3(max_rows), a);
#undef K_
  }
#define K_(N) moe_combine_rows_kernel<float, N>
  PULSAR_NPER_DISPATCH(a.D, K_, dim3(max_rows), a);
#undef K_
}
int launch_pulse_output(const PulseOutputArgs& a, int dtype, int max_rows, hipStream_t s) {
  PULSAR_DISPATCH(dtype, pulse_output_kernel, dim3(max_rows), 256, a);
}
int launch_prefill_stem(const int32_t* ids, const void* emb, const float* anchor_w,
                        const float* conv_w, void* a_buf, void* e_buf, int B, int T_, int D,
                        float eps, int dtype, hipStream_t s) {
  const int n = B * T_;
  const int64_t total = (int64_t)n * D;
  if (dtype == PULSAR_BF16) {
    prefill_embed_kernel<bf16><<<n, 256, 0, s>>>(ids, (const bf16*)emb, anchor_w, (bf16*)a_buf, D,
                                                 n, eps);
    prefill_conv_kernel<bf16><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
        (const bf16*)a_buf, conv_w, (bf16*)e_buf, T_, D, total);
  } else {
    prefill_embed_kernel<float><<<n, 256, 0, s>>>(ids, (const float*)emb, anchor_w, (float*)a_buf,
                                                  D, n, eps);
    prefill_conv_kernel<float><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
        (const float*)a_buf, conv_w, (float*)e_buf, T_, D, total);
  }
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

}  // namespace pulsar
