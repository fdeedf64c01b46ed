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

__device__ __forceinline__ void store8(bf16* p, const float* v) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)f2bf(v[2 * i]).u |
           ((uint32_t)f2bf(v[2 * i + 1]).u << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ void store8(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
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

__device__ __forceinline__ float lerp_ref(float s, float e, float w) {
  // torch.lerp: start + w*(end-start) for |w| < 0.5, else end - (end-start)*(1-w)
  return fabsf(w) < 0.5f ? s + w * (e - s) : e - (e - s) * (1.0f - w);
}

}  // namespace

// ---------------------------------------------------------------------------
// Pulse input. pulse 0: stem (decode: embed, anchor norm, conv over one token) + step
// embedding. pulse >= 1: rank-r re-injection gate on (anchor, state-normed previous pulse).
// ---------------------------------------------------------------------------
// RT: rank bound of the re-injection gate; EXACT: the rank equals RT (no rank guards).
template <typename T, int EPL, int RT, bool EXACT>
__global__ void __launch_bounds__(64) pulse_input_kernel(PulseInputArgs a) {
  // one wave per row; lane owns elements [lane*EPL, lane*EPL + EPL)
  const int lane = threadIdx.x;
  if (blockIdx.x == 0 && a.zero_counts) {
    for (int i = lane; i < a.n_zero; i += 64) a.zero_counts[i] = 0;
  }
  const int r = blockIdx.x;
  // the row descriptor is read with the row count (the rows buffer holds a descriptor for
  // every block of the grid; the empty asm keeps the load ahead of the count test), and the
  // pulse-indexed vectors, the next layer norm's included, right after it
  const RowDesc rd = a.rows[r];
  asm volatile("" ::: "memory");
  if (r >= a.ctl->n_rows) return;
  const int D = a.D, i0 = lane * EPL;
  const int st = a.prefill ? rd.pos + rd.seq * a.prefill_T : rd.seq * a.slots + rd.sslot;
  T* e = reinterpret_cast<T*>(a.e_state) + (int64_t)st * D;
  const T* step = reinterpret_cast<const T*>(a.step_emb) + (int64_t)rd.pulse * D;
  float hv[EPL], nw[EPL];
  // the step vector stays in its storage type until its use inside the branches below
  // (converted here, its loads made the branches' loads wait for them)
  T stp_raw[EPL];
  if constexpr ((EPL * sizeof(T)) % 16 == 0) {
#pragma unroll
    for (int w = 0; w < (int)(EPL * sizeof(T) / 16); ++w)
      reinterpret_cast<uint4*>(stp_raw)[w] = reinterpret_cast<const uint4*>(step + i0)[w];
  } else {
#pragma unroll
    for (int c = 0; c < EPL; ++c) stp_raw[c] = step[i0 + c];
  }
  auto stp = [&](int c) { return to_f(stp_raw[c]); };
  if (a.norm_w) ldv<EPL>(a.norm_w + (int64_t)rd.pulse * D + i0, nw);
  if (rd.pulse == 0) {
    if (!a.prefill) {
      const T* x0 = reinterpret_cast<const T*>(a.tok_emb) + (int64_t)rd.token * D;
      float x[EPL], an[EPL];
      ldv<EPL>(x0 + i0, x);
      ldv<EPL>(a.anchor_norm + i0, an);
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < EPL; ++c) ss += x[c] * x[c];
      const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
      float ev[EPL];
#pragma unroll
      for (int c = 0; c < EPL; ++c) {
        float v = rnd<T>(x[c] * inv * an[c]);
        if (a.conv_w) v = rnd<T>(v + a.conv_w[(i0 + c) * 4] * v);
        ev[c] = v;
        hv[c] = rnd<T>(v + stp(c));
      }
      stv<EPL>(e + i0, ev);
    } else {
      float ev[EPL];
      ldv<EPL>(e + i0, ev);
#pragma unroll
      for (int c = 0; c < EPL; ++c) hv[c] = rnd<T>(ev[c] + stp(c));
    }
  } else if constexpr (EXACT && sizeof(T) == 2 && EPL % 8 == 0 && EPL <= 16) {
    // The same re-injection as the general branch below, with every load of the row (state,
    // norm, bias and all 2R + D/64 weight vectors of this lane) issued before the first
    // reduction: one memory round trip instead of one per rank.
    const bf16* hp = reinterpret_cast<const bf16*>(a.hout_state) + (int64_t)st * D;
    const bf16* wd = reinterpret_cast<const bf16*>(a.reinject_down) + (int64_t)rd.pulse * RT * 2 * D;
    const bf16* wu = reinterpret_cast<const bf16*>(a.reinject_up) + (int64_t)rd.pulse * D * RT;
    const bf16* bu = reinterpret_cast<const bf16*>(a.reinject_bias) + (int64_t)rd.pulse * D;
    constexpr int QV = EPL / 8, QU = RT / 8;
    uint4 rwe[RT][QV], rwr[RT][QV], rwu[EPL][QU];
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int q = 0; q < QV; ++q) {
        rwe[j][q] = *reinterpret_cast<const uint4*>(wd + (int64_t)j * 2 * D + i0 + 8 * q);
        rwr[j][q] = *reinterpret_cast<const uint4*>(wd + (int64_t)j * 2 * D + D + i0 + 8 * q);
      }
#pragma unroll
    for (int c = 0; c < EPL; ++c)
#pragma unroll
      for (int q = 0; q < QU; ++q)
        rwu[c][q] = *reinterpret_cast<const uint4*>(wu + (int64_t)(i0 + c) * RT + 8 * q);
    float ev[EPL], hpv[EPL], sn[EPL], bv[EPL];
    ldv<EPL>(e + i0, ev);
    ldv<EPL>(hp + i0, hpv);
    ldv<EPL>(a.state_norm + i0, sn);
    ldv<EPL>(bu + i0, bv);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < EPL; ++c) ss += hpv[c] * hpv[c];
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
    float rv[EPL];
#pragma unroll
    for (int c = 0; c < EPL; ++c) rv[c] = rnd<T>(hpv[c] * inv * sn[c]);
    float gh[RT];
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      float we[EPL], wr[EPL];
#pragma unroll
      for (int q = 0; q < QV; ++q) {
        unpack_bf16x8(rwe[j][q], we + 8 * q);
        unpack_bf16x8(rwr[j][q], wr + 8 * q);
      }
      float pe = 0.f, pr = 0.f;
#pragma unroll
      for (int c = 0; c < EPL; ++c) {
        pe += ev[c] * we[c];
        pr += rv[c] * wr[c];
      }
      gh[j] = rnd<T>(rnd<T>(wave_sum(pe)) + rnd<T>(wave_sum(pr)));
    }
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      float wv[RT];
#pragma unroll
      for (int q = 0; q < QU; ++q) unpack_bf16x8(rwu[c][q], wv + 8 * q);
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < RT; ++j) acc += gh[j] * wv[j];
      const float mix = rnd<T>(sigmoidf_(rnd<T>(acc + bv[c])));
      hv[c] = rnd<T>(rnd<T>(lerp_ref(rv[c], ev[c], mix)) + stp(c));
    }
  } else {
    // rank-R re-injection: g = T(T(e . wd[j][:D]) + T(r . wd[j][D:])), mix = sigmoid(up g + b)
    const T* hp = reinterpret_cast<const T*>(a.hout_state) + (int64_t)st * D;
    const int R = EXACT ? RT : a.rank;
    const T* wd = reinterpret_cast<const T*>(a.reinject_down) + (int64_t)rd.pulse * R * 2 * D;
    const T* wu = reinterpret_cast<const T*>(a.reinject_up) + (int64_t)rd.pulse * D * R;
    const T* bu = reinterpret_cast<const T*>(a.reinject_bias) + (int64_t)rd.pulse * D;
    float ev[EPL], hpv[EPL], sn[EPL], bv[EPL];
    ldv<EPL>(e + i0, ev);
    ldv<EPL>(hp + i0, hpv);
    ldv<EPL>(a.state_norm + i0, sn);
    ldv<EPL>(bu + i0, bv);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < EPL; ++c) ss += hpv[c] * hpv[c];
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
    float rv[EPL];
#pragma unroll
    for (int c = 0; c < EPL; ++c) rv[c] = rnd<T>(hpv[c] * inv * sn[c]);
    float gh[RT];
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int jj = j < R ? j : 0;  // ranks past R load rank 0 and are dropped
      float we[EPL], wr[EPL];
      ldv<EPL>(wd + (int64_t)jj * 2 * D + i0, we);
      ldv<EPL>(wd + (int64_t)jj * 2 * D + D + i0, wr);
      float pe = 0.f, pr = 0.f;
#pragma unroll
      for (int c = 0; c < EPL; ++c) {
        pe += ev[c] * we[c];
        pr += rv[c] * wr[c];
      }
      gh[j] = 0.f;
      if (EXACT || j < R) gh[j] = rnd<T>(rnd<T>(wave_sum(pe)) + rnd<T>(wave_sum(pr)));
    }
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      float wv[RT];
      if (EXACT) {
        ldv<RT>(wu + (int64_t)(i0 + c) * RT, wv);
      } else {
#pragma unroll
        for (int j = 0; j < RT; ++j) wv[j] = j < R ? ld(wu, (int64_t)(i0 + c) * R + j) : 0.f;
      }
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < RT; ++j)
        if (EXACT || j < R) acc += gh[j] * wv[j];
      const float mix = rnd<T>(sigmoidf_(rnd<T>(acc + bv[c])));
      hv[c] = rnd<T>(rnd<T>(lerp_ref(rv[c], ev[c], mix)) + stp(c));
    }
  }
  T* h_in = reinterpret_cast<T*>(a.h_in) + (int64_t)r * D;
  T* h = reinterpret_cast<T*>(a.h) + (int64_t)r * D;
  stv<EPL>(h_in + i0, hv);
  stv<EPL>(h + i0, hv);
  if (a.norm_w) {
    float ss = 0.f, y[EPL];
#pragma unroll
    for (int c = 0; c < EPL; ++c) ss += hv[c] * hv[c];
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
#pragma unroll
    for (int c = 0; c < EPL; ++c) y[c] = rnd<T>(nw[c] * (hv[c] * inv));
    stv<EPL>(reinterpret_cast<T*>(a.xn) + (int64_t)r * D + i0, y);
  }
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
// A block of 256 threads normalises RPB rows; thread t holds elements t, t + 256, ... of
// each (D <= 256 EPT), summed in that order, then the wave sums and the 4 wave partials in
// wave order: each row's arithmetic is the same for every RPB. Every load of the block,
// the norm weights included, is issued before the first reduction: with the loads behind a
// per-element bounds branch each one waited for the last (prefill of 16 x 2048 tokens:
// 59.6 -> 38.8 us per launch; the weights loaded up front 39.4 -> 35.7 us at 8 rows per
// block, 27.7 us at 4, 28.9 us at 2). Prefill takes 4 rows per block, decode steps and
// logits rows one.
// ---------------------------------------------------------------------------
template <typename T, int RPB, int EPT>
__global__ void __launch_bounds__(256) norm_rows_kernel(NormArgs a) {
  __shared__ float red[RPB][4];
  const int n = a.use_lrows ? a.ctl->n_lrows : a.ctl->n_rows;
  const int r0 = blockIdx.x * RPB;
  if (r0 >= n) return;
  const int D = a.D, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  float xv[RPB][EPT], wt[RPB][EPT], inv[RPB];
  // loads branch-free (a load on one side of a branch makes the join wait for every load
  // in flight): elements past D read element D - 1 and count as zero; the norm weights go
  // out with the rows, ahead of the reduction
#pragma unroll
  for (int j = 0; j < RPB; ++j) {
    const int r = min(r0 + j, n - 1);  // rows past n recompute the last row, never stored
    const int src = a.use_lrows ? a.lrow_src[r] : r;
    const int pulse = a.use_lrows ? 0 : a.rows[r].pulse;
    const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)src * a.ldx;
    const float* w = a.w + (int64_t)pulse * a.w_pulse_stride;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      xv[j][k] = ld(x, min(t + 256 * k, D - 1));
      wt[j][k] = w[min(t + 256 * k, D - 1)];
    }
  }
#pragma unroll
  for (int j = 0; j < RPB; ++j) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const float v = xv[j][k];
      if (t + 256 * k < D) ss += v * v;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[j][wv] = ss;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < RPB; ++j) {
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) tot += red[j][i];
    inv[j] = 1.0f / sqrtf(tot / (float)D + a.eps);
  }
#pragma unroll
  for (int j = 0; j < RPB; ++j) {
    if (r0 + j >= n) break;
    T* y = reinterpret_cast<T*>(a.y) + (int64_t)(r0 + j) * a.D;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int i = t + 256 * k;
      if (i < D) y[i] = from_f<T>(wt[j][k] * (xv[j][k] * inv[j]));
    }
  }
}

// ---------------------------------------------------------------------------
// QK-norm + RoPE (+YaRN) on q heads, value residual + K-norm + RoPE on kv heads and the
// cache write. One wave per head vector (lane = element, rotate-half partner = lane^32);
// a wave takes head hh of RPW consecutive rows, their loads issued before the first
// reduction (prefill: 8 rows; decode: 1). The value cache is dimension-major: 8 rows of one
// sequence at consecutive positions from a multiple of 8 leave each lane 8 adjacent values
// of its dimension row, stored as one vector (16 x 2048 tokens: 117 us per launch with one
// row per wave and element stores, 104 with 2 rows, 95 with 8 rows and vector stores).
// Prefill and fp32 decode; bf16 decode does the same arithmetic inside
// attn_decode_unit_kernel.
// ---------------------------------------------------------------------------
template <typename T, int RPW>
__global__ void __launch_bounds__(256) qk_post_kernel(QKPostArgs a) {
  const int n = a.ctl->n_rows;
  const int r0 = blockIdx.x * RPW;
  if (r0 >= n) return;
  const int hh = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int H = a.H, Hk = a.Hkv;
  if (hh >= H + Hk) return;
  const int lane = threadIdx.x & 63;
  const int j = lane & 31;
  // the wave's rows: r0 .. r0 + RPW - 1 (rows past n recompute the last row, never stored);
  // every load of a path is issued before its first reduction, branch-free (a load on one
  // side of a branch makes the join wait for every load in flight)
  auto row_of = [&](int i) { return min(r0 + i, n - 1); };
  auto norm_rope = [&](float xx, const float* w, float c, float sv) {
    const float ss = wave_sum(xx * xx);
    const float inv = 1.0f / sqrtf(ss / 64.0f + a.eps);
    const float y = rnd<T>(w[lane] * (xx * inv));
    const float p = __shfl_xor(y, 32, 64);
    return rnd<T>(lane < 32 ? y * c - p * sv : y * c + p * sv);
  };
  RowDesc rd[RPW];
  float x[RPW], cs[RPW], sn[RPW];
  if (hh < H) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = row_of(i);
      rd[i] = a.rows[r];
      x[i] = ld(reinterpret_cast<const T*>(a.qkv) + (int64_t)r * a.ldq, hh * 64 + lane);
      cs[i] = a.cos[(int64_t)rd[i].pos * 32 + j];
      sn[i] = a.sin[(int64_t)rd[i].pos * 32 + j];
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      if (r0 + i >= n) break;
      const int pulse = rd[i].pulse, pos = rd[i].pos;
      float y = norm_rope(x[i], a.q_norm + ((int64_t)pulse * H + hh) * 64, cs[i], sn[i]);
      if (!a.prefill && !a.is_local && pos + 1 > a.base_seq_len) {
        const double base = (double)a.base_seq_len;
        const double pp = (double)(pos + 1) > base ? (double)(pos + 1) : base;
        const float scale = (float)(1.0 + 0.1 * log(pp / base));
        y = rnd<T>(y * scale);
      }
      reinterpret_cast<T*>(a.qkv)[(int64_t)(r0 + i) * a.ldq + hh * 64 + lane] = from_f<T>(y);
    }
    return;
  }
  const int g = hh - H;
  float v[RPW], vf0[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = row_of(i);
    rd[i] = a.rows[r];
    const T* q = reinterpret_cast<const T*>(a.qkv) + (int64_t)r * a.ldq;
    x[i] = ld(q, H * 64 + g * 64 + lane);
    v[i] = ld(q, H * 64 + Hk * 64 + g * 64 + lane);
    // value-first element, used by pulse-0 rows of layers after the first (layer 0 writes it)
    vf0[i] = to_f(reinterpret_cast<const T*>(a.v_first)[(int64_t)r * Hk * 64 + g * 64 + lane]);
    cs[i] = a.cos[(int64_t)rd[i].pos * 32 + j];
    sn[i] = a.sin[(int64_t)rd[i].pos * 32 + j];
  }
  bool keep[RPW];  // row stored (exists and not before a prefill's window)
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    keep[i] = false;
    if (r0 + i >= n) break;
    const int r = r0 + i;
    const int pulse = rd[i].pulse, pos = rd[i].pos;
    float vv = v[i];
    if (pulse == 0) {
      T* vf = reinterpret_cast<T*>(a.v_first) + (int64_t)r * Hk * 64 + g * 64 + lane;
      if (a.layer == 0) {
        *vf = from_f<T>(vv);
      } else {
        const float lv = a.v_lambda[pulse];
        vv = rnd<T>(rnd<T>(rnd<T>(1.0f - lv) * vv) + rnd<T>(lv * vf0[i]));
      }
    }
    v[i] = vv;
    const float k = norm_rope(x[i], a.k_norm + ((int64_t)pulse * Hk + g) * 64, cs[i], sn[i]);
    if (a.prefill && a.is_local && pos < a.prefill_T - a.window) continue;
    keep[i] = true;
    reinterpret_cast<T*>(a.kv.k[a.layer])[kv_offset(a.kv, a.layer, rd[i].seq, g, pos) + lane] =
        from_f<T>(k);
  }
  // V is stored dimension-major: 8 stored rows of one sequence at consecutive positions from
  // a multiple of 8 are 8 adjacent elements of the lane's dimension row, written as one
  // vector; other row sets go element by element
  T* Vc = reinterpret_cast<T*>(a.kv.v[a.layer]);
  bool vec = RPW % 8 == 0 && (rd[0].pos & 7) == 0 &&
             (!kv_is_local(a.kv, a.layer) || (a.kv.lcap & 7) == 0);
#pragma unroll
  for (int i = 0; i < (RPW % 8 == 0 ? 8 : 0); ++i)
    vec = vec && keep[i] && rd[i].seq == rd[0].seq && rd[i].pos == rd[0].pos + i;
  if (vec) {
    T* vp = Vc + kv_offset_v(a.kv, a.layer, rd[0].seq, g, rd[0].pos, lane);
    store8(vp, v);
#pragma unroll
    for (int i = 8; i < RPW; ++i)
      if (keep[i]) Vc[kv_offset_v(a.kv, a.layer, rd[i].seq, g, rd[i].pos, lane)] = from_f<T>(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < RPW; ++i)
      if (keep[i]) Vc[kv_offset_v(a.kv, a.layer, rd[i].seq, g, rd[i].pos, lane)] = from_f<T>(v[i]);
  }
}

// ---------------------------------------------------------------------------
// Decode attention for fp32 caches (the bf16 path runs on the matrix cores below), split
// over keys: block (row, kv head, split) serves the 4 query heads of the group over up to
// 256 keys, 64 per wave. Lane l owns key group (l >> 3), i.e. keys
// kbeg + (l >> 3) + 8i for i < 8, and dims 8*(l & 7) .. +8, so each K and V load is 128
// contiguous bits and every 8 lanes read one 128-byte key row: the wave reads 1 KB of
// contiguous cache per load instruction (V, stored dimension-major, is gathered per
// element: this path is for exactness, not speed). Scores are reduced over the 8 lanes of a key
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
#pragma unroll
    for (int d = 0; d < 8; ++d)
      vf[i][d] = valid[i] ? ld(Vc, kv_offset_v(a.kv, a.layer, rd.seq, g, key, dc * 8 + d)) : 0.f;
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
// Decode attention on the matrix cores (bf16 caches): shared types and the unit key range.
// A unit is the rows of one sequence in a step, at consecutive positions pos0 + i (the
// current token and the speculative token one position later, or the rows of a draft
// block); they read each key block of the cache once. Row i sees keys
// [lo(pos0 + i), pos0 + i]: row 0 has the lowest bound, the last row the highest key.
// ---------------------------------------------------------------------------
typedef __bf16 attn_bf16x8 __attribute__((ext_vector_type(8)));
typedef float attn_f32x4 __attribute__((ext_vector_type(4)));

// Splits of SPLIT keys start at multiples of SPLIT, so the 64-key blocks a row's keys fall
// in, the wave and split that compute each block, and the order of every sum (within a wave,
// across the waves, across the splits) are fixed by the row's own position: a row gives the
// same result alone or in a unit with other rows (the speculative row of the exact schedule,
// the rows of a draft block).
template <int SPLIT>
__device__ __forceinline__ void unit_range(const AttnArgs& a, const AttnUnit& un, int& base,
                                           int& uhi) {
  const int lo0 = a.is_local ? max(0, un.pos0 - a.window + 1) : 0;
  uhi = un.pos0 + un.n - 1;
  base = lo0 / SPLIT * SPLIT;
}

// Row of unit row z (z < NZ), -1 past the unit's rows: a select chain, so the unit stays
// in registers (no indexed register access).
template <int NZ>
__device__ __forceinline__ int unit_row(const AttnUnit& un, int z) {
  int row = -1;
#pragma unroll
  for (int i = 0; i < NZ; ++i)
    if (z == i) row = un.row[i];
  return z < un.n ? row : -1;
}

// Last split block of (unit u, kv head g): merge the split partials (device-coherent loads),
// normalise, round as the SDPA output and apply the head gate. Query column c = 4 z + h
// (unit row z, head h of the group); element t = 32 c + e0 / 2 (two dims of one column).
// A thread takes elements t, t + 256, ... of the unit's columns and issues the partial loads
// of all of them (kMergeChunk splits at a time) before the first use: one round trip per
// chunk however many rows the unit holds. Per element the splits are summed in order, so
// a row's result does not depend on the unit's other rows.
template <int COLS>
__device__ __forceinline__ void attn_merge_splits(const AttnArgs& a, int u, int g,
                                                  const AttnUnit& un, int nsplit) {
  constexpr int NT = 64 * kUnitWaves;
  constexpr int EPT = (COLS * 32 + NT - 1) / NT;  // elements per thread
  constexpr int CH = EPT > 2 ? 8 : 16;            // splits loaded per round trip
  const int nel = min(un.n, COLS / 4) * 4 * 32;  // a multiple of 128: whole waves drop out
  const int wbase = threadIdx.x & ~63;
  const float* part = a.part + (((int64_t)u * a.Hkv + g) * a.max_splits) * COLS * 66;
  float Mx[EPT], Ls[EPT], Oa[EPT], Ob[EPT], gate[EPT];
  int off[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int t = min((int)threadIdx.x + NT * e, nel - 1), c = t >> 5;
    off[e] = c * 66 + (t & 31) * 2;
    gate[e] = 0.f;
    if (NT * e + wbase < nel)
      gate[e] = to_f(reinterpret_cast<const bf16*>(a.gate)[(int64_t)unit_row<COLS / 4>(un, c >> 2) *
                                                           a.H + g * 4 + (c & 3)]);
    Mx[e] = -INFINITY;
    Ls[e] = Oa[e] = Ob[e] = 0.f;
  }
  for (int c0 = 0; c0 < nsplit; c0 += CH) {
    float pm[EPT][CH], pl[EPT][CH], pa[EPT][CH], pb[EPT][CH];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (NT * e + wbase >= nel) continue;
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const float* p = part + (int64_t)min(c0 + k, nsplit - 1) * COLS * 66;
        pm[e][k] = __hip_atomic_load(p + off[e] - (off[e] % 66), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pl[e][k] = __hip_atomic_load(p + off[e] - (off[e] % 66) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pa[e][k] = __hip_atomic_load(p + off[e] + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pb[e][k] = __hip_atomic_load(p + off[e] + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (NT * e + wbase >= nel) continue;
      float cm = Mx[e];
#pragma unroll
      for (int k = 0; k < CH; ++k)
        if (c0 + k < nsplit) cm = fmaxf(cm, pm[e][k]);
      const float f0 = Mx[e] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(Mx[e] - cm);
      Ls[e] *= f0;
      Oa[e] *= f0;
      Ob[e] *= f0;
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        if (c0 + k < nsplit && pm[e][k] != -INFINITY) {
          const float f = __builtin_amdgcn_exp2f(pm[e][k] - cm);
          Ls[e] += pl[e][k] * f;
          Oa[e] += pa[e][k] * f;
          Ob[e] += pb[e][k] * f;
        }
      }
      Mx[e] = cm;
    }
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int t = threadIdx.x + NT * e;
    if (t >= nel) continue;
    const int c = t >> 5, e0 = (t & 31) * 2;
    const int row = unit_row<COLS / 4>(un, c >> 2);
    bf16* dst = reinterpret_cast<bf16*>(a.out) + (int64_t)row * a.H * 64 + (g * 4 + (c & 3)) * 64 + e0;
    dst[0] = f2bf(rnd<bf16>(Oa[e] / Ls[e]) * gate[e]);
    dst[1] = f2bf(rnd<bf16>(Ob[e] / Ls[e]) * gate[e]);
  }
}

// ---------------------------------------------------------------------------
// Decode attention, one workgroup per (unit, kv head, split of kUnitSplit keys): kUnitWaves
// waves stride over the split's 64-key blocks, each keeping an online softmax over its
// blocks; the waves merge in LDS, and only a unit whose keys span several splits goes
// through the split partials. Products are formed transposed, as in the prefill kernel:
// S^T = K Q^T (A = 16 keys x 32 dims of the position-major K block, B = 16 query columns:
// column c = 4 z + h is head h of unit row z; COLS columns in COLS/16 tiles), so P^T stays
// in registers for O^T = V^T P^T, whose A operand is one 16-byte run of the dimension-major
// V block per lane (attn_key_of). P = exp(S - max) in fp32 is split into bf16 hi + lo (hi + lo =
// P to 2^-16 relative), two products each. The last split block to count in merges the
// split partials, normalises, rounds as the SDPA output and applies the head gate.
// The step's q/k/v post-processing is fused in (no separate launch): qkv holds the raw
// projection; every split finishes the unit's queries, and the split holding a row's own
// position finishes its key and value, patches them into the loaded block and stores them
// to the caches at the end (the arithmetic of qk_post_kernel, bit for bit).
// COLS = 8 serves units of up to 2 rows (exact mode), 16 up to 4, 32 up to 8. BPW = 64-key
// blocks per wave and split: long caches take BPW = 8 (2048-key splits) in the global
// layers and 4 in the sliding-window layers, shorter ones 2 (512-key splits). Holding the next block in registers while
// computing the current one (64 more registers: one wave per SIMD) and touching the next
// blocks' lines ahead of their loads were both measured slower at 64 x 8192 positions, and
// so was staging the blocks through LDS with direct global-to-LDS loads (2-stage rings of
// 16 KB per wave, 4-8 waves): slower at batch 16 x 2048 and 64 x 8192, 3 % faster only at
// 4 x 8192.
// ---------------------------------------------------------------------------
typedef __bf16 attn_bf16x4 __attribute__((ext_vector_type(4)));

struct AttnKV {
  attn_bf16x8 k[4][2];
  attn_bf16x4 vl[4][2], vh[4][2];
};

// Key order within a 64-key block: row m of S^T tile kt is key
// 32 (kt >> 1) + 8 (m >> 2) + 4 (kt & 1) + (m & 3). The S^T product leaves lane (m16, kq)
// rows 4 kq + j of each tile; the 8 P values it feeds the B operand of the s2-th O^T = V^T P^T
// product (tiles 2 s2 and 2 s2 + 1) are then keys 32 s2 + 8 kq .. + 7, consecutive, so the
// V^T operand (dimension-major V) is one 16-byte load per lane like the K operand (with keys
// in plain order it takes two 8-byte loads: 11.9 against 13.0 us per launch at batch 16).
__device__ __forceinline__ int attn_key_of(int kt, int m) {
  return 32 * (kt >> 1) + 8 * (m >> 2) + 4 * (kt & 1) + (m & 3);
}

// Lane (m16, kq): K rows attn_key_of(kt, m16), dims 32 ks + 8 kq (16 bytes); V^T rows (dims)
// 16 mt + m16, keys 32 s2 + 8 kq .. + 7 (16 bytes).
__device__ __forceinline__ void attn_load_block(const bf16* Kc, const bf16* Vc, const KVBlock& blk,
                                                int m16, int kq, AttnKV& r) {
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      r.k[kt][ks] = *reinterpret_cast<const attn_bf16x8*>(Kc + blk.k0 + attn_key_of(kt, m16) * 64 +
                                                          ks * 32 + kq * 8);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const bf16* vp = Vc + blk.v0 + (int64_t)(mt * 16 + m16) * blk.vstride + s2 * 32 + kq * 8;
      const attn_bf16x8 v8 = *reinterpret_cast<const attn_bf16x8*>(vp);
      r.vl[mt][s2] = __builtin_shufflevector(v8, v8, 0, 1, 2, 3);
      r.vh[mt][s2] = __builtin_shufflevector(v8, v8, 4, 5, 6, 7);
    }
}

// Pulse of step row `row` from the step's pulse row ranges [ps[q], ps[q] + pc[q]) (rows of
// a step are sorted by pulse).
__device__ __forceinline__ int step_row_pulse(const int* ps, const int* pc, int row) {
  int p = 0;
#pragma unroll
  for (int q = 1; q < kMaxPulses; ++q)
    if (row >= ps[q] && row < ps[q] + pc[q]) p = q;
  return p;
}

// Replace, in a loaded block at kb, the keys and values of positions [f_lo, f_hi] (rows
// z = pos - pos0 of the unit, finished in LDS by this workgroup) by their new values.
// Lane (m16, kq) holds K rows attn_key_of(kt, m16), dims 32 ks + 8 kq .. + 7, and V^T rows
// (dims) 16 mt + m16 of keys 32 s2 + 8 kq + e.
__device__ __forceinline__ void attn_patch_fresh(AttnKV& r, int kb, int f_lo, int f_hi, int pos0,
                                                 int m16, int kq, const uint16_t (*fk)[64],
                                                 const uint16_t (*fv)[64]) {
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const int p = kb + attn_key_of(kt, m16);
    if (p >= f_lo && p <= f_hi) {
      const int z = p - pos0;
      r.k[kt][0] = *reinterpret_cast<const attn_bf16x8*>(&fk[z][kq * 8]);
      r.k[kt][1] = *reinterpret_cast<const attn_bf16x8*>(&fk[z][32 + kq * 8]);
    }
  }
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int p = kb + 32 * s2 + 8 * kq + e;
      if (p >= f_lo && p <= f_hi) {
        const int z = p - pos0;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const __bf16 v = __builtin_bit_cast(__bf16, fv[z][16 * mt + m16]);
          if (e < 4)
            r.vl[mt][s2][e] = v;
          else
            r.vh[mt][s2][e - 4] = v;
        }
      }
    }
}

template <int COLS, int BPW>
__global__ void __launch_bounds__(64 * kUnitWaves)
__attribute__((amdgpu_waves_per_eu(COLS <= 16 ? 3 : 2))) attn_decode_unit_kernel(AttnArgs a) {
  constexpr int NQT = (COLS + 15) / 16;
  constexpr int NZ = COLS / 4;
  constexpr int SPLIT = kUnitSplit * BPW;
  __shared__ float wm[kUnitWaves][COLS], wl[kUnitWaves][COLS];
  __shared__ float wo[kUnitWaves][COLS][65];
  const int u = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
  // the unit descriptor is read together with the unit count (grid.x never exceeds the
  // units array), so the two loads share one round trip; the empty asm keeps the compiler
  // from sinking the descriptor load below the exit branch
  const int n_units = a.ctl->n_units;
  const AttnUnit un = a.units[u];
  // the step's pulse row ranges and the value-residual weight, read with the unit: scalar
  // loads ahead of every store and asm statement of the kernel (after either, the compiler
  // reads them with vector loads, each a round trip)
  int ps[kMaxPulses], pc[kMaxPulses];
#pragma unroll
  for (int q = 0; q < kMaxPulses; ++q) {
    ps[q] = a.ctl->pulse_start[q];
    pc[q] = a.ctl->pulse_count[q];
  }
  const float lv0 = a.v_lambda[0];
  asm volatile("" ::"s"(un.seq), "s"(un.n), "s"(un.pos0), "s"(un.row[0]), "s"(un.row[1]),
               "s"(un.row[2]), "s"(un.row[3]), "s"(un.row[4]), "s"(un.row[5]), "s"(un.row[6]),
               "s"(un.row[7]), "s"(ps[1]), "s"(ps[2]), "s"(pc[1]), "s"(pc[2]), "s"(lv0));
  asm volatile("" ::"s"(a.kl.k), "s"(a.kl.v), "s"(a.kl.lcap), "s"(a.kl.max_pages),
               "s"(a.kl.page_table),
               "s"(a.is_local), "s"(a.window), "s"(a.Hkv), "s"(a.qkv), "s"(a.ldq));
  if (u >= n_units) return;
  int base, uhi;
  unit_range<SPLIT>(a, un, base, uhi);
  const int nsplit = (uhi + 1 - base + SPLIT - 1) / SPLIT;
  if (s >= nsplit) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m16 = lane & 15, kq = lane >> 4;
  const attn_bf16x8 zero = {};
  const bf16* Kc = reinterpret_cast<const bf16*>(a.kl.k);
  const bf16* Vc = reinterpret_cast<const bf16*>(a.kl.v);
  const int s_lo = base + s * SPLIT;
  const int s_hi = min(uhi, s_lo + SPLIT - 1);
  constexpr int kStride = kUnitWaves * 64;
  // the wave's first block: blocks wholly before the unit's first key (sliding-window
  // layers: the first row's window start) are masked for every row and would leave the
  // wave's running max, sum and output at their initial values, so the wave skips them
  const int lo_blk = (a.is_local ? max(0, un.pos0 - a.window + 1) : 0) & ~63;
  const int kbw = s_lo + wv * 64;
  const int kb0 = kbw + (lo_blk > kbw ? (lo_blk - kbw + kStride - 1) / kStride * kStride : 0);
  // The wave's first block (a wave without blocks loads the split's last block and does not
  // use it). Global layers: its pool page is a scalar load (the block index is uniform per
  // wave) issued before the post operands below: the block's loads wait for it in the scalar
  // counter, not for every operand load in flight (local layers read an in-bounds entry and
  // ignore it: no branch around the load).
  const int kbf = min(kb0, s_hi / 64 * 64);
  const int pt_idx = __builtin_amdgcn_readfirstlane(
      un.seq * a.kl.max_pages + min(kbf / kPage, a.kl.max_pages - 1));
  const int pg_first =
      ((const __attribute__((address_space(4))) int32_t*)(uintptr_t)a.kl.page_table)[pt_idx];
  __builtin_amdgcn_sched_barrier(0);
  // Post-processing of the step's projections (what qk_post_kernel does, fused): every split
  // finishes the unit's query columns (wave per column, lane = dimension: RMSNorm over the
  // head, RoPE, YaRN query scale); the split whose keys hold a unit row's own position
  // finishes that row's key and value (value residual, cache stores) and patches them into
  // the block registers it loaded, so no load waits for the stores. Loads first (queries,
  // fresh rows), then the first key block, then the arithmetic.
  constexpr int NQ = COLS / kUnitWaves;  // query columns per wave
  constexpr int NF = NZ / 2;             // fresh (row, key | value) tasks per wave
  __shared__ __align__(16) uint16_t qs[COLS][64];
  __shared__ __align__(16) uint16_t fk[NZ][64], fv[NZ][64];
  const int zlo = max(0, s_lo - un.pos0), zhi = min(un.n - 1, s_hi - un.pos0);
  const bf16* qkv = reinterpret_cast<const bf16*>(a.qkv);
  const int H = a.H, Hkv = a.Hkv, jr = lane & 31;
  // Loads without branches (addresses clamped into range, results unused where invalid): a
  // load on one side of a branch makes the join wait for every load in flight. Order: the
  // first block's page, the post operands, then the wave's first block.
  // Query column c = wv + 4 i of this wave is unit row z = i; in the 16- and 32-column
  // launches rows past the unit's (a unit of a draft step holds one row) issue no loads (a
  // uniform branch; the 8-column launch measured faster without it)
  // bf16 inputs stay raw bits until their use: converted inside the branch of their load, a
  // column's input made the next column's loads wait for it (one round trip per column).
  // Skipped inputs start at a zero the compiler cannot see as a constant, which keeps it from
  // folding the conversion back into the branch.
  uint32_t opaque_zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(opaque_zero));
  uint32_t qx[NQ];
  float qw[NQ], qcs[NQ], qsn[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    qx[i] = opaque_zero;
    qw[i] = qcs[i] = qsn[i] = 0.f;
    if (NQ > 2 && ((wv + kUnitWaves * i) >> 2) >= un.n) continue;
    const int c = wv + kUnitWaves * i, z = c >> 2, head = g * 4 + (c & 3);
    const int row = max(unit_row<NZ>(un, z), 0);
    const int pos = z < un.n ? un.pos0 + z : un.pos0, pulse = step_row_pulse(ps, pc, row);
    qx[i] = qkv[(int64_t)row * a.ldq + head * 64 + lane].u;
    qw[i] = a.q_norm[((int64_t)pulse * H + head) * 64 + lane];
    qcs[i] = a.cos[(int64_t)pos * 32 + jr];
    qsn[i] = a.sin[(int64_t)pos * 32 + jr];
  }
  uint32_t fx[NF], fvf[NF];
  float fw[NF], fcs[NF], fsn[NF];
  int fpg[NF];  // global layers: pool page of the fresh position
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    fx[i] = fvf[i] = opaque_zero;
    fw[i] = fcs[i] = fsn[i] = 0.f;
    fpg[i] = 0;
    if (NF > 1 && zlo + ((wv + kUnitWaves * i) >> 1) > zhi) continue;
    const int t = wv + kUnitWaves * i, z = min(zlo + (t >> 1), max(zhi, 0));
    const int row = max(unit_row<NZ>(un, z), 0), pos = un.pos0 + z;
    const int pulse = step_row_pulse(ps, pc, row);
    const int col = (t & 1) == 0 ? (H + g) * 64 : (H + Hkv + g) * 64;
    fx[i] = qkv[(int64_t)row * a.ldq + col + lane].u;
    fw[i] = a.k_norm[((int64_t)pulse * Hkv + g) * 64 + lane];
    fcs[i] = a.cos[(int64_t)pos * 32 + jr];
    fsn[i] = a.sin[(int64_t)pos * 32 + jr];
    fvf[i] = reinterpret_cast<const bf16*>(a.v_first)[(int64_t)row * Hkv * 64 + g * 64 + lane].u;
    fpg[i] = a.kl.page_table[(int64_t)un.seq * a.kl.max_pages + pos / kPage];
  }
  AttnKV cur;
  attn_load_block(Kc, Vc, kv_block_layer_page(a.kl, a.is_local, Hkv, un.seq, g, kbf, pg_first),
                  m16, kq, cur);
  auto norm_rope = [&](float x, float w, float cs, float sn) {
    const float ss = wave_sum(x * x);
    const float inv = 1.0f / sqrtf(ss / 64.0f + a.eps);
    const float y = rnd<bf16>(w * (x * inv));
    const float p = __shfl_xor(y, 32, 64);
    return rnd<bf16>(lane < 32 ? y * cs - p * sn : y * cs + p * sn);
  };
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int c = wv + kUnitWaves * i, z = c >> 2;
    float o = 0.f;
    if (unit_row<NZ>(un, z) >= 0) {
      o = norm_rope(__uint_as_float(qx[i] << 16), qw[i], qcs[i], qsn[i]);
      const int pos = un.pos0 + z;
      if (!a.is_local && pos + 1 > a.base_seq_len) {
        const double b0 = (double)a.base_seq_len;
        const double pp = (double)(pos + 1) > b0 ? (double)(pos + 1) : b0;
        const float sc = (float)(1.0 + 0.1 * log(pp / b0));
        o = rnd<bf16>(o * sc);
      }
    }
    qs[c][lane] = f2bf(o).u;
  }
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    const int t = wv + kUnitWaves * i, z = zlo + (t >> 1);
    if (z > zhi) continue;
    if ((t & 1) == 0) {
      fk[z][lane] = f2bf(norm_rope(__uint_as_float(fx[i] << 16), fw[i], fcs[i], fsn[i])).u;
    } else {
      float v = __uint_as_float(fx[i] << 16);
      if (step_row_pulse(ps, pc, unit_row<NZ>(un, z)) == 0 && a.layer > 0)
        v = rnd<bf16>(rnd<bf16>(rnd<bf16>(1.0f - lv0) * v) +
                      rnd<bf16>(lv0 * __uint_as_float(fvf[i] << 16)));
      fv[z][lane] = f2bf(v).u;
    }
  }
  // the fresh keys and values go to the caches at the end of the kernel (stores count in
  // the same counter as loads: issued here, the block loads' wait would include them)
  auto store_fresh = [&]() {
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      const int t = wv + kUnitWaves * i, z = zlo + (t >> 1);
      if (z > zhi) continue;
      const int pos = un.pos0 + z;
      if ((t & 1) == 0) {
        bf16* kc = reinterpret_cast<bf16*>(const_cast<void*>(a.kl.k));
        const int64_t ko = a.is_local
            ? (((int64_t)un.seq * Hkv + g) * a.kl.lcap + pos % a.kl.lcap) * kHeadDim
            : (((int64_t)fpg[i] * Hkv + g) * kPage + pos % kPage) * kHeadDim;
        kc[ko + lane].u = fk[z][lane];
      } else {
        const int row = unit_row<NZ>(un, z);
        bf16 v;
        v.u = fv[z][lane];
        if (a.layer == 0 && step_row_pulse(ps, pc, row) == 0)
          reinterpret_cast<bf16*>(a.v_first)[(int64_t)row * Hkv * 64 + g * 64 + lane] = v;
        bf16* vc = reinterpret_cast<bf16*>(const_cast<void*>(a.kl.v));
        const int64_t vo = a.is_local
            ? (((int64_t)un.seq * Hkv + g) * kHeadDim + lane) * a.kl.lcap + pos % a.kl.lcap
            : (((int64_t)fpg[i] * Hkv + g) * kHeadDim + lane) * kPage + pos % kPage;
        vc[vo] = v;
      }
    }
  };
  __syncthreads();
  int qlo[NQT], qhi[NQT];
  attn_bf16x8 qb[NQT][2];
#pragma unroll
  for (int t = 0; t < NQT; ++t) {
    const int c = t * 16 + m16, z = c >> 2;
    const int qrow = c < COLS ? unit_row<NZ>(un, z) : -1;
    const int qpos = un.pos0 + z;
    qlo[t] = a.is_local ? max(0, qpos - a.window + 1) : 0;
    qhi[t] = qrow < 0 ? -1 : qpos;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      qb[t][ks] = c < COLS ? *reinterpret_cast<const attn_bf16x8*>(&qs[c < COLS ? c : 0][ks * 32 + kq * 8])
                           : zero;
  }
  float mrun[NQT], lrun[NQT];
  attn_f32x4 o[NQT][4];
#pragma unroll
  for (int t = 0; t < NQT; ++t) {
    mrun[t] = -INFINITY;
    lrun[t] = 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[t][mt] = attn_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // scores in the base-2 domain: exp(x - m) = exp2(x log2e - m log2e)
  const float scale2 = a.scale * 1.4426950408889634f;
  // keys every row of the unit sees: [lo of the last row, position of the first row]
  const int full_lo = a.is_local ? max(0, uhi - a.window + 1) : 0;
  const int full_hi = un.pos0;
  const int f_lo = un.pos0 + zlo, f_hi = un.pos0 + zhi;  // this split's fresh positions
  for (int kb = kb0; kb <= s_hi; kb += kStride) {
    if (kb != kb0)
      attn_load_block(Kc, Vc, kv_block_layer(a.kl, a.is_local, a.Hkv, un.seq, g, kb), m16, kq,
                      cur);
    if (kb <= f_hi && kb + 63 >= f_lo) attn_patch_fresh(cur, kb, f_lo, f_hi, un.pos0, m16, kq, fk, fv);
    const auto& kk = cur.k;
    const auto& vl = cur.vl;
    const auto& vh = cur.vh;
#pragma unroll
    for (int t = 0; t < NQT; ++t) {
      if (t > 0 && 4 * t >= un.n) break;  // query tile t holds unit rows 4 t .. 4 t + 3
      attn_f32x4 sv[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        attn_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kk[kt][0], qb[t][0], acc, 0, 0, 0);
        sv[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kk[kt][1], qb[t][1], acc, 0, 0, 0);
      }
      // lane holds keys kb + attn_key_of(kt, 4 kq + j) of query column 16 t + m16; a block inside
      // every row's key range needs no mask (unused columns hold zero queries: finite)
      float mx = -INFINITY;
      if (kb >= full_lo && kb + 63 <= full_hi) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            sv[kt][j] *= scale2;
            mx = fmaxf(mx, sv[kt][j]);
          }
      } else {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = kb + attn_key_of(kt, kq * 4 + j);
            const float v = (key >= qlo[t] && key <= qhi[t]) ? sv[kt][j] * scale2 : -INFINITY;
            sv[kt][j] = v;
            mx = fmaxf(mx, v);
          }
      }
      mx = fmaxf(mx, swz_xor16(mx));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(mrun[t], mx);
      const float muse = mnew == -INFINITY ? 0.f : mnew;
      // exp2(-inf) = 0 covers an empty running state and masked keys
      const float f = __builtin_amdgcn_exp2f(mrun[t] - muse);
      mrun[t] = mnew;
      lrun[t] *= f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) o[t][mt] *= f;
      attn_bf16x8 ph[2], pl[2];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p = __builtin_amdgcn_exp2f(sv[kt][j] - muse);
          lrun[t] += p;
          const __bf16 hi = (__bf16)p;
          ph[kt >> 1][(kt & 1) * 4 + j] = hi;
          pl[kt >> 1][(kt & 1) * 4 + j] = (__bf16)(p - (float)hi);
        }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const attn_bf16x8 av = __builtin_shufflevector(vl[mt][s2], vh[mt][s2], 0, 1, 2, 3, 4, 5, 6, 7);
          o[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, ph[s2], o[t][mt], 0, 0, 0);
          o[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pl[s2], o[t][mt], 0, 0, 0);
        }
    }
  }
  // wave partials: query column 16 t + m16 < COLS; lane holds dims 16 mt + 4 kq + j
#pragma unroll
  for (int t = 0; t < NQT; ++t) {
    float lr = lrun[t];
    lr += swz_xor16(lr);
    lr += __shfl_xor(lr, 32, 64);
    const int c = t * 16 + m16;
    if (c < COLS) {
      if (kq == 0) {
        wm[wv][c] = mrun[t];
        wl[wv][c] = lr;
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) wo[wv][c][mt * 16 + kq * 4 + j] = o[t][mt][j];
    }
  }
  __syncthreads();
  // merge the waves: element t -> query column hr, dim d; the block's threads cover the
  // unit's columns (hr < 4 n) x 64 elements whatever its size
  const int ncol = min(un.n, NZ) * 4;
  for (int t = threadIdx.x; t < ncol * 64; t += blockDim.x) {
    const int hr = t >> 6, d = t & 63;
    const int row = unit_row<NZ>(un, hr >> 2);
    float M = -INFINITY, L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kUnitWaves; ++w) M = fmaxf(M, wm[w][hr]);
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kUnitWaves; ++w) {
        if (wm[w][hr] == -INFINITY) continue;
        const float f = __builtin_amdgcn_exp2f(wm[w][hr] - M);
        L += wl[w][hr] * f;
        O += wo[w][hr][d] * f;
      }
    }
    if (nsplit == 1) {
      const int head = g * 4 + (hr & 3);
      const float gate = to_f(reinterpret_cast<const bf16*>(a.gate)[(int64_t)row * a.H + head]);
      reinterpret_cast<bf16*>(a.out)[(int64_t)row * a.H * 64 + head * 64 + d] =
          f2bf(rnd<bf16>(O / L) * gate);
    } else {
      // several splits: device-coherent partials; the last block to count in merges
      float* out = a.part + ((((int64_t)u * a.Hkv + g) * a.max_splits + s) * COLS + hr) * 66;
      __hip_atomic_store(out + 2 + d, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(out, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(out + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (nsplit == 1) {
    store_fresh();
    return;
  }
  // Hand-off to the merging block without a release/acquire pair. Every partial is written
  // and read with agent-scope atomics, which gfx950 issues as `global_store ... sc1` /
  // `global_load ... sc1`: coherent at device scope on their own (written through and read
  // past the XCD's L2). What the memory model would add with acq_rel on the counter is
  // ordering against *other* accesses, as `buffer_wbl2 sc1` before and `buffer_inv sc1`
  // after the add: a write-back and invalidate of the whole L2, measured slower. The order
  // that matters is kept in hardware and by the compiler: `s_waitcnt vmcnt(0)` below waits
  // for every partial store of this workgroup to be acknowledged before the barrier, so all
  // of them complete before thread 0's counter add is issued; the merging block issues its
  // partial loads only after the add has returned (through LDS and a barrier, which the
  // compiler does not move memory operations across).
  __builtin_amdgcn_s_waitcnt(0);
  __shared__ int s_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t* cnt = a.split_done + (int64_t)u * a.Hkv + g;
    const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == nsplit - 1;
    if (s_last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  store_fresh();
  if (!s_last) return;
  attn_merge_splits<COLS>(a, u, g, un, nsplit);
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
      Ks[kk][d] = key <= thi ? ld(Kc, kv_offset(a.kv, a.layer, b, g, key) + d) : 0.f;
    }
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
      const int kk = i & 63, d = i >> 6;  // V is dimension-major: consecutive keys per thread
      const int key = k0 + kk;
      Vs[kk][d] = key <= thi ? ld(Vc, kv_offset_v(a.kv, a.layer, b, g, key, d)) : 0.f;
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
// Prefill attention in bf16 on the matrix cores (same key ranges as attn_prefill_kernel).
// Block = (sequence, 64-query tile, kv head); wave w takes query head 4g + w % 4 over
// 16·NQ of the tile's 64 queries, so each 64-key block staged in LDS serves every head and
// query of the block. Per block:
// S^T = K Q^T (keys x queries), online softmax per query, O^T += V^T P^T (dims x queries).
// In this orientation P never leaves the registers: the D tile of S^T gives lane l keys
// 4*(l/16) + j (j < 4) of query l % 16, and the B operand of the second product takes 8
// keys of query l % 16 -- here the 4 keys of key tile 2s and the 4 of tile 2s + 1, a
// permutation of the reduction index that the V^T operand repeats (V^T is staged with those
// 8 keys in consecutive slots: one 16-byte LDS read per fragment).
// Scores use exp2 with log2(e) folded into the scale; P is rounded to bf16 for the second
// product, the running max, sum and output accumulate in fp32.
// ---------------------------------------------------------------------------

// At least 4 waves per SIMD (at most 128 registers per lane): with NQ = 2 two workgroups of
// 8 waves share a CU, so one computes while the other waits at its barriers.
template <int NQ>
__global__ void __launch_bounds__(256 * (4 / NQ), 4) attn_prefill_mfma_kernel(AttnArgs a) {
  // NQ 16-query tiles per wave: the 64 queries of the block are split over 4 / NQ waves
  // per head, so the block has 4 heads x (4 / NQ) waves
  constexpr int kThreads = 256 * (4 / NQ);
  // 16-byte chunks of each staged tile per staging thread (the first 512 threads stage)
  constexpr int CH = kThreads >= 512 ? 1 : 512 / kThreads;
  const bool stager = threadIdx.x < 512;
  constexpr int kLd = 72;  // LDS row stride in bf16: 16 bytes of padding against bank conflicts
  __shared__ __attribute__((aligned(16))) __bf16 Ks[64][kLd];  // [key][dim]
  // [dim][key slot]: within each 32-key half, lane kq's 8 keys of the second product (keys
  // 4 kq .. 4 kq + 3 of both 16-key tiles) sit in slots 8 kq .. 8 kq + 7
  __shared__ __attribute__((aligned(16))) __bf16 Vs[64][kLd];
  const int T_ = a.prefill_T;
  const int ntile = (T_ + 63) / 64;
  const int b = (int)blockIdx.x / ntile;
  const int qt = ntile - 1 - (int)blockIdx.x % ntile;  // longest key ranges first
  const int g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int m16 = lane & 15, kq = lane >> 4;
  const int head = g * 4 + (wv & 3);
  const int qoff = (wv >> 2) * 16 * NQ;  // this wave's first query within the block
  const bool quirk = a.is_local && T_ > a.window;
  const int q0 = qt * 64;
  const int qlast = min(q0 + 63, T_ - 1);
  const int tlo = quirk ? T_ - a.window : 0;
  const int thi = quirk ? T_ - a.window + min(qlast, a.window - 1) : qlast;
  // keys every query of the tile sees: blocks inside [flo, fhi] need no mask
  const int flo = tlo;
  const int fhi = quirk ? T_ - a.window + min(q0, a.window - 1) : q0;

  int qlo[NQ], qhi[NQ];
  attn_bf16x8 qb[NQ][2];  // Q^T operand: column = query m16 of tile nt, dims kq*8 + 32*ks
#pragma unroll
  for (int nt = 0; nt < NQ; ++nt) {
    const int t = q0 + qoff + nt * 16 + m16;
    const int tc = min(t, T_ - 1);
    qlo[nt] = tlo;
    qhi[nt] = t >= T_ ? -1 : (quirk ? T_ - a.window + min(tc, a.window - 1) : tc);
    const bf16* qp = reinterpret_cast<const bf16*>(a.qkv) + ((int64_t)b * T_ + tc) * a.ldq +
                     head * 64 + kq * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qb[nt][ks] = *reinterpret_cast<const attn_bf16x8*>(qp + ks * 32);
  }
  attn_f32x4 o[4][NQ];  // O^T tile (dim tile mt, query tile nt)
  float mrun[NQ], lrun[NQ];
#pragma unroll
  for (int nt = 0; nt < NQ; ++nt) {
    mrun[nt] = -INFINITY;
    lrun[nt] = 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[mt][nt] = attn_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float sl2 = a.scale * 1.4426950408889634f;

  // staging: thread -> CH 16-byte chunks of K row sr (dims from sc) and of V row sr (keys)
  const int sr = ((tid & 511) * CH) >> 3, sc16 = (((tid & 511) * CH) & 7) * 8;
  const bf16* Kc = reinterpret_cast<const bf16*>(a.kv.k[a.layer]);
  const bf16* Vc = reinterpret_cast<const bf16*>(a.kv.v[a.layer]);
  attn_bf16x8 kr[CH], vr[CH];
  auto fetch = [&](int kb) {
    const KVBlock blk = kv_block(a.kv, a.layer, b, g, kb);
    const bf16* kp = Kc + blk.k0 + sr * 64 + sc16;
    const bf16* vp = Vc + blk.v0 + (int64_t)sr * blk.vstride + sc16;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      kr[c] = *reinterpret_cast<const attn_bf16x8*>(kp + 8 * c);
      vr[c] = *reinterpret_cast<const attn_bf16x8*>(vp + 8 * c);
    }
  };
  const int kb0 = tlo & ~63;
  fetch(kb0);
  for (int kb = kb0; kb <= thi; kb += 64) {
    __syncthreads();  // the previous block's LDS reads are done
    if (stager) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        *reinterpret_cast<attn_bf16x8*>(&Ks[sr][sc16 + 8 * c]) = kr[c];
        // keys k0 .. k0 + 7 of the block: the two 4-key halves go to the slots of lanes
        // kq and kq + 1 of the same key-tile parity
        const int k0 = sc16 + 8 * c, w0 = k0 & 31, kqa = (w0 >> 2) & 3;
        bf16* vrow = reinterpret_cast<bf16*>(&Vs[sr][(k0 & 32) + (w0 >> 4) * 4]);
        *reinterpret_cast<attn_bf16x4*>(vrow + kqa * 8) =
            __builtin_shufflevector(vr[c], vr[c], 0, 1, 2, 3);
        *reinterpret_cast<attn_bf16x4*>(vrow + (kqa + 1) * 8) =
            __builtin_shufflevector(vr[c], vr[c], 4, 5, 6, 7);
      }
    }
    __syncthreads();
    if (kb + 64 <= thi) fetch(kb + 64);  // in flight during this block's products

    attn_f32x4 sv[4][NQ];  // S^T tile (key tile kt, query tile nt)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const attn_bf16x8 k0 = *reinterpret_cast<const attn_bf16x8*>(&Ks[kt * 16 + m16][kq * 8]);
      const attn_bf16x8 k1 = *reinterpret_cast<const attn_bf16x8*>(&Ks[kt * 16 + m16][32 + kq * 8]);
#pragma unroll
      for (int nt = 0; nt < NQ; ++nt) {
        attn_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qb[nt][0], acc, 0, 0, 0);
        sv[kt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qb[nt][1], acc, 0, 0, 0);
      }
    }
    const bool full = kb >= flo && kb + 63 <= fhi;  // uniform per block
    attn_bf16x8 pb[NQ][2];
#pragma unroll
    for (int nt = 0; nt < NQ; ++nt) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v = sv[kt][nt][j] * sl2;
          if (!full) {
            const int key = kb + kt * 16 + kq * 4 + j;
            v = (key >= qlo[nt] && key <= qhi[nt]) ? v : -INFINITY;
          }
          sv[kt][nt][j] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, swz_xor16(mx));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(mrun[nt], mx);
      const float muse = mnew == -INFINITY ? 0.f : mnew;
      const float f = __builtin_amdgcn_exp2f(mrun[nt] - muse);
      mrun[nt] = mnew;
      float ls = lrun[nt] * f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) o[mt][nt] *= f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p = __builtin_amdgcn_exp2f(sv[kt][nt][j] - muse);
          ls += p;
          pb[nt][kt >> 1][(kt & 1) * 4 + j] = (__bf16)p;
        }
      lrun[nt] = ls;
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const attn_bf16x8 av = *reinterpret_cast<const attn_bf16x8*>(&Vs[mt * 16 + m16][ks * 32 + kq * 8]);
#pragma unroll
        for (int nt = 0; nt < NQ; ++nt)
          o[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[nt][ks], o[mt][nt], 0, 0, 0);
      }
  }
  // lane holds O[query q0 + 16 nt + m16][dims 16 mt + 4 kq + j]
#pragma unroll
  for (int nt = 0; nt < NQ; ++nt) {
    float l = lrun[nt];
    l += swz_xor16(l);
    l += __shfl_xor(l, 32, 64);
    const int t = q0 + qoff + nt * 16 + m16;
    if (t >= T_) continue;
    const int64_t row = (int64_t)b * T_ + t;
    const float gate = bf2f(reinterpret_cast<const bf16*>(a.gate)[row * a.H + head]);
    const float inv = 1.0f / l;
    bf16* op = reinterpret_cast<bf16*>(a.out) + row * a.H * 64 + head * 64 + kq * 4;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      attn_bf16x4 w;
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = (__bf16)(rnd<bf16>(o[mt][nt][j] * inv) * gate);
      *reinterpret_cast<attn_bf16x4*>(op + mt * 16) = w;
    }
  }
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
// Decode: mlp_norm of the residual stream fused with the router. Block = 4 waves per row;
// every wave normalises the row (wave 0 stores it), wave w computes the logits of experts
// [w*E/4, (w+1)*E/4); wave 0 then ranks the experts in parallel (lane = expert).
template <typename T, int E, int EPL>
__global__ void __launch_bounds__(256) norm_router_kernel(RouterArgs a) {
  constexpr int EW = E / 4;
  __shared__ float lg[E];
  const int r = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int D = a.D, i0 = lane * EPL;
  // The row goes out first (in bounds for every block: the grid is the engine's row
  // capacity), with the control block's row count and pulse ranges in one scalar read; the
  // empty asm (a memory clobber, no operand) keeps the row's loads ahead of the row-count
  // test without waiting for them. Blocks past the step's rows leave before their weight
  // loads; the pulse-indexed weights of live rows wait one scalar round trip.
  int ps[kMaxPulses], pc[kMaxPulses];
#pragma unroll
  for (int q = 0; q < kMaxPulses; ++q) {
    ps[q] = a.ctl->pulse_start[q];
    pc[q] = a.ctl->pulse_count[q];
  }
  const int n_rows = a.ctl->n_rows;
  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)r * D;
  float xv[EPL], nw[EPL], wt[EW][EPL];
  ldv<EPL>(x + i0, xv);
  // (the weight pointers are read here too, so the weights do not wait for them)
  const float* wbase = a.w;
  const float* nbase = a.norm_w;
  asm volatile("" ::"s"(wbase), "s"(nbase) : "memory");
  if (r >= n_rows) return;
  const bool live = true;
  const int pulse = step_row_pulse(ps, pc, r);
  const float* W = wbase + ((int64_t)pulse * E + wv * EW) * D;
  ldv<EPL>(nbase + (int64_t)pulse * D + i0, nw);
#pragma unroll
  for (int q = 0; q < EW; ++q) ldv<EPL>(W + (int64_t)q * D + i0, wt[q]);
  // the ranking wave's bias goes out with the weights (after the logits exchange it would be
  // one more round trip); lanes past the experts read expert 0's and do not use it
  const float bias_l = a.bias[(int64_t)pulse * E + (lane < E ? lane : 0)];
  // the weight loads go out before the row's arithmetic, which waits for the row
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < EPL; ++c) ss += xv[c] * xv[c];
  const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
  float y[EPL];
#pragma unroll
  for (int c = 0; c < EPL; ++c) y[c] = rnd<T>(nw[c] * (xv[c] * inv));
  if (wv == 0 && live) stv<EPL>(reinterpret_cast<T*>(a.xn) + (int64_t)r * D + i0, y);
#pragma unroll
  for (int q = 0; q < EW; ++q) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < EPL; ++c) acc += y[c] * wt[q][c];
    acc = wave_sum(acc);
    if (lane == 0) lg[wv * EW + q] = acc;
  }
  __syncthreads();
  if (wv != 0 || !live) return;
  // sigmoid of mean-centred logits, + bias; rank = #experts ahead (value desc, index asc)
  const bool act = lane < E;
  const float l = act ? lg[lane] : 0.f;
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < E; ++j) sum += lane_bcast(l, j);
  const float cen = l - sum / (float)E;
  const float sc = 1.0f / (1.0f + expf(-cen));
  const float bsc = sc + (act ? bias_l : 0.f);
  int rank = 0;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float bj = lane_bcast(bsc, j);
    rank += (bj > bsc || (bj == bsc && j < lane)) ? 1 : 0;
  }
  const int K = a.K;
  float tot = 0.f;
  for (int k = 0; k < K; ++k) {
    const uint64_t m = __ballot(act && rank == k);
    tot += lane_bcast(sc, __ffsll((unsigned long long)m) - 1);
  }
  tot += 1e-6f;
  if (act && rank < K) {
    const int64_t o = (int64_t)r * K + rank;
    a.topk_idx[o] = lane;
    a.topk_w[o] = rnd<T>(sc / tot);
    if (a.lists) {
      const int p = atomicAdd(&a.list_count[lane], 1);
      a.lists[(int64_t)lane * a.list_stride + p] = (int)o;
    }
  }
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

// Prefill router in bf16 on the matrix cores: logits[rows][E] = X . bf16(W)^T with fp32
// accumulation, E <= 16 experts as the 16 columns of one v_mfma_f32_16x16x32_bf16 tile;
// a wave owns 16 rows, a workgroup of 8 waves converts the weights into LDS once for its
// 128 rows (16 x 2048 tokens: 28.1 -> 21.4 us per launch against every wave loading and
// converting them itself). The logits, rounded to bf16, go through LDS to the shared top-k
// routine (one lane per row), so routing is the same as router_prefill_kernel's.
constexpr int kRouterWaves = 8;     // 16-row tiles per workgroup
constexpr int kRouterMaxD = 1024;   // model widths the staged weights cover
__global__ void __launch_bounds__(64 * kRouterWaves) router_prefill_mfma_kernel(RouterArgs a) {
  // the pulse's weights, rounded to bf16 once per workgroup, in B-operand order: k step t,
  // lane (expert m16, k chunk kq) -> W[m16][32 t + 8 kq .. + 7] (zero for m16 >= E)
  __shared__ attn_bf16x8 sw[kRouterMaxD / 32][64];
  __shared__ float lg[kRouterWaves][16][17];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int m16 = lane & 15, kq = lane >> 4;
  const int r0 = ((int)blockIdx.x * kRouterWaves + wv) * 16;
  const int D = a.D, E = a.E, KS = D / 32;
  const bf16* xp = reinterpret_cast<const bf16*>(a.x) +
                   (int64_t)min(r0 + m16, a.m_fixed - 1) * D + kq * 8;
  const attn_bf16x8 zero = {};
  // the first rows' loads go out ahead of the weight staging
  attn_bf16x8 xa[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) xa[u] = *reinterpret_cast<const attn_bf16x8*>(xp + 32 * u);
  const float* wbase = a.w + (int64_t)a.pulse * E * D;
  for (int f = tid; f < KS * 64; f += 64 * kRouterWaves) {
    const int t = f >> 6, l = f & 63, ex = l & 15;
    const float* src = wbase + (int64_t)min(ex, E - 1) * D + t * 32 + (l >> 4) * 8;
    const float4 w0 = *reinterpret_cast<const float4*>(src);
    const float4 w1 = *reinterpret_cast<const float4*>(src + 4);
    attn_bf16x8 v;
    v[0] = (__bf16)w0.x; v[1] = (__bf16)w0.y; v[2] = (__bf16)w0.z; v[3] = (__bf16)w0.w;
    v[4] = (__bf16)w1.x; v[5] = (__bf16)w1.y; v[6] = (__bf16)w1.z; v[7] = (__bf16)w1.w;
    sw[t][l] = ex < E ? v : zero;
  }
  __syncthreads();
  attn_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < D; k += 256) {
    if (k > 0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) xa[u] = *reinterpret_cast<const attn_bf16x8*>(xp + k + 32 * u);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[u], sw[(k >> 5) + u][lane], acc, 0, 0, 0);
  }
  // lane holds the logits of rows 4 kq + j for expert m16
#pragma unroll
  for (int j = 0; j < 4; ++j) lg[wv][kq * 4 + j][m16] = rnd<bf16>(acc[j]);
  __syncthreads();
  if (lane < 16 && r0 + lane < a.m_fixed)
    route_topk<bf16>(lg[wv][lane], E, a.K, a.bias + (int64_t)a.pulse * E, r0 + lane, a);
}

// ---------------------------------------------------------------------------
// Prefill capacity: within each sequence, the assignments of an expert beyond its
// capacity C are dropped, ranked in (weight desc, flat index asc) order via the float key
// e - 0.5*w/(1+w). Kept assignments are appended to the expert lists.
// ---------------------------------------------------------------------------
// One block per (sequence, expert). A first pass counts the sequence's assignments to the
// expert and stages up to kCapStage of them in LDS (loads batched ahead of their tests, one
// LDS atomic per wave; prefill of 16 x 2048 tokens: 97 -> 84 us per launch). Under
// capacity every one is kept; over capacity the C first in (key asc, flat index asc) order
// are: the C-th smallest key found by bisection over the keys' ordered bits, in LDS when
// staged, else over the sequence's assignments in memory, and the assignments on that key
// ranked by flat index. The block then reserves its kept count in the expert's list with
// one atomic and writes its entries there.
__device__ int block_excl_scan_int(int v, int* scratch, int* total) {
  const int tid = threadIdx.x, nt = blockDim.x;
  __syncthreads();  // previous users of the scratch are done
  scratch[tid] = v;
  __syncthreads();
  for (int off = 1; off < nt; off <<= 1) {
    const int add = tid >= off ? scratch[tid - off] : 0;
    __syncthreads();
    scratch[tid] += add;
    __syncthreads();
  }
  *total = scratch[nt - 1];
  return scratch[tid] - v;
}
// Order-preserving map of a float onto unsigned integers.
__device__ __forceinline__ uint32_t ordered_bits(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// Block-wide sum and exclusive prefix sum of one int per thread (blockDim.x <= 1024,
// scratch of blockDim.x ints); every thread returns the same total.
__device__ int block_sum_int(int v, int* scratch) {
  int tot;
  block_excl_scan_int(v, scratch, &tot);
  return tot;
}
// Sum of one small count per thread over a block of 256 threads (exact: counts stay far
// below 2^24); every thread returns the same total.
__device__ __forceinline__ int block_count(int v, float* red4) {
  const float f = wave_sum((float)v);
  __syncthreads();  // the previous call's readers are done
  if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = f;
  __syncthreads();
  return (int)(red4[0] + red4[1] + red4[2] + red4[3]);
}
constexpr int kCapStage = 4096;
constexpr int kTieBits = 32768;  // flat indices of a sequence's assignments the tie bitmap holds
__global__ void __launch_bounds__(256) prefill_select_kernel(
    const int32_t* __restrict__ idx, const float* __restrict__ w, int32_t* __restrict__ keep,
    int32_t* __restrict__ lists, int32_t* __restrict__ lcount, int64_t list_stride, int T_, int K,
    int E, int C) {
  __shared__ int s_n, s_base;
  __shared__ int s_off[256];
  __shared__ float s_red[4];
  __shared__ uint32_t tbits[kTieBits / 32];  // assignments on the threshold key, by flat index
  __shared__ int tpre[kTieBits / 32];        // set bits in the words before each word
  __shared__ int sidx[kCapStage];
  __shared__ float skey[kCapStage];
  __shared__ uint8_t skept[kCapStage];
  const int b = (int)blockIdx.x / E, e = (int)blockIdx.x % E;
  const int64_t per = (int64_t)T_ * K, s0 = (int64_t)b * per;
  const int tid = threadIdx.x, nt = blockDim.x;
  auto key_w = [&](float wr) {
    const float wi = fmaxf(wr, 0.f);
    return (float)e - (wi / (1.0f + wi)) * 0.5f;
  };
  auto key_of = [&](int64_t i) { return key_w(w[i]); };
  if (tid == 0) s_n = 0;
  __syncthreads();
  // the sequence's assignments in chunks of kSelLoads per thread, every load of a chunk
  // issued before the first test (a load behind a branch on the previous one waits for it);
  // positions past the end re-read the last assignment and are not counted
  constexpr int kSelLoads = 16;
  for (int64_t c0 = s0; c0 < s0 + per; c0 += (int64_t)nt * kSelLoads) {
    int v[kSelLoads];
    float wv[kSelLoads];
#pragma unroll
    for (int u = 0; u < kSelLoads; ++u) {
      const int64_t i = c0 + tid + (int64_t)u * nt;
      const int64_t ic = i < s0 + per ? i : s0 + per - 1;
      v[u] = idx[ic];
      wv[u] = w[ic];
    }
#pragma unroll
    for (int u = 0; u < kSelLoads; ++u) {
      const int64_t i = c0 + tid + (int64_t)u * nt;
      const bool hit = i < s0 + per && v[u] == e;
      // one LDS atomic per wave: the wave's hits take consecutive slots in lane order
      const uint64_t m = __ballot(hit);
      if (m == 0) continue;
      const int lane = tid & 63;
      int q0 = 0;
      if (lane == __ffsll((unsigned long long)m) - 1) q0 = atomicAdd(&s_n, __popcll(m));
      q0 = __shfl(q0, __ffsll((unsigned long long)m) - 1, 64);
      const int q = q0 + __popcll(m & ((1ull << lane) - 1ull));
      if (hit && q < kCapStage) {
        sidx[q] = (int)(i - s0);
        skey[q] = key_w(wv[u]);
      }
    }
  }
  __syncthreads();
  const int n = s_n;
  const bool staged = n <= kCapStage;
  int mine = 0;
  if (staged) {
    // Over capacity, an assignment is kept when fewer than C others precede it in (key,
    // flat index) order: the C-th smallest key uc by bisection over the staged keys' ordered
    // bits (one counting pass per step), then keys below uc are kept, keys above dropped,
    // and those on uc ranked by flat index among themselves. The keys are e - 0.5 w/(1+w)
    // with w >= 0 (never -0 or NaN), so the ordered bits compare as the floats do.
    uint32_t uc = 0xffffffffu;
    int below = 0;
    bool tie_bits = false, lone_tie = false;
    if (n > C) {
      uint32_t lo = 0u, hi = 0xffffffffu;
      while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        int c = 0;
        for (int q = tid; q < n; q += nt) c += ordered_bits(skey[q]) <= mid ? 1 : 0;
        if (block_count(c, s_red) >= C)
          hi = mid;
        else
          lo = mid + 1;
      }
      uc = lo;
      int c = 0, ct = 0;
      for (int q = tid; q < n; q += nt) {
        const uint32_t uk = ordered_bits(skey[q]);
        c += uk < uc ? 1 : 0;
        ct += uk == uc ? 1 : 0;
      }
      below = block_count(c, s_red);
      // the assignments on uc as a bitmap of flat indices with per-word prefix counts, so
      // each one's rank among them is one lookup (saturated routing scores make ties
      // common; ranking each against every staged key was up to 150 us per launch)
      const int nties = block_count(ct, s_red);  // at least one: uc is a staged key
      lone_tie = nties == 1;
      tie_bits = nties > 1 && per <= kTieBits;
      if (tie_bits) {
        const int nw = (int)((per + 31) / 32);
        for (int w = tid; w < nw; w += nt) tbits[w] = 0u;
        __syncthreads();
        for (int q = tid; q < n; q += nt)
          if (ordered_bits(skey[q]) == uc) atomicOr(&tbits[sidx[q] >> 5], 1u << (sidx[q] & 31));
        __syncthreads();
        const int wpt = (nw + nt - 1) / nt, w0 = tid * wpt, w1 = min(nw, w0 + wpt);
        int cnt = 0;
        for (int w = w0; w < w1; ++w) cnt += __popc(tbits[w]);
        int tot_ties;
        int run = block_excl_scan_int(cnt, s_off, &tot_ties);
        for (int w = w0; w < w1; ++w) {
          tpre[w] = run;
          run += __popc(tbits[w]);
        }
        __syncthreads();
      }
    }
    for (int q = tid; q < n; q += nt) {
      bool kept = true;
      if (n > C) {
        const uint32_t uk = ordered_bits(skey[q]);
        if (uk == uc) {
          const int iq = sidx[q];
          int ties = 0;
          if (lone_tie) {
            ties = 0;
          } else if (tie_bits) {
            ties = tpre[iq >> 5] + __popc(tbits[iq >> 5] & ((1u << (iq & 31)) - 1u));
          } else {
            for (int u = 0; u < n; ++u)
              ties += (ordered_bits(skey[u]) == uc && sidx[u] < iq) ? 1 : 0;
          }
          kept = below + ties < C;
        } else {
          kept = uk < uc;
        }
      }
      keep[s0 + sidx[q]] = kept ? 1 : 0;
      skept[q] = kept ? 1 : 0;
      mine += kept ? 1 : 0;
    }
  } else if (n <= C) {
    for (int64_t i = s0 + tid; i < s0 + per; i += nt)
      if (idx[i] == e) {
        keep[i] = 1;
        ++mine;
      }
  } else {
    // Too many to stage: the C-th smallest key by bisection over its ordered bits (one
    // counting pass per step), then the assignments on that key ranked by flat index with
    // an ordered scan over chunks of nt consecutive assignments.
    uint32_t lo = 0u, hi = 0xffffffffu;
    while (lo < hi) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      int c = 0;
      for (int64_t i = s0 + tid; i < s0 + per; i += nt)
        c += (idx[i] == e && ordered_bits(key_of(i)) <= mid) ? 1 : 0;
      if (block_sum_int(c, s_off) >= C)
        hi = mid;
      else
        lo = mid + 1;
    }
    const uint32_t uc = lo;
    int c = 0;
    for (int64_t i = s0 + tid; i < s0 + per; i += nt)
      c += (idx[i] == e && ordered_bits(key_of(i)) < uc) ? 1 : 0;
    const int below = block_sum_int(c, s_off);
    int run = 0;  // assignments on the threshold key in earlier chunks
    for (int64_t c0 = s0; c0 < s0 + per; c0 += nt) {
      const int64_t i = c0 + tid;
      const bool my = i < s0 + per && idx[i] == e;
      const uint32_t uk = my ? ordered_bits(key_of(i)) : 0u;
      int tot;
      const int before = block_excl_scan_int(my && uk == uc ? 1 : 0, s_off, &tot);
      if (my) {
        const bool kept = uk < uc || (uk == uc && below + run + before < C);
        keep[i] = kept ? 1 : 0;
        mine += kept ? 1 : 0;
      }
      run += tot;
    }
  }
  int tot;
  const int my_off = block_excl_scan_int(mine, s_off, &tot);
  if (tid == 0) s_base = tot ? atomicAdd(&lcount[e], tot) : 0;
  __syncthreads();
  int32_t* out = lists + (int64_t)e * list_stride + s_base + my_off;
  if (staged) {
    for (int q = tid; q < n; q += nt)
      if (skept[q]) *out++ = (int32_t)(s0 + sidx[q]);
  } else {
    for (int64_t i = s0 + tid; i < s0 + per; i += nt)
      if (idx[i] == e && keep[i]) *out++ = (int32_t)i;
  }
}

// ---------------------------------------------------------------------------
// MoE combine + residual.
// decode: routed = sum_k T(out_k * w_k) in T, mlp = T(shared + T(routed * rs)), h += mlp.
// prefill: routed = index_add of T(w_k * out_k) in T (dropped = 0), mlp = T(shared + routed).
// ---------------------------------------------------------------------------
template <typename T, int EPL, int KT>
__global__ void __launch_bounds__(64) moe_combine_rows_kernel(CombineArgs a) {
  // one wave per row; lane owns elements [lane*EPL, lane*EPL + EPL)
  const int r = blockIdx.x;
  const int K = a.K, D = a.D, lane = threadIdx.x, i0 = lane * EPL;
  // The row's operands go out first (every block's row is in bounds: the grid is the row
  // capacity), the routing weights as one vector load (lane k holds slot k: per-slot scalar
  // loads would each sit in a block of their own behind a wait), then the control block's
  // row count and pulse ranges in one scalar read; the empty asm (a memory clobber, no
  // operand) keeps the loads ahead of the row-count test without waiting for them, and
  // blocks past the step's rows leave before the pulse-indexed loads.
  const T* shp = reinterpret_cast<const T*>(a.shared) + (int64_t)r * D + i0;
  const T* rop = reinterpret_cast<const T*>(a.routed) + (int64_t)r * K * D + i0;
  T* h = reinterpret_cast<T*>(a.h) + (int64_t)r * D + i0;
  float hv[EPL], sh[EPL], rs[EPL], ro[KT][EPL];
  ldv<EPL>(h, hv);
  ldv<EPL>(shp, sh);
#pragma unroll
  for (int k = 0; k < KT; ++k) ldv<EPL>(rop + (int64_t)(k < K ? k : 0) * D, ro[k]);
  const float wl = a.topk_w[(int64_t)r * K + min(lane, K - 1)];
  // the folded pulse output's row operands go out with the rest; launches without it re-read
  // the row's h instead (no branch around the load: converted inside one, the load made the
  // control block's reads and the pulse-indexed loads wait for every row operand)
  const bool pout = a.hout_state != nullptr;
  float hin[EPL];
  ldv<EPL>(pout ? reinterpret_cast<const T*>(a.h_in) + (int64_t)r * D + i0 : h, hin);
  RowDesc rd{};
  if (pout) rd = a.rows[r];
  int n = a.m_fixed, pulse = a.pulse;
  if (a.ctl) {
    int ps[kMaxPulses], pc[kMaxPulses];
#pragma unroll
    for (int q = 0; q < kMaxPulses; ++q) {
      ps[q] = a.ctl->pulse_start[q];
      pc[q] = a.ctl->pulse_count[q];
    }
    n = a.ctl->n_rows;
    pulse = step_row_pulse(ps, pc, r);
  }
  asm volatile("" ::: "memory");
  if (r >= n) return;
  const bool live = true;
  // the pulse-indexed operands go out before the routing weights' lane shuffles (which wait
  // for the row operands issued ahead of them)
  ldv<EPL>(reinterpret_cast<const T*>(a.routed_scale) + (int64_t)pulse * D + i0, rs);
  float nwn[EPL];
  if (a.next_norm) ldv<EPL>(a.next_norm + (int64_t)pulse * D + i0, nwn);
  float rso[EPL], fn[EPL];
  if (pout) {
    ldv<EPL>(reinterpret_cast<const T*>(a.res_scale) + (int64_t)pulse * D + i0, rso);
    ldv<EPL>(a.final_norm + i0, fn);
  }
  float w[KT];
#pragma unroll
  for (int k = 0; k < KT; ++k) w[k] = __shfl(wl, k < K ? k : 0, 64);
  bool kept[KT];
#pragma unroll
  for (int k = 0; k < KT; ++k) kept[k] = true;
  if (a.keep) {
    const int kl = a.keep[(int64_t)r * K + min(lane, K - 1)];
#pragma unroll
    for (int k = 0; k < KT; ++k) kept[k] = __shfl(kl, k < K ? k : 0, 64) != 0;
  }
  // K is uniform: one branch per top-k slot, the element loops inside
  float routed[EPL];
#pragma unroll
  for (int c = 0; c < EPL; ++c) routed[c] = 0.f;
  if (!a.prefill) {
#pragma unroll
    for (int k = 0; k < KT; ++k) {
      if (k < K) {
#pragma unroll
        for (int c = 0; c < EPL; ++c) routed[c] = rnd<T>(routed[c] + rnd<T>(ro[k][c] * w[k]));
      }
    }
#pragma unroll
    for (int c = 0; c < EPL; ++c) hv[c] = rnd<T>(hv[c] + rnd<T>(sh[c] + rnd<T>(routed[c] * rs[c])));
  } else {
#pragma unroll
    for (int k = 0; k < KT; ++k) {
      if (k < K) {
        const float wk = kept[k] ? w[k] : 0.f;
#pragma unroll
        for (int c = 0; c < EPL; ++c)
          routed[c] = rnd<T>(routed[c] + (kept[k] ? rnd<T>(wk * ro[k][c]) : 0.f));
      }
    }
#pragma unroll
    for (int c = 0; c < EPL; ++c) hv[c] = rnd<T>(hv[c] + rnd<T>(sh[c] + routed[c]));
  }
  if (!live) return;
  stv<EPL>(h, hv);
  if (pout) {
    // pulse_output_kernel's arithmetic: out = h_in + (h - h_in) * res_scale, each step
    // rounded to T; logits rows also get final_norm(out)
    float o[EPL];
#pragma unroll
    for (int c = 0; c < EPL; ++c) o[c] = rnd<T>(hin[c] + rnd<T>(rnd<T>(hv[c] - hin[c]) * rso[c]));
    stv<EPL>(reinterpret_cast<T*>(a.hout_state) + ((int64_t)rd.seq * a.slots + rd.sslot) * D + i0, o);
    if (rd.lrow >= 0) {
      float ss = 0.f, y[EPL];
#pragma unroll
      for (int c = 0; c < EPL; ++c) ss += o[c] * o[c];
      const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
#pragma unroll
      for (int c = 0; c < EPL; ++c) y[c] = rnd<T>(fn[c] * (o[c] * inv));
      stv<EPL>(reinterpret_cast<T*>(a.xn_final) + (int64_t)rd.lrow * D + i0, y);
    }
  }
  if (a.next_norm) {
    float ss = 0.f, y[EPL];
#pragma unroll
    for (int c = 0; c < EPL; ++c) ss += hv[c] * hv[c];
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
#pragma unroll
    for (int c = 0; c < EPL; ++c) y[c] = rnd<T>(nwn[c] * (hv[c] * inv));
    stv<EPL>(reinterpret_cast<T*>(a.xn) + (int64_t)r * D + i0, y);
  }
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
  const int st = a.prefill ? rd.pos + rd.seq * a.prefill_T : rd.seq * a.slots + rd.sslot;
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
// Wave-per-row kernels: EPL = D / 64 elements per lane.
#define PULSAR_EPL_DISPATCH(D, KERNEL_T, grid, block, arg)                                   \
  do {                                                                                       \
    switch ((D) % 256 == 0 ? (D) / 64 : 0) {                                                 \
      case 4: KERNEL_T(4)<<<(grid), (block), 0, s>>>(arg); break;                            \
      case 8: KERNEL_T(8)<<<(grid), (block), 0, s>>>(arg); break;                            \
      case 16: KERNEL_T(16)<<<(grid), (block), 0, s>>>(arg); break;                          \
      case 32: KERNEL_T(32)<<<(grid), (block), 0, s>>>(arg); break;                          \
      default: return fail(PULSAR_ERR_UNSUPPORTED, "d_model must be 256, 512, 1024 or 2048"); \
    }                                                                                        \
    PULSAR_LAUNCH_CHECK();                                                                   \
    return PULSAR_OK;                                                                        \
  } while (0)

int launch_pulse_input(const PulseInputArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (a.rank < 1 || a.rank > kMaxRank)
    return fail(PULSAR_ERR_UNSUPPORTED, "pulse_input: reinject rank must be 1..16");
  if (a.rank == 8) {
    if (dtype == PULSAR_BF16) {
#define K_(N) pulse_input_kernel<bf16, N, 8, true>
      PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 64, a);
#undef K_
    }
#define K_(N) pulse_input_kernel<float, N, 8, true>
    PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 64, a);
#undef K_
  }
  if (dtype == PULSAR_BF16) {
#define K_(N) pulse_input_kernel<bf16, N, 16, false>
    PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 64, a);
#undef K_
  }
#define K_(N) pulse_input_kernel<float, N, 16, false>
  PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 64, a);
#undef K_
}
// Row sets of this many rows or more (prefill) take several rows per block / wave.
constexpr int kManyRows = 1024;
constexpr int kNormRowsPerBlock = 4;
constexpr int kPostRowsPerWave = 8;

template <typename T, int RPB>
void launch_norm_rows_t(const NormArgs& a, int max_rows, hipStream_t s) {
  const dim3 grid((unsigned)((max_rows + RPB - 1) / RPB));
  if (a.D <= 256)
    norm_rows_kernel<T, RPB, 1><<<grid, 256, 0, s>>>(a);
  else if (a.D <= 512)
    norm_rows_kernel<T, RPB, 2><<<grid, 256, 0, s>>>(a);
  else if (a.D <= 1024)
    norm_rows_kernel<T, RPB, 4><<<grid, 256, 0, s>>>(a);
  else
    norm_rows_kernel<T, RPB, 8><<<grid, 256, 0, s>>>(a);
}
int launch_norm_rows(const NormArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (a.D > 2048) return fail(PULSAR_ERR_UNSUPPORTED, "norm rows: D above 2048");
  if (max_rows <= 0) return PULSAR_OK;
  const bool many = max_rows >= kManyRows;
  if (dtype == PULSAR_BF16) {
    if (many) launch_norm_rows_t<bf16, kNormRowsPerBlock>(a, max_rows, s);
    else launch_norm_rows_t<bf16, 1>(a, max_rows, s);
  } else {
    if (many) launch_norm_rows_t<float, kNormRowsPerBlock>(a, max_rows, s);
    else launch_norm_rows_t<float, 1>(a, max_rows, s);
  }
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}
int launch_qk_post(const QKPostArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (max_rows <= 0) return PULSAR_OK;
  const int rpw = max_rows >= kManyRows ? kPostRowsPerWave : 1;
  const dim3 grid((unsigned)((max_rows + rpw - 1) / rpw), (unsigned)((a.H + a.Hkv + 3) / 4));
  if (dtype == PULSAR_BF16) {
    if (rpw > 1) qk_post_kernel<bf16, kPostRowsPerWave><<<grid, 256, 0, s>>>(a);
    else qk_post_kernel<bf16, 1><<<grid, 256, 0, s>>>(a);
  } else {
    if (rpw > 1) qk_post_kernel<float, kPostRowsPerWave><<<grid, 256, 0, s>>>(a);
    else qk_post_kernel<float, 1><<<grid, 256, 0, s>>>(a);
  }
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}
int launch_attn_decode(const AttnArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (dtype == PULSAR_BF16) {
    // Key split per launch, from the layer type, the engine's context length and, for
    // shorter contexts, whether the engine holds kWideSplitUnits sequences or more: results
    // are the same for engines on the same side of each threshold. Engines whose context
    // needs more than kLongCacheSplits 256-key splits take 2048-key splits (8 blocks per
    // wave) in the global layers, which spread each workgroup's fixed start and merge costs
    // over 8x the keys, and 1024-key splits in the sliding-window layers (at most window +
    // unit rows keys: two splits).
    const bool lng = a.max_splits_unit > kLongCacheSplits;
    // engines of few sequences keep 256-key splits in the sliding-window layers: 1024-key
    // splits would leave most CUs idle there (two workgroups per unit and kv head)
    const bool few = a.max_units < kManyUnits;
    // shorter engines: 512-key splits (two blocks per wave). Every split repeats the unit's
    // query post-processing and adds a partial to merge; against 256-key splits: c2
    // draft-block 25.4k -> 25.9k tokens/s, c2 reference schedule 18.5k -> 18.9k, c5 85.3k
    // -> 87.1k (1024-key splits for draft blocks: 24.8k). Engines of kWideSplitUnits
    // sequences or more have workgroups enough at 1024-key splits, which leave most units
    // one split and no merge: 256 x 1024 positions, reference schedule 116.8k -> 124.3k
    // tokens/s, draft length 6 104.4k -> 111.5k.
    const int short_bpw = a.max_units >= kWideSplitUnits ? 4 : kShortCacheBlocks;
    const int bpw = !lng ? short_bpw : (a.is_local ? (few ? 1 : 4) : 8);
    const int split = kUnitSplit * bpw;
    // a unit's keys [lo, hi] lie in the splits from lo's to hi's: at most max_ctx keys, and in
    // sliding-window layers window + rows - 1 keys, which can straddle one more split
    int zs = (a.max_ctx + split - 1) / split;
    if (a.is_local) zs = std::min(zs, (a.window + a.unit_rows - 1 + split - 1) / split + 1);
    const dim3 grid(a.max_units, a.Hkv, zs);
    if (!a.post || !a.q_norm || !a.k_norm || !a.v_lambda || !a.v_first || !a.cos || !a.sin)
      return fail(PULSAR_ERR_INVALID, "decode attention: bf16 takes the q/k/v post operands");
    AttnArgs b = a;
    b.kl.k = a.kv.k[a.layer];
    b.kl.v = a.kv.v[a.layer];
    b.kl.lcap = a.kv.lcap;
    b.kl.max_pages = a.kv.max_pages;
    b.kl.page_table = a.kv.page_table;
    if (((a.kv.local_mask >> a.layer) & 1u) != (a.is_local ? 1u : 0u))
      return fail(PULSAR_ERR_INVALID, "decode attention: layer type mismatch");
#define PULSAR_ATTN_UNIT(C)                                                         \
  do {                                                                              \
    if (bpw == 8)                                                                   \
      attn_decode_unit_kernel<C, 8><<<grid, 64 * kUnitWaves, 0, s>>>(b);            \
    else if (bpw == 4)                                                              \
      attn_decode_unit_kernel<C, 4><<<grid, 64 * kUnitWaves, 0, s>>>(b);            \
    else if (bpw == 2)                                                              \
      attn_decode_unit_kernel<C, 2><<<grid, 64 * kUnitWaves, 0, s>>>(b);            \
    else                                                                            \
      attn_decode_unit_kernel<C, 1><<<grid, 64 * kUnitWaves, 0, s>>>(b);            \
  } while (0)
    if (a.unit_rows <= 2)
      PULSAR_ATTN_UNIT(8);
    else if (a.unit_rows <= 4)
      PULSAR_ATTN_UNIT(16);
    else if (a.unit_rows <= kMaxBlock)
      PULSAR_ATTN_UNIT(32);
    else
      return fail(PULSAR_ERR_UNSUPPORTED, "decode attention: at most 8 rows per unit");
#undef PULSAR_ATTN_UNIT
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  }
  attn_decode_kernel<float><<<dim3(max_rows, a.Hkv, a.max_splits), 256, 0, s>>>(a);
  PULSAR_LAUNCH_CHECK();
  attn_combine_kernel<float><<<dim3(max_rows, a.H / 4), 256, 0, s>>>(a);
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}
int launch_attn_prefill(const AttnArgs& a, int dtype, int B, hipStream_t s) {
  const int ntile = (a.prefill_T + 63) / 64;
  if (a.H != 4 * a.Hkv)
    return fail(PULSAR_ERR_UNSUPPORTED, "prefill attention: four query heads per kv head");
  if (dtype == PULSAR_BF16) {
    // two 16-query tiles per wave: each K and V fragment read from LDS feeds two products
    // (16 x 2048 tokens: 289 -> 260 us per launch against one tile per wave at 16 waves;
    // 352 us with two tiles at 136 registers, where one workgroup fills a CU)
    attn_prefill_mfma_kernel<2><<<dim3(B * ntile, a.Hkv), 512, 0, s>>>(a);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  }
  PULSAR_DISPATCH(dtype, attn_prefill_kernel, dim3(B * ntile, a.Hkv), 256, a);
}
int launch_router_decode(const RouterArgs& a, int dtype, int max_rows, hipStream_t s) {
  PULSAR_DISPATCH(dtype, router_decode_kernel, dim3(max_rows), 256, a);
}
int launch_norm_router(const RouterArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (a.K < 1 || a.K > 8 || a.K > a.E)
    return fail(PULSAR_ERR_UNSUPPORTED, "norm_router: top_k must be 1..8 and <= n_experts");
  if (a.E == 16) {
    if (dtype == PULSAR_BF16) {
#define K_(N) norm_router_kernel<bf16, 16, N>
      PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 256, a);
#undef K_
    }
#define K_(N) norm_router_kernel<float, 16, N>
    PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 256, a);
#undef K_
  }
  if (a.E == 8) {
    if (dtype == PULSAR_BF16) {
#define K_(N) norm_router_kernel<bf16, 8, N>
      PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 256, a);
#undef K_
    }
#define K_(N) norm_router_kernel<float, 8, N>
    PULSAR_EPL_DISPATCH(a.D, K_, dim3(max_rows), 256, a);
#undef K_
  }
  return fail(PULSAR_ERR_UNSUPPORTED, "norm_router: n_experts must be 8 or 16");
}
int launch_router_prefill(const RouterArgs& a, int dtype, hipStream_t s) {
  if (a.E > 32) return fail(PULSAR_ERR_UNSUPPORTED, "router: at most 32 experts");
  if (dtype == PULSAR_BF16 && a.E <= 16 && a.D % 256 == 0 && a.D <= kRouterMaxD) {
    const int rows = 16 * kRouterWaves;
    router_prefill_mfma_kernel<<<dim3((unsigned)((a.m_fixed + rows - 1) / rows)), 64 * kRouterWaves,
                                 0, s>>>(a);
    PULSAR_LAUNCH_CHECK();
    return PULSAR_OK;
  }
  PULSAR_DISPATCH(dtype, router_prefill_kernel, dim3(a.m_fixed), 256, a);
}
int launch_prefill_capacity(const int32_t* idx, const float* w, int32_t* keep, int32_t* lists,
                            int32_t* lcount, int64_t list_stride, int B, int T_, int K, int E,
                            int C, hipStream_t s) {
  if (B < 1 || E < 1) return PULSAR_OK;
  prefill_select_kernel<<<(unsigned)(B * E), 256, 0, s>>>(idx, w, keep, lists, lcount, list_stride,
                                                           T_, K, E, C);
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}
int launch_moe_combine(const CombineArgs& a, int dtype, int max_rows, hipStream_t s) {
  if (a.K < 1 || a.K > 8) return fail(PULSAR_ERR_UNSUPPORTED, "moe_combine: top_k must be 1..8");
  const int kt = a.K <= 2 ? 2 : (a.K <= 4 ? 4 : 8);
#define PULSAR_COMBINE_CASE(KT)                                     \
  if (kt == KT) {                                                   \
    if (dtype == PULSAR_BF16) {                                     \
      PULSAR_EPL_DISPATCH(a.D, K_BF, dim3(max_rows), 64, a);        \
    }                                                               \
    PULSAR_EPL_DISPATCH(a.D, K_F32, dim3(max_rows), 64, a);         \
  }
#define K_BF(N) moe_combine_rows_kernel<bf16, N, 2>
#define K_F32(N) moe_combine_rows_kernel<float, N, 2>
  PULSAR_COMBINE_CASE(2)
#undef K_BF
#undef K_F32
#define K_BF(N) moe_combine_rows_kernel<bf16, N, 4>
#define K_F32(N) moe_combine_rows_kernel<float, N, 4>
  PULSAR_COMBINE_CASE(4)
#undef K_BF
#undef K_F32
#define K_BF(N) moe_combine_rows_kernel<bf16, N, 8>
#define K_F32(N) moe_combine_rows_kernel<float, N, 8>
  PULSAR_COMBINE_CASE(8)
#undef K_BF
#undef K_F32
#undef PULSAR_COMBINE_CASE
  return fail(PULSAR_ERR_UNSUPPORTED, "moe_combine: top_k");
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
