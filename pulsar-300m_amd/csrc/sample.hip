// Sampling and the speculative controller, both on the device so that a captured step
// graph can be replayed without host round trips.
//
// Sampling (reference src/infer.py:658-685): repetition penalty over the seen set
// (divide positive, multiply non-positive), greedy argmax (first maximum) when the
// temperature is <= 1e-4, else temperature scaling, top-p (keep the smallest set of
// highest-scoring tokens whose mass strictly above each kept token is <= top_p, found by
// bisection on the order-preserving integer key of the scaled logits) and an inverse-CDF
// draw over the kept tokens in index order. Two independent draws are produced per row.
//
// Controller (reference src/infer.py:623-731): per sequence, the current token c runs its
// pulses; in speculative mode the pulse-0 logits of a "tested" token give the reference's
// draft d, which is also the speculative next token s whose pulse 0 runs in the same step
// as c's last pulse (it attends to c's last-pulse K/V written earlier in that step). The
// verify draw v decides acceptance exactly as the reference (d == v and d not a stop id);
// on rejection the next token is a fresh draw, and s's work is kept when it equals that
// draw. After an accepted draft the next token is a plain draw, as in the reference;
// s is then the pulse-0 argmax guess of the accepted token, which changes which work is
// speculative but never the emitted distribution.
#include <mutex>

#include "sample.h"

namespace pulsar {

namespace {

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ float uniform01(uint64_t seed, int seq, uint32_t ctr, int d) {
  uint64_t k = mix64(seed + 0x9E3779B97F4A7C15ull * (uint64_t)(seq + 1));
  k = mix64(k ^ ((uint64_t)ctr << 8) ^ (uint64_t)d);
  return (float)(k >> 40) * (1.0f / 16777216.0f);
}

// Block-wide exclusive scan of one float per thread (blockDim <= 1024). `red` needs
// blockDim / 64 floats.
__device__ float block_excl_scan(float v, float* red, float* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  float incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  __syncthreads();
  if (lane == 63) red[w] = incl;
  __syncthreads();
  float base = 0.f, tot = 0.f;
  for (int i = 0; i < nw; ++i) {
    if (i < w) base += red[i];
    tot += red[i];
  }
  *total = tot;
  return base + incl - v;
}

struct ArgMax {
  float v;
  int i;
};

__device__ __forceinline__ ArgMax better(ArgMax a, ArgMax b) {
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}

__device__ ArgMax block_argmax(ArgMax x, ArgMax* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    ArgMax o;
    o.v = __shfl_xor(x.v, off, 64);
    o.i = __shfl_xor(x.i, off, 64);
    x = better(x, o);
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = x;
  __syncthreads();
  ArgMax r = red[0];
  for (int i = 1; i < nw; ++i) r = better(r, red[i]);
  return r;
}

}  // namespace

#ifndef PULSAR_SAMPLE_THREADS
#define PULSAR_SAMPLE_THREADS 1024
#endif
constexpr int kSampleThreads = PULSAR_SAMPLE_THREADS;

template <typename T, int PER, int NT>
__global__ void __launch_bounds__(NT) sample_kernel(SampleArgs a) {
  __shared__ float red[32];
  __shared__ ArgMax ared[16];
  const int lr = blockIdx.x;
  // the row's sequence and extra seen tokens are read with the row count (their buffers
  // hold an entry for every block of the grid; the empty asm keeps the loads ahead of the
  // count test), so the logits and the seen bits go out one round trip later, together
  const int seq = a.lrow_seq[lr];
  int xt[kMaxExtra];
#pragma unroll
  for (int x = 0; x < kMaxExtra; ++x)
    xt[x] = x < a.n_extra ? a.lrow_extra[(int64_t)lr * a.extra_stride + x] : -1;
  asm volatile("" ::: "memory");
  if (lr >= a.ctl->n_lrows) return;
  if (a.n_seq > 0 && (seq < 0 || seq >= a.n_seq)) {
    if (threadIdx.x < 3) (threadIdx.x == 0 ? a.out_argmax[lr] : a.out_draw[lr * 2 + threadIdx.x - 1]) = -1;
    return;
  }
  const float* lg = a.logits + (int64_t)lr * a.V;
  const uint32_t* seen = a.seen + (int64_t)seq * (a.V / 32);
  const int base = threadIdx.x * PER;
  // tokens counted as seen for this row beyond the sequence's bitmap, as a mask over this
  // thread's PER logits
  uint64_t xmask = 0;
  bool has_extra = false;
  float l[PER];
#pragma unroll
  for (int i = 0; i < PER; i += 4) {
    const float4 v = *reinterpret_cast<const float4*>(lg + base + i);
    l[i] = v.x;
    l[i + 1] = v.y;
    l[i + 2] = v.z;
    l[i + 3] = v.w;
  }
#pragma unroll
  for (int x = 0; x < kMaxExtra; ++x) {
    if (xt[x] < 0) continue;
    has_extra = true;
    const int off = xt[x] - base;
    if (off >= 0 && off < PER) xmask |= 1ull << off;
  }
  if (a.out_maxprob) {
    // early-exit test (src/infer.py:540-541): max of softmax(logits) = 1 / sum exp(l - max),
    // on the logits before penalty and temperature, rounded like the reference's softmax
    // output in the activation dtype
    float rm = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) rm = fmaxf(rm, l[i]);
    rm = block_max(rm, red);
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) z += expf(l[i] - rm);
    z = block_sum(z, red);
    if (threadIdx.x == 0) a.out_maxprob[lr] = rnd<T>(1.0f / z);
  }
  if (a.rep_penalty != 1.0f) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = base + i;
      const bool s = ((seen[idx >> 5] >> (idx & 31)) & 1u) || ((xmask >> i) & 1u);
      if (s) l[i] = l[i] > 0.f ? rnd<T>(l[i] / a.rep_penalty) : rnd<T>(l[i] * a.rep_penalty);
    }
  }
  ArgMax am{-INFINITY, 0x7fffffff};
#pragma unroll
  for (int i = 0; i < PER; ++i) am = better(am, ArgMax{l[i], base + i});
  am = block_argmax(am, ared);
  // Non-finite logits compare false everywhere and leave no maximum: a token id outside the
  // vocabulary is never emitted (it would index the embedding table out of bounds).
  if (am.i < 0 || am.i >= a.V) am.i = 0;
  if (a.greedy) {
    if (threadIdx.x == 0) {
      a.out_argmax[lr] = am.i;
      a.out_draw[lr * 2] = am.i;
      a.out_draw[lr * 2 + 1] = am.i;
    }
    return;
  }
  // x / temperature for every score: the quotient by the correctly rounded reciprocal and
  // one fma correction (Markstein's theorem: RN(q + (x - q t) r) = RN(x / t) when r =
  // RN(1 / t) and no intermediate over- or underflows), three instructions in place of the
  // full-precision divide; a non-finite product is kept as it is. The map (this quotient,
  // then the rounding to T) is monotone, so the largest scaled score is the scaled maximum:
  // no reduction of its own.
  const float tmp = a.temperature, rtmp = 1.0f / tmp;
  auto scaled = [&](float x) {
    const float q = x * rtmp;
    const float q2 = fmaf(fmaf(-q, tmp, x), rtmp, q);
    return rnd<T>(__builtin_isfinite(q) ? q2 : q);
  };
#pragma unroll
  for (int i = 0; i < PER; ++i) l[i] = scaled(l[i]);
  const float mx = scaled(am.v);
  // Unnormalised probabilities and order keys, computed once. bf16-rounded scores carry
  // no information in the low 16 key bits (all zero for positive, all one for negative
  // values, so equal high halves mean equal keys): the threshold search runs on the high
  // half there, 16 steps instead of 32, with the same kept set.
  // The 16-bit keys of bf16 scores are stored two per register.
  constexpr int kLow = sizeof(T) == 2 ? 16 : 0;
  constexpr int kPack = sizeof(T) == 2 ? 2 : 1;
  float pr[PER];
  uint32_t kw[PER / kPack];
#pragma unroll
  for (int i = 0; i < PER / kPack; ++i) kw[i] = 0u;
  float zl = 0.f, at_max = 0.f;
  const uint32_t kmax = order_key(mx) >> kLow;
  // exp(l - mx) as the hardware base-2 exponential of the scaled difference (a few ulps;
  // the same values feed Z, the threshold search and the draws)
  constexpr float kLog2e = 1.4426950408889634f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    pr[i] = __builtin_amdgcn_exp2f((l[i] - mx) * kLog2e);
    const uint32_t k = order_key(l[i]) >> kLow;
    kw[i / kPack] |= kPack == 2 ? k << (16 * (i & 1)) : k;
    zl += pr[i];
    at_max += k == kmax ? 1.f : 0.f;
  }
#define KEY(i) (kPack == 2 ? (kw[(i) / kPack] >> (16 * ((i) & 1))) & 0xffffu : kw[(i) / kPack])
  // Z, and the number of scores at the maximum (each with probability weight exp(0) = 1):
  // one reduction, Z summed in the same order as a reduction of its own
  float Z, n_max;
  {
    const float zw = wave_sum(zl), cw = wave_sum(at_max);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) {
      red[w] = zw;
      red[16 + w] = cw;
    }
    __syncthreads();
    Z = 0.f;
    n_max = 0.f;
    for (int i = 0; i < nw; ++i) {
      Z += red[i];
      n_max += red[16 + i];
    }
  }
  uint32_t kstar = 0;
  // When the scores tied at the maximum hold more than top_p of the mass (mass above any
  // lower key >= n_max > top_p Z, mass above the maximum's key 0), the threshold search
  // would end at the maximum's key: take it directly. A single such score is then the only
  // token kept, and both draws are the argmax.
  const bool max_only = a.top_p < 1.0f && n_max > a.top_p * Z;
  if (max_only && n_max == 1.f) {
    if (threadIdx.x == 0) {
      a.out_argmax[lr] = am.i;
      a.out_draw[lr * 2] = am.i;
      a.out_draw[lr * 2 + 1] = am.i;
    }
    return;
  }
  if (max_only) {
    kstar = kmax;
  } else if (a.top_p < 1.0f) {
    // smallest m with mass(key > m) <= top_p * Z; the maximum's key always qualifies.
    // Bisection (per-step cost is the 32-element pass, so wider probes do not pay); one
    // barrier per step: partials alternate between two LDS buffers.
    __shared__ float part[2][16];
    const float lim = a.top_p * Z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t lo = 0, hi = order_key(mx) >> kLow;
    int buf = 0;
    while (lo < hi) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      float f = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) f += KEY(i) > mid ? pr[i] : 0.f;
      f = wave_sum(f);
      if (lane == 0) part[buf][w] = f;
      __syncthreads();
      float t = 0.f;
      for (int i = 0; i < nw; ++i) t += part[buf][i];
      buf ^= 1;
      if (t <= lim)
        hi = mid;
      else
        lo = mid + 1;
    }
    kstar = lo;
  }
  float own = 0.f;
  int last_kept = -1;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (KEY(i) >= kstar) {
      own += pr[i];
      last_kept = base + i;
    }
  }
  float total;
  const float pre = block_excl_scan(own, red, &total);
  ArgMax lk = block_argmax(ArgMax{(float)last_kept, 0}, ared);
  __shared__ int pick[2];
  if (threadIdx.x < 2) pick[threadIdx.x] = (int)lk.v;
  __syncthreads();
  // stream: the row's own counter (draft-block mode), else the step counter of the
  // sequence and whether this is the speculative row
  const uint32_t ctr = a.lrow_ctr ? a.lrow_ctr[lr] : a.state[seq].ctr * 2u + (has_extra ? 1u : 0u);
  for (int d = 0; d < 2; ++d) {
    const float target = uniform01(*a.seed, seq, ctr, d) * total;
    if (own > 0.f && target >= pre && target < pre + own) {
      float run = pre;
      int choice = -1;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if (KEY(i) >= kstar) {
          run += pr[i];
          if (choice < 0 && target < run) choice = base + i;
        }
      }
      if (choice < 0) choice = last_kept;
      pick[d] = choice;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    a.out_argmax[lr] = am.i;
#pragma unroll
    for (int d = 0; d < 2; ++d)
      a.out_draw[lr * 2 + d] = (pick[d] >= 0 && pick[d] < a.V) ? pick[d] : am.i;
  }
#undef KEY
}

// ---------------------------------------------------------------------------
// Controller: one thread per sequence (B <= 256); block scans lay out the next step.
// ---------------------------------------------------------------------------
namespace {

// LDS copies of what the step's controller reads by an index it learns from the state (the
// last step's argmax and draws) and of the stop ids, loaded by the whole block together
// with the state, so that the state's round trip is the only one before the layout.
constexpr int kCtlMaxLrows = 2048;
struct CtlShared {
  int draw[2 * kCtlMaxLrows];
  int argmax[kCtlMaxLrows];
  int stop[8];
};
__shared__ CtlShared ctl_lds;

__device__ __forceinline__ bool is_stop(const ControllerArgs& a, int tok) {
  for (int i = 0; i < a.n_stop; ++i)
    if (ctl_lds.stop[i] == tok) return true;
  return false;
}

// Append tok to the sequence's output; kind 1 marks an accepted draft, 0 a drawn token.
__device__ __forceinline__ void emit(const ControllerArgs& a, SeqState& s, int b, int tok, int kind = 0) {
  a.out_tokens[(int64_t)b * a.max_new + s.produced] = tok;
  if (a.out_kinds) a.out_kinds[(int64_t)b * a.max_new + s.produced] = kind;
  s.produced += 1;
  // only this thread writes the sequence's row: a no-return atomic sets the bit without
  // reading the word back first (one round trip less)
  atomicOr(&a.seen[(int64_t)b * (a.V / 32) + (tok >> 5)], 1u << (tok & 31));
  if (s.produced >= s.max_new) s.done = 1;
}

// c <- s (whose pulse 0 ran this step). kind = kind of the new current token.
__device__ __forceinline__ void promote(const ControllerArgs& a, SeqState& s, int kind) {
  s.c_tok = s.s_tok;
  s.c_pos = s.c_pos + 1;
  s.c_slot = 1 - s.c_slot;
  s.c_kind = kind;
  s.c_pulse = 1;
  s.s_valid = 0;
  // the new current token's pulse-0 logits are those of the s row
  const int lr = s.lrow_s;
  if (kind == KIND_TESTED) {
    s.d_tok = ctl_lds.draw[lr * 2];
    s.s_valid = !is_stop(a, s.d_tok);
    s.s_tok = s.d_tok;
  } else {
    const int g = ctl_lds.argmax[lr];
    s.s_valid = !is_stop(a, g);
    s.s_tok = g;
  }
}

__device__ __forceinline__ void fresh(SeqState& s, int tok) {
  s.c_tok = tok;
  s.c_pos = s.c_pos + 1;
  s.c_slot = 1 - s.c_slot;
  s.c_kind = KIND_TESTED;
  s.c_pulse = 0;
  s.s_valid = 0;
}

}  // namespace

// Tokens whose pulses the reference runs through decode_step, the only place its early
// exit applies: every decoded token in plain mode (src/infer.py:620), an accepted draft in
// speculative mode (:728); the tested tokens' draft/verify passes never exit (:700-714).
__device__ __forceinline__ bool exit_eligible(const ControllerArgs& a, const SeqState& s) {
  return a.early_exit && (!a.speculative || s.c_kind == KIND_PLAIN);
}

// Plain decode with early exit: the reference's loop runs decode_step on the last emitted
// token as well (src/infer.py:619-620), and counts its exit; keep the sequence running for
// that token's pulses (it emits nothing after them).
__device__ __forceinline__ void keep_for_tail(const ControllerArgs& a, SeqState& s) {
  if (s.done && a.early_exit && !a.speculative) {
    s.done = 0;
    s.tail = 1;
  }
}

// The current token is done without a draft test (plain mode, an accepted draft, or an
// early exit): the next token is a draw from logits row lr; a speculative row that ran
// with that very token is kept.
__device__ __forceinline__ void finish_untested(const ControllerArgs& a, SeqState& s, int b, int lr, bool s_ran) {
  const int t = ctl_lds.draw[lr * 2];
  if (is_stop(a, t)) {
    s.done = 1;
    return;
  }
  emit(a, s, b, t);
  keep_for_tail(a, s);
  if (s.done) return;
  if (a.speculative && s_ran && s.s_tok == t)
    promote(a, s, KIND_TESTED);
  else
    fresh(s, t);
}

// Advance one sequence's state after the step whose rows it ran.
__device__ __forceinline__ void update_seq(const ControllerArgs& a, SeqState& s, int b) {
  const int P = a.n_pulses;
  s.ctr += 1;
  const int pulse_ran = s.c_pulse;
  bool last = pulse_ran >= P - 1;
  if (exit_eligible(a, s)) {
    // exit after pulse_ran when the top-1 probability of its logits reaches the threshold
    // (src/infer.py:536-543); a token that runs every pulse counts at the last (:546-547)
    if (!last && (double)a.maxprob[s.lrow_c] >= a.exit_thr) last = true;
    if (last) a.exit_counts[b * 4 + min(pulse_ran, P - 1)] += 1;
  }
  if (last && s.tail) {
    s.done = 1;
    return;
  }
  if (!last) {
    if (pulse_ran == 0 && a.speculative) {
      const int lr = s.lrow_c;
      if (s.c_kind == KIND_TESTED) {
        s.d_tok = ctl_lds.draw[lr * 2];
        s.s_valid = !is_stop(a, s.d_tok);
        s.s_tok = s.d_tok;
      } else {
        const int g = ctl_lds.argmax[lr];
        s.s_valid = !is_stop(a, g);
        s.s_tok = g;
      }
    }
    s.c_pulse = pulse_ran + 1;
    return;
  }
  const int lr = s.lrow_c;
  const bool s_ran = s.row_s >= 0;
  if (a.speculative && s.c_kind == KIND_TESTED) {
    const int v = ctl_lds.draw[lr * 2];
    s.tests += 1;
    if (s.d_tok == v && !is_stop(a, s.d_tok)) {
      s.accepted += 1;
      emit(a, s, b, s.d_tok, 1);
      if (!s.done) {
        const int lr_s = s.lrow_s;
        promote(a, s, KIND_PLAIN);
        // the accepted draft's pulse 0 ran as this step's speculative row, so the exit
        // test after its pulse 0 (src/infer.py:536-543) reads that row's logits
        if (exit_eligible(a, s) && P > 1 && (double)a.maxprob[lr_s] >= a.exit_thr) {
          a.exit_counts[b * 4] += 1;
          finish_untested(a, s, b, lr_s, false);
        }
      }
    } else {
      const int t = ctl_lds.draw[lr * 2 + 1];
      if (is_stop(a, t)) {
        s.done = 1;
      } else {
        emit(a, s, b, t);
        if (!s.done) {
          if (s_ran && s.s_tok == t)
            promote(a, s, KIND_TESTED);
          else
            fresh(s, t);
        }
      }
    }
  } else {
    finish_untested(a, s, b, lr, s_ran);
  }
}

// Global-layer KV pages for sequence b's positions up to hi, taken from the pool in order
// of request; false (and the pool's spent flag set) when the pool cannot cover them. have:
// the sequence's page count, read at the kernel's start.
__device__ __forceinline__ bool ensure_pages(const ControllerArgs& a, int b, int hi, int have) {
  if (!a.page_table) return true;
  const int need = hi / kPage + 1;
  if (have >= need) return true;
  const int n = need - have;
  const int first = take_pages(a.pool, n, a.pool_pages);
  if (first < 0) return false;
  for (int i = 0; i < n; ++i) a.page_table[(int64_t)b * a.max_pages + have + i] = first + i;
  a.page_count[b] = need;
  return true;
}

// Exclusive scan of N counters over the block (blockDim 256): wave prefix sums by lane
// shifts, then the 4 wave totals through LDS (two barriers).
template <int N>
__device__ void scan_counts(int* v, int* sh, int* total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int inc[N];
#pragma unroll
  for (int k = 0; k < N; ++k) {
    int x = v[k];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    inc[k] = x;
    if (lane == 63) sh[k * 4 + w] = x;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < N; ++k) {
    int pre = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int wt = sh[k * 4 + i];
      if (i < w) pre += wt;
      tot += wt;
    }
    total[k] = tot;
    v[k] = pre + inc[k] - v[k];
  }
  __syncthreads();
}

// NL loads of draws per thread (2 max_lrows <= 256 NL), issued before any store.
template <int NL>
__device__ void ctl_preload(const ControllerArgs& a) {
  CtlShared& c = ctl_lds;
  constexpr int NA = (NL + 1) / 2;
  const int t = threadIdx.x;
  const int nd = 2 * a.max_lrows, na = a.max_lrows;
  int d[NL], m[NA];
#pragma unroll
  for (int k = 0; k < NL; ++k) d[k] = a.draw[min(t + 256 * k, nd - 1)];
#pragma unroll
  for (int k = 0; k < NA; ++k) m[k] = a.argmax[min(t + 256 * k, na - 1)];
  const int st = a.stop_ids[min(t, 7)];
#pragma unroll
  for (int k = 0; k < NL; ++k)
    if (t + 256 * k < nd) c.draw[t + 256 * k] = d[k];
#pragma unroll
  for (int k = 0; k < NA; ++k)
    if (t + 256 * k < na) c.argmax[t + 256 * k] = m[k];
  if (t < a.n_stop) c.stop[t] = st;
}


// One thread per sequence: advance the state, then lay out the next step's rows grouped by
// pulse (sequence order within a pulse) and its logits rows. Also snapshots the rows and
// control block of the step that just ran (readable for testing).
// The sequence state moves between memory and registers as 16-byte words at constant
// offsets: a struct copy leaves the fields a kernel never names in scratch memory.
static_assert(sizeof(SeqState) % 16 == 0 && alignof(SeqState) <= 16, "SeqState words");
constexpr int kStateWords = (int)(sizeof(SeqState) / 16);
// The state's words go out as loads first (no wait); state_commit, after the kernel's other
// loads are issued, passes them through registers into the state (no memory-to-memory copy
// of the fields a kernel never names). Passed one by one right after their loads, each word
// waited for its load before the next load went out: one round trip per word.
__device__ __forceinline__ void state_issue(int4 (&v)[kStateWords], const SeqState* p) {
#pragma unroll
  for (int k = 0; k < kStateWords; ++k) v[k] = reinterpret_cast<const int4*>(p)[k];
}
__device__ __forceinline__ void state_commit(SeqState& s, int4 (&v)[kStateWords]) {
#pragma unroll
  for (int k = 0; k < kStateWords; ++k)
    asm volatile("" : "+v"(v[k].x), "+v"(v[k].y), "+v"(v[k].z), "+v"(v[k].w));
#pragma unroll
  for (int k = 0; k < kStateWords; ++k) reinterpret_cast<int4*>(&s)[k] = v[k];
}
__device__ __forceinline__ void state_store(SeqState* p, const SeqState& s) {
  constexpr int W = (int)(sizeof(SeqState) / 16);
#pragma unroll
  for (int k = 0; k < W; ++k) reinterpret_cast<int4*>(p)[k] = reinterpret_cast<const int4*>(&s)[k];
}

template <int NL>
__global__ void __launch_bounds__(256) controller_kernel(ControllerArgs a) {
  __shared__ int sh[5 * 4];
  const int b = threadIdx.x;
  StepCtl* ctl = a.ctl;
  const int P = a.n_pulses;
  // the sequence's state and page count are read with the snapshot of the last step's rows
  // and control block and the LDS copies (one round trip for all, before the barrier that
  // retires the snapshot)
  const bool act = b < a.B;
  alignas(16) SeqState s{};
  int4 sw[kStateWords];  // threads past the batch read the last sequence's and drop it
  state_issue(sw, a.state + min(b, a.B - 1));
  const int have = act && a.page_table ? a.page_count[b] : 0;
  ctl_preload<NL>(a);
  const int n_prev = ctl->n_rows;
  for (int i = b; i < n_prev; i += blockDim.x) a.last_rows[i] = a.rows[i];
  if (b == 0) *a.last_ctl = *ctl;
  if (act) state_commit(s, sw);
  __syncthreads();
  if (act) {
    if (a.init) {
      s = SeqState{};
      s.max_new = a.max_new;
      s.c_pos = a.prompt_len - 1;
      s.c_slot = 1;
      // the first token was drawn with counter 0 (state cleared before that draw); step
      // draws use counters 2 * ctr (+1 for the speculative row), so ctr starts at 1 and no
      // later draw reuses the first token's uniform
      s.ctr = 1;
      const int t = ctl_lds.draw[b * 2];
      if (is_stop(a, t) || s.max_new <= 0) {
        s.done = 1;
      } else {
        emit(a, s, b, t);
        keep_for_tail(a, s);
        fresh(s, t);
      }
    } else if (!s.done) {
      update_seq(a, s, b);
    }
    // pages for the next step's positions: the current token's, and the speculative row's
    // one position later; a sequence the pool cannot serve stops here
    if (!s.done && !ensure_pages(a, b, s.c_pos + (a.speculative && s.c_pulse == P - 1 &&
                                                  s.s_valid ? 1 : 0), have))
      s.done = 1;
  }
  // rows of the next step
  const bool live = act && !s.done;
  const bool crow = live;
  const bool srow = live && a.speculative && s.c_pulse == P - 1 && s.s_valid;
  // logits of c: at its last pulse (the next draw; not for a tail token, which draws
  // nothing), at pulse 0 when it drafts, and after every earlier pulse when it may exit
  const bool cwant = crow && (a.all_logits || (s.c_pulse == P - 1 && !s.tail) ||
                              (a.speculative && s.c_pulse == 0) ||
                              (exit_eligible(a, s) && s.c_pulse < P - 1));
  int v[5] = {0, 0, 0, 0, 0};  // rows of pulse 0, 1, 2; logits rows; attention units
  if (crow) v[s.c_pulse] += 1;
  if (srow) v[0] += 1;
  v[3] = (cwant ? 1 : 0) + (srow ? 1 : 0);
  v[4] = live ? 1 : 0;
  int total[5];
  scan_counts<5>(v, sh, total);
  int base[4] = {0, total[0], total[0] + total[1], 0};
  int lr = v[3];
  s.row_c = s.row_s = s.lrow_c = s.lrow_s = -1;
  if (srow) {
    const int idx = base[0] + v[0];
    s.lrow_s = lr++;
    a.lrow_seq[s.lrow_s] = b;
    a.lrow_extra[s.lrow_s] = s.s_tok;
    a.rows[idx] = RowDesc{b, 1 - s.c_slot, 0, s.c_pos + 1, s.s_tok, s.lrow_s, s.s_tok, 1 - s.c_slot};
    s.row_s = idx;
  }
  if (crow) {
    const int p = s.c_pulse;
    const int idx = base[p] + v[p] + ((p == 0 && srow) ? 1 : 0);
    if (cwant) {
      s.lrow_c = lr++;
      a.lrow_seq[s.lrow_c] = b;
      a.lrow_extra[s.lrow_c] = -1;
    }
    a.rows[idx] = RowDesc{b, s.c_slot, p, s.c_pos, s.c_tok, s.lrow_c, -1, s.c_slot};
    s.row_c = idx;
    AttnUnit un{};
    un.seq = b;
    un.n = srow ? 2 : 1;
    un.pos0 = s.c_pos;
    un.row[0] = idx;
    un.row[1] = s.row_s;
    for (int i = 2; i < kMaxBlock; ++i) un.row[i] = -1;
    a.units[v[4]] = un;
  }
  if (act) state_store(a.state + b, s);
  if (b == 0) {
    for (int p = 0; p < 4; ++p) {
      ctl->pulse_start[p] = p < 3 ? base[p] : total[0] + total[1] + total[2];
      ctl->pulse_count[p] = p < 3 ? total[p] : 0;
    }
    ctl->n_rows = total[0] + total[1] + total[2];
    ctl->n_lrows = total[3];
    ctl->n_units = total[4];
    ctl->active = total[4];
    ctl->step += 1;
  }
}

// ---------------------------------------------------------------------------
// Draft-block controller (draft_len > 0). A round starts from an emitted token t = blk[0]
// at position c_pos. Draft steps run pulse 0 of block row j alone (slot j, position
// c_pos + j) and draw blk[j + 1] from its logits (a stop id ends the block); verify steps
// run pulse k of every block row; after the last pulse, the draft of row i + 1 is accepted
// iff it equals draw 0 of row i and is not a stop id. The first rejection (row i) emits
// draw 1 of row i (an independent draw from the same logits); a block without rejection
// emits draw 0 of its last row. Accepted rows keep the last pulse's keys/values at their
// positions; the next round starts one position after the last accepted row. A logits row
// counts block tokens 1..i of its row i as seen. Matches the oracle's
// block_speculative_ids.
//
// Pipelined rounds (block_pipelined): the verify's pulse-0 pass also yields the penalised
// argmax of the last block row, a guess of the next round's first token (the token that
// follows when every draft is accepted). The last verify step then runs one more row for
// the sequence: the guess at the position after the block, pulse 0, in the slot past the
// block's, attending the block's last-pulse keys written earlier in the same layer. If
// every draft is accepted and the emitted token equals the guess, that row was the next
// round's first draft step (same keys, same logits, same draw counter and seen tokens), so
// the round goes straight to its second draft; otherwise the row's work is dropped. The
// emitted streams are those of unpipelined rounds.
// ---------------------------------------------------------------------------
namespace {

// The block tokens while the controller works on them: a vector value, whose elements at
// run-time indices are register selects. (Indexed at run time inside the state struct,
// they kept the whole struct in scratch memory: 176 bytes per lane.) The struct's copy is
// read and written only at constant offsets, at the kernel's start and end.
typedef int32_t BlkVec __attribute__((ext_vector_type(kMaxBlock)));
static_assert(kMaxBlock == 8, "BlkVec holds the block tokens");

__device__ __forceinline__ void new_round(const ControllerArgs& a, SeqState& s, BlkVec& bk,
                                          int tok) {
  // block row i keeps its token state in slot (blk_base + i) % S; the base steps back one
  // slot per round, so the row the previous round's last verify step ran one slot past its
  // block (slot base - 1) is this round's row 0
  const int S = engine_slots(a.draft_len);
  s.blk_base = (s.blk_base + S - 1) % S;
#pragma unroll
  for (int i = 0; i < kMaxBlock; ++i) bk[i] = i == 0 ? tok : -1;
  s.blk_n = 1;
  s.ctr += 1;
  s.s_valid = 0;
  // drafts beyond the tokens still wanted are never emitted
  s.blk_g = min(a.draft_len, s.max_new - s.produced - 1);
  s.blk_phase = s.blk_g > 0 ? 0 : 1;
  s.blk_step = 0;
}

// The verify's pulse 0 runs only rows whose pulse 0 no draft step ran: a draft step ran
// pulse 0 of its row over the committed cache and the block's earlier pulse-0 keys, which is
// the verify's rule, so that row's keys, values and token state are the verify's pulse 0
// already (the kernels' results do not depend on the other rows of a step). That leaves
// the block's last row when a draft was drawn from the row before it, and none when a stop
// id ended the block: the verify then starts at pulse 1, and the pipelined round's guess is
// the stopping draft row's own penalised argmax.
__device__ __forceinline__ void enter_verify(const ControllerArgs& a, SeqState& s, bool last_ran, int lrow) {
  s.blk_phase = 1;
  s.blk_step = 0;
  if (last_ran && a.n_pulses > 1) {
    s.blk_step = 1;
    if (block_pipelined(a.draft_len)) {
      s.s_tok = ctl_lds.argmax[lrow];
      s.s_valid = !is_stop(a, s.s_tok);
    }
  }
}

__device__ __forceinline__ void update_block(const ControllerArgs& a, SeqState& s, BlkVec& bk,
                                             int b) {
  const int P = a.n_pulses;
  if (s.blk_phase == 0) {
    const int j = s.blk_step;
    const int d = ctl_lds.draw[s.lrow_c * 2];
    if (is_stop(a, d)) {
      enter_verify(a, s, true, s.lrow_c);
      return;
    }
    bk[j + 1] = d;
    s.blk_n = j + 2;
    if (j + 1 >= s.blk_g) {
      enter_verify(a, s, false, -1);
    } else {
      s.blk_step = j + 1;
    }
    return;
  }
  if (s.blk_step < P - 1) {
    if (s.blk_step == 0 && s.lrow_s >= 0) {
      // guess of the next round's first token (pipelined rounds)
      s.s_tok = ctl_lds.argmax[s.lrow_s];
      s.s_valid = !is_stop(a, s.s_tok);
    }
    s.blk_step += 1;
    return;
  }
  const bool spec_ran = s.row_s >= 0;
  const int spec_lrow = s.lrow_s, guess = s.s_tok;
  const int n = s.blk_n, lr0 = s.lrow_c;
  // every draw the round's end may read, loaded together (rows past the block re-read its
  // last row; the speculative row's first draw too)
  int dv[kMaxBlock], dw[kMaxBlock];
#pragma unroll
  for (int i = 0; i < kMaxBlock; ++i) {
    const int r = lr0 + min(i, n - 1);
    dv[i] = ctl_lds.draw[r * 2];
    dw[i] = ctl_lds.draw[r * 2 + 1];
  }
  const int d_spec = ctl_lds.draw[max(spec_lrow, 0) * 2];
  int acc = 0, nxt = -1;
#pragma unroll
  for (int i = 0; i < kMaxBlock; ++i) {
    if (i >= n) break;
    if (i < n - 1) {
      const int v = dv[i];
      s.tests += 1;
      if (v == bk[i + 1] && !is_stop(a, v)) {
        s.accepted += 1;
        emit(a, s, b, v, 1);
        acc = i + 1;
        if (s.done) return;
        continue;
      }
      nxt = dw[i];
    } else {
      nxt = dv[i];
    }
    break;
  }
  s.c_pos += acc + 1;
  if (is_stop(a, nxt)) {
    s.done = 1;
    return;
  }
  emit(a, s, b, nxt);
  if (s.done) return;
  new_round(a, s, bk, nxt);
  if (spec_ran && acc == n - 1 && nxt == guess && s.blk_phase == 0) {
    // the speculative row was this round's first draft step
    const int d = d_spec;
    if (is_stop(a, d)) {
      enter_verify(a, s, true, spec_lrow);
    } else {
      bk[1] = d;
      s.blk_n = 2;
      if (s.blk_g <= 1) enter_verify(a, s, false, -1);
      else s.blk_step = 1;
    }
  }
}

}  // namespace

template <int NL>
__global__ void __launch_bounds__(256) controller_block_kernel(ControllerArgs a) {
  __shared__ int sh[5 * 4];
  const int b = threadIdx.x;
  StepCtl* ctl = a.ctl;
  const int P = a.n_pulses;
  // the sequence's state and page count are read with the snapshot of the last step's rows
  // and control block and the LDS copies (one round trip for all, before the barrier that
  // retires the snapshot)
  const bool act = b < a.B;
  alignas(16) SeqState s{};
  int4 sw[kStateWords];  // threads past the batch read the last sequence's and drop it
  state_issue(sw, a.state + min(b, a.B - 1));
  const int have = act && a.page_table ? a.page_count[b] : 0;
  ctl_preload<NL>(a);
  const int n_prev = ctl->n_rows;
  for (int i = b; i < n_prev; i += blockDim.x) a.last_rows[i] = a.rows[i];
  if (b == 0) *a.last_ctl = *ctl;
  if (act) state_commit(s, sw);
  BlkVec bk;
#pragma unroll
  for (int i = 0; i < kMaxBlock; ++i) bk[i] = s.blk[i];
  __syncthreads();
  if (act) {
    if (a.init) {
      s = SeqState{};
      bk = 0;
      s.max_new = a.max_new;
      s.c_pos = a.prompt_len;
      const int t = ctl_lds.draw[b * 2];
      if (is_stop(a, t) || s.max_new <= 0) {
        s.done = 1;
      } else {
        emit(a, s, b, t);
        if (!s.done) new_round(a, s, bk, t);
      }
    } else if (!s.done) {
      update_block(a, s, bk, b);
    }
  }
  bool live = act && !s.done;
  const bool pipe = block_pipelined(a.draft_len);
  int nrow = 0, pulse = 0, lrows = 0, pos0 = 0, slot0 = 0;
  bool guess_row = false, spec = false;
  if (live) {
    if (s.blk_phase == 0) {
      nrow = 1;
      lrows = 1;
      slot0 = s.blk_step;
    } else {
      nrow = s.blk_n;
      pulse = s.blk_step;
      if (pulse == 0 && P > 1) {  // the verify's pulse 0: the block's last row alone
        slot0 = s.blk_n - 1;
        nrow = 1;
      }
      lrows = (pulse == P - 1 || a.all_logits) ? nrow : 0;
      // pulse 0 of a verify: the last row's logits give the guess
      guess_row = pipe && pulse == 0 && P > 1;
      if (guess_row && lrows == 0) lrows = 1;
      // last pulse: the guessed next token's first row, when a next round can follow
      spec = pipe && pulse == P - 1 && P > 1 && s.s_valid && s.produced + nrow < s.max_new;
    }
    pos0 = s.c_pos + slot0;
    // pages for the step's positions; a sequence the pool cannot serve stops here
    if (!ensure_pages(a, b, spec ? s.c_pos + nrow : pos0 + nrow - 1, have)) {
      s.done = 1;
      live = false;
      nrow = lrows = 0;
      guess_row = spec = false;
    }
  }
  int v[5] = {0, 0, 0, 0, 0};  // rows of pulse 0, 1, 2; logits rows; attention units
  v[0] = pulse == 0 ? nrow : 0;
  v[1] = pulse == 1 ? nrow : 0;
  v[2] = pulse == 2 ? nrow : 0;
  if (spec) v[0] += 1;
  v[3] = lrows + (spec ? 1 : 0);
  v[4] = live ? 1 : 0;
  int total[5];
  scan_counts<5>(v, sh, total);
  const int base[3] = {0, total[0], total[0] + total[1]};
  s.row_c = s.row_s = s.lrow_c = s.lrow_s = -1;
  if (live) {
    const int r0 = pulse == 0 ? v[0] : pulse == 1 ? base[1] + v[1] : base[2] + v[2];
    const int lr0 = v[3];
    s.row_c = r0;
    s.lrow_c = lrows ? lr0 : -1;
    const int S = engine_slots(a.draft_len);
    AttnUnit un{};
    un.seq = b;
    un.n = nrow + (spec ? 1 : 0);
    un.pos0 = pos0;
#pragma unroll
    for (int i = 0; i < kMaxBlock; ++i) un.row[i] = i < nrow ? r0 + i : -1;
    if (guess_row) s.lrow_s = lrows == nrow ? lr0 + nrow - 1 : lr0;
#pragma unroll
    for (int i = 0; i < kMaxBlock; ++i) {
      if (i >= nrow) break;
      const int slot = slot0 + i;
      const int lr = lrows == nrow ? lr0 + i : (lrows && i == nrow - 1 ? lr0 : -1);
      a.rows[r0 + i] = RowDesc{b, slot, pulse, pos0 + i, bk[slot], lr, -1,
                               (s.blk_base + slot) % S};
      if (lr >= 0) {
        a.lrow_seq[lr] = b;
#pragma unroll
        for (int x = 0; x < kMaxExtra; ++x)
          a.lrow_extra[(int64_t)lr * kMaxExtra + x] = x < slot ? bk[1 + x] : -1;
        // distinct stream per (round, draft or verify, block row)
        a.lrow_ctr[lr] = (s.ctr * 2u + (s.blk_phase == 0 ? 0u : 1u)) * (uint32_t)kMaxBlock + slot;
      }
    }
    if (spec) {
      // next round's first row: position after the block, the slot past the block's; its
      // draw is the next round's first draft (that round's counter, seen tokens = this
      // round's drafts and the guess)
      const int r = base[0] + v[0] + (pulse == 0 ? nrow : 0);
      const int lr = lr0 + lrows;
      a.rows[r] = RowDesc{b, S - 1, 0, s.c_pos + nrow, s.s_tok, lr, -1, (s.blk_base + S - 1) % S};
#pragma unroll
      for (int i = 0; i < kMaxBlock; ++i) un.row[i] = i == nrow ? r : un.row[i];
      s.row_s = r;
      s.lrow_s = lr;
      a.lrow_seq[lr] = b;
#pragma unroll
      for (int x = 0; x < kMaxExtra; ++x)
        a.lrow_extra[(int64_t)lr * kMaxExtra + x] =
            x < nrow - 1 ? bk[1 + x] : (x == nrow - 1 ? s.s_tok : -1);
      a.lrow_ctr[lr] = ((s.ctr + 1u) * 2u) * (uint32_t)kMaxBlock;
    }
    a.units[v[4]] = un;
  }
#pragma unroll
  for (int i = 0; i < kMaxBlock; ++i) s.blk[i] = bk[i];
  if (act) state_store(a.state + b, s);
  if (b == 0) {
    for (int p = 0; p < 4; ++p) {
      ctl->pulse_start[p] = p < 3 ? base[p] : total[0] + total[1] + total[2];
      ctl->pulse_count[p] = p < 3 ? total[p] : 0;
    }
    ctl->n_rows = total[0] + total[1] + total[2];
    ctl->n_lrows = total[3];
    ctl->n_units = total[4];
    ctl->active = total[4];
    ctl->step += 1;
  }
}

int launch_sample(const SampleArgs& a, int dtype, int max_lrows, hipStream_t s) {
  // kSampleThreads threads per logits row, PER = V / kSampleThreads logits per thread
  if (a.V % 4096 != 0 || a.V > 65536)
    return fail(PULSAR_ERR_UNSUPPORTED, "sample: vocab must be a multiple of 4096 and <= 65536");
  const int per = a.V / kSampleThreads;
#define PULSAR_SAMPLE_CASE(N)                                                                   \
  case N:                                                                                       \
    if (dtype == PULSAR_BF16)                                                                   \
      sample_kernel<bf16, N, kSampleThreads><<<max_lrows, kSampleThreads, 0, s>>>(a);          \
    else                                                                                        \
      sample_kernel<float, N, kSampleThreads><<<max_lrows, kSampleThreads, 0, s>>>(a);         \
    break;
  switch (per) {
    PULSAR_SAMPLE_CASE(4)
    PULSAR_SAMPLE_CASE(8)
    PULSAR_SAMPLE_CASE(16)
    PULSAR_SAMPLE_CASE(32)
    PULSAR_SAMPLE_CASE(64)
    default:
      return fail(PULSAR_ERR_UNSUPPORTED, "sample: vocab / 4096 must be a power of two");
  }
#undef PULSAR_SAMPLE_CASE
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

namespace {
// Control block, seed word and per-sequence counters of a standalone sampling call.
__global__ void sample_setup_kernel(StepCtl* ctl, uint64_t* seed_dev, SeqState* st,
                                    const uint32_t* ctr, int n_rows, int n_seq, uint64_t seed) {
  int32_t* c = reinterpret_cast<int32_t*>(ctl);
  for (int i = threadIdx.x; i < (int)(sizeof(StepCtl) / 4); i += blockDim.x) c[i] = 0;
  __syncthreads();
  if (threadIdx.x == 0) {
    ctl->n_lrows = n_rows;
    *seed_dev = seed;
  }
  for (int i = threadIdx.x; i < n_seq; i += blockDim.x) {
    SeqState z{};
    z.ctr = ctr[i];
    st[i] = z;
  }
}
}  // namespace

size_t sample_workspace_bytes(int n_seq) {
  return 256 + 256 + (size_t)n_seq * sizeof(SeqState);
}

int launch_sample_rows(const float* logits, int n_rows, int V, int dtype, const uint32_t* seen,
                       const int32_t* row_seq, const int32_t* row_extra, const uint32_t* seq_ctr,
                       int n_seq, uint64_t seed, float temperature, float top_p, float rep_penalty,
                       int greedy, int32_t* out_argmax, int32_t* out_draw, void* workspace,
                       hipStream_t s) {
  static_assert(sizeof(StepCtl) <= 256, "control block fits its workspace slot");
  char* ws = static_cast<char*>(workspace);
  StepCtl* ctl = reinterpret_cast<StepCtl*>(ws);
  uint64_t* seed_dev = reinterpret_cast<uint64_t*>(ws + 256);
  SeqState* st = reinterpret_cast<SeqState*>(ws + 512);
  sample_setup_kernel<<<1, 256, 0, s>>>(ctl, seed_dev, st, seq_ctr, n_rows, n_seq, seed);
  PULSAR_LAUNCH_CHECK();
  SampleArgs a{};
  a.ctl = ctl;
  a.logits = logits;
  a.lrow_seq = row_seq;
  a.lrow_extra = row_extra;
  a.extra_stride = 1;
  a.n_extra = 1;
  a.seen = seen;
  a.state = st;
  a.V = V;
  a.greedy = greedy;
  a.temperature = temperature;
  a.top_p = top_p;
  a.rep_penalty = rep_penalty;
  a.seed = seed_dev;
  a.out_argmax = out_argmax;
  a.out_draw = out_draw;
  a.n_seq = n_seq;
  return launch_sample(a, dtype, n_rows, s);
}

template <int NL>
void launch_controller_nl(const ControllerArgs& a, hipStream_t s) {
  if (a.draft_len > 0)
    controller_block_kernel<NL><<<1, 256, 0, s>>>(a);
  else
    controller_kernel<NL><<<1, 256, 0, s>>>(a);
}

int launch_controller(const ControllerArgs& a, hipStream_t s) {
  if (a.B > 256) return fail(PULSAR_ERR_UNSUPPORTED, "controller: at most 256 sequences");
  if (a.max_lrows < a.B || a.max_lrows > kCtlMaxLrows)
    return fail(PULSAR_ERR_INVALID, "controller: max_lrows must be in [B, 2048]");
  if (a.n_stop < 0 || a.n_stop > 8) return fail(PULSAR_ERR_INVALID, "controller: n_stop");
  if (a.draft_len > 0 && (a.draft_len >= kMaxBlock || a.n_pulses > 3 || !a.lrow_ctr))
    return fail(PULSAR_ERR_INVALID, "controller: draft-block mode arguments");
  // draws per thread of the LDS copy: 2 max_lrows over 256 threads
  const int nl = (2 * a.max_lrows + 255) / 256;
  if (nl <= 1) launch_controller_nl<1>(a, s);
  else if (nl <= 2) launch_controller_nl<2>(a, s);
  else if (nl <= 4) launch_controller_nl<4>(a, s);
  else if (nl <= 8) launch_controller_nl<8>(a, s);
  else launch_controller_nl<16>(a, s);
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

}  // namespace pulsar

// ---------------------------------------------------------------------------
// Allocation-free sampling entry: pulsar_sample_rows with its workspace (control block, seed
// word, per-sequence states) in a file-scope device array instead of a caller buffer, for
// callers that cannot allocate device memory (code under HIP graph capture, serving loops).
// Each GPU holds its own copy of the array until the process ends; host code reaches it only
// through the address hipGetSymbolAddress returns for the current device, looked up once per
// device on the entry's first call there. Calls that overlap on one GPU share the array and
// race; calls on one stream are ordered.
// ---------------------------------------------------------------------------
namespace pulsar {
namespace {

constexpr int kStaticSampleSeqs = 4096;
constexpr size_t kStaticSampleBytes = 512 + (size_t)kStaticSampleSeqs * sizeof(SeqState);
static_assert(kStaticSampleBytes >= 512 + 4096 * 128, "scratch holds 4096 sequence states");

static __device__ __align__(256) char scratch[kStaticSampleBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's scratch (looked up once per device, with it current).
int scratch_address(void** out) {
  int dev = -1;
  PULSAR_CHECK_HIP(hipGetDevice(&dev));
  PULSAR_REQUIRE(dev >= 0 && dev < kMaxDevices, "sample_rows_static: device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(PULSAR_ERR_HIP,
                  std::string("sample_rows_static: hipGetSymbolAddress(scratch): ") +
                      hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PULSAR_OK;
}

}  // namespace
}  // namespace pulsar

extern "C" int pulsar_sample_rows_static(const float* logits, int32_t n_rows, int32_t V,
                                         int32_t dtype, const uint32_t* seen,
                                         const int32_t* row_seq, const int32_t* row_extra,
                                         const uint32_t* seq_ctr, int32_t n_seq, uint64_t seed,
                                         float temperature, float top_p,
                                         float repetition_penalty, int32_t greedy,
                                         int32_t* out_argmax, int32_t* out_draw,
                                         hipStream_t stream) {
  using namespace pulsar;
  PULSAR_REQUIRE(logits && seen && row_seq && row_extra && seq_ctr && out_argmax && out_draw,
                 "sample_rows_static: null argument");
  PULSAR_REQUIRE(n_rows >= 0 && n_seq >= 1, "sample_rows_static: n_rows >= 0 and n_seq >= 1");
  PULSAR_REQUIRE(n_seq <= kStaticSampleSeqs,
                 "sample_rows_static: n_seq > 4096 (the size of its static scratch); use "
                 "pulsar_sample_rows with a workspace");
  PULSAR_REQUIRE(dtype == PULSAR_BF16 || dtype == PULSAR_F32, "sample_rows_static: dtype");
  PULSAR_REQUIRE(temperature > 0.f && top_p > 0.f && top_p <= 1.f && repetition_penalty > 0.f,
                 "sample_rows_static: temperature > 0, 0 < top_p <= 1, repetition_penalty > 0");
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != PULSAR_OK) return rc;
  if (n_rows == 0) return PULSAR_OK;
  return launch_sample_rows(logits, n_rows, V, dtype, seen, row_seq, row_extra, seq_ctr, n_seq,
                            seed, temperature, top_p, repetition_penalty, greedy, out_argmax,
                            out_draw, ws, stream);
}
