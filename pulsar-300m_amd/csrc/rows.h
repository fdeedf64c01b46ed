// Argument blocks and launchers of the per-row kernels (rows.hip).
#pragma once

#include "engine.h"

namespace pulsar {

constexpr int kSplitLen = 256;  // keys per decode-attention block (fp32 path)
// bf16 decode attention: waves per workgroup, and keys per split workgroup at one 64-key
// block per wave (the unit in which split counts and partial slots are sized; launches
// take 2-8 blocks per wave)
constexpr int kUnitWaves = 4;
constexpr int kUnitSplit = kUnitWaves * 64;
// engines whose context needs more 256-key splits than this use 2048-key splits in the
// global layers
constexpr int kLongCacheSplits = 16;
// engines of at least this many sequences (units) take 1024-key splits in the long
// engines' sliding-window layers, fewer keep 256-key splits
constexpr int kManyUnits = 16;
// 64-key blocks per wave and split in engines below the long-cache threshold, and in
// those of at least kWideSplitUnits sequences (many workgroups already: 1024-key splits)
constexpr int kShortCacheBlocks = 2;
constexpr int kWideSplitUnits = 128;
static_assert(kUnitSplit >= kSplitLen, "split partial slots are sized for kSplitLen");
constexpr int kMaxRank = 16;    // re-injection gate rank bound

// KV cache addressing. Local (sliding-window) layers: a per-sequence ring of `lcap`
// positions (a multiple of 64). Global layers: pages of 64 positions from a pool shared by
// the batch; page_table[b * max_pages + p] is the pool page holding positions
// [64 p, 64 p + 64) of sequence b (the same page index in every global layer). Pages are
// given out when a sequence first writes a position in them (prefill and fill_kv for the
// prompt, the controller as decoding reaches a new page). K is stored position-major
// ([..][pos][64]); V is stored transposed, dimension-major ([..][64][pos]), so that the
// keys of one dimension are contiguous: the layout the P.V matrix-core operand reads.
//   local  K: [B][Hkv][lcap][64]            V: [B][Hkv][64][lcap]
//   global K: [pool pages][Hkv][64 pos][64]  V: [pool pages][Hkv][64][64 pos]
struct KVDesc {
  void* k[kMaxLayers];
  void* v[kMaxLayers];
  uint32_t local_mask;
  int Hkv;
  int lcap;
  int max_pages;                // page-table entries per sequence
  const int32_t* page_table;    // [B][max_pages] pool page ids
};

// Pool page of sequence b's positions [64 p, 64 p + 64) in the global layers.
__device__ __forceinline__ int64_t kv_page(const int32_t* table, int max_pages, int b, int pos) {
  return table[(int64_t)b * max_pages + pos / kPage];
}

__device__ __forceinline__ bool kv_is_local(const KVDesc& c, int layer) {
  return (c.local_mask >> layer) & 1u;
}

// K element (pos, 0).
__device__ __forceinline__ int64_t kv_offset(const KVDesc& c, int layer, int b, int g, int pos) {
  if (kv_is_local(c, layer)) {
    return (((int64_t)b * c.Hkv + g) * c.lcap + (pos % c.lcap)) * kHeadDim;
  }
  const int64_t page = kv_page(c.page_table, c.max_pages, b, pos);
  return ((page * c.Hkv + g) * kPage + (pos % kPage)) * kHeadDim;
}

// V element (pos, dim).
__device__ __forceinline__ int64_t kv_offset_v(const KVDesc& c, int layer, int b, int g, int pos,
                                               int dim) {
  if (kv_is_local(c, layer)) {
    return (((int64_t)b * c.Hkv + g) * kHeadDim + dim) * c.lcap + (pos % c.lcap);
  }
  const int64_t page = kv_page(c.page_table, c.max_pages, b, pos);
  return ((page * c.Hkv + g) * kHeadDim + dim) * kPage + (pos % kPage);
}

// A 64-aligned block of 64 positions starting at kb is contiguous in both caches:
// K(kb + i, d) = k0 + i*64 + d and V(kb + i, d) = v0 + d*vstride + i.
struct KVBlock {
  int64_t k0, v0;
  int vstride;
};
__device__ __forceinline__ KVBlock kv_block(const KVDesc& c, int layer, int b, int g, int kb) {
  KVBlock r;
  if (kv_is_local(c, layer)) {
    const int64_t bg = (int64_t)b * c.Hkv + g;
    const int ring = kb % c.lcap;
    r.k0 = (bg * c.lcap + ring) * kHeadDim;
    r.v0 = bg * kHeadDim * c.lcap + ring;
    r.vstride = c.lcap;
  } else {
    const int64_t pg = kv_page(c.page_table, c.max_pages, b, kb) * c.Hkv + g;
    r.k0 = pg * kPage * kHeadDim;
    r.v0 = pg * kHeadDim * kPage;
    r.vstride = kPage;
  }
  return r;
}

struct PulseInputArgs {
  const StepCtl* ctl;
  const RowDesc* rows;
  int D, rank, prefill, prefill_T;
  int slots;                // token-state slots per sequence (decode state = seq*slots+slot)
  float eps;
  const void* tok_emb;
  const float* anchor_norm;
  const float* conv_w;      // nullable
  const float* state_norm;
  const void* step_emb;     // [P][D] T
  const void* reinject_down;  // [P][rank][2D] T
  const void* reinject_up;    // [P][D][rank] T
  const void* reinject_bias;  // [P][D] T
  void* e_state;            // anchor embedding per state
  void* hout_state;         // previous pulse output per state
  void* h_in;
  void* h;
  int32_t* zero_counts;     // zeroed by block 0 (expert list counts of the step)
  int n_zero;
  const float* norm_w;      // [P][D] attn_norm of the first layer (nullable)
  void* xn;                 // normed h_in output when norm_w is set
};

struct NormArgs {
  const StepCtl* ctl;
  const RowDesc* rows;
  int use_lrows;
  const int32_t* lrow_src;
  const void* x;
  int64_t ldx;
  const float* w;
  int64_t w_pulse_stride;
  void* y;
  int D;
  float eps;
};

struct QKPostArgs {
  const StepCtl* ctl;
  const RowDesc* rows;
  void* qkv;
  int64_t ldq;
  int H, Hkv, layer, is_local, prefill, prefill_T, window, base_seq_len;
  float eps;
  const float* q_norm;    // [P][H][64]
  const float* k_norm;    // [P][Hkv][64]
  const float* v_lambda;  // [P] sigmoid(lambda) rounded through T
  void* v_first;          // [rows][Hkv*64]
  const float* cos;       // [positions][32]
  const float* sin;
  KVDesc kv;
};

// One layer's caches, resolved on the host (the kernel reads them straight from its
// arguments instead of indexing the per-layer pointer arrays by layer).
struct KVLayer {
  const void* k;
  const void* v;
  int lcap, max_pages;
  const int32_t* page_table;
};

// Block of key position kb of sequence b, KV head g; global layers take the pool page of
// the block from the caller (`page`, read from the page table beforehand).
__device__ __forceinline__ KVBlock kv_block_layer_page(const KVLayer& c, bool local, int Hkv,
                                                       int b, int g, int kb, int64_t page) {
  KVBlock r;
  if (local) {
    const int64_t bg = (int64_t)b * Hkv + g;
    const int ring = kb % c.lcap;
    r.k0 = (bg * c.lcap + ring) * kHeadDim;
    r.v0 = bg * kHeadDim * c.lcap + ring;
    r.vstride = c.lcap;
  } else {
    const int64_t pg = page * Hkv + g;
    r.k0 = pg * kPage * kHeadDim;
    r.v0 = pg * kHeadDim * kPage;
    r.vstride = kPage;
  }
  return r;
}

__device__ __forceinline__ KVBlock kv_block_layer(const KVLayer& c, bool local, int Hkv, int b,
                                                  int g, int kb) {
  return kv_block_layer_page(c, local, Hkv, b, g, kb,
                             local ? 0 : kv_page(c.page_table, c.max_pages, b, kb));
}

struct AttnArgs {
  const StepCtl* ctl;
  const RowDesc* rows;
  const AttnUnit* units;  // decode, matrix-core path: units of the step (ctl->n_units)
  KVLayer kl;             // decode, matrix-core path: set by launch_attn_decode
  const void* qkv;
  int64_t ldq;
  const void* gate;  // [rows][H] T
  void* out;         // [rows][H*64] T
  float* part;       // decode split partials
  int32_t* split_done;  // decode: per (unit, kv head) count of finished splits (self-resetting)
  int max_splits;       // split partial slots per (unit or row, kv head)
  int max_splits_unit;  // bf16 path: splits of kUnitSplit keys
  int max_units;
  int unit_rows;        // bf16 path: most rows a unit of this launch holds (1..kMaxBlock)
  int max_ctx;          // positions per sequence of the engine (bounds a unit's key range)
  int H, Hkv, layer, is_local, window, prefill_T;
  float scale;
  KVDesc kv;
  // bf16 decode: q/k/v post-processing (what qk_post_kernel does) fused into the attention;
  // qkv then holds the raw projection (q | k | v columns)
  int post;
  int base_seq_len;
  float eps;
  const float* q_norm;    // [P][H][64]
  const float* k_norm;    // [P][Hkv][64]
  const float* v_lambda;  // [P]
  void* v_first;          // [rows][Hkv*64]
  const float* cos;       // [positions][32]
  const float* sin;
};

struct RouterArgs {
  const StepCtl* ctl;
  const RowDesc* rows;
  const void* x;
  const float* w;      // [P][E][D] fp32
  const float* bias;   // [P][E]
  int E, K, D, pulse, m_fixed;
  int32_t* topk_idx;   // [rows][K]
  float* topk_w;       // [rows][K] (values rounded through T)
  int32_t* lists;      // [E][list_stride] assignment ids (decode), nullable
  int32_t* list_count; // [E]
  int64_t list_stride;
  const float* norm_w; // norm_router: [P][D] mlp_norm weight
  void* xn;            // norm_router: normed output [rows][D]
  float eps;
};

struct CombineArgs {
  const StepCtl* ctl;  // null for prefill (m_fixed rows)
  const RowDesc* rows;
  int m_fixed, pulse, prefill, K, D;
  const void* shared;  // [rows][D]
  const void* routed;  // [rows*K][D]
  const float* topk_w;
  const int32_t* keep; // [rows*K] or null
  const void* routed_scale;  // [P][D] T
  void* h;
  const float* next_norm;    // [P][D] attn_norm of the next layer (nullable)
  void* xn;                  // normed h output when next_norm is set
  float eps;
  // decode, last layer (nullable hout_state: no pulse output here): the pulse output of
  // pulse_output_kernel folded in — harmonic residual into the row's token state and, for
  // logits rows, the final norm
  const void* h_in;          // [rows][D] pulse input
  const void* res_scale;     // [P][D] T
  void* hout_state;          // [B * slots][D]
  int slots;
  const float* final_norm;   // [D]
  void* xn_final;            // [lrows][D]
};

struct PulseOutputArgs {
  const StepCtl* ctl;
  const RowDesc* rows;
  int D, prefill, prefill_T;
  int slots;                // token-state slots per sequence
  float eps;
  const void* h_in;
  const void* h;
  const void* res_scale;  // [P][D] T
  void* hout_state;
  const float* final_norm;
  void* xn_final;         // [lrows][D]
};

// route_topk for compile-time E and K: every loop unrolled and every array index a
// constant, so the arrays stay in registers (with runtime bounds the selected experts'
// scores are read with lane-dependent indices). The same operations in the same order as
// the generic form below, so the results are identical.
template <typename T, int E, int K>
__device__ __forceinline__ void route_topk_fixed(const float* lg, const float* bias, int r,
                                                 const RouterArgs& a) {
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) sum += lg[e];
  const float mean = sum / (float)E;
  float s[E], b[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float c = lg[e] - mean;
    s[e] = 1.0f / (1.0f + expf(-c));
    b[e] = s[e] + bias[e];
  }
  // sorted (descending) selection with its experts' scores; the initial entries name
  // expert 0, as the generic form's do
  int bi[K];
  float bv[K], bs[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    bi[k] = 0;
    bv[k] = -INFINITY;
    bs[k] = s[0];
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float v = b[e];
    if (v > bv[K - 1]) {
      int p = K - 1;
#pragma unroll
      for (int q = K - 1; q > 0; --q)
        if (p == q && v > bv[q - 1]) {
          bv[q] = bv[q - 1];
          bi[q] = bi[q - 1];
          bs[q] = bs[q - 1];
          p = q - 1;
        }
#pragma unroll
      for (int q = 0; q < K; ++q)
        if (p == q) {
          bv[q] = v;
          bi[q] = e;
          bs[q] = s[e];
        }
    }
  }
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) tot += bs[k];
  tot += 1e-6f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    a.topk_idx[(int64_t)r * K + k] = bi[k];
    a.topk_w[(int64_t)r * K + k] = rnd<T>(bs[k] / tot);
    if (a.lists) {
      const int p = atomicAdd(&a.list_count[bi[k]], 1);
      a.lists[(int64_t)bi[k] * a.list_stride + p] = r * K + k;
    }
  }
}

// Shared top-k routine of the router kernels (single thread).
template <typename T>
__device__ __forceinline__ void route_topk(const float* lg, int E, int K, const float* bias, int r,
                                           const RouterArgs& a) {
  if (E == 16 && K == 4) {
    route_topk_fixed<T, 16, 4>(lg, bias, r, a);
    return;
  }
  float sum = 0.f;
  for (int e = 0; e < E; ++e) sum += lg[e];
  const float mean = sum / (float)E;
  float s[32], b[32];
  for (int e = 0; e < E; ++e) {
    const float c = lg[e] - mean;
    s[e] = 1.0f / (1.0f + expf(-c));
    b[e] = s[e] + bias[e];
  }
  int bi[8];
  float bv[8];
  for (int k = 0; k < K; ++k) {
    bi[k] = 0;
    bv[k] = -INFINITY;
  }
  for (int e = 0; e < E; ++e) {
    const float v = b[e];
    if (v > bv[K - 1]) {
      int p = K - 1;
      while (p > 0 && v > bv[p - 1]) {
        bv[p] = bv[p - 1];
        bi[p] = bi[p - 1];
        --p;
      }
      bv[p] = v;
      bi[p] = e;
    }
  }
  float tot = 0.f;
  for (int k = 0; k < K; ++k) tot += s[bi[k]];
  tot += 1e-6f;
  for (int k = 0; k < K; ++k) {
    a.topk_idx[(int64_t)r * K + k] = bi[k];
    a.topk_w[(int64_t)r * K + k] = rnd<T>(s[bi[k]] / tot);
    if (a.lists) {
      const int p = atomicAdd(&a.list_count[bi[k]], 1);
      a.lists[(int64_t)bi[k] * a.list_stride + p] = r * K + k;
    }
  }
}

int launch_pulse_input(const PulseInputArgs& a, int dtype, int max_rows, hipStream_t s);
int launch_norm_rows(const NormArgs& a, int dtype, int max_rows, hipStream_t s);
int launch_qk_post(const QKPostArgs& a, int dtype, int max_rows, hipStream_t s);
int launch_attn_decode(const AttnArgs& a, int dtype, int max_rows, hipStream_t s);
int launch_attn_prefill(const AttnArgs& a, int dtype, int B, hipStream_t s);
int launch_router_decode(const RouterArgs& a, int dtype, int max_rows, hipStream_t s);
// mlp_norm + router fused: a.x = residual stream h, a.norm_w/a.xn the norm weight/output.
int launch_norm_router(const RouterArgs& a, int dtype, int max_rows, hipStream_t s);
int launch_router_prefill(const RouterArgs& a, int dtype, hipStream_t s);
int launch_prefill_capacity(const int32_t* idx, const float* w, int32_t* keep, int32_t* lists,
                            int32_t* lcount, int64_t list_stride, int B, int T_, int K, int E,
                            int C, hipStream_t s);
int launch_moe_combine(const CombineArgs& a, int dtype, int max_rows, hipStream_t s);
int launch_pulse_output(const PulseOutputArgs& a, int dtype, int max_rows, hipStream_t s);
int launch_prefill_stem(const int32_t* ids, const void* emb, const float* anchor_w,
                        const float* conv_w, void* a_buf, void* e_buf, int B, int T_, int D,
                        float eps, int dtype, hipStream_t s);

}  // namespace pulsar
