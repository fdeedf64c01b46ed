/*
 * pulsar_hip.h — C ABI of libpulsar_hip.so, the MI355X (gfx950) implementation of
 * Pulsar's KV-cache self-speculative decode path.
 *
 * Conventions
 *   - Every entry returns an int status (PULSAR_OK = 0). On failure
 *     pulsar_last_error() returns a thread-local message; no C++ exception crosses
 *     the boundary.
 *   - Pointers are device pointers unless the name says host_. The caller allocates
 *     every input and output (the library keeps no allocation across calls except
 *     inside an engine handle).
 *   - Work is enqueued on the given HIP stream; no entry synchronises the host unless
 *     documented. Kernels launched here are capturable in a HIP graph.
 *   - dtype selects the element type of activation tensors: PULSAR_F32 or PULSAR_BF16
 *     (bf16 as raw 16-bit words, round-to-nearest-even). The reference op surface is
 *     bf16-only; fp32 instantiations are extra.
 *
 * Each op entry cites the reference binding it replaces
 * (csrc/pulsar_cuda.cpp = pybind module, csrc/kernels.cu = CUDA kernels).
 */
#ifndef PULSAR_HIP_H_
#define PULSAR_HIP_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PULSAR_OK 0
#define PULSAR_ERR_INVALID 1     /* bad shape, dtype or argument (reference: TORCH_CHECK) */
#define PULSAR_ERR_HIP 2         /* HIP runtime or launch error */
#define PULSAR_ERR_UNSUPPORTED 3 /* configuration this build does not implement */

#define PULSAR_F32 0
#define PULSAR_BF16 1

/* Thread-local message of the last failing call on this thread. */
const char* pulsar_last_error(void);
/* ABI version of this header (bumped on any signature change). */
int pulsar_abi_version(void);

/* ---------------------------------------------------------------------------------
 * Op surface of the reference's pulsar_cuda module
 * ------------------------------------------------------------------------------- */

/* rmsnorm_forward(x, weight, eps) -> (y, rsqrt)
 * Replaces csrc/pulsar_cuda.cpp:202 / csrc/kernels.cu:224-266.
 * x, y: [rows, dim] contiguous; w: fp32 [dim]; rsqrt_out: fp32 [rows] (nullable). */
int pulsar_rmsnorm_forward(const void* x, const float* w, void* y, float* rsqrt_out,
                           int64_t rows, int64_t dim, float eps, int dtype,
                           hipStream_t stream);

/* rope_forward(qk, cos, sin) -> out, rotate-half with fp32 tables.
 * Replaces csrc/pulsar_cuda.cpp:211 / csrc/kernels.cu:935-965.
 * x, y: contiguous [rows, head_dim] where row = ((b*H)+h)*T + t; table row t = row % T;
 * cos, sin: fp32 [T, head_dim/2]. */
int pulsar_rope_forward(const void* x, void* y, const float* cos, const float* sin,
                        int64_t rows, int64_t T, int64_t head_dim, int dtype,
                        hipStream_t stream);

/* qk_rmsnorm_rope_forward(x, weight, cos, sin, T, eps) -> (y, rsqrt)
 * Replaces csrc/pulsar_cuda.cpp:225-226 / csrc/kernels.cu:2716-2765.
 * x: [B,H,T,64] with element strides (sB, sH, sT, 1); w: fp32 [H,64];
 * cos, sin: fp32 [T,32]; y: contiguous [B,H,T,64]; rsqrt_out: fp32 [B*H*T] (nullable).
 * head_dim must be 64 (error message contains "head_dim == 64"). */
int pulsar_qk_rmsnorm_rope_forward(const void* x, int64_t sB, int64_t sH, int64_t sT,
                                   int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                   const float* w, const float* cos, const float* sin,
                                   void* y, float* rsqrt_out, float eps, int dtype,
                                   hipStream_t stream);

/* fused_attn_gate_forward(attn_out, gate_logits) -> out
 * Replaces csrc/pulsar_cuda.cpp:230-231 / csrc/kernels.cu:2930-2958.
 * attn: contiguous [B,H,T,64]; gate_logits: fp32 [B,T,H]; out: [B,T,H*64]. */
int pulsar_fused_attn_gate_forward(const void* attn, const float* gate_logits, void* out,
                                   int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                   int dtype, hipStream_t stream);

/* causal_depthwise_conv1d_k4_forward(x, weight) -> y = x + sum_k w[:,k] x[t-k]
 * Replaces csrc/pulsar_cuda.cpp:274-276 / csrc/kernels.cu:3653-3691.
 * x, y: contiguous [B,T,D]; w: fp32 [D,4]. */
int pulsar_causal_conv1d_k4_forward(const void* x, const float* w, void* y, int64_t B,
                                    int64_t T, int64_t D, int dtype, hipStream_t stream);

/* fused_swiglu_forward(gu, d_ff) -> silu(gu[..,:d_ff]) * gu[..,d_ff:]
 * Replaces csrc/pulsar_cuda.cpp:209 / csrc/kernels.cu:825-863.
 * gu: contiguous [rows, 2*d_ff]; out: [rows, d_ff]. */
int pulsar_fused_swiglu_forward(const void* gu, void* out, int64_t rows, int64_t d_ff,
                                int dtype, hipStream_t stream);

/* moe_router_topk_forward(logits, expert_bias, top_k, z_loss_weight)
 *   -> (topk_idx int64 [N,K], topk_weights bf16 [N,K], z_loss fp32 [], probs_mean fp32 [E])
 * Replaces csrc/pulsar_cuda.cpp:255-266 / csrc/kernels.cu:2417-2491.
 * Centred-sigmoid scores, top-K of score+bias (ties to the lower index), weights
 * s/(sum s + 1e-6). z_loss = w_z * mean(logsumexp(centred)^2) (0 when w_z <= 0),
 * probs_mean = mean sigmoid score; both reduced deterministically. E <= 32, K <= 8. */
int pulsar_moe_router_topk_forward(const void* logits, int logits_dtype, const float* bias,
                                   int64_t* topk_idx, uint16_t* topk_w_bf16, float* z_loss,
                                   float* probs_mean, int64_t N, int64_t E, int64_t K,
                                   float z_loss_weight, hipStream_t stream);

/* The same with a caller workspace of pulsar_moe_router_workspace_bytes(N, E) bytes (device
 * memory, any contents): the statistics are then summed per workgroup of 128 tokens inside
 * the top-k launch and the partials merged in workgroup order (deterministic), instead of
 * one workgroup reading every token again. Same results up to the summation order of the
 * statistics; the indices and weights are identical. The Python op surface uses this entry.
 * pulsar_moe_router_workspace_bytes returns -1 for E outside [1, 32] or N < 0. */
int64_t pulsar_moe_router_workspace_bytes(int64_t N, int64_t E);
int pulsar_moe_router_topk_forward_ws(const void* logits, int logits_dtype, const float* bias,
                                      int64_t* topk_idx, uint16_t* topk_w_bf16, float* z_loss,
                                      float* probs_mean, int64_t N, int64_t E, int64_t K,
                                      float z_loss_weight, float* workspace,
                                      hipStream_t stream);

/* moe_dispatch_forward(x, topk_idx, token_to_slot, E, C, expert_counts) -> [E,C,D]
 * Replaces csrc/pulsar_cuda.cpp:213-215 / csrc/kernels.cu:1548-1605.
 * Slots >= count[e] (or all unused slots when expert_counts is NULL) are zeroed. */
int pulsar_moe_dispatch_forward(const void* x, const int64_t* topk_idx, const int32_t* slots,
                                const int64_t* expert_counts, void* expert_inputs, int64_t N,
                                int64_t D, int64_t K, int64_t E, int64_t C, int dtype,
                                hipStream_t stream);

/* moe_combine_forward(expert_outputs, topk_idx, topk_weights, token_to_slot, shared_out)
 *   out[t] = shared[t] + sum_k w[t,k] * expert_out[e,slot]   (fp32 accumulate)
 * Replaces csrc/pulsar_cuda.cpp:217-219 / csrc/kernels.cu:1633-1664.
 * shared_out nullable; weights are bf16 words. */
int pulsar_moe_combine_forward(const void* expert_outputs, const int64_t* topk_idx,
                               const uint16_t* topk_w_bf16, const int32_t* slots,
                               const void* shared_out, void* out, int64_t N, int64_t D,
                               int64_t K, int64_t E, int64_t C, int dtype, hipStream_t stream);

/* moe_slots_from_order(flat_e, order, E, C) -> (slots int32 [M], counts int64 [E])
 * Replaces csrc/pulsar_cuda.cpp:235-236 / csrc/kernels.cu:3058-3095.
 * slot = rank of the assignment within its expert in `order`, -1 when >= C. */
int pulsar_moe_slots_from_order(const int64_t* flat_e, const int64_t* order, int32_t* slots,
                                int64_t* counts, int64_t M, int64_t E, int64_t C,
                                hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Backward ops of the same surface (the training path through model.forward).
 * fp32 arithmetic; activation gradients in the activation dtype, norm / conv weight
 * gradients fp32 (zeroed by the call, then summed with atomics, so their last bits
 * depend on scheduling order).
 * ------------------------------------------------------------------------------- */

/* rmsnorm_backward(dy, x, weight, rsqrt) -> (dx, dweight)
 * Replaces csrc/pulsar_cuda.cpp:203 / csrc/kernels.cu:268-310.
 * dy, x, dx: [rows, dim] contiguous; w, dw: fp32 [dim]; rsqrt: the forward's fp32 [rows].
 * dim <= 8192. */
int pulsar_rmsnorm_backward(const void* dy, const void* x, const float* w, const float* rsqrt,
                            void* dx, float* dw, int64_t rows, int64_t dim, int dtype,
                            hipStream_t stream);

/* qk_rmsnorm_rope_backward(dy, x, weight, rsqrt_in, cos, sin, T) -> (dx, dweight)
 * Replaces csrc/pulsar_cuda.cpp:227-228 / csrc/kernels.cu:2767-2835.
 * dy: contiguous [B,H,T,64]; x: strides (sB, sH, sT, 1); dx: strides (dB, dH, dT, 1);
 * w, dw: fp32 [H,64]; rsqrt: fp32 [B*H*T]; cos, sin: fp32 [T,32]. */
int pulsar_qk_rmsnorm_rope_backward(const void* dy, const void* x, int64_t sB, int64_t sH,
                                    int64_t sT, void* dx, int64_t dB, int64_t dH, int64_t dT,
                                    int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                    const float* w, const float* rsqrt, const float* cos,
                                    const float* sin, float* dw, int dtype,
                                    hipStream_t stream);

/* fused_attn_gate_backward(grad_out, attn_out, gate_logits) -> (d_attn, d_gate)
 * Replaces csrc/pulsar_cuda.cpp:232-233 / csrc/kernels.cu:2960-2992.
 * grad_out: [B,T,H*64]; attn, d_attn: [B,H,T,64]; gate_logits, d_gate: fp32 [B,T,H]. */
int pulsar_fused_attn_gate_backward(const void* grad_out, const void* attn,
                                    const float* gate_logits, void* d_attn, float* d_gate,
                                    int64_t B, int64_t H, int64_t T, int64_t head_dim,
                                    int dtype, hipStream_t stream);

/* fused_swiglu_backward(dout, gu, d_ff) -> dgu = [d_gate | d_up]
 * Replaces csrc/pulsar_cuda.cpp:210 / csrc/kernels.cu:865-900.
 * dout: [rows, d_ff]; gu, dgu: [rows, 2*d_ff]. */
int pulsar_fused_swiglu_backward(const void* dout, const void* gu, void* dgu, int64_t rows,
                                 int64_t d_ff, int dtype, hipStream_t stream);

/* moe_dispatch_backward(d_expert_inputs, topk_idx, token_to_slot, N, D) -> dx [N,D]
 * Replaces csrc/pulsar_cuda.cpp:216 / csrc/kernels.cu:1607-1631.
 * dx[t] = sum of d_expert_inputs[e, slot] over t's kept assignments, in top-k order. */
int pulsar_moe_dispatch_backward(const void* d_expert_inputs, const int64_t* topk_idx,
                                 const int32_t* slots, void* dx, int64_t N, int64_t D,
                                 int64_t K, int64_t E, int64_t C, int dtype,
                                 hipStream_t stream);

/* moe_combine_backward(d_routed_out, expert_outputs, topk_idx, topk_weights, token_to_slot)
 *   -> (d_expert_outputs [E,C,D], d_topk_weights bf16 [N,K])
 * Replaces csrc/pulsar_cuda.cpp:220-222 / csrc/kernels.cu:1666-1711.
 * Rows of d_expert_outputs no kept assignment names are zero; dropped assignments get
 * d_topk_weights = 0. Weights are bf16 words. */
int pulsar_moe_combine_backward(const void* d_routed_out, const void* expert_outputs,
                                const int64_t* topk_idx, const uint16_t* topk_w_bf16,
                                const int32_t* slots, void* d_expert_outputs,
                                uint16_t* d_topk_w_bf16, int64_t N, int64_t D, int64_t K,
                                int64_t E, int64_t C, int dtype, hipStream_t stream);

/* moe_router_topk_backward(d_topk_weights, logits, topk_idx, z_loss_weight, d_z_loss,
 *                          d_probs_mean) -> d_logits (logits' dtype)
 * Replaces csrc/pulsar_cuda.cpp:267-269 / csrc/kernels.cu:2493-2578.
 * Adjoint of pulsar_moe_router_topk_forward with the selection held fixed: through the
 * weight normalisation, the z-loss (scaled by d_z_loss[0] when given) and probs_mean
 * (d_probs_mean fp32 [E], nullable), then the centring. E <= 32, K <= 8. */
int pulsar_moe_router_topk_backward(const uint16_t* d_topk_w_bf16, const void* logits,
                                    int logits_dtype, const int64_t* topk_idx,
                                    float z_loss_weight, const float* d_z_loss,
                                    const float* d_probs_mean, void* d_logits, int64_t N,
                                    int64_t E, int64_t K, hipStream_t stream);

/* causal_depthwise_conv1d_k4_backward(dout, x, weight) -> (dx, dweight)
 * Replaces csrc/pulsar_cuda.cpp:277-279 / csrc/kernels.cu:3693-3732.
 * dout, x, dx: contiguous [B,T,D]; w, dw: fp32 [D,4]. */
int pulsar_causal_conv1d_k4_backward(const void* dout, const void* x, const float* w, void* dx,
                                     float* dw, int64_t B, int64_t T, int64_t D, int dtype,
                                     hipStream_t stream);


/* ---------------------------------------------------------------------------------
 * Decode engine: prefill + self-speculative decode of a batch of sequences.
 * Replaces the reference's PulsarInferenceEngine (src/infer.py:181-731) and
 * UnifiedKVCache (src/infer.py:64-178). No reference C entry exists for these: the
 * reference drives the same math from Python; a binding mirrors its Python interface.
 * ------------------------------------------------------------------------------- */

#define PULSAR_MAX_LAYERS 16

/* GEMM weight layout. fp32 weights are row-major [N][K]. bf16 weights (wqkvg, wo, shared_gu,
 * shared_down, routed_gu, routed_down, lm_head) are stored in matrix-core tiles: each
 * [N][K] matrix becomes [N/16][K/32][64][8], tile (n, k) holding rows 16n..16n+15 and
 * columns 32k..32k+31 in the order the 16x16x32 bf16 MFMA B operand reads them (lane l:
 * row 16n + l%16, columns 32k + 8*(l/16) .. +8), so every wave load is 1 KB contiguous.
 * N must be a multiple of 16 and K of 256. */

/* Architecture constants plus device pointers to the kernel-format weights.
 * T = element type selected by dtype. Per-pulse tensors hold the first n_pulses pulses.
 * Host-side preparation (see pulsar_engine/model.py) merges the per-pulse LoRA into the
 * projections exactly as the reference (src/model.py:716-727), appends the attention-gate
 * rows to the merged qkv weight, transposes routed experts to [E][out][in], and rounds
 * fp32-kept parameters through T where the reference casts them (.to(x.dtype)). */
typedef struct PulsarModelDesc {
  int32_t vocab, d_model, n_heads, n_kv_heads, head_dim, d_expert, d_shared, n_layers;
  int32_t n_pulses, n_experts, top_k, window, base_seq_len, reinject_rank, dtype;
  uint32_t local_mask;      /* bit L set: layer L is a sliding-window layer */
  float rms_eps, softcap;
  int32_t rope_len;         /* rows of the RoPE tables (>= max positions) */
  const void* tok_emb;      /* [V][D] T, tied output head */
  const float* anchor_norm; /* [D] */
  const float* state_norm;  /* [D] */
  const float* final_norm;  /* [D] */
  const float* conv_w;      /* [D][4] or NULL */
  const void* step_emb;     /* [P][D] T */
  const void* reinject_down;/* [P][r][2D] T */
  const void* reinject_up;  /* [P][D][r] T */
  const void* reinject_bias;/* [P][D] T */
  const void* res_scale;    /* [P][D] T */
  const float* rope_cos_local;  /* [rope_len][head_dim/2] */
  const float* rope_sin_local;
  const float* rope_cos_global;
  const float* rope_sin_global;
  const float* attn_norm[PULSAR_MAX_LAYERS];   /* [P][D] */
  const float* mlp_norm[PULSAR_MAX_LAYERS];    /* [P][D] */
  const void* wqkvg[PULSAR_MAX_LAYERS];        /* [P][qkv+H][D] T: merged qkv | gate rows */
  const void* gate_bias[PULSAR_MAX_LAYERS];    /* [P][H] T */
  const void* wo[PULSAR_MAX_LAYERS];           /* [P][D][H*hd] T merged */
  const float* q_norm[PULSAR_MAX_LAYERS];      /* [P][H][hd] */
  const float* k_norm[PULSAR_MAX_LAYERS];      /* [P][Hkv][hd] */
  const float* v_lambda[PULSAR_MAX_LAYERS];    /* [P] sigmoid(lambda) rounded through T */
  const void* shared_gu[PULSAR_MAX_LAYERS];    /* [2 d_shared][D] T */
  const void* shared_down[PULSAR_MAX_LAYERS];  /* [D][d_shared] T */
  const void* routed_gu[PULSAR_MAX_LAYERS];    /* [E][2 d_expert][D] T */
  const void* routed_down[PULSAR_MAX_LAYERS];  /* [E][D][d_expert] T */
  const float* router[PULSAR_MAX_LAYERS];      /* [P][E][D] */
  const float* expert_bias[PULSAR_MAX_LAYERS]; /* [P][E] */
  const void* routed_scale[PULSAR_MAX_LAYERS]; /* [P][D] T */
  const void* lm_head;      /* output head (tied to tok_emb) in the GEMM weight layout */
} PulsarModelDesc;

/* Generation settings (the reference's generate() arguments, src/infer.py:733-743). */
typedef struct PulsarEngineConfig {
  int32_t max_batch;     /* sequences */
  int32_t max_prompt;    /* prompt tokens per sequence */
  int32_t max_new;       /* max_new_tokens */
  int32_t max_ctx;       /* positions per sequence (>= max_prompt + max_new + 1) */
  int32_t speculative;   /* 1: self-speculative (generate(speculative=True)); 0: plain */
  int32_t all_logits;    /* 1: compute logits for every pulse pass (testing) */
  float temperature;     /* <= 1e-4 selects greedy */
  float top_p;
  float repetition_penalty;
  int32_t n_stop;
  int32_t stop_ids[8];
  uint64_t seed;
  /* 0: the reference's exact self-speculation (one pulse-0 draft per token, pipelined).
   * 1..7: draft-block mode, a multi-token draft with no reference counterpart: per round,
   * up to draft_len drafts from pulse 0 alone, then one verify of the block [t, drafts]
   * with every pulse (row i attends the cache plus the block's same-pulse keys at positions
   * <= its own, the reference prefill's rule), drafts accepted down the block by the
   * reference's equal-draw rule (src/infer.py:704-725). Needs max_ctx >= max_prompt +
   * max_new + 2 + draft_len. */
  int32_t draft_len;
  /* Adaptive early exit (the reference's set_early_exit_threshold, src/infer.py:198-232,
   * :536-547). early_exit = 1: a token run by decode_step (every decoded token in plain
   * mode, an accepted draft in speculative mode) stops after pulse k < n_pulses - 1 when
   * the top-1 probability of softmax(its pulse-k logits), rounded to the activation dtype,
   * is >= early_exit_threshold; it then keeps pulse k's keys/values and the next token is
   * drawn from pulse k's logits. Exits are counted per pulse (PULSAR_BUF_EXIT_COUNTS). In
   * plain mode the last emitted token still runs its pulses, as the reference's loop does,
   * so that its exit is counted. Exact schedule only (draft_len = 0). */
  int32_t early_exit;
  double early_exit_threshold;
  /* Pages of 64 positions in the global layers' KV pool, shared by the batch (0: enough for
   * every sequence to reach max_ctx). Prefill (and fill_kv) give each sequence the pages of
   * its prompt; decoding takes one more page from the pool when a sequence first writes a
   * position in it. A sequence that finds the pool spent stops there (PULSAR_BUF_KV_PAGES
   * reports it); a prompt set that does not fit fails prefill with an error. No reference
   * counterpart: the reference grows each global layer's cache tensor by concatenation
   * (src/infer.py:139-150). */
  int32_t kv_pages;
} PulsarEngineConfig;

/* Buffers readable with pulsar_engine_read. */
#define PULSAR_BUF_TOKENS 0    /* int32 [B][max_new] emitted ids */
#define PULSAR_BUF_SEQSTATE 1  /* int32 [B][32] controller state: [0]=done [1]=produced
                                  [4]=position of the current token or block
                                  [11]=tests [12]=accepted */
#define PULSAR_BUF_LOGITS 2    /* fp32 [n_lrows][V] logits of the last step */
#define PULSAR_BUF_ROWS 3      /* int32 [n_rows][8] rows of the next step
                                  (seq, slot, pulse, pos, token, lrow, extra, state slot):
                                  slot = c/s token or block row, state slot = the token
                                  state the row reads and writes (draft-block mode: rotates
                                  per round) */
#define PULSAR_BUF_CTL 4       /* int32 [16] n_rows, n_lrows, pulse_start[4],
                                  pulse_count[4], active, step, n_units */
#define PULSAR_BUF_LAST_ROWS 5 /* int32 [n_rows][8] rows of the last executed step */
#define PULSAR_BUF_LAST_CTL 6  /* int32 [16] control block of the last executed step */
#define PULSAR_BUF_EXPERT_COUNTS 7 /* int32 [n_layers][E] rows routed to each expert, last step */
#define PULSAR_BUF_EXIT_COUNTS 8   /* int32 [B][4] tokens that left after pulse k (early exit),
                                      since the last prefill or rewind */
#define PULSAR_BUF_TOPK_IDX 9      /* int32 [n_layers][max_rows][top_k] router top-k expert ids
                                      of each row of the last executed step, in that step's row
                                      order (PULSAR_BUF_LAST_ROWS), in the router's ranking
                                      order */
#define PULSAR_BUF_KV_LAYOUT 11    /* int32 [4] cache layout: ring positions of a sliding-
                                      window layer (lcap), page-table entries per sequence
                                      of a global layer, positions per page, kv heads (host copy, no
                                      device access) */
#define PULSAR_BUF_KV_PAGES 12     /* int32 [3] global KV pages: pool size, pages handed out
                                      (at most the pool size), 1 if a request found the pool
                                      spent since the last prefill, fill_kv or rewind */
#define PULSAR_BUF_TOKEN_KINDS 10  /* int32 [B][max_new] per emitted token: 1 = an accepted
                                      draft, 0 = a drawn token */

/* Kernel classes of the per-class timing (pulsar_engine_profile_read). */
#define PULSAR_PROF_CLASSES 17
/* 0 pulse input, 1 rmsnorm, 2 qkv+gate GEMM, 3 qk-norm/rope/KV write, 4 attention,
 * 5 wo GEMM, 6 router, 7 shared gate/up, 8 routed gate/up, 9 shared down, 10 routed down,
 * 11 MoE combine, 12 pulse output, 13 lm_head, 14 sampling, 15 controller,
 * 16 an empty event pair (the timing overhead included in every other class's span) */

int pulsar_engine_create(const PulsarModelDesc* model, const PulsarEngineConfig* cfg,
                         void** handle);
int pulsar_engine_destroy(void* handle);
/* Prefill B prompts of T tokens (host ids, row-major [B][T]), fill the KV cache, draw the
 * first token of every sequence. Synchronises the stream at the end. */
int pulsar_engine_prefill(void* handle, const int32_t* host_ids, int32_t B, int32_t T,
                          hipStream_t stream);
/* Run n pulse steps. use_graph=1 replays a captured HIP graph of one step. */
int pulsar_engine_step(void* handle, int32_t n_steps, int32_t use_graph, hipStream_t stream);
/* Steps until every sequence is done (or max_steps), checking every `check_every` steps. */
int pulsar_engine_generate(void* handle, int32_t max_steps, int32_t check_every,
                           hipStream_t stream, int32_t* steps_run);
/* Block verify: n tokens per sequence (host ids [B][n]) at positions P0 .. P0 + n - 1, where
 * P0 is the prefilled prompt length (or fill_kv's ctx), run through every pulse: pulse k is
 * one pass over the B*n rows, a row attending the cache and the block's pulse-k keys at
 * positions <= its own. The last pass's logits (row b*n + i) are readable as
 * PULSAR_BUF_LOGITS. n <= draft_len + 1 (<= 2 in exact mode). The decode state is not
 * touched; the block positions' keys/values are overwritten. host_tokens == NULL re-runs
 * the last uploaded block without a host synchronisation (timing); otherwise the upload
 * synchronises the stream; an upload whose positions need more global-layer KV pages
 * than the pool has left fails with PULSAR_ERR_INVALID before any launch. use_graph=1
 * replays a captured HIP graph of the passes.
 * No reference counterpart: it is the verify step of the draft-block mode, and of the
 * verify microbenchmark (a 5-token verify over pre-filled caches). */
int pulsar_engine_verify(void* handle, const int32_t* host_tokens, int32_t n, int32_t use_graph,
                         hipStream_t stream);
/* Synthetic cache: every key and value element of every layer ~ N(0,1) (counter-based
 * generator keyed by seed), positions [0, ctx) then count as cached context for
 * pulsar_engine_verify. Decoding afterwards needs a prefill. Synchronises the stream. */
int pulsar_engine_fill_kv(void* handle, int32_t ctx, uint64_t seed, hipStream_t stream);
/* Restart decoding from the prefilled cache with a new sampling seed: the first token is
 * drawn again from the saved prefill logits. Synchronises the stream. */
int pulsar_engine_rewind(void* handle, uint64_t seed, hipStream_t stream);
/* Enable (1) or disable (0) per-class event timing; steps then run eagerly (no graph) with
 * a HIP event pair around every kernel group, preceded by a short fixed-length sleep
 * kernel so that the pair brackets the kernels rather than host launch latency.
 * Enabling resets the counters. */
int pulsar_engine_profile(void* handle, int32_t enable);
/* Accumulated milliseconds and launch counts per class, [PULSAR_PROF_CLASSES] each. */
int pulsar_engine_profile_read(void* handle, double* host_ms, int64_t* host_launches);
/* Copy an engine buffer to host memory (synchronises the stream). */
int pulsar_engine_read(void* handle, int32_t what, void* host_dst, int64_t bytes,
                       hipStream_t stream);

/* The engine's sampler on caller buffers. No counterpart in the reference's C surface: it
 * is the device form of the reference's _sample (src/infer.py:658-685) for hosts that hold
 * their own logits, and lets tests check the sampling rule kernel against the oracle.
 *   logits [n_rows][V] fp32; seen [n_seq][V/32] bitmaps of the tokens each sequence has
 *   seen; row_seq [n_rows] its sequence; row_extra [n_rows] one more token counted as seen
 *   (-1: none); seq_ctr [n_seq] the per-sequence draw counters. dtype (PULSAR_BF16 or
 *   PULSAR_F32) is the activation dtype whose rounding the penalty and temperature follow.
 *   Outputs: out_argmax [n_rows] (penalised argmax, lowest index on ties) and out_draw
 *   [n_rows][2] (two independent draws from the top-p set; equal to the argmax when
 *   greedy). workspace: pulsar_sample_workspace_bytes(n_seq) bytes of device memory,
 *   256-byte aligned. V must be a multiple of 4096 with V / 1024 a power of two <= 64. */
int64_t pulsar_sample_workspace_bytes(int32_t n_seq);
int pulsar_sample_rows(const float* logits, int32_t n_rows, int32_t V, int32_t dtype,
                       const uint32_t* seen, const int32_t* row_seq, const int32_t* row_extra,
                       const uint32_t* seq_ctr, int32_t n_seq, uint64_t seed, float temperature,
                       float top_p, float repetition_penalty, int32_t greedy, int32_t* out_argmax,
                       int32_t* out_draw, void* workspace, hipStream_t stream);

/* pulsar_sample_rows without a workspace argument: the same sampling on caller buffers,
 * with its workspace in a static device array of the library instead (one per GPU, 525 KB,
 * held until the process ends). No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops, harnesses
 * that forbid allocation). It allocates nothing; n_seq <= 4096 (larger requests fail with
 * PULSAR_ERR_INVALID). Calls that overlap on one GPU share the array and race. */
int pulsar_sample_rows_static(const float* logits, int32_t n_rows, int32_t V, int32_t dtype,
                              const uint32_t* seen, const int32_t* row_seq,
                              const int32_t* row_extra, const uint32_t* seq_ctr, int32_t n_seq,
                              uint64_t seed, float temperature, float top_p,
                              float repetition_penalty, int32_t greedy, int32_t* out_argmax,
                              int32_t* out_draw, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PULSAR_HIP_H_ */
