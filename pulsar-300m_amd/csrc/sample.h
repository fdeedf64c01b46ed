// Sampling and controller argument blocks (sample.hip).
#pragma once

#include "engine.h"

namespace pulsar {

constexpr int KIND_TESTED = 0;  // token drawn at the top of the reference loop (gets a draft test)
constexpr int KIND_PLAIN = 1;   // accepted draft (its successor is a plain draw)

constexpr int kMaxExtra = kMaxBlock;  // extra seen tokens per logits row (draft-block mode)

// Draft-block rounds are pipelined (the next round's first pulse-0 row rides in the last
// verify step, one slot past the block) when a block plus that row fits a unit.
__host__ __device__ constexpr bool block_pipelined(int draft_len) {
  return draft_len + 2 <= kMaxBlock;
}
// Token-state slots (rows of one sequence in a step) of an engine.
__host__ __device__ constexpr int engine_slots(int draft_len) {
  return draft_len <= 0 ? 2 : (block_pipelined(draft_len) ? draft_len + 2 : draft_len + 1);
}

// Per-sequence decode state, owned by the controller.
struct SeqState {
  int32_t done, produced, max_new;
  int32_t c_tok, c_pos, c_pulse, c_kind, c_slot;
  int32_t s_valid, s_tok, d_tok;
  int32_t tests, accepted;
  int32_t row_c, row_s, lrow_c, lrow_s;
  uint32_t ctr;
  int32_t tail;  // plain mode with early exit: the last emitted token runs for its exit count
  int32_t blk_base;  // draft-block mode: token-state slot of block row 0 (rotates per round)
  // draft-block mode: block tokens (blk[0] = the round's emitted token at position c_pos),
  // tokens known, phase (0 draft, 1 verify), step within the phase (draft index or verify
  // pulse), drafts wanted this round
  int32_t blk_n, blk_phase, blk_step, blk_g;
  int32_t blk[kMaxBlock];
};

struct SampleArgs {
  const StepCtl* ctl;
  const float* logits;  // [lrows][V]
  const int32_t* lrow_seq;
  const int32_t* lrow_extra;  // [lrows][extra_stride], first n_extra entries read (-1: none)
  int extra_stride, n_extra;
  const uint32_t* lrow_ctr;   // per logits row draw counter (nullable: state ctr scheme)
  const uint32_t* seen;  // [B][V/32]
  const SeqState* state;
  int V, greedy;
  float temperature, top_p, rep_penalty;
  const uint64_t* seed;  // device word, so a captured graph follows re-seeding
  int32_t* out_argmax;  // [lrows]
  int32_t* out_draw;    // [lrows][2]
  int n_seq;            // > 0: rows naming a sequence outside [0, n_seq) output -1
  float* out_maxprob;   // nullable: [lrows] top-1 probability of softmax(raw logits), rounded
                        // to the activation dtype (the early-exit test)
};

struct ControllerArgs {
  StepCtl* ctl;
  StepCtl* last_ctl;    // snapshot of the control block of the step that ran
  RowDesc* last_rows;   // snapshot of its rows
  SeqState* state;
  RowDesc* rows;
  AttnUnit* units;      // decode attention units of the next step
  int32_t* lrow_seq;
  int32_t* lrow_extra;  // [lrows][kMaxExtra] in draft-block mode, [lrows] otherwise
  uint32_t* lrow_ctr;   // draft-block mode: per logits row draw counter
  uint32_t* seen;
  int32_t* out_tokens;  // [B][max_new]
  int32_t* out_kinds;   // nullable: [B][max_new] 1 = accepted draft, 0 = drawn token
  const int32_t* argmax;
  const int32_t* draw;
  const int32_t* stop_ids;
  int n_stop, B, V, n_pulses, max_new, speculative, all_logits, init, prompt_len;
  int draft_len;        // > 0: draft-block mode with up to draft_len drafts per round
  // adaptive early exit (exact schedule): per logits row top-1 probability, per-sequence
  // exit counts [B][4], threshold
  int early_exit;
  const float* maxprob;
  int32_t* exit_counts;
  double exit_thr;
  // global-layer KV pages: page table [B][max_pages], pages per sequence [B], pool counter
  // and spent flag [2], pool size (nullable table: no page allocation)
  int32_t* page_table;
  int32_t* page_count;
  int32_t* pool;
  int pool_pages, max_pages;
  int max_lrows;  // logits rows of the largest step (sizes the LDS copy of argmax / draw)
};

int launch_sample(const SampleArgs& a, int dtype, int max_lrows, hipStream_t s);
// Standalone sampling of n_rows logits rows (the engine's kernel on caller buffers).
size_t sample_workspace_bytes(int n_seq);
int launch_sample_rows(const float* logits, int n_rows, int V, int dtype, const uint32_t* seen,
                       const int32_t* row_seq, const int32_t* row_extra, const uint32_t* seq_ctr,
                       int n_seq, uint64_t seed, float temperature, float top_p, float rep_penalty,
                       int greedy, int32_t* out_argmax, int32_t* out_draw, void* workspace,
                       hipStream_t s);
int launch_controller(const ControllerArgs& a, hipStream_t s);

}  // namespace pulsar
