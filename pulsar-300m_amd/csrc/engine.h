// Internal interfaces of the decode/prefill engine (not part of the C ABI).
#pragma once

#include "common.h"

namespace pulsar {

constexpr int kMaxLayers = 16;
constexpr int kMaxPulses = 3;
constexpr int kHeadDim = 64;
constexpr int kPage = 64;  // positions per KV page

// Take n consecutive pages from a KV page pool (pool[0]: pages handed out, pool[1]: spent
// flag, pool_pages: pool size). Returns the first page, or -1 after setting the spent flag
// when fewer than n are left. The counter only moves on success, so a request the pool
// cannot serve leaves its pages to smaller requests; each failed compare-and-swap means
// another request took pages, so the loop ends after at most one pass per competitor.
__device__ __forceinline__ int take_pages(int32_t* pool, int n, int pool_pages) {
  int cur = __hip_atomic_load(&pool[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (cur + n <= pool_pages) {
    const int prev = atomicCAS(&pool[0], cur, cur + n);
    if (prev == cur) return cur;
    cur = prev;
  }
  atomicOr(&pool[1], 1);
  return -1;
}

// One (token, pulse) evaluation inside a step. Rows of a step are sorted by pulse.
struct RowDesc {
  int32_t seq;    // sequence index
  int32_t slot;   // the row's slot: c/s token (0 or 1, exact mode), block row (draft-block)
  int32_t pulse;  // 0..n_pulses-1
  int32_t pos;    // absolute position of the token
  int32_t token;  // token id
  int32_t lrow;   // logits row, or -1 when this pass needs no logits
  int32_t extra_seen;  // token counted as seen when sampling this row (-1 = none)
  int32_t sslot;  // token-state slot the pulse kernels read and write (seq * slots + sslot)
};

// Step control block, written by the controller (or the host for prefill).
struct StepCtl {
  int32_t n_rows;
  int32_t n_lrows;
  int32_t pulse_start[4];
  int32_t pulse_count[4];
  int32_t active;      // sequences not finished
  int32_t step;        // step counter
  int32_t n_units;     // decode attention units (sequences with rows in the step)
  int32_t pad[3];
};

constexpr int kMaxBlock = 8;  // rows of one sequence in a step (draft block + 1)

// Decode attention work unit: the rows of one sequence in a step that read the same cache,
// at consecutive positions pos0, pos0 + 1, ... (exact mode: the current token and, when
// present, the speculative token one position later; draft-block mode: the block's rows).
struct AttnUnit {
  int32_t seq;
  int32_t n;     // rows (1..kMaxBlock)
  int32_t pos0;  // position of row[0]; row[i] sits at pos0 + i
  int32_t pad;
  int32_t row[kMaxBlock];
};

// GEMM epilogues.
enum Epi : int {
  EPI_STORE = 0,      // C[r][n] = T(acc)
  EPI_QKVG = 1,       // columns < n_main: store; tail columns: sigmoid gate with bias
  EPI_RESID = 2,      // C[r][n] = T(C[r][n] + T(acc))
  EPI_SWIGLU = 3,     // act = T(silu(T(acc_gate)) * T(acc_up))
  EPI_LOGITS = 4,     // softcapped logits, fp32 store of T-rounded values
  EPI_LOGITS_RAW = 5, // T-rounded logits without softcap (prefill)
  EPI_SCALE = 6,      // C = T(T(acc) * scale[n])  (prefill routed down with routed_scale)
};

// Row-set modes of a GEMM launch.
enum RowMode : int {
  ROWS_PULSE = 0,   // group g = pulse: rows [pulse_start[g], +pulse_count[g]) of the step
  ROWS_LIST = 1,    // group g: rows list[g][0..count[g]) ; A row = a_map(entry), C row = entry
  ROWS_ALL = 2,     // single group: rows [0, n) with n from ctl->n_rows or m_fixed
  ROWS_LOGITS = 3,  // logits rows i < ctl->n_lrows (A row = C row = i)
};

struct GemmArgs {
  const void* A;           // activations, row stride lda (elements)
  int64_t lda;
  const void* W;           // weights [groups][N][K] row-major
  int64_t w_group_stride;  // elements between groups (0 = shared weight)
  int64_t ldw;
  void* C;                 // output rows, stride ldc
  int64_t ldc;
  int K;
  int N;                   // output columns (for SWIGLU: act columns; weights hold 2N rows)
  int n_main;              // EPI_QKVG: number of non-gate columns
  int row_mode;
  int group_offset;        // first group index covered by grid.y == 0
  int m_fixed;             // ROWS_ALL with ctl == nullptr
  const StepCtl* ctl;
  const int32_t* list;        // ROWS_LIST: [groups][list_stride]
  const int32_t* list_count;  // ROWS_LIST: [groups]
  int64_t list_stride;
  int a_div;               // ROWS_LIST: A row = entry / a_div (1 = same as entry)
  // epilogue operands
  void* C2;                // EPI_QKVG: gate output [rows][n_gate]
  int64_t ldc2;
  const void* bias;        // EPI_QKVG: [groups][n_gate] T ; EPI_SCALE: [N] T
  int64_t bias_group_stride;
  float softcap;
  int c_row_offset;        // added to C row index (prefill chunking)
  // Optional extra group 0 computed over all rows with its own operands (the shared expert
  // fused into the routed-expert launch); list groups then start at grid.y == 1.
  int has_g0;
  int K0;                  // K of group 0 (K or 2K)
  const void* A0;
  int64_t lda0;
  const void* W0;
  int64_t ldw0;
  void* C0;
  int64_t ldc0;
  int N0;
  // ROWS_LIST, bf16 SwiGLU with K0 == K: stream every group's weights and first rows
  // without waiting for its row count (for launches where nearly every group has rows; an
  // empty group's weights are then read for nothing)
  int eager_w;
  int a_rows, a_rows0;  // rows of A and A0 (eager_w clamps speculative row indices into them)
  int grid_x, grid_y, grid_z;  // decode bf16 launches: (column block, group, row tile) extents
  int g0_split;  // decode bf16 launches with group 0: grid.y rows of group 0 (its row tiles
                 // spread over g0_split x grid_z workgroups per column block)
};

int launch_gemm(const GemmArgs& a, int dtype, int epi, int groups, int max_rows,
                hipStream_t s);
// Same contract, for row sets of hundreds to tens of thousands of rows (prefill): bf16
// launches without a fused all-rows group use 128 x 256 output tiles; others fall back to
// launch_gemm. The two kernels sum K in different orders, so a caller that wants results
// independent of batch composition picks one by a per-sequence property (prompt length).
int launch_gemm_wide(const GemmArgs& a, int dtype, int epi, int groups, int max_rows,
                     hipStream_t s);
// Same contract and identical results as launch_gemm (the same summation order), for row
// sets of tens to hundreds of rows per group: 64-row tiles of 64 (rows of a pulse, all
// rows) or 128 (expert lists) weight columns staged through LDS, so that weights are read
// once per 64 rows. bf16 with the store, qkv + gate, residual and SwiGLU epilogues; other
// launches go to launch_gemm.
int launch_gemm_mid(const GemmArgs& a, int dtype, int epi, int groups, int max_rows,
                    hipStream_t s);

}  // namespace pulsar
