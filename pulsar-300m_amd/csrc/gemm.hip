// Row-set GEMMs for decode and prefill: C[rows, N] = epi(A[rows, K] . W[N, K]^T), bf16
// weights stored in matrix-core tile order [N/16][K/32][64 lanes][8].
//
// Decode (gemm_bf16_kernel): a workgroup of 8 waves owns 16 output columns and walks the
// group's 32-row tiles; the waves split K, each runs v_mfma_f32_16x16x32_bf16 on two
// 16-row blocks that share the weight operand, so every weight byte is read once per
// launch. Partial tiles are summed through LDS (one tile value per wave) before the fused
// epilogue. Row sets come from the step control block (rows of one pulse, rows of one
// expert, all rows, or logits rows), so one launch serves every pulse / expert group and
// groups without rows exit before touching their weights.
//
// Prefill (gemm_bf16_lds_kernel): 128 x 256 output tiles staged through LDS for row sets
// of thousands of rows, where the work is matrix-core bound rather than weight-bound.
//
// fp32: one wave per output column, lanes split K with 128-bit loads, wave64 reduction.
#include <algorithm>

#include "engine.h"

namespace pulsar {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

namespace {

__device__ __forceinline__ bf16x8_t load_bf16x8(const bf16* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}
// Non-temporal (streaming) load: for weights a launch reads once, so that they do not push
// out of the caches what later kernels read again (attention keys/values, activations).
__device__ __forceinline__ bf16x8_t load_bf16x8_nt(const bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(p));
}

// Resolve the (A row, C row) pairs of this workgroup's 32-row tile into LDS.
// Returns the number of valid rows (0 => nothing to do).
__device__ int resolve_rows(const GemmArgs& g, int group, int tile, int* a_row, int* c_row) {
  __shared__ int s_n;
  const int mode = (g.has_g0 && group < 0) ? ROWS_ALL : g.row_mode;
  if (threadIdx.x == 0) {
    int n = 0;
    switch (mode) {
      case ROWS_PULSE: {
        const int cnt = g.ctl->pulse_count[group];
        n = cnt - tile * 32;
        break;
      }
      case ROWS_LIST:
        n = g.list_count[group] - tile * 32;
        break;
      case ROWS_ALL: {
        const int tot = g.ctl ? g.ctl->n_rows : g.m_fixed;
        n = tot - tile * 32;
        break;
      }
      case ROWS_LOGITS:
        n = g.ctl->n_lrows - tile * 32;
        break;
    }
    s_n = n < 0 ? 0 : (n > 32 ? 32 : n);
  }
  __syncthreads();
  const int n = s_n;
  if (threadIdx.x < 32) {
    const int m = threadIdx.x;
    int ar = -1, cr = -1;
    if (m < n) {
      const int i = tile * 32 + m;
      switch (mode) {
        case ROWS_PULSE:
          ar = cr = g.ctl->pulse_start[group] + i;
          break;
        case ROWS_LIST: {
          const int e = g.list[(int64_t)group * g.list_stride + i];
          ar = e / g.a_div;
          cr = e;
          break;
        }
        case ROWS_ALL:
          ar = cr = i;
          break;
        case ROWS_LOGITS:
          ar = cr = i;
          break;
      }
    }
    a_row[m] = ar;
    c_row[m] = cr < 0 ? -1 : cr + g.c_row_offset;
  }
  __syncthreads();
  return n;
}

template <typename T>
__device__ __forceinline__ void epilogue(const GemmArgs& g, int epi, int group, void* Cv,
                                         int64_t ldc, int crow, int col, float acc, float acc_up) {
  T* C = reinterpret_cast<T*>(Cv);
  switch (epi) {
    case EPI_STORE:
      C[(int64_t)crow * ldc + col] = from_f<T>(acc);
      break;
    case EPI_QKVG:
      if (col < g.n_main) {
        C[(int64_t)crow * ldc + col] = from_f<T>(acc);
      } else {
        const int h = col - g.n_main;
        const T* b = reinterpret_cast<const T*>(g.bias) + (int64_t)group * g.bias_group_stride;
        const float v = rnd<T>(acc + to_f(b[h]));
        reinterpret_cast<T*>(g.C2)[(int64_t)crow * g.ldc2 + h] = from_f<T>(sigmoidf_(v));
      }
      break;
    case EPI_RESID: {
      T* p = C + (int64_t)crow * ldc + col;
      *p = from_f<T>(to_f(*p) + rnd<T>(acc));
      break;
    }
    case EPI_SWIGLU: {
      const float gt = rnd<T>(acc), up = rnd<T>(acc_up);
      C[(int64_t)crow * ldc + col] = from_f<T>(gt * sigmoidf_(gt) * up);
      break;
    }
    case EPI_LOGITS: {
      float l = rnd<T>(acc);
      if (g.softcap > 0.f) {
        float t = rnd<T>(l / g.softcap);
        t = rnd<T>(tanhf(t));
        l = rnd<T>(g.softcap * t);
      }
      reinterpret_cast<float*>(Cv)[(int64_t)crow * ldc + col] = l;
      break;
    }
    case EPI_LOGITS_RAW:
      reinterpret_cast<float*>(Cv)[(int64_t)crow * ldc + col] = rnd<T>(acc);
      break;
    case EPI_SCALE: {
      const T* s = reinterpret_cast<const T*>(g.bias);
      C[(int64_t)crow * ldc + col] = from_f<T>(rnd<T>(acc) * to_f(s[col]));
      break;
    }
  }
}

// Entry i of the group: the row index (pulse / all / logits modes) or the assignment id
// (list mode; the all-rows group -1 of a fused launch takes row i). Branch-free in the row
// mode, which is a template parameter: a load pending on one path of a runtime switch
// would make the join wait for every load in flight, weights included.
template <int MODE>
__device__ __forceinline__ int entry_load(const GemmArgs& g, int group, int i) {
  if constexpr (MODE == ROWS_PULSE) return g.ctl->pulse_start[group] + i;
  if constexpr (MODE == ROWS_LIST) return g.list[(int64_t)max(group, 0) * g.list_stride + i];
  return i;
}
// Applied after the weight loads are issued (the only use of the loaded value).
template <int MODE>
__device__ __forceinline__ int entry_fix(int group, int i, int v) {
  if constexpr (MODE == ROWS_LIST) return group < 0 ? i : v;
  return v;
}
template <int MODE>
__device__ __forceinline__ int a_row_of(const GemmArgs& g, int group, int raw) {
  if constexpr (MODE == ROWS_LIST) {
    if (group < 0) return raw;
    // a_div is 1 (expert output rows) or the top-k count (token rows). A power of two takes
    // a shift instead of the ~30-instruction integer division; entries are non-negative
    // (only the spare-capacity entries of eager launches may not be, and their rows are
    // clamped, computed and never stored).
    const int d = g.a_div;
    if ((d & (d - 1)) == 0) return raw >> __builtin_ctz((unsigned)d);
    return raw / d;
  }
  return raw;
}
template <int MODE>
__device__ __forceinline__ int group_rows(const GemmArgs& g, int group) {
  if constexpr (MODE == ROWS_PULSE) return g.ctl->pulse_count[group];
  if constexpr (MODE == ROWS_LOGITS) return g.ctl->n_lrows;
  if constexpr (MODE == ROWS_LIST) {
    // the fused all-rows group (-1) exists only in launches with a step control block
    return group >= 0 ? g.list_count[group] : g.ctl->n_rows;
  }
  return g.ctl ? g.ctl->n_rows : g.m_fixed;
}

// Workgroup: 16 output columns of one group; 8 waves split K (few registers per wave, so
// a launch's workgroups are resident at once). The workgroup walks the
// group's 32-row tiles z, z + gridDim.z, ... keeping its weight slice in registers, so a
// launch needs only as many workgroups along z as the largest row set needs for
// parallelism (one for decode batches of up to 32 rows per group). KMUL0 > 1: the
// all-rows group has K0 = KMUL0 * K and runs KMUL0 passes over K-slices (the shared expert
// down projection fused into the routed one).
constexpr int kGemmWaves = 8;
constexpr int kXcds = 8;  // MI355X: consecutive workgroups go to the 8 XCDs in turn

// A launch with several row tiles per group is a 1-D grid over (column block x, group y,
// row tile z), ordered so that the z workgroups of one (x, y) run one after another on the
// same XCD: workgroup L goes to XCD L % 8, and within an XCD the slots enumerate (x, y)
// pairs with z fastest. They then share that XCD's L2 for the weight slice instead of each
// fetching it from HBM. Pairs are padded to a multiple of 8; padding workgroups exit.
// With one row tile (decode batches) the grid is the plain (x, y) grid: no index
// arithmetic ahead of the weight loads.
struct GemmBlock {
  int x, y, z;
  bool valid;
};
template <bool XCD>
__device__ __forceinline__ GemmBlock gemm_block(const GemmArgs& g) {
  if constexpr (!XCD) return GemmBlock{(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z, true};
  const int L = blockIdx.x, slot = L / kXcds;
  const int pair = (slot / g.grid_z) * kXcds + L % kXcds;
  GemmBlock b;
  b.z = slot % g.grid_z;
  b.x = pair % g.grid_x;
  b.y = pair / g.grid_x;
  b.valid = b.y < g.grid_y;
  return b;
}

// s_waitcnt vmcnt(n) for an n that is a constant once the caller's loops are unrolled.
__device__ __forceinline__ void wait_vmcnt_unrolled(int n) {
  switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    default: wait_vmcnt<0>(); break;
  }
}

template <int EPI, int KITER, int MODE, int KMUL0, bool EAGER, bool XCD>
__global__ void __launch_bounds__(64 * kGemmWaves) gemm_bf16_kernel(GemmArgs g) {
  // two weight column tiles share each A operand: SwiGLU's gate and up columns, and the
  // output head's columns c and N + c (the host halves N: the head's A rows are then read
  // once per 32 vocabulary columns, not per 16)
  constexpr bool kPair = (EPI == EPI_SWIGLU || EPI == EPI_LOGITS);
  constexpr int kKPass = KITER * 32 * kGemmWaves;  // K covered by one pass of the waves
  static_assert(!EAGER || MODE == ROWS_LIST, "eager weight loads are for expert lists");
  // One LDS slice per wave: first the wave's A rows of a 16-row block (one 1 KB tile per
  // k tile and pass), then its partial tile values [value][lane] for the K-split sum (the
  // lanes of one value are consecutive words: conflict-free writes and reducing reads;
  // lane-major rows of 16 values put every 4th lane on one bank, 16-way conflicts). A wave
  // only writes its own slice, so the A staging needs no barrier.
  constexpr int kAFrags = KITER * KMUL0;
  constexpr int kRedFloats = (kPair ? 16 : 8) * 64;
  constexpr int kSliceFloats = kAFrags * 256 > kRedFloats ? kAFrags * 256 : kRedFloats;
  __shared__ __attribute__((aligned(16))) float lds_slices[kGemmWaves * kSliceFloats];
  const GemmBlock blk = gemm_block<XCD>(g);
  if (!blk.valid) return;
  // grid.y < g0_split: the optional all-rows group (group -1) when has_g0 is set. Its row
  // tiles go to g0_split x Z workgroups per column block (tile y Z + z, stride g0_split Z),
  // those of a list group to Z (tile z, stride Z): the all-rows group holds about K / E
  // times the rows of a routed expert, and one workgroup walking all of them would be the
  // launch's longest chain of dependent tiles.
  const int s0 = g.has_g0 ? g.g0_split : 0;
  const bool g0 = blk.y < s0;
  const int group = g0 ? -1 : blk.y - s0 + g.group_offset;
  const int N = g0 ? g.N0 : g.N;
  const int col0 = blk.x * 16;
  if (col0 >= N) return;
  const int zs = XCD ? g.grid_z : (int)gridDim.z;
  const int tstep = (g0 ? s0 * zs : zs) * 32;
  int tile0 = (g0 ? blk.y * zs + blk.z : blk.z) * 32;
  int cnt = 0;
  if constexpr (!EAGER) {
    cnt = group_rows<MODE>(g, group);  // uniform per workgroup
    if (tile0 >= cnt) return;
  } else {
    // the all-rows group's later tiles exist for parallelism at large steps: they check
    // the step's row count before streaming weights (the first tile never waits for it)
    if (g0 && tile0 > 0) {
      cnt = group_rows<MODE>(g, group);
      if (tile0 >= cnt) return;
    }
  }

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m = lane & 15, kq = lane >> 4;
  const int64_t lda = g0 ? g.lda0 : g.lda;
  const bf16* W = g0 ? reinterpret_cast<const bf16*>(g.W0)
                     : reinterpret_cast<const bf16*>(g.W) + (int64_t)group * g.w_group_stride;
  // Weights in matrix-core tiles [N/16][K/32][64 lanes][8]: this lane's 16 bytes of tile
  // (column tile, k tile) sit at ((ct * KT + kt) * 64 + lane) * 8, and the wave's load of a
  // tile is 1 KB contiguous. The up-projection rows of SwiGLU are column tiles N/16 on.
  const int KT = (g0 ? g.K0 : g.K) / 32;
  const bool vc = col0 + m < N;  // N is a multiple of 16: always true; kept as a guard
  const bf16* w0 = W + ((int64_t)(col0 / 16) * KT * 64 + lane) * 8;
  const bf16* w1 = W + ((int64_t)((N + col0) / 16) * KT * 64 + lane) * 8;
  const bf16* A = reinterpret_cast<const bf16*>(g0 ? g.A0 : g.A);
  void* Cout = g0 ? g.C0 : g.C;
  const int64_t ldc = g0 ? g.ldc0 : g.ldc;
  const int passes = g0 ? KMUL0 : 1;
  const int kb = wv * (KITER * 32) + kq * 8;
  const bf16x8_t zero = {};
  // every pass's weights stay in registers (the all-rows group of a KMUL0 launch loads its
  // second K half with the first, not one round trip after the first half's products)
  bf16x8_t bw[KITER * KMUL0], bu[KITER], xa[KITER];
  // k tile of step i of this wave in pass p: p * (K / 32 per pass) + wv * KITER + i
#define PULSAR_LOAD_W(pass)                                                              \
  do {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < KITER; ++i) {                                  \
      const int64_t kt = (int64_t)(pass) * (kKPass / 32) + wv * KITER + i;               \
      bw[(pass) * KITER + i] = XCD ? load_bf16x8(w0 + kt * 512) : load_bf16x8_nt(w0 + kt * 512); \
      if constexpr (kPair)                                                               \
        bu[i] = XCD ? load_bf16x8(w1 + kt * 512) : load_bf16x8_nt(w1 + kt * 512);        \
    }                                                                                    \
  } while (0)
#define PULSAR_LOAD_W_REST()                                                             \
  do {                                                                                   \
    if constexpr (KMUL0 > 1) {                                                           \
      if (g0) {                                                                          \
        _Pragma("unroll") for (int p = 1; p < KMUL0; ++p) PULSAR_LOAD_W(p);              \
      }                                                                                  \
    }                                                                                    \
  } while (0)

  // Row entries of the first tile first, then the weights, then (after a scheduling
  // barrier) the A rows: vector loads retire in issue order, so waiting for the few entry
  // loads leaves every weight load in flight. Lanes past the last row re-read the last
  // entry (always in bounds) and use a zero A operand. Each lane loads two entries per
  // block: that of its fragment row m (for the A operand's zero test and the stores) and
  // that of the row sr = lane / 4 whose 16 bytes it stages into LDS.
  const int sr = lane >> 2;
  int n, i0, i1, l0, l1, si0, si1, ls0, ls1;
  if constexpr (EAGER) {
    // Most experts have rows (the host decides from the batch size): the first tile's
    // entries and the weights go out before the row count, whose scalar load retires apart
    // from them, instead of one round trip later. Entries past the count are read from the
    // list's spare capacity; the rows they name are clamped, computed and never stored.
    const int64_t cap = g.list_stride - 1;
    i0 = tile0 + m;
    i1 = tile0 + m + 16;
    const int32_t* lst = g.list + (int64_t)max(group, 0) * g.list_stride;
    si0 = tile0 + sr;
    si1 = tile0 + sr + 16;
    l0 = lst[min((int64_t)i0, cap)];
    l1 = lst[min((int64_t)i1, cap)];
    ls0 = lst[min((int64_t)si0, cap)];
    ls1 = lst[min((int64_t)si1, cap)];
    __builtin_amdgcn_sched_barrier(0);
    PULSAR_LOAD_W(0);
    // no early exit on the count: a branch on it would let the compiler test it before
    // issuing the weight loads. A workgroup without rows runs on clamped rows and stores
    // nothing.
    cnt = group_rows<MODE>(g, group);
    // Use the entries here: the wait for them then leaves the weight loads behind them in
    // flight, and the compiler cannot merge these loads into the next tile's (which would
    // put them behind the weights and the count).
    asm volatile("" ::"v"(l0), "v"(l1), "v"(ls0), "v"(ls1));
    n = max(0, min(32, cnt - tile0));
  } else {
    n = min(32, cnt - tile0);
    i0 = tile0 + min(m, n - 1);
    i1 = tile0 + min(m + 16, n - 1);
    si0 = tile0 + min(sr, n - 1);
    si1 = tile0 + min(sr + 16, n - 1);
    l0 = entry_load<MODE>(g, group, i0);
    l1 = entry_load<MODE>(g, group, i1);
    ls0 = entry_load<MODE>(g, group, si0);
    ls1 = entry_load<MODE>(g, group, si1);
    PULSAR_LOAD_W(0);
    PULSAR_LOAD_W_REST();
  }
  // One row tile (32 rows) of the group. The first tile runs outside the loop: in a
  // loop, the wait for the entries of a later tile (issued last) would also stand at the
  // first tile's A loads and make them wait for the whole weight slice.
  auto run_tile = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    const bool two = n > 16;  // second 16-row block present (uniform per workgroup)
    const int e0 = entry_fix<MODE>(group, i0, l0), e1 = entry_fix<MODE>(group, i1, l1);
    const int es0 = entry_fix<MODE>(group, si0, ls0), es1 = entry_fix<MODE>(group, si1, ls1);
    int ar0, ar1, as0, as1;  // ar: fragment row's A row (-1: zero operand); as: staged row
    if constexpr (EAGER) {
      // every lane of the first row block loads a row (clamped into the A buffer): rows
      // past the count are computed and never stored, so no A load waits on the count
      const int lim = (g0 ? g.a_rows0 : g.a_rows) - 1;
      ar0 = min(max(a_row_of<MODE>(g, group, e0), 0), lim);
      ar1 = m + 16 < n ? min(max(a_row_of<MODE>(g, group, e1), 0), lim) : -1;
      as0 = min(max(a_row_of<MODE>(g, group, es0), 0), lim);
      as1 = min(max(a_row_of<MODE>(g, group, es1), 0), lim);
    } else {
      ar0 = m < n ? a_row_of<MODE>(g, group, e0) : -1;
      ar1 = m + 16 < n ? a_row_of<MODE>(g, group, e1) : -1;
      as0 = a_row_of<MODE>(g, group, es0);  // rows past the count re-read the last row
      as1 = a_row_of<MODE>(g, group, es1);
    }
    // A rows through the wave's LDS slice: tile (pass p, k tile i) holds the block's 16
    // rows x 32 k as (row r, k chunk q) at slot 4 r + (q ^ 2 (r >> 3)); the load's lanes
    // 4 j .. 4 j + 3 fetch row j's 64 contiguous bytes (a register load's 16 lanes touched
    // 16 rows), and the fragment read (lane = row m, chunk kq) is free of bank conflicts.
    // With one pass the fragment reads wait for their own tile only (the A loads retire in
    // issue order, after the weights); a compiler barrier keeps each read behind its wait.
    bf16x8_t* astage = reinterpret_cast<bf16x8_t*>(lds_slices + wv * kSliceFloats);
    const int acl = (lane & 3) ^ ((lane >> 5) << 1);
    const int aslot = m * 4 + (kq ^ ((m >> 3) << 1));
    auto stage_a = [&](int as) {  // as: A row of block row sr
      const bf16* src = A + (int64_t)as * lda + wv * (KITER * 32) + acl * 8;
#pragma unroll
      for (int pass = 0; pass < KMUL0; ++pass) {
        if (pass >= passes) break;
#pragma unroll
        for (int i = 0; i < KITER; ++i)
          load_lds16(src + pass * kKPass + 32 * i, astage + (pass * KITER + i) * 64);
      }
    };
    f32x4_t c00 = {0.f, 0.f, 0.f, 0.f}, c10 = c00, c01 = c00, c11 = c00;
    auto wait_a = [&](int i) {  // before the fragment read of k tile i of the first pass
      if constexpr (KMUL0 == 1) {
        wait_vmcnt_unrolled(KITER - 1 - i);
        asm volatile("" ::: "memory");
      } else if (i == 0) {
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
      }
    };
    stage_a(as0);
#pragma unroll
    for (int pass = 0; pass < KMUL0; ++pass) {
      if (pass >= passes) break;
#pragma unroll
      for (int i = 0; i < KITER; ++i) {
        if (pass == 0) wait_a(i);
        xa[i] = (EAGER || ar0 >= 0) ? astage[(pass * KITER + i) * 64 + aslot] : zero;
      }
#pragma unroll
      for (int i = 0; i < KITER; ++i) {
        c00 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[i], bw[pass * KITER + i], c00, 0, 0, 0);
        if constexpr (kPair) c01 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[i], bu[i], c01, 0, 0, 0);
      }
    }
    if (two) {  // the second 16-row block reuses the slice once the first block's reads are in
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      stage_a(as1);
#pragma unroll
      for (int pass = 0; pass < KMUL0; ++pass) {
        if (pass >= passes) break;
#pragma unroll
        for (int i = 0; i < KITER; ++i) {
          if (pass == 0) wait_a(i);
          xa[i] = ar1 >= 0 ? astage[(pass * KITER + i) * 64 + aslot] : zero;
        }
#pragma unroll
        for (int i = 0; i < KITER; ++i) {
          c10 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[i], bw[pass * KITER + i], c10, 0, 0, 0);
          if constexpr (kPair) c11 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[i], bu[i], c11, 0, 0, 0);
        }
      }
    }
    // the partial values overwrite the slice: its A reads are done
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // Partial tiles to LDS; then wave w reduces and stores tile value w of every lane:
    // row block w / 4, accumulator element w % 4 (with its up-projection twin for SwiGLU).
    float* red_w = lds_slices + wv * kSliceFloats;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      red_w[j * 64 + lane] = c00[j];
      red_w[(4 + j) * 64 + lane] = c10[j];
      if constexpr (kPair) {
        red_w[(8 + j) * 64 + lane] = c01[j];
        red_w[(12 + j) * 64 + lane] = c11[j];
      }
    }
    __syncthreads();
    {
      static_assert(kGemmWaves == 8, "one tile value per wave");
      const int blk = wv >> 2, j = wv & 3;
      float acc = 0.f, accu = 0.f;
#pragma unroll
      for (int w = 0; w < kGemmWaves; ++w) {
        acc += lds_slices[w * kSliceFloats + (blk * 4 + j) * 64 + lane];
        if constexpr (kPair) accu += lds_slices[w * kSliceFloats + (8 + blk * 4 + j) * 64 + lane];
      }
      // D layout of 16x16 MFMA: lane holds rows (lane/16)*4 + j, column lane%16; the C row
      // of tile row r is the entry held by lane r % 16 (rows 0-15: e0, 16-31: e1).
      const int crow = __shfl(blk ? e1 : e0, kq * 4 + j, 64);
      const int row = blk * 16 + kq * 4 + j;
      if (vc && row < n) {
        epilogue<bf16>(g, EPI, group, Cout, ldc, crow + g.c_row_offset, col0 + m, acc, accu);
        if constexpr (EPI == EPI_LOGITS)
          epilogue<bf16>(g, EPI, group, Cout, ldc, crow + g.c_row_offset, N + col0 + m, accu, 0.f);
      }
    }
  };
  run_tile();
  tile0 += tstep;
  while (tile0 < cnt) {
    __syncthreads();  // the partial sums in LDS are consumed before the next tile's writes
    n = min(32, cnt - tile0);
    i0 = tile0 + min(m, n - 1);
    i1 = tile0 + min(m + 16, n - 1);
    si0 = tile0 + min(sr, n - 1);
    si1 = tile0 + min(sr + 16, n - 1);
    l0 = entry_load<MODE>(g, group, i0);
    l1 = entry_load<MODE>(g, group, i1);
    ls0 = entry_load<MODE>(g, group, si0);
    ls1 = entry_load<MODE>(g, group, si1);
    run_tile();
    tile0 += tstep;
  }
#undef PULSAR_LOAD_W
#undef PULSAR_LOAD_W_REST
}

// fp32: 4 waves per workgroup, one output column per wave, 32-row tile.
template <int EPI>
__global__ void __launch_bounds__(256) gemm_f32_kernel(GemmArgs g) {
  constexpr bool kPair = (EPI == EPI_SWIGLU);
  __shared__ int a_row[32], c_row[32];
  const int group = (int)blockIdx.y + g.group_offset - (g.has_g0 ? 1 : 0);
  const bool g0 = group < 0;
  const int N = g0 ? g.N0 : g.N;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col = blockIdx.x * 4 + wv;
  if (blockIdx.x * 4 >= N) return;
  const int n = resolve_rows(g, group, blockIdx.z, a_row, c_row);
  if (n == 0 || col >= N) return;
  const float* A = reinterpret_cast<const float*>(g0 ? g.A0 : g.A);
  const int64_t lda = g0 ? g.lda0 : g.lda, ldw = g0 ? g.ldw0 : g.ldw;
  const float* W = g0 ? reinterpret_cast<const float*>(g.W0)
                      : reinterpret_cast<const float*>(g.W) + (int64_t)group * g.w_group_stride;
  void* Cout = g0 ? g.C0 : g.C;
  const int64_t ldc = g0 ? g.ldc0 : g.ldc;
  const float* w0 = W + (int64_t)col * ldw;
  const float* w1 = W + (int64_t)(N + col) * ldw;
  const int Kg = g0 ? g.K0 : g.K;
  for (int r = 0; r < n; ++r) {
    const float* a = A + (int64_t)a_row[r] * lda;
    float s0 = 0.f, s1 = 0.f;
    for (int k = lane * 4; k < Kg; k += 256) {
      const float4 av = *reinterpret_cast<const float4*>(a + k);
      const float4 bv = *reinterpret_cast<const float4*>(w0 + k);
      s0 += av.x * bv.x + av.y * bv.y + av.z * bv.z + av.w * bv.w;
      if constexpr (kPair) {
        const float4 uv = *reinterpret_cast<const float4*>(w1 + k);
        s1 += av.x * uv.x + av.y * uv.y + av.z * uv.z + av.w * uv.w;
      }
    }
    s0 = wave_sum(s0);
    if constexpr (kPair) s1 = wave_sum(s1);
    if (lane == (r & 63)) epilogue<float>(g, EPI, group, Cout, ldc, c_row[r], col, s0, s1);
  }
}

// Four consecutive output columns of one row (col0 % 4 == 0, never straddling n_main).
__device__ __forceinline__ void epilogue4(const GemmArgs& g, int epi, int group, void* Cv,
                                          int64_t ldc, int crow, int col0, const float* v,
                                          const float* u) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16* C = reinterpret_cast<bf16*>(Cv);
  bf16x4_t o;
  switch (epi) {
    case EPI_STORE:
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (__bf16)v[j];
      break;
    case EPI_RESID: {
      const bf16x4_t h = *reinterpret_cast<const bf16x4_t*>(C + (int64_t)crow * ldc + col0);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (__bf16)((float)h[j] + rnd<bf16>(v[j]));
      break;
    }
    case EPI_SWIGLU:
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float gt = rnd<bf16>(v[j]), up = rnd<bf16>(u[j]);
        o[j] = (__bf16)(gt * sigmoidf_(gt) * up);
      }
      break;
    case EPI_SCALE: {
      const bf16x4_t sc = *reinterpret_cast<const bf16x4_t*>(reinterpret_cast<const bf16*>(g.bias) + col0);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (__bf16)(rnd<bf16>(v[j]) * (float)sc[j]);
      break;
    }
    case EPI_LOGITS:
    case EPI_LOGITS_RAW: {
      // fp32 store of bf16-rounded logits, softcapped with the scalar epilogue's roundings
      float4 lv;
      float* lp = &lv.x;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float l = rnd<bf16>(v[j]);
        if (epi == EPI_LOGITS && g.softcap > 0.f) {
          float t = rnd<bf16>(l / g.softcap);
          t = rnd<bf16>(tanhf(t));
          l = rnd<bf16>(g.softcap * t);
        }
        lp[j] = l;
      }
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(Cv) + (int64_t)crow * ldc + col0) = lv;
      return;
    }
    default:  // EPI_QKVG: q/k/v columns stored, gate columns through the scalar epilogue
      if (col0 >= g.n_main) {
#pragma unroll
        for (int j = 0; j < 4; ++j) epilogue<bf16>(g, epi, group, Cv, ldc, crow, col0 + j, v[j], 0.f);
        return;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (__bf16)v[j];
      break;
  }
  *reinterpret_cast<bf16x4_t*>(C + (int64_t)crow * ldc + col0) = o;
}

// LDS-staged tiles for wide row sets: a workgroup of 4 waves owns 128 rows x 256 output
// columns (SwiGLU: 128 gate columns and their 128 up-projection twins); wave (wr, wc)
// computes 64 rows x 128 columns as 4 x 8 MFMA tiles (128 accumulators). Per 32-wide k
// step the workgroup stages the A tile (8 row tiles of 16 rows, gathered rows in MFMA lane
// order) and 16 weight tiles (1 KB each, stored in lane order) in LDS with direct
// global-to-LDS loads (16 bytes per lane, no staging registers): a wave's load instruction
// fills one 1 KB tile, lane l at +16 l, which is the lane's own MFMA operand. A ring of
// kWideStages buffers keeps kWideStages - 1 k steps in flight while one is computed; one
// barrier per step both publishes the step's tiles to all waves and frees the buffer the
// next load overwrites. Each staged byte feeds 2 waves from LDS, and each wave's 12
// fragment reads feed 32 products. The weights go in as the A operand and the rows as B,
// so a lane ends with 4 consecutive output columns of its own row: 8-byte epilogue loads
// and stores, and the C row is an entry the lane loads itself.
constexpr int kTileRows = 128;
constexpr int kWideStages = 3;

// Row-set launches of the wide kernel are 1-D grids. The tiles that hold rows, in the order
// (group, row tile, column block) with column blocks fastest, are cut into 8 equal
// contiguous ranges, one per XCD (workgroup L runs on XCD L % 8, as slot L / 8 of its
// range). The column blocks of a row tile then follow one another on one XCD, which
// fetches the tile's rows into its L2 once for all of them, and a group's weights are read
// by the one or two XCDs whose ranges hold its tiles. Row counts are read on the device, so
// every XCD gets an equal share of the tiles that exist; workgroups past the end exit.
template <int MODE>
__device__ __forceinline__ bool wide_tile(const GemmArgs& g, int& bx, int& group, int& bz) {
  const int L = (int)blockIdx.x, xcd = L % kXcds, slot = L / kXcds;
  const int lane = (int)threadIdx.x & 63;
  // row tiles of each group, 64 groups per pass (one per lane)
  int total = 0;
  for (int y0 = 0; y0 < g.grid_y; y0 += 64) {
    const int y = y0 + lane;
    const int nt = y < g.grid_y
        ? min((group_rows<MODE>(g, y + g.group_offset) + kTileRows - 1) / kTileRows, g.grid_z)
        : 0;
    for (int j = 0; j < 64 && y0 + j < g.grid_y; ++j) total += __builtin_amdgcn_readlane(nt, j);
  }
  total *= g.grid_x;
  const int per = (total + kXcds - 1) / kXcds;
  int item = xcd * per + slot;
  if (slot >= per || item >= total) return false;
  bx = item % g.grid_x;
  int t = item / g.grid_x;
  for (int y0 = 0; y0 < g.grid_y; y0 += 64) {
    const int y = y0 + lane;
    const int nt = y < g.grid_y
        ? min((group_rows<MODE>(g, y + g.group_offset) + kTileRows - 1) / kTileRows, g.grid_z)
        : 0;
    for (int j = 0; j < 64 && y0 + j < g.grid_y; ++j) {
      const int ntj = __builtin_amdgcn_readlane(nt, j);
      if (t < ntj) {
        group = y0 + j + g.group_offset;
        bz = t;
        return true;
      }
      t -= ntj;
    }
  }
  return false;
}

template <int EPI, int MODE>
__global__ void __launch_bounds__(256, 2) gemm_bf16_lds_kernel(GemmArgs g) {
  constexpr bool kPair = (EPI == EPI_SWIGLU);
  constexpr int S = kWideStages;
  __shared__ bf16x8_t sA[S][8][64];   // [buffer][row tile][lane]
  __shared__ bf16x8_t sW[S][16][64];  // [buffer][column tile][lane]
  int bx = (int)blockIdx.x, group = (int)blockIdx.y + g.group_offset, bz = (int)blockIdx.z;
  if constexpr (MODE != ROWS_LOGITS) {
    if (!wide_tile<MODE>(g, bx, group, bz)) return;
  }
  const int N = g.N;
  const int KT = g.K / 32;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wr = wv >> 1, wc = wv & 1;
  const int m16 = lane & 15, kq = lane >> 4;
  const int cnt = group_rows<MODE>(g, group);
  if constexpr (MODE == ROWS_LOGITS) {
    // output head (one group): workgroup L runs on XCD L % 8; give each XCD a contiguous
    // range of column tiles with their row tiles one after another, so the row tiles of a
    // column tile read its weights through one L2
    const int nz = (int)gridDim.z, total = (int)gridDim.x * nz;
    if (nz > 1 && total % 8 == 0) {
      const int L = bx + (int)gridDim.x * bz;
      const int w = (L & 7) * (total >> 3) + (L >> 3);
      bx = w / nz;
      bz = w % nz;
    }
  }
  const int r_wg = bz * kTileRows;
  if (r_wg >= cnt) return;
  const int ct_wg = bx * (kPair ? 8 : 16);  // first (gate) column tile
  if (ct_wg * 16 >= N) return;
  const bf16* A = reinterpret_cast<const bf16*>(g.A);
  const bf16* W = reinterpret_cast<const bf16*>(g.W) + (int64_t)group * g.w_group_stride;

  // staging: wave wv fills row tiles wv + 4 h (h < 2) and weight tiles wv + 4 h (h < 4).
  // A row tile's 64 16-byte chunks sit in LDS as (row m, k chunk q) at slot
  // 4 m + (q ^ (m >> 2 & 3)): the load's lane l carries row 16 t + (l >> 2), so 16 lanes
  // fetch the 64 contiguous bytes of 4 rows, and the XOR puts the 16 rows of one k chunk
  // that a fragment read takes on 16 different 16-byte bank groups
  const bf16* ga[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = (wv + 4 * h) * 16 + (lane >> 2);
    const int i = min(r_wg + r, cnt - 1);
    const int e = entry_load<MODE>(g, group, i);
    ga[h] = A + (int64_t)a_row_of<MODE>(g, group, e) * g.lda + ((lane & 3) ^ (lane >> 4 & 3)) * 8;
  }
  const int aslot = m16 * 4 + (kq ^ (m16 >> 2 & 3));  // this lane's fragment chunk
  const bf16* gw[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int c = wv + 4 * h;
    int ct;
    if constexpr (kPair)
      ct = c < 8 ? ct_wg + c : N / 16 + ct_wg + (c - 8);
    else
      ct = min(ct_wg + c, N / 16 - 1);  // tiles past N re-read the last one (never stored)
    gw[h] = W + ((int64_t)ct * KT * 64 + lane) * 8;
  }
  // k step kt into ring buffer b: 6 loads per wave, counted by vmcnt
  auto fetch = [&](int kt, int b) {
#pragma unroll
    for (int h = 0; h < 4; ++h) load_lds16(gw[h] + (int64_t)kt * 512, &sW[b][wv + 4 * h][0]);
#pragma unroll
    for (int h = 0; h < 2; ++h) load_lds16(ga[h] + kt * 32, &sA[b][wv + 4 * h][0]);
  };
  // this wave's column tiles in the staged set: 8 of 16 (SwiGLU: 4 gate + their 4 up)
  int wcol[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) wcol[j] = kPair ? (j < 4 ? wc * 4 + j : 8 + wc * 4 + (j - 4)) : wc * 8 + j;

  f32x4_t acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < S - 1; ++k)
    if (k < KT) fetch(k, k);
  int buf = 0;
  for (int kt = 0; kt < KT; ++kt) {
    // this wave's loads of step kt are done once at most the S - 2 younger steps' loads
    // are outstanding (all of them near the end); the barrier then makes every wave's
    // tiles of step kt visible and retires step kt - 1, whose buffer the next fetch fills
    if (kt + S - 2 < KT)
      wait_vmcnt<6 * (S - 2)>();
    else
      wait_vmcnt<0>();
    lds_barrier();
    if (kt + S - 1 < KT) fetch(kt + S - 1, buf == 0 ? S - 1 : buf - 1);
    bf16x8_t fa[4], fw[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = sA[buf][wr * 4 + i][aslot];
#pragma unroll
    for (int j = 0; j < 8; ++j) fw[j] = sW[buf][wcol[j]][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[j], fa[i], acc[i][j], 0, 0, 0);
    buf = buf == S - 1 ? 0 : buf + 1;
  }
  // lane holds columns 4 kq + e of column tile wcol[j] for row m16 of row tile wr * 4 + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r_wg + wr * 64 + i * 16 + m16;
    if (r >= cnt) continue;
    const int crow = entry_fix<MODE>(group, r, entry_load<MODE>(g, group, r)) + g.c_row_offset;
#pragma unroll
    for (int j = 0; j < (kPair ? 4 : 8); ++j) {
      const int col0 = (ct_wg + wcol[j]) * 16 + kq * 4;
      if (col0 >= N) continue;
      float v[4], u[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = acc[i][j][e];
        u[e] = kPair ? acc[i][j + 4][e] : 0.f;
      }
      epilogue4(g, EPI, group, g.C, g.ldc, crow, col0, v, u);
    }
  }
}

// Mid-size row sets (tens to a few hundred rows per group: block verifies, large decode
// batches). A workgroup of 4 waves owns R = 64 RB rows of one group and CT weight column
// tiles of 16 (CT = 4: 64 output columns, SwiGLU 32 gate columns and their 32 up twins;
// CT = 8: twice that); wave w computes rows 16 RB w .. 16 RB (w + 1) - 1 against all CT
// tiles. The weight tiles of each 32-wide k step go through a ring of S LDS buffers with
// direct global-to-LDS loads (each wave fetches CT / 4 of the 1 KB tiles, all 4 waves read
// all CT); the wave's own rows go through the same ring (one 1 KB direct load per 16-row
// block, read back by the wave alone: 320-row verify 3.15 -> 3.06 ms against loading them
// into registers, whose 16 lanes of a load touched 16 rows). The launch moves rows x (weight rows) x K x 2 (1/(16 CT) + 1/R) bytes from L2 to
// the CUs, which bounds it (about 10 TB/s measured: timing copies without the k loop or
// without the products put the 320-row verify's routed gate/up at 6.2 and 22.9 of its
// 22.7 us, and rings of 4 to 10 buffers or 2 to 4 k tiles per stage ran alike; lanes past
// the row count re-read the last row, whose lines their wave's load fetches once). The
// expert launches take 64 x 128 tiles (RB = 1, CT = 8; 320-row verify: routed gate/up 22.8
// us in 64 x 64 tiles, 21.1 in 64 x 128, 21.8 in 128 x 128 at one wave per SIMD, 24.4 in
// 128 x 64) and the attention projections, whose few hundred dense rows need the
// workgroups, 64 x 64 (RB = 1, CT = 4).
//
// Summation order: K is cut into the 8 chunks of gemm_bf16_kernel (wave w of that kernel
// takes k tiles p K/32 + w KITER + i, pass p, i < KITER), each chunk summed by one chain
// of matrix-core products from zero and the chunks added in order 0..7 to a zero start,
// as that kernel's LDS reduction does: the two kernels give identical results, so a
// caller picks either one by speed alone.
constexpr int kMidWaves = 4;

// Tile of a 1-D mid-size launch: the tiles that hold rows, ordered (group, row tile,
// column block) with column blocks fastest and the fused all-rows group (has_g0) first,
// are cut into 8 contiguous ranges, one per XCD, as in wide_tile.
template <int MODE, int CW, int R>
__device__ __forceinline__ bool mid_tile(const GemmArgs& g, int& cb, int& group, int& rt,
                                         int& cnt) {
  const int L = (int)blockIdx.x, xcd = L % kXcds, slot = L / kXcds;
  const int lane = (int)threadIdx.x & 63;
  const int s0 = g.has_g0 ? 1 : 0;
  const int ng = g.grid_y + s0;  // at most 64 (host check)
  int rows = 0, nx = 0, items = 0;
  if (lane < ng) {
    const int grp = lane < s0 ? -1 : lane - s0 + g.group_offset;
    rows = group_rows<MODE>(g, grp);
    nx = ((lane < s0 ? g.N0 : g.N) + CW - 1) / CW;
    items = min((rows + R - 1) / R, g.grid_z) * nx;
  }
  int total = 0;
  for (int j = 0; j < ng; ++j) total += __builtin_amdgcn_readlane(items, j);
  const int per = (total + kXcds - 1) / kXcds;
  int it = xcd * per + slot;
  if (slot >= per || it >= total) return false;
  for (int j = 0; j < ng; ++j) {
    const int ij = __builtin_amdgcn_readlane(items, j);
    if (it < ij) {
      const int nxj = __builtin_amdgcn_readlane(nx, j);
      group = j < s0 ? -1 : j - s0 + g.group_offset;
      rt = it / nxj;
      cb = it % nxj;
      cnt = __builtin_amdgcn_readlane(rows, j);
      return true;
    }
    it -= ij;
  }
  return false;
}

// The k loop of one mid-size tile: PASSES passes of 8 KITER k tiles, visited chunk by chunk
// (chunk w: tiles p 8 KITER + w KITER + i, p < PASSES, i < KITER). wsrc[h]: the wave's
// weight tile h (tile wv + 4 h of the block) at k tile 0, lane offset included; arow: the
// wave's A rows at k 0 (lane offset included). tot: the chunk sums added in chunk
// order.
template <int KITER, int PASSES, int RB, int CT, int SR>
__device__ __forceinline__ void mid_kloop(const bf16* const (&wsrc)[CT / 4],
                                          const bf16* const (&arow)[RB], bf16x8_t (*sW)[CT][64],
                                          bf16x8_t (*sA)[kMidWaves * RB][64], int aslot, int wv,
                                          int lane, f32x4_t (&tot)[RB][CT]) {
  constexpr int CK = KITER * PASSES, STEPS = 8 * CK, KB = 8 * KITER;
  constexpr int S = SR < STEPS ? SR : STEPS;  // ring buffers in use (at most sW's SR)
  static_assert(S >= 2, "ring of at least 2 buffers");
  constexpr int LOADS = CT / 4 + RB;  // vector loads of one wave per step
  static_assert((S - 2) * LOADS <= 63, "vmcnt range");
  // k tile of step t of the chunk-ordered sequence
  auto ktile = [](int t) { return ((t % CK) / KITER) * KB + (t / CK) * KITER + (t % CK) % KITER; };
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  f32x4_t acc[RB][CT];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int c = 0; c < CT; ++c) tot[rb][c] = zero;
  auto fetch = [&](int j) {
    const int kt = ktile(j);
#pragma unroll
    for (int h = 0; h < CT / 4; ++h)
      load_lds16(wsrc[h] + (int64_t)kt * 512, &sW[j % S][wv + 4 * h][0]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) load_lds16(arow[rb] + kt * 32, &sA[j % S][wv * RB + rb][0]);
  };
#pragma unroll
  for (int j = 0; j < S - 1; ++j) fetch(j);
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    // steps stay in program order (the scheduler would otherwise keep several chunks'
    // accumulators live at once)
    __builtin_amdgcn_sched_barrier(0);
    // step s's loads are done once at most the S - 2 younger steps' loads are
    // outstanding; the barrier publishes every wave's weight tiles of step s and retires
    // step s - 1, whose buffer the next fetch fills
    if (s + S - 2 < STEPS)
      wait_vmcnt<(S - 2) * LOADS>();
    else
      wait_vmcnt<0>();
    lds_barrier();
    if (s + S - 1 < STEPS) fetch(s + S - 1);
    bf16x8_t fw[CT], xa[RB];
#pragma unroll
    for (int c = 0; c < CT; ++c) fw[c] = sW[s % S][c][lane];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) xa[rb] = sA[s % S][wv * RB + rb][aslot];
    // a chunk's chain starts from zero
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int c = 0; c < CT; ++c)
        acc[rb][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[rb], fw[c],
                                                            s % CK == 0 ? zero : acc[rb][c], 0, 0, 0);
    if ((s + 1) % CK == 0) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int c = 0; c < CT; ++c) tot[rb][c] += acc[rb][c];
    }
  }
}

template <int EPI, int MODE, int KITER, int KMUL0, int RB, int CT, int S>
__global__ void __launch_bounds__(64 * kMidWaves, 2) gemm_bf16_mid_kernel(GemmArgs g) {
  constexpr bool kPair = (EPI == EPI_SWIGLU);
  constexpr int CW = kPair ? CT * 8 : CT * 16;  // output columns per column block
  constexpr int R = kMidWaves * RB * 16;
  static_assert(CT == 4 || CT == 8, "4 or 8 weight tiles per workgroup");
  __shared__ bf16x8_t sW[S][CT][64];
  // each wave's A rows of a k step go through the same ring: 16 rows x 32 k per row block,
  // chunk (row m, k chunk q) at slot 4 m + (q ^ 2 (m >> 3)): the load's lanes 4 j .. 4 j + 3
  // fetch row j's 64 contiguous bytes, and the fragment read (lane = row m, chunk kq) is
  // free of LDS bank conflicts
  __shared__ bf16x8_t sA[S][kMidWaves * RB][64];
  int cb, group, rt, cnt;
  if (!mid_tile<MODE, CW, R>(g, cb, group, rt, cnt)) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m = lane & 15, kq = lane >> 4;
  const bool g0 = group < 0;
  const int N = g0 ? g.N0 : g.N;
  const int KT = (g0 ? g.K0 : g.K) / 32;
  const bf16* W = g0 ? reinterpret_cast<const bf16*>(g.W0)
                     : reinterpret_cast<const bf16*>(g.W) + (int64_t)group * g.w_group_stride;
  const bf16* A = reinterpret_cast<const bf16*>(g0 ? g.A0 : g.A);
  const int64_t lda = g0 ? g.lda0 : g.lda;
  void* Cout = g0 ? g.C0 : g.C;
  const int64_t ldc = g0 ? g.ldc0 : g.ldc;
  // weight tile c of the block: SwiGLU gate tiles (CT/2) cb + c for c < CT/2 and their up
  // twins N/16 on; otherwise tiles CT cb + c (tiles past N re-read the last one, never
  // stored). Wave wv fetches tiles wv + 4 h.
  const bf16* wsrc[CT / 4];
#pragma unroll
  for (int h = 0; h < CT / 4; ++h) {
    const int c = wv + 4 * h;
    int ct;
    if constexpr (kPair)
      ct = (c < CT / 2 ? 0 : N / 16 - CT / 2) + cb * (CT / 2) + c;
    else
      ct = min(cb * CT + c, N / 16 - 1);
    wsrc[h] = W + ((int64_t)ct * KT * 64 + lane) * 8;
  }
  // rows of the wave: 16-row block rb holds tile rows 16 (RB wv + rb) + 0..15; lanes past
  // the count re-read the last row (computed, never stored). Lane l loads row l >> 2 of
  // the block (its entry is lane (l >> 2)'s), chunk (l & 3) ^ 2 (l >> 5).
  const int r0 = rt * R + wv * RB * 16;
  int ent[RB];
  const bf16* arow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int i = min(r0 + rb * 16 + m, cnt - 1);
    ent[rb] = entry_fix<MODE>(group, i, entry_load<MODE>(g, group, i));
    const int el = __shfl(ent[rb], lane >> 2, 64);
    arow[rb] = A + (int64_t)a_row_of<MODE>(g, group, el) * lda + ((lane & 3) ^ ((lane >> 5) << 1)) * 8;
  }
  const int aslot = m * 4 + (kq ^ ((m >> 3) << 1));  // this lane's fragment chunk
  f32x4_t tot[RB][CT];
  if (g0 && KMUL0 > 1)
    mid_kloop<KITER, KMUL0, RB, CT, S>(wsrc, arow, sW, sA, aslot, wv, lane, tot);
  else
    mid_kloop<KITER, 1, RB, CT, S>(wsrc, arow, sW, sA, aslot, wv, lane, tot);
  // D layout of 16x16 MFMA: lane holds rows 4 kq + j of its block, column m; the C row of
  // block row r is the entry held by lane r
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int crow = __shfl(ent[rb], kq * 4 + j, 64);
      if (r0 + rb * 16 + kq * 4 + j >= cnt) continue;
      if constexpr (kPair) {
#pragma unroll
        for (int c = 0; c < CT / 2; ++c)
          epilogue<bf16>(g, EPI, group, Cout, ldc, crow + g.c_row_offset,
                         (cb * (CT / 2) + c) * 16 + m, tot[rb][c][j], tot[rb][c + CT / 2][j]);
      } else {
#pragma unroll
        for (int c = 0; c < CT; ++c) {
          const int col = (cb * CT + c) * 16 + m;
          if (col < N)
            epilogue<bf16>(g, EPI, group, Cout, ldc, crow + g.c_row_offset, col, tot[rb][c][j], 0.f);
        }
      }
    }
  }
}

template <int EPI, int MODE, int KMUL0, bool EAGER, bool XCD>
void launch_bf16_kx(const GemmArgs& a, dim3 grid, hipStream_t s) {
  constexpr int T = 64 * kGemmWaves;
  switch (a.K) {
    case 256: gemm_bf16_kernel<EPI, 1, MODE, KMUL0, EAGER, XCD><<<grid, T, 0, s>>>(a); break;
    case 512: gemm_bf16_kernel<EPI, 2, MODE, KMUL0, EAGER, XCD><<<grid, T, 0, s>>>(a); break;
    case 1024: gemm_bf16_kernel<EPI, 4, MODE, KMUL0, EAGER, XCD><<<grid, T, 0, s>>>(a); break;
    default: gemm_bf16_kernel<EPI, 8, MODE, KMUL0, EAGER, XCD><<<grid, T, 0, s>>>(a); break;
  }
}

template <int EPI, int MODE, int KMUL0, bool EAGER = false>
void launch_bf16_k(const GemmArgs& a, dim3 grid, hipStream_t s) {
  if (a.grid_z > 1) {
    // 1-D launch in the XCD-aware order of gemm_block
    const int pairs = (a.grid_x * a.grid_y + kXcds - 1) / kXcds * kXcds;
    launch_bf16_kx<EPI, MODE, KMUL0, EAGER, true>(a, dim3((unsigned)(pairs * a.grid_z)), s);
  } else {
    launch_bf16_kx<EPI, MODE, KMUL0, EAGER, false>(a, grid, s);
  }
}

// Row tiles walked by one workgroup of an expert-list or logits launch (weights stay in
// registers across them). Launches over the rows of a pulse (the attention projections,
// whose weights are a few MiB) give every 32-row tile its own workgroup: their tiles run
// in parallel, and the re-read weight slices come from the XCD's L2 (XCD-aware order
// below). The output head (64 MiB) measured slower that way at 320 rows (61 -> 75 us).
constexpr int kTilesPerWorkgroup = 4;
constexpr int kG0Split = 4;

template <int EPI>
int launch_one(const GemmArgs& a, int dtype, int groups, int max_rows, hipStream_t s) {
  const int tiles = (max_rows + 31) / 32;
  if (tiles <= 0 || groups <= 0) return PULSAR_OK;
  int gy = groups + (a.has_g0 ? 1 : 0);
  const int nmax = a.has_g0 ? std::max(a.N, a.N0) : a.N;
  const int k0 = a.has_g0 ? a.K0 : a.K;
  if (dtype == PULSAR_BF16) {
    if (a.K != 256 && a.K != 512 && a.K != 1024 && a.K != 2048)
      return fail(PULSAR_ERR_UNSUPPORTED, "gemm: K must be 256, 512, 1024 or 2048");
    if (a.has_g0 && (a.row_mode != ROWS_LIST || a.ctl == nullptr))
      return fail(PULSAR_ERR_INVALID,
                  "gemm: the all-rows group fuses into list launches with a control block only");
    if (k0 != a.K && k0 != 2 * a.K)
      return fail(PULSAR_ERR_UNSUPPORTED, "gemm: the all-rows group needs K0 = K or 2K");
    const int per_wg = a.row_mode == ROWS_PULSE ? 1 : kTilesPerWorkgroup;
    const int gz = (tiles + per_wg - 1) / per_wg;
    // the all-rows group: one row tile per workgroup, up to kG0Split rows of the grid
    const int s0 = a.has_g0 ? std::min(kG0Split, (tiles + gz - 1) / gz) : 0;
    gy = groups + s0;
    dim3 grid((unsigned)((nmax + 15) / 16), (unsigned)gy, (unsigned)gz);
    GemmArgs ga = a;
    ga.g0_split = s0;
    ga.grid_x = (int)grid.x;
    ga.grid_y = (int)grid.y;
    ga.grid_z = (int)grid.z;
    switch (a.row_mode) {
      case ROWS_PULSE: launch_bf16_k<EPI, ROWS_PULSE, 1>(ga, grid, s); break;
      case ROWS_LIST:
        if (a.eager_w) {
          if (EPI != EPI_SWIGLU || k0 != a.K)
            return fail(PULSAR_ERR_UNSUPPORTED,
                        "gemm: eager expert launches are SwiGLU with K0 == K");
          if (a.a_rows < 1 || (a.has_g0 && a.a_rows0 < 1))
            return fail(PULSAR_ERR_INVALID, "gemm: eager expert launches need A row counts");
          if constexpr (EPI == EPI_SWIGLU) launch_bf16_k<EPI, ROWS_LIST, 1, true>(ga, grid, s);
        } else {
          if (k0 == a.K)
            launch_bf16_k<EPI, ROWS_LIST, 1>(ga, grid, s);
          else
            launch_bf16_k<EPI, ROWS_LIST, 2>(ga, grid, s);
        }
        break;
      case ROWS_ALL: launch_bf16_k<EPI, ROWS_ALL, 1>(ga, grid, s); break;
      case ROWS_LOGITS: launch_bf16_k<EPI, ROWS_LOGITS, 1>(ga, grid, s); break;
      default: return fail(PULSAR_ERR_INVALID, "gemm: row mode");
    }
  } else {
    dim3 grid((unsigned)((nmax + 3) / 4), (unsigned)gy, (unsigned)tiles);
    gemm_f32_kernel<EPI><<<grid, 256, 0, s>>>(a);
  }
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

template <int EPI, int MODE, int KMUL0, int RB, int CT, int S>
void launch_mid_k(const GemmArgs& a, dim3 grid, hipStream_t s) {
  switch (a.K) {
    case 256: gemm_bf16_mid_kernel<EPI, MODE, 1, KMUL0, RB, CT, S><<<grid, 64 * kMidWaves, 0, s>>>(a); break;
    case 512: gemm_bf16_mid_kernel<EPI, MODE, 2, KMUL0, RB, CT, S><<<grid, 64 * kMidWaves, 0, s>>>(a); break;
    case 1024: gemm_bf16_mid_kernel<EPI, MODE, 4, KMUL0, RB, CT, S><<<grid, 64 * kMidWaves, 0, s>>>(a); break;
    default: gemm_bf16_mid_kernel<EPI, MODE, 8, KMUL0, RB, CT, S><<<grid, 64 * kMidWaves, 0, s>>>(a); break;
  }
}

// Tile shape of a mid-size launch: expert lists in 64 x 128 tiles, rows of a pulse or all
// rows (one dense group) in 64 x 64 tiles; rings of 6 buffers.
template <int EPI, int RB, int CT, int S>
int launch_mid_shape(const GemmArgs& a, int groups, int max_rows, hipStream_t s) {
  constexpr int R = kMidWaves * RB * 16;
  constexpr int CW = EPI == EPI_SWIGLU ? CT * 8 : CT * 16;
  const int ncol = EPI == EPI_SWIGLU ? CT * 8 : 16;
  if (a.N % ncol != 0 || (a.has_g0 && a.N0 % ncol != 0))
    return fail(PULSAR_ERR_UNSUPPORTED, "gemm: mid-size tiles need N % 16 == 0 (SwiGLU: a "
                                        "multiple of the column block)");
  GemmArgs ga = a;
  ga.grid_y = groups;
  ga.grid_z = (max_rows + R - 1) / R;
  int64_t items = (int64_t)groups * ga.grid_z * ((a.N + CW - 1) / CW);
  if (a.has_g0) items += (int64_t)ga.grid_z * ((a.N0 + CW - 1) / CW);
  if (items > (int64_t)1 << 30) return fail(PULSAR_ERR_INVALID, "gemm: mid-size launch too large");
  const dim3 grid((unsigned)((items + kXcds - 1) / kXcds * kXcds));
  const bool k2 = a.has_g0 && a.K0 == 2 * a.K;
  switch (a.row_mode) {
    case ROWS_PULSE: launch_mid_k<EPI, ROWS_PULSE, 1, RB, CT, S>(ga, grid, s); break;
    case ROWS_ALL: launch_mid_k<EPI, ROWS_ALL, 1, RB, CT, S>(ga, grid, s); break;
    case ROWS_LIST:
      if (k2)
        launch_mid_k<EPI, ROWS_LIST, 2, RB, CT, S>(ga, grid, s);
      else
        launch_mid_k<EPI, ROWS_LIST, 1, RB, CT, S>(ga, grid, s);
      break;
    default: return fail(PULSAR_ERR_INVALID, "gemm: row mode of a mid-size launch");
  }
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

template <int EPI>
int launch_mid(const GemmArgs& a, int groups, int max_rows, hipStream_t s) {
  if (groups <= 0 || max_rows <= 0) return PULSAR_OK;
  if (a.K != 256 && a.K != 512 && a.K != 1024 && a.K != 2048)
    return fail(PULSAR_ERR_UNSUPPORTED, "gemm: K must be 256, 512, 1024 or 2048");
  if (a.has_g0 && (a.row_mode != ROWS_LIST || a.ctl == nullptr))
    return fail(PULSAR_ERR_INVALID,
                "gemm: the all-rows group fuses into list launches with a control block only");
  if (a.has_g0 && a.K0 != a.K && a.K0 != 2 * a.K)
    return fail(PULSAR_ERR_UNSUPPORTED, "gemm: the all-rows group needs K0 = K or 2K");
  if (groups + (a.has_g0 ? 1 : 0) > 64)
    return fail(PULSAR_ERR_UNSUPPORTED, "gemm: mid-size tiles take at most 64 groups");
  if (a.row_mode == ROWS_LIST) return launch_mid_shape<EPI, 1, 8, 6>(a, groups, max_rows, s);
  return launch_mid_shape<EPI, 1, 4, 6>(a, groups, max_rows, s);
}

template <int EPI>
int launch_wide(const GemmArgs& a, int groups, int max_rows, hipStream_t s) {
  const int colw = EPI == EPI_SWIGLU ? 128 : 256;
  dim3 grid((unsigned)((a.N + colw - 1) / colw), (unsigned)groups,
            (unsigned)((max_rows + kTileRows - 1) / kTileRows));
  // row-set modes: a 1-D grid over (column block, group, row tile), split by wide_tile
  GemmArgs ga = a;
  ga.grid_x = (int)grid.x;
  ga.grid_y = (int)grid.y;
  ga.grid_z = (int)grid.z;
  const int64_t tiles = (int64_t)ga.grid_x * ga.grid_y * ga.grid_z;
  if (tiles > (int64_t)1 << 30) return fail(PULSAR_ERR_INVALID, "gemm: wide launch too large");
  const dim3 g1((unsigned)((tiles + kXcds - 1) / kXcds * kXcds));
  switch (a.row_mode) {
    case ROWS_PULSE: gemm_bf16_lds_kernel<EPI, ROWS_PULSE><<<g1, 256, 0, s>>>(ga); break;
    case ROWS_LIST: gemm_bf16_lds_kernel<EPI, ROWS_LIST><<<g1, 256, 0, s>>>(ga); break;
    case ROWS_ALL: gemm_bf16_lds_kernel<EPI, ROWS_ALL><<<g1, 256, 0, s>>>(ga); break;
    case ROWS_LOGITS:
      if constexpr (EPI == EPI_LOGITS || EPI == EPI_LOGITS_RAW) {
        gemm_bf16_lds_kernel<EPI, ROWS_LOGITS><<<grid, 256, 0, s>>>(a);
        break;
      }
      return fail(PULSAR_ERR_INVALID, "gemm: logits rows take a logits epilogue");
    default: return fail(PULSAR_ERR_INVALID, "gemm: row mode of a wide launch");
  }
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

}  // namespace

int launch_gemm_wide(const GemmArgs& a, int dtype, int epi, int groups, int max_rows,
                     hipStream_t s) {
  if (dtype != PULSAR_BF16 || a.has_g0)
    return launch_gemm(a, dtype, epi, groups, max_rows, s);
  if (groups <= 0) return PULSAR_OK;
  if (a.K % 256 != 0 || a.N % 16 != 0 || (epi == EPI_SWIGLU && a.N % 128 != 0))
    return fail(PULSAR_ERR_UNSUPPORTED, "gemm: wide tiles need K % 256 == 0 and N % 16 == 0 "
                                        "(SwiGLU: N % 128 == 0)");
  switch (epi) {
    case EPI_STORE: return launch_wide<EPI_STORE>(a, groups, max_rows, s);
    case EPI_QKVG: return launch_wide<EPI_QKVG>(a, groups, max_rows, s);
    case EPI_RESID: return launch_wide<EPI_RESID>(a, groups, max_rows, s);
    case EPI_SWIGLU: return launch_wide<EPI_SWIGLU>(a, groups, max_rows, s);
    case EPI_SCALE: return launch_wide<EPI_SCALE>(a, groups, max_rows, s);
    case EPI_LOGITS: return launch_wide<EPI_LOGITS>(a, groups, max_rows, s);
    case EPI_LOGITS_RAW: return launch_wide<EPI_LOGITS_RAW>(a, groups, max_rows, s);
  }
  return launch_gemm(a, dtype, epi, groups, max_rows, s);
}

int launch_gemm_mid(const GemmArgs& a, int dtype, int epi, int groups, int max_rows,
                    hipStream_t s) {
  if (dtype != PULSAR_BF16) return launch_gemm(a, dtype, epi, groups, max_rows, s);
  switch (epi) {
    case EPI_STORE: return launch_mid<EPI_STORE>(a, groups, max_rows, s);
    case EPI_QKVG: return launch_mid<EPI_QKVG>(a, groups, max_rows, s);
    case EPI_RESID: return launch_mid<EPI_RESID>(a, groups, max_rows, s);
    case EPI_SWIGLU: return launch_mid<EPI_SWIGLU>(a, groups, max_rows, s);
  }
  return launch_gemm(a, dtype, epi, groups, max_rows, s);
}

int launch_gemm(const GemmArgs& a, int dtype, int epi, int groups, int max_rows, hipStream_t s) {
  if (a.K % 256 != 0)
    return fail(PULSAR_ERR_UNSUPPORTED, "gemm: K must be a multiple of 256");
  switch (epi) {
    case EPI_STORE: return launch_one<EPI_STORE>(a, dtype, groups, max_rows, s);
    case EPI_QKVG: return launch_one<EPI_QKVG>(a, dtype, groups, max_rows, s);
    case EPI_RESID: return launch_one<EPI_RESID>(a, dtype, groups, max_rows, s);
    case EPI_SWIGLU: return launch_one<EPI_SWIGLU>(a, dtype, groups, max_rows, s);
    case EPI_LOGITS:
      if (dtype == PULSAR_BF16) {
        // column pairs (c, N/2 + c) per workgroup
        if (a.N % 32 != 0) return fail(PULSAR_ERR_UNSUPPORTED, "gemm: logits N % 32 != 0");
        GemmArgs h = a;
        h.N = a.N / 2;
        return launch_one<EPI_LOGITS>(h, dtype, groups, max_rows, s);
      }
      return launch_one<EPI_LOGITS>(a, dtype, groups, max_rows, s);
    case EPI_LOGITS_RAW: return launch_one<EPI_LOGITS_RAW>(a, dtype, groups, max_rows, s);
    case EPI_SCALE: return launch_one<EPI_SCALE>(a, dtype, groups, max_rows, s);
  }
  return fail(PULSAR_ERR_INVALID, "gemm: unknown epilogue");
}

}  // namespace pulsar
