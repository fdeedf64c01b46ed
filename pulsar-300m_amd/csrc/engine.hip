// Decode engine: owns the KV cache, per-row work buffers and controller state of a batch
// of sequences; runs prefill eagerly and decode as a step (one pulse of every active row)
// that can be captured once into a HIP graph and replayed.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

#include "rows.h"
#include "sample.h"

namespace pulsar {

struct Engine {
  PulsarModelDesc m{};
  PulsarEngineConfig cfg{};
  int dtype = 0, es = 4;
  int D = 0, H = 0, Hkv = 0, qkv = 0, qkvg = 0, E = 0, K = 0, de = 0, ds = 0, L = 0, P = 0, V = 0;
  int B = 0, max_rows = 0, R = 0, max_pages = 0, lcap = 0, max_splits = 0, max_splits_unit = 0;
  int G = 0;  // drafts per round (draft-block mode), 0 = exact mode
  int mid_rows = 0;  // steps of this many rows or more run the mid-size projection GEMMs
  int S = 2;  // token-state slots per sequence: rows of one sequence in a step
  std::vector<void*> allocs;

  StepCtl* ctl = nullptr;
  StepCtl* last_ctl = nullptr;
  RowDesc* rows = nullptr;
  RowDesc* last_rows = nullptr;
  AttnUnit* units = nullptr;
  int32_t* split_done = nullptr;  // [B][Hkv] decode attention split counters
  SeqState* state = nullptr;
  int32_t *lrow_seq = nullptr, *lrow_extra = nullptr, *argmax = nullptr, *draw = nullptr;
  uint32_t* lrow_ctr = nullptr;  // draft-block mode: per logits row draw counter
  int32_t *tokens = nullptr, *stop_ids = nullptr;
  int32_t* kinds = nullptr;  // [B][max_new] 1 = emitted as an accepted draft
  uint32_t* seen = nullptr;
  void *e_state = nullptr, *hout_state = nullptr;
  void *h_in = nullptr, *h = nullptr, *xn = nullptr, *qkvbuf = nullptr, *gate = nullptr;
  void *attn_out = nullptr, *v_first = nullptr, *act_s = nullptr, *act_r = nullptr;
  void *out_s = nullptr, *out_r = nullptr, *xn_final = nullptr;
  float *part = nullptr, *logits = nullptr, *topk_w = nullptr;
  float* plogits = nullptr;   // prefill logits [B][V], kept for rewind
  uint64_t* d_seed = nullptr;
  // per-kernel-class event timing of eager steps
  bool prof_on = false;
  std::vector<hipEvent_t> ev_pool;
  int ev_used = 0;
  std::vector<std::array<int, 3>> spans;  // (class, start event, end event)
  double prof_ms[PULSAR_PROF_CLASSES] = {};
  int64_t prof_n[PULSAR_PROF_CLASSES] = {};
  int32_t *topk_idx = nullptr, *keep = nullptr;
  int32_t* dec_topk = nullptr;     // decode router top-k ids per layer [L][max_rows][K]
  float* maxprob = nullptr;        // early exit: top-1 probability per logits row
  int32_t* exit_counts = nullptr;  // early exit: [B][4] exits per pulse
  int32_t *lists = nullptr, *list_count = nullptr;      // decode: [L][E][max_rows*K], [L][E]
  int32_t *p_lists = nullptr, *p_lcount = nullptr;  // prefill
  int32_t* p_ids = nullptr;
  RowDesc* p_rows = nullptr;  // [P][R]
  StepCtl* p_ctl = nullptr;   // [P]
  KVDesc kv{};
  // global-layer KV pages: pool size, page table [B][max_pages] (unassigned entries name
  // the spare page pool_pages, never written by a sequence), pages per sequence [B], pool
  // counter and spent flag [2]; the *_save copies hold the state the last prefill or
  // fill_kv left, which rewind restores
  int pool_pages = 0;
  int32_t *page_table = nullptr, *page_count = nullptr, *pool = nullptr;
  int32_t *page_table_save = nullptr, *page_count_save = nullptr, *pool_save = nullptr;
  void* ring_save_k[kMaxLayers] = {};  // sliding-window rings as the last prefill left them
  void* ring_save_v[kMaxLayers] = {};
  int prompt_len = 0;
  int v_n = 0;  // rows per sequence of the uploaded verify block (0: none since prefill/fill_kv)
  bool prefilled = false;
  bool kv_ready = false;  // the cache holds positions [0, prompt_len) (prefill or fill_kv)
  // block verify: host-built rows, control blocks and units of its passes
  RowDesc* v_rows = nullptr;  // [P][max_rows]
  StepCtl* v_ctl = nullptr;   // [P]
  AttnUnit* v_units = nullptr;  // [P][B]
  hipGraphExec_t vexec = nullptr;
  hipGraph_t vgraph = nullptr;

  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec_multi = nullptr;  // kGraphSteps steps in one graph
  hipGraph_t graph_multi = nullptr;
  hipStream_t capture_stream = nullptr;  // graphs are captured here (never the legacy stream)
  // pulsar_engine_generate: two pinned readback slots (control block + every sequence's
  // state) and their completion events
  void* host_rb = nullptr;
  hipEvent_t rb_ev[2] = {nullptr, nullptr};

  ~Engine() {
    for (hipEvent_t ev : rb_ev)
      if (ev) hipEventDestroy(ev);
    if (host_rb) hipHostFree(host_rb);
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    if (exec_multi) hipGraphExecDestroy(exec_multi);
    if (graph_multi) hipGraphDestroy(graph_multi);
    if (vexec) hipGraphExecDestroy(vexec);
    if (vgraph) hipGraphDestroy(vgraph);
    if (capture_stream) hipStreamDestroy(capture_stream);
    for (hipEvent_t ev : ev_pool) hipEventDestroy(ev);
    for (void* p : allocs) hipFree(p);
  }

  template <typename X>
  int alloc(X** p, size_t bytes) {
    void* q = nullptr;
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(&q, bytes);
    if (e != hipSuccess)
      return fail(PULSAR_ERR_HIP, std::string("hipMalloc(") + std::to_string(bytes) +
                                      "): " + hipGetErrorString(e));
    allocs.push_back(q);
    *p = reinterpret_cast<X*>(q);
    return PULSAR_OK;
  }
};

#define PULSAR_TRY(expr)          \
  do {                            \
    int _rc = (expr);             \
    if (_rc != PULSAR_OK) return _rc; \
  } while (0)

namespace {

int validate(const PulsarModelDesc& m, const PulsarEngineConfig& c) {
  PULSAR_REQUIRE(m.dtype == PULSAR_F32 || m.dtype == PULSAR_BF16, "model dtype");
  PULSAR_REQUIRE(m.head_dim == kHeadDim, "engine requires head_dim == 64");
  PULSAR_REQUIRE(m.n_heads % m.n_kv_heads == 0 && m.n_heads / m.n_kv_heads == 4,
                 "engine requires 4 query heads per kv head");
  PULSAR_REQUIRE(m.n_layers >= 1 && m.n_layers <= PULSAR_MAX_LAYERS, "n_layers");
  PULSAR_REQUIRE(m.n_pulses >= 1 && m.n_pulses <= kMaxPulses, "n_pulses must be 1..3");
  PULSAR_REQUIRE(m.n_experts >= 1 && m.n_experts <= 32 && m.top_k >= 1 && m.top_k <= 8,
                 "experts");
  PULSAR_REQUIRE(m.d_model % 256 == 0 && m.d_expert % 256 == 0 && m.d_shared % 256 == 0,
                 "d_model, d_expert, d_shared must be multiples of 256");
  PULSAR_REQUIRE(m.reinject_rank >= 1 && m.reinject_rank <= 16, "reinject rank");
  PULSAR_REQUIRE(m.vocab % 4096 == 0, "vocab must be a multiple of 4096");
  PULSAR_REQUIRE(c.max_batch >= 1 && c.max_batch <= 256, "max_batch must be 1..256");
  PULSAR_REQUIRE(c.max_prompt >= 1 && c.max_new >= 0, "max_prompt/max_new");
  PULSAR_REQUIRE(c.draft_len >= 0 && c.draft_len < kMaxBlock, "draft_len must be 0..7");
  PULSAR_REQUIRE(c.draft_len == 0 || m.n_pulses <= 3, "draft-block mode needs n_pulses <= 3");
  PULSAR_REQUIRE(c.max_ctx >= c.max_prompt + c.max_new + 2 + c.draft_len,
                 "max_ctx < max_prompt + max_new + 2 + draft_len");
  PULSAR_REQUIRE(m.rope_len >= c.max_ctx, "rope tables shorter than max_ctx");
  PULSAR_REQUIRE(c.n_stop >= 0 && c.n_stop <= 8, "n_stop must be 0..8");
  PULSAR_REQUIRE(c.early_exit == 0 || c.early_exit == 1, "early_exit must be 0 or 1");
  PULSAR_REQUIRE(c.kv_pages >= 0, "kv_pages must be >= 0 (0: every sequence up to max_ctx)");
  if (c.early_exit) {
    PULSAR_REQUIRE(c.draft_len == 0,
                   "early exit applies to the exact schedule only (draft_len == 0)");
    PULSAR_REQUIRE(std::isfinite(c.early_exit_threshold), "early_exit_threshold must be finite");
  }
  return PULSAR_OK;
}

__global__ void set_seen_kernel(const int32_t* ids, uint32_t* seen, int T, int V, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int b = i / T;
  const int tok = ids[i];
  atomicOr(&seen[(int64_t)b * (V / 32) + (tok >> 5)], 1u << (tok & 31));
}

void kv_desc(Engine& e) {
  e.kv.local_mask = e.m.local_mask;
  e.kv.Hkv = e.Hkv;
  e.kv.lcap = e.lcap;
  e.kv.max_pages = e.max_pages;
  e.kv.page_table = e.page_table;
}

int prof_mark(Engine& e, hipStream_t s) {
  if (!e.prof_on) return -1;
  if (e.ev_used == (int)e.ev_pool.size()) {
    // timing-only events: no system-scope cache writeback/invalidate around the kernels
    hipEvent_t ev;
    if (hipEventCreateWithFlags(&ev, hipEventDisableSystemFence) != hipSuccess) return -1;
    e.ev_pool.push_back(ev);
  }
  const int i = e.ev_used++;
  if (hipEventRecord(e.ev_pool[i], s) != hipSuccess) return -1;
  return i;
}

void prof_span(Engine& e, int cls, int a, int b) {
  if (a >= 0 && b >= 0) e.spans.push_back({cls, a, b});
}

int prof_collect(Engine& e, hipStream_t s) {
  if (!e.prof_on) return PULSAR_OK;
  PULSAR_CHECK_HIP(hipStreamSynchronize(s));
  for (const auto& sp : e.spans) {
    float ms = 0.f;
    PULSAR_CHECK_HIP(hipEventElapsedTime(&ms, e.ev_pool[sp[1]], e.ev_pool[sp[2]]));
    e.prof_ms[sp[0]] += ms;
    e.prof_n[sp[0]] += 1;
  }
  e.spans.clear();
  e.ev_used = 0;
  return PULSAR_OK;
}

// Profiling runs eagerly; a fixed-length sleep kernel ahead of each timed group keeps the
// device busy while the host enqueues the group's start event, kernels and end event, so
// the span measures the kernels, not host launch latency.
__global__ void prof_delay_kernel(int n) {
  for (int i = 0; i < n; ++i) __builtin_amdgcn_s_sleep(127);
}

int prof_delay(Engine& e, hipStream_t s) {
  if (!e.prof_on) return PULSAR_OK;
  prof_delay_kernel<<<1, 64, 0, s>>>(12);
  PULSAR_LAUNCH_CHECK();
  return PULSAR_OK;
}

#define PULSAR_TIMED(cls, expr)          \
  do {                                   \
    PULSAR_TRY(prof_delay(e, s));        \
    const int _a = prof_mark(e, s);      \
    PULSAR_TRY(expr);                    \
    prof_span(e, (cls), _a, prof_mark(e, s)); \
  } while (0)

enum ProfClass {
  PC_INPUT = 0, PC_NORM, PC_QKVG, PC_QKPOST, PC_ATTN, PC_WO, PC_ROUTER, PC_SHARED_GU,
  PC_ROUTED_GU, PC_SHARED_DOWN, PC_ROUTED_DOWN, PC_COMBINE, PC_OUTPUT, PC_LMHEAD, PC_SAMPLE,
  PC_CONTROL, PC_EVENT_PAIR
};

// From kMidRows rows up to kWideRows the projections run in the mid-size tiles of
// launch_gemm_mid (64-row tiles, weights staged through LDS). They give results
// identical to the row-tile kernel's, so the threshold is a matter of speed only; the
// environment variable PULSAR_GEMM_MID_ROWS (read when an engine is created) overrides it.
constexpr int kMidRows = 128;

int create(const PulsarModelDesc& m, const PulsarEngineConfig& c, Engine** out) {
  PULSAR_TRY(validate(m, c));
  Engine* e = new Engine();
  std::unique_ptr<Engine> guard(e);
  e->m = m;
  e->cfg = c;
  e->dtype = m.dtype;
  e->es = m.dtype == PULSAR_BF16 ? 2 : 4;
  e->D = m.d_model;
  e->H = m.n_heads;
  e->Hkv = m.n_kv_heads;
  e->qkv = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
  e->qkvg = e->qkv + m.n_heads;
  e->E = m.n_experts;
  e->K = m.top_k;
  e->de = m.d_expert;
  e->ds = m.d_shared;
  e->L = m.n_layers;
  e->P = m.n_pulses;
  e->V = m.vocab;
  e->B = c.max_batch;
  e->G = c.draft_len;
  e->S = engine_slots(c.draft_len);
  e->max_rows = e->S * c.max_batch;
  e->mid_rows = kMidRows;
  if (const char* v = std::getenv("PULSAR_GEMM_MID_ROWS")) {
    char* end = nullptr;
    const long r = std::strtol(v, &end, 10);
    PULSAR_REQUIRE(end != v && *end == 0 && r >= 0, "PULSAR_GEMM_MID_ROWS must be a row count");
    e->mid_rows = (int)std::min<long>(r, 1L << 30);
  }
  e->R = std::max(e->max_rows, c.max_batch * c.max_prompt);
  e->max_pages = (c.max_ctx + kPage - 1) / kPage;
  // ring capacity: the window plus the rows one step writes (at most kMaxBlock), so that a
  // step's writes never overwrite a key some row of it still attends (the reference keeps
  // the newest `window` entries, src/infer.py:142-148); rewind restores the ring from the
  // copy prefill leaves (ring_save)
  e->lcap = (m.window + kMaxBlock + kPage - 1) / kPage * kPage;
  static_assert(kMaxBlock <= kPage, "ring slack holds a draft block");
  // decode splits start at a 64-aligned position at most 63 keys before the first key
  e->max_splits = (c.max_ctx + kPage - 1 + kSplitLen - 1) / kSplitLen;
  e->max_splits_unit = (c.max_ctx + kPage - 1 + kUnitSplit - 1) / kUnitSplit;
  const size_t es = e->es, D = e->D, R = e->R, MR = e->max_rows;
  Engine& x = *e;
  PULSAR_TRY(x.alloc(&x.ctl, sizeof(StepCtl)));
  PULSAR_TRY(x.alloc(&x.last_ctl, sizeof(StepCtl)));
  PULSAR_TRY(x.alloc(&x.rows, sizeof(RowDesc) * MR));
  PULSAR_TRY(x.alloc(&x.last_rows, sizeof(RowDesc) * MR));
  // every slot holds a valid descriptor from the start (snapshots copy whole row sets)
  PULSAR_CHECK_HIP(hipMemset(x.rows, 0, sizeof(RowDesc) * MR));
  PULSAR_CHECK_HIP(hipMemset(x.last_rows, 0, sizeof(RowDesc) * MR));
  PULSAR_TRY(x.alloc(&x.units, sizeof(AttnUnit) * x.B));
  PULSAR_TRY(x.alloc(&x.v_rows, sizeof(RowDesc) * x.P * MR));
  PULSAR_TRY(x.alloc(&x.v_ctl, sizeof(StepCtl) * x.P));
  PULSAR_TRY(x.alloc(&x.v_units, sizeof(AttnUnit) * x.P * x.B));
  PULSAR_TRY(x.alloc(&x.split_done, 4 * (size_t)x.B * x.Hkv));
  PULSAR_CHECK_HIP(hipMemset(x.split_done, 0, 4 * (size_t)x.B * x.Hkv));
  PULSAR_TRY(x.alloc(&x.state, sizeof(SeqState) * x.B));
  PULSAR_TRY(x.alloc(&x.lrow_seq, 4 * MR));
  PULSAR_TRY(x.alloc(&x.lrow_extra, 4 * MR * kMaxExtra));
  PULSAR_TRY(x.alloc(&x.lrow_ctr, 4 * MR));
  PULSAR_TRY(x.alloc(&x.argmax, 4 * MR));
  PULSAR_TRY(x.alloc(&x.draw, 8 * MR));
  PULSAR_TRY(x.alloc(&x.tokens, 4 * (size_t)x.B * std::max(1, c.max_new)));
  PULSAR_TRY(x.alloc(&x.kinds, 4 * (size_t)x.B * std::max(1, c.max_new)));
  PULSAR_TRY(x.alloc(&x.stop_ids, 4 * 8));
  PULSAR_TRY(x.alloc(&x.seen, 4 * (size_t)x.B * (x.V / 32)));
  PULSAR_TRY(x.alloc(&x.e_state, es * R * D));
  PULSAR_TRY(x.alloc(&x.hout_state, es * R * D));
  PULSAR_TRY(x.alloc(&x.h_in, es * R * D));
  PULSAR_TRY(x.alloc(&x.h, es * R * D));
  PULSAR_TRY(x.alloc(&x.xn, es * R * D));
  PULSAR_TRY(x.alloc(&x.qkvbuf, es * R * x.qkv));
  PULSAR_TRY(x.alloc(&x.gate, es * R * x.H));
  PULSAR_TRY(x.alloc(&x.attn_out, es * R * x.H * kHeadDim));
  PULSAR_TRY(x.alloc(&x.v_first, es * R * x.Hkv * kHeadDim));
  PULSAR_TRY(x.alloc(&x.act_s, es * R * x.ds));
  PULSAR_TRY(x.alloc(&x.act_r, es * R * x.K * x.de));
  PULSAR_TRY(x.alloc(&x.out_s, es * R * D));
  PULSAR_TRY(x.alloc(&x.out_r, es * R * x.K * D));
  PULSAR_TRY(x.alloc(&x.xn_final, es * std::max<size_t>(MR, x.B) * D));
  PULSAR_TRY(x.alloc(&x.logits, 4 * std::max<size_t>(MR, x.B) * x.V));
  PULSAR_TRY(x.alloc(&x.plogits, 4 * (size_t)x.B * x.V));
  PULSAR_TRY(x.alloc(&x.d_seed, 8));
  PULSAR_TRY(x.alloc(&x.topk_idx, 4 * R * x.K));
  PULSAR_TRY(x.alloc(&x.topk_w, 4 * R * x.K));
  PULSAR_TRY(x.alloc(&x.keep, 4 * R * x.K));
  PULSAR_TRY(x.alloc(&x.dec_topk, 4 * (size_t)x.L * MR * x.K));
  PULSAR_CHECK_HIP(hipMemset(x.dec_topk, 0xff, 4 * (size_t)x.L * MR * x.K));
  PULSAR_TRY(x.alloc(&x.maxprob, 4 * std::max<size_t>(MR, x.B)));
  PULSAR_TRY(x.alloc(&x.exit_counts, 4 * 4 * (size_t)x.B));
  PULSAR_CHECK_HIP(hipMemset(x.exit_counts, 0, 4 * 4 * (size_t)x.B));
  // split partials: fp32 path per (row, kv head, split, head); bf16 path per (unit, kv
  // head, split, query column), up to 32 columns per unit (8 rows x 4 heads)
  PULSAR_TRY(x.alloc(&x.part, 4 * std::max<size_t>(MR * 4, (size_t)x.B * 4 * kMaxBlock) * x.Hkv *
                                  x.max_splits * 66));
  PULSAR_TRY(x.alloc(&x.lists, 4 * (size_t)x.L * x.E * MR * x.K));
  PULSAR_TRY(x.alloc(&x.list_count, 4 * (size_t)x.L * x.E));
  PULSAR_TRY(x.alloc(&x.p_lists, 4 * (size_t)x.E * R * x.K));
  PULSAR_TRY(x.alloc(&x.p_lcount, 4 * (size_t)x.E));
  PULSAR_TRY(x.alloc(&x.p_ids, 4 * (size_t)x.B * c.max_prompt));
  PULSAR_TRY(x.alloc(&x.p_rows, sizeof(RowDesc) * x.P * (size_t)x.B * c.max_prompt));
  PULSAR_TRY(x.alloc(&x.p_ctl, sizeof(StepCtl) * x.P));
  // KV cache; the global layers' pool holds one spare page past pool_pages, which the
  // page-table entries not assigned yet name
  x.pool_pages = c.kv_pages > 0 ? c.kv_pages : x.B * x.max_pages;
  const size_t pt = (size_t)x.B * x.max_pages;
  PULSAR_TRY(x.alloc(&x.page_table, 4 * pt));
  PULSAR_TRY(x.alloc(&x.page_table_save, 4 * pt));
  PULSAR_TRY(x.alloc(&x.page_count, 4 * (size_t)x.B));
  PULSAR_TRY(x.alloc(&x.page_count_save, 4 * (size_t)x.B));
  PULSAR_TRY(x.alloc(&x.pool, 8));
  PULSAR_TRY(x.alloc(&x.pool_save, 8));
  {
    const std::vector<int32_t> spare(pt, x.pool_pages);
    PULSAR_CHECK_HIP(hipMemcpy(x.page_table, spare.data(), 4 * pt, hipMemcpyHostToDevice));
    PULSAR_CHECK_HIP(hipMemcpy(x.page_table_save, spare.data(), 4 * pt, hipMemcpyHostToDevice));
    PULSAR_CHECK_HIP(hipMemset(x.page_count, 0, 4 * (size_t)x.B));
    PULSAR_CHECK_HIP(hipMemset(x.page_count_save, 0, 4 * (size_t)x.B));
    PULSAR_CHECK_HIP(hipMemset(x.pool, 0, 8));
    PULSAR_CHECK_HIP(hipMemset(x.pool_save, 0, 8));
  }
  const size_t local_elems = (size_t)x.B * x.Hkv * x.lcap * kHeadDim;
  const size_t global_elems = ((size_t)x.pool_pages + 1) * x.Hkv * kPage * kHeadDim;
  for (int l = 0; l < x.L; ++l) {
    const bool loc = (m.local_mask >> l) & 1u;
    const size_t n = loc ? local_elems : global_elems;
    PULSAR_TRY(x.alloc(&x.kv.k[l], es * n));
    PULSAR_TRY(x.alloc(&x.kv.v[l], es * n));
    if (loc) {
      PULSAR_TRY(x.alloc(&x.ring_save_k[l], es * n));
      PULSAR_TRY(x.alloc(&x.ring_save_v[l], es * n));
    }
    // never-written positions are read (masked) by the block-wise decode attention: keep
    // them finite
    PULSAR_CHECK_HIP(hipMemset(x.kv.k[l], 0, es * n));
    PULSAR_CHECK_HIP(hipMemset(x.kv.v[l], 0, es * n));
  }
  std::vector<int32_t> stops(8, -1);
  for (int i = 0; i < c.n_stop; ++i) stops[i] = c.stop_ids[i];
  PULSAR_CHECK_HIP(hipMemcpy(x.stop_ids, stops.data(), 32, hipMemcpyHostToDevice));
  PULSAR_CHECK_HIP(hipMemset(x.ctl, 0, sizeof(StepCtl)));
  PULSAR_CHECK_HIP(hipMemset(x.last_ctl, 0, sizeof(StepCtl)));
  PULSAR_CHECK_HIP(hipMemset(x.state, 0, sizeof(SeqState) * x.B));
  PULSAR_CHECK_HIP(hipMemset(x.list_count, 0, 4 * (size_t)x.L * x.E));
  PULSAR_CHECK_HIP(hipStreamCreateWithFlags(&x.capture_stream, hipStreamNonBlocking));
  kv_desc(x);
  *out = guard.release();
  return PULSAR_OK;
}

GemmArgs gemm_base(const Engine& e) {
  GemmArgs g{};
  g.a_div = 1;
  g.softcap = 0.f;
  return g;
}

// Engines whose steps hold kWideHeadRows rows or more (verify blocks, batches of 64+) run
// the output head in the 128 x 256 LDS tiles of the prefill GEMMs (its 64 MiB of weights
// read once per 128 rows instead of once per 32); from kWideRows rows (the draft-block
// mode at batch 256) the decode projections too. Below that the row-tile and mid-size
// GEMMs are faster: 128 x 256 tiles leave most CUs idle at a few hundred rows (320-row
// verify: 3.78 against 5.35 ms with every projection in wide tiles). The wide tiles sum K
// in another order than the row-tile and mid-size kernels (which agree exactly), so an
// engine's logits can differ from an engine's on the other side of a wide threshold by
// bf16 rounding; engines on the same side agree exactly.
constexpr int kWideHeadRows = 128;
constexpr int kWideRows = 1024;

// One pass over a row set (the rows of a step, or of one pulse of a block verify): pulse
// input, every layer, pulse output and the logits of the rows that need them.
// Per layer: qkv+gate GEMM, qk-norm/RoPE/KV write, attention (+ split combine), wo GEMM with
// residual, mlp-norm + router, shared+routed gate/up GEMM, shared+routed down GEMM, MoE
// combine with residual and the next layer's attn-norm (the first layer's attn-norm is
// fused into the pulse-input kernel). `head` false leaves out the output head, for passes
// the host knows to have no logits rows.
int enqueue_pass(Engine& e, const StepCtl* ctl, const RowDesc* rows, const AttnUnit* units,
                 hipStream_t s, bool head = true) {
  const PulsarModelDesc& m = e.m;
  const int D = e.D, MR = e.max_rows, dt = e.dtype;
  // at two or more assignments per expert on average, nearly every expert has rows: the
  // routed gate/up GEMM then streams weights and rows without first waiting for each
  // expert's row count (12.2 -> 11.5 us at batch 16; the down GEMM measured no gain)
  const int eager_experts = (int64_t)MR * e.K >= 2 * (int64_t)e.E ? 1 : 0;
  const bool wide = dt == PULSAR_BF16 && MR >= kWideRows;
  const bool wide_head = dt == PULSAR_BF16 && MR >= kWideHeadRows;
  const bool mid = dt == PULSAR_BF16 && !wide && e.mid_rows > 0 && MR >= e.mid_rows;
  // projection GEMMs below the wide-tile threshold
  auto gemm = [&](const GemmArgs& g, int epi, int groups) {
    return mid ? launch_gemm_mid(g, dt, epi, groups, MR, s) : launch_gemm(g, dt, epi, groups, MR, s);
  };
  // bf16: the decode attention finishes q, k and v itself (no qk_post launch)
  const bool fuse_post = dt == PULSAR_BF16;
  if (e.prof_on) {
    // an empty timed group: the fixed cost of an event pair around a kernel launch
    PULSAR_TRY(prof_delay(e, s));
    const int _a = prof_mark(e, s);
    prof_span(e, PC_EVENT_PAIR, _a, prof_mark(e, s));
  }
  PulseInputArgs pi{};
  pi.ctl = ctl;
  pi.rows = rows;
  pi.D = D;
  pi.slots = e.S;
  pi.rank = m.reinject_rank;
  pi.eps = m.rms_eps;
  pi.tok_emb = m.tok_emb;
  pi.anchor_norm = m.anchor_norm;
  pi.conv_w = m.conv_w;
  pi.state_norm = m.state_norm;
  pi.step_emb = m.step_emb;
  pi.reinject_down = m.reinject_down;
  pi.reinject_up = m.reinject_up;
  pi.reinject_bias = m.reinject_bias;
  pi.e_state = e.e_state;
  pi.hout_state = e.hout_state;
  pi.h_in = e.h_in;
  pi.h = e.h;
  pi.zero_counts = e.list_count;
  pi.n_zero = e.L * e.E;
  pi.norm_w = m.attn_norm[0];
  pi.xn = e.xn;
  PULSAR_TIMED(PC_INPUT, launch_pulse_input(pi, dt, MR, s));
  const int64_t lstride = (int64_t)MR * e.K;
  for (int l = 0; l < e.L; ++l) {
    const bool loc = (m.local_mask >> l) & 1u;
    GemmArgs g = gemm_base(e);
    g.A = e.xn;
    g.lda = D;
    g.W = m.wqkvg[l];
    g.w_group_stride = (int64_t)e.qkvg * D;
    g.ldw = D;
    g.C = e.qkvbuf;
    g.ldc = e.qkv;
    g.K = D;
    g.N = e.qkvg;
    g.n_main = e.qkv;
    g.row_mode = ROWS_PULSE;
    g.ctl = ctl;
    g.C2 = e.gate;
    g.ldc2 = e.H;
    g.bias = m.gate_bias[l];
    g.bias_group_stride = e.H;
    PULSAR_TIMED(PC_QKVG, wide ? launch_gemm_wide(g, dt, EPI_QKVG, e.P, MR, s)
                               : gemm(g, EPI_QKVG, e.P));
    QKPostArgs qa{};
    qa.ctl = ctl;
    qa.rows = rows;
    qa.qkv = e.qkvbuf;
    qa.ldq = e.qkv;
    qa.H = e.H;
    qa.Hkv = e.Hkv;
    qa.layer = l;
    qa.is_local = loc;
    qa.window = m.window;
    qa.base_seq_len = m.base_seq_len;
    qa.eps = m.rms_eps;
    qa.q_norm = m.q_norm[l];
    qa.k_norm = m.k_norm[l];
    qa.v_lambda = m.v_lambda[l];
    qa.v_first = e.v_first;
    qa.cos = loc ? m.rope_cos_local : m.rope_cos_global;
    qa.sin = loc ? m.rope_sin_local : m.rope_sin_global;
    qa.kv = e.kv;
    if (!fuse_post) PULSAR_TIMED(PC_QKPOST, launch_qk_post(qa, dt, MR, s));
    AttnArgs aa{};
    aa.ctl = ctl;
    aa.rows = rows;
    aa.qkv = e.qkvbuf;
    aa.ldq = e.qkv;
    aa.gate = e.gate;
    aa.out = e.attn_out;
    aa.units = units;
    aa.split_done = e.split_done;
    aa.max_units = e.B;
    aa.unit_rows = e.S;
    aa.part = e.part;
    aa.max_splits = e.max_splits;
    aa.max_splits_unit = e.max_splits_unit;
    aa.max_ctx = e.cfg.max_ctx;
    aa.H = e.H;
    aa.Hkv = e.Hkv;
    aa.layer = l;
    aa.is_local = loc;
    aa.window = m.window;
    aa.scale = 0.125f;
    aa.kv = e.kv;
    if (fuse_post) {
      aa.post = 1;
      aa.base_seq_len = m.base_seq_len;
      aa.eps = m.rms_eps;
      aa.q_norm = m.q_norm[l];
      aa.k_norm = m.k_norm[l];
      aa.v_lambda = m.v_lambda[l];
      aa.v_first = e.v_first;
      aa.cos = qa.cos;
      aa.sin = qa.sin;
    }
    PULSAR_TIMED(PC_ATTN, launch_attn_decode(aa, dt, MR, s));
    g = gemm_base(e);
    g.A = e.attn_out;
    g.lda = (int64_t)e.H * kHeadDim;
    g.W = m.wo[l];
    g.w_group_stride = (int64_t)D * e.H * kHeadDim;
    g.ldw = (int64_t)e.H * kHeadDim;
    g.C = e.h;
    g.ldc = D;
    g.K = e.H * kHeadDim;
    g.N = D;
    g.row_mode = ROWS_PULSE;
    g.ctl = ctl;
    PULSAR_TIMED(PC_WO, wide ? launch_gemm_wide(g, dt, EPI_RESID, e.P, MR, s)
                             : gemm(g, EPI_RESID, e.P));
    RouterArgs ra{};
    ra.ctl = ctl;
    ra.rows = rows;
    ra.x = e.h;
    ra.w = m.router[l];
    ra.bias = m.expert_bias[l];
    ra.E = e.E;
    ra.K = e.K;
    ra.D = D;
    ra.topk_idx = e.dec_topk + (int64_t)l * MR * e.K;
    ra.topk_w = e.topk_w;
    ra.lists = e.lists + (int64_t)l * e.E * lstride;
    ra.list_count = e.list_count + (int64_t)l * e.E;
    ra.list_stride = lstride;
    ra.norm_w = m.mlp_norm[l];
    ra.xn = e.xn;
    ra.eps = m.rms_eps;
    PULSAR_TIMED(PC_ROUTER, launch_norm_router(ra, dt, MR, s));
    // shared expert (group 0, all rows) + routed experts (assignment lists): gate/up + SwiGLU
    g = gemm_base(e);
    g.A = e.xn;
    g.lda = D;
    g.W = m.routed_gu[l];
    g.w_group_stride = (int64_t)2 * e.de * D;
    g.ldw = D;
    g.C = e.act_r;
    g.ldc = e.de;
    g.K = D;
    g.N = e.de;
    g.row_mode = ROWS_LIST;
    g.list = ra.lists;
    g.list_count = ra.list_count;
    g.list_stride = lstride;
    g.a_div = e.K;
    g.ctl = ctl;
    g.eager_w = eager_experts;
    g.a_rows = MR;
    g.a_rows0 = MR;
    if (wide) {
      // wide tiles: the shared expert over all rows, then the routed experts' lists
      GemmArgs gs = gemm_base(e);
      gs.A = e.xn;
      gs.lda = D;
      gs.W = m.shared_gu[l];
      gs.ldw = D;
      gs.C = e.act_s;
      gs.ldc = e.ds;
      gs.K = D;
      gs.N = e.ds;
      gs.row_mode = ROWS_ALL;
      gs.ctl = ctl;
      PULSAR_TIMED(PC_SHARED_GU, launch_gemm_wide(gs, dt, EPI_SWIGLU, 1, MR, s));
      PULSAR_TIMED(PC_ROUTED_GU, launch_gemm_wide(g, dt, EPI_SWIGLU, e.E, MR, s));
    } else {
      g.has_g0 = 1;
      g.K0 = D;
      g.A0 = e.xn;
      g.lda0 = D;
      g.W0 = m.shared_gu[l];
      g.ldw0 = D;
      g.C0 = e.act_s;
      g.ldc0 = e.ds;
      g.N0 = e.ds;
      PULSAR_TIMED(PC_ROUTED_GU, gemm(g, EPI_SWIGLU, e.E));
    }
    // shared + routed down projections
    g = gemm_base(e);
    g.A = e.act_r;
    g.lda = e.de;
    g.W = m.routed_down[l];
    g.w_group_stride = (int64_t)D * e.de;
    g.ldw = e.de;
    g.C = e.out_r;
    g.ldc = D;
    g.K = e.de;
    g.N = D;
    g.row_mode = ROWS_LIST;
    g.list = ra.lists;
    g.list_count = ra.list_count;
    g.list_stride = lstride;
    g.a_div = 1;
    g.ctl = ctl;
    if (!wide && (e.ds == e.de || e.ds == 2 * e.de)) {
      g.has_g0 = 1;
      g.K0 = e.ds;
      g.A0 = e.act_s;
      g.lda0 = e.ds;
      g.W0 = m.shared_down[l];
      g.ldw0 = e.ds;
      g.C0 = e.out_s;
      g.ldc0 = D;
      g.N0 = D;
      PULSAR_TIMED(PC_ROUTED_DOWN, gemm(g, EPI_STORE, e.E));
    } else {
      // the fused launch takes K0 = K or 2K for the shared group; other widths and wide
      // tiles: two launches
      PULSAR_TIMED(PC_ROUTED_DOWN, wide ? launch_gemm_wide(g, dt, EPI_STORE, e.E, MR, s)
                                        : gemm(g, EPI_STORE, e.E));
      GemmArgs gs = gemm_base(e);
      gs.A = e.act_s;
      gs.lda = e.ds;
      gs.W = m.shared_down[l];
      gs.ldw = e.ds;
      gs.C = e.out_s;
      gs.ldc = D;
      gs.K = e.ds;
      gs.N = D;
      gs.row_mode = ROWS_ALL;
      gs.ctl = ctl;
      PULSAR_TIMED(PC_SHARED_DOWN, wide ? launch_gemm_wide(gs, dt, EPI_STORE, 1, MR, s)
                                        : gemm(gs, EPI_STORE, 1));
    }
    CombineArgs ca{};
    ca.ctl = ctl;
    ca.rows = rows;
    ca.K = e.K;
    ca.D = D;
    ca.shared = e.out_s;
    ca.routed = e.out_r;
    ca.topk_w = e.topk_w;
    ca.routed_scale = m.routed_scale[l];
    ca.h = e.h;
    ca.next_norm = l + 1 < e.L ? m.attn_norm[l + 1] : nullptr;
    ca.xn = e.xn;
    ca.eps = m.rms_eps;
    if (fuse_post && l + 1 == e.L) {
      // bf16: the last layer's combine also does the pulse output (no separate launch)
      ca.h_in = e.h_in;
      ca.res_scale = m.res_scale;
      ca.hout_state = e.hout_state;
      ca.slots = e.S;
      ca.final_norm = m.final_norm;
      ca.xn_final = e.xn_final;
    }
    PULSAR_TIMED(PC_COMBINE, launch_moe_combine(ca, dt, MR, s));
  }
  if (!fuse_post) {
    PulseOutputArgs po{};
    po.ctl = ctl;
    po.rows = rows;
    po.D = D;
    po.slots = e.S;
    po.eps = m.rms_eps;
    po.h_in = e.h_in;
    po.h = e.h;
    po.res_scale = m.res_scale;
    po.hout_state = e.hout_state;
    po.final_norm = m.final_norm;
    po.xn_final = e.xn_final;
    PULSAR_TIMED(PC_OUTPUT, launch_pulse_output(po, dt, MR, s));
  }
  if (!head) return PULSAR_OK;
  GemmArgs g = gemm_base(e);
  g.A = e.xn_final;
  g.lda = D;
  g.W = m.lm_head ? m.lm_head : m.tok_emb;
  g.ldw = D;
  g.C = e.logits;
  g.ldc = e.V;
  g.K = D;
  g.N = e.V;
  g.row_mode = ROWS_LOGITS;
  g.ctl = ctl;
  g.softcap = m.softcap;
  if (wide_head)
    PULSAR_TIMED(PC_LMHEAD, launch_gemm_wide(g, dt, EPI_LOGITS, 1, MR, s));
  else
    PULSAR_TIMED(PC_LMHEAD, launch_gemm(g, dt, EPI_LOGITS, 1, MR, s));
  return PULSAR_OK;
}

// One step: a pass over the step's rows, sampling of its logits rows and the controller,
// which lays out the next step.
int enqueue_step(Engine& e, hipStream_t s) {
  PULSAR_TRY(enqueue_pass(e, e.ctl, e.rows, e.units, s));
  SampleArgs sa{};
  sa.ctl = e.ctl;
  sa.logits = e.logits;
  sa.lrow_seq = e.lrow_seq;
  sa.lrow_extra = e.lrow_extra;
  sa.extra_stride = e.G > 0 ? kMaxExtra : 1;
  sa.n_extra = sa.extra_stride;
  sa.lrow_ctr = e.G > 0 ? e.lrow_ctr : nullptr;
  sa.seen = e.seen;
  sa.state = e.state;
  sa.V = e.V;
  sa.greedy = e.cfg.temperature <= 1e-4f;
  sa.temperature = std::max(e.cfg.temperature, 1e-5f);
  sa.top_p = e.cfg.top_p;
  sa.rep_penalty = e.cfg.repetition_penalty;
  sa.seed = e.d_seed;
  sa.out_argmax = e.argmax;
  sa.out_draw = e.draw;
  sa.out_maxprob = e.cfg.early_exit ? e.maxprob : nullptr;
  PULSAR_TIMED(PC_SAMPLE, launch_sample(sa, e.dtype, e.max_rows, s));
  PULSAR_TRY(prof_delay(e, s));
  const int _pc = prof_mark(e, s);
  ControllerArgs co{};
  co.last_ctl = e.last_ctl;
  co.last_rows = e.last_rows;
  co.ctl = e.ctl;
  co.state = e.state;
  co.rows = e.rows;
  co.units = e.units;
  co.lrow_seq = e.lrow_seq;
  co.lrow_extra = e.lrow_extra;
  co.lrow_ctr = e.lrow_ctr;
  co.draft_len = e.G;
  co.seen = e.seen;
  co.out_tokens = e.tokens;
  co.out_kinds = e.kinds;
  co.argmax = e.argmax;
  co.draw = e.draw;
  co.stop_ids = e.stop_ids;
  co.n_stop = e.cfg.n_stop;
  co.B = e.B;
  co.V = e.V;
  co.n_pulses = e.P;
  co.max_new = e.cfg.max_new;
  co.speculative = e.cfg.speculative;
  co.all_logits = e.cfg.all_logits;
  co.prompt_len = e.prompt_len;
  co.early_exit = e.cfg.early_exit;
  co.maxprob = e.maxprob;
  co.exit_counts = e.exit_counts;
  co.exit_thr = e.cfg.early_exit_threshold;
  co.page_table = e.page_table;
  co.page_count = e.page_count;
  co.pool = e.pool;
  co.pool_pages = e.pool_pages;
  co.max_pages = e.max_pages;
  co.max_lrows = e.max_rows;
  PULSAR_TRY(launch_controller(co, s));
  prof_span(e, PC_CONTROL, _pc, prof_mark(e, s));
  return PULSAR_OK;
}

// Global-layer pages of a fresh cache holding positions [0, npos) of every sequence:
// sequence b gets pool pages [b * need, (b + 1) * need), need = ceil(npos / 64), the rest of
// its table names the spare page; the same state goes to the saved copies rewind restores.
int assign_prompt_pages(Engine& e, int npos, hipStream_t s) {
  const int need = (npos + kPage - 1) / kPage;
  PULSAR_REQUIRE((int64_t)e.B * need <= e.pool_pages,
                 "KV page pool too small for the prompts: " + std::to_string(e.B) + " x " +
                     std::to_string(need) + " pages > kv_pages " +
                     std::to_string(e.pool_pages));
  const size_t pt = (size_t)e.B * e.max_pages;
  std::vector<int32_t> table(pt, e.pool_pages), count(e.B, need);
  for (int b = 0; b < e.B; ++b)
    for (int p = 0; p < need; ++p) table[(size_t)b * e.max_pages + p] = b * need + p;
  const int32_t pool[2] = {e.B * need, 0};
  for (int32_t* dst : {e.page_table, e.page_table_save})
    PULSAR_CHECK_HIP(hipMemcpyAsync(dst, table.data(), 4 * pt, hipMemcpyHostToDevice, s));
  for (int32_t* dst : {e.page_count, e.page_count_save})
    PULSAR_CHECK_HIP(hipMemcpyAsync(dst, count.data(), 4 * (size_t)e.B, hipMemcpyHostToDevice, s));
  for (int32_t* dst : {e.pool, e.pool_save})
    PULSAR_CHECK_HIP(hipMemcpyAsync(dst, pool, 8, hipMemcpyHostToDevice, s));
  // the host vectors must outlive the copies
  PULSAR_CHECK_HIP(hipStreamSynchronize(s));
  return PULSAR_OK;
}

// Back to the pages the last prefill or fill_kv left (pages decoding took return to the
// pool).
int restore_pages(Engine& e, hipStream_t s) {
  const size_t pt = (size_t)e.B * e.max_pages;
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.page_table, e.page_table_save, 4 * pt,
                                  hipMemcpyDeviceToDevice, s));
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.page_count, e.page_count_save, 4 * (size_t)e.B,
                                  hipMemcpyDeviceToDevice, s));
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.pool, e.pool_save, 8, hipMemcpyDeviceToDevice, s));
  return PULSAR_OK;
}

// Pages for the positions of the block verify's units (unit b: sequence b's block), taken
// in order of request; when the pool is spent the entries keep naming the spare page and
// the spent flag is set. Reads the positions from the uploaded units, so a captured verify
// follows later uploads.
__global__ void kv_ensure_pages_kernel(const AttnUnit* units, int32_t* table, int32_t* count,
                                       int32_t* pool, int pool_pages, int max_pages, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const AttnUnit un = units[b];
  const int need = (un.pos0 + un.n - 1) / kPage + 1;
  const int have = count[un.seq];
  if (have >= need) return;
  const int n = need - have;
  const int first = take_pages(pool, n, pool_pages);
  if (first < 0) return;
  for (int i = 0; i < n; ++i) table[(int64_t)un.seq * max_pages + have + i] = first + i;
  count[un.seq] = need;
}

// Copy the sliding-window rings to their saved copies (restore = false) or back (restore =
// true). Decoding overwrites ring slots of prompt positions; the global layers' prompt
// positions are never written after prefill.
int save_rings(Engine& e, hipStream_t s, bool restore) {
  const size_t bytes = (size_t)e.es * e.B * e.Hkv * e.lcap * kHeadDim;
  for (int l = 0; l < e.L; ++l) {
    if (!((e.m.local_mask >> l) & 1u)) continue;
    void* ring[2] = {e.kv.k[l], e.kv.v[l]};
    void* save[2] = {e.ring_save_k[l], e.ring_save_v[l]};
    for (int i = 0; i < 2; ++i)
      PULSAR_CHECK_HIP(hipMemcpyAsync(restore ? ring[i] : save[i], restore ? save[i] : ring[i], bytes,
                                      hipMemcpyDeviceToDevice, s));
  }
  return PULSAR_OK;
}

// Draw the first token of every sequence from the prefill logits and (re)initialise the
// controller state; the KV cache of the prompt is left as prefill wrote it.
int first_token(Engine& e, uint64_t seed, hipStream_t s) {
  const int T = e.prompt_len, BT = e.B * T;
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.d_seed, &seed, 8, hipMemcpyHostToDevice, s));
  PULSAR_CHECK_HIP(hipMemsetAsync(e.state, 0, sizeof(SeqState) * e.B, s));
  PULSAR_CHECK_HIP(hipMemsetAsync(e.exit_counts, 0, 4 * 4 * (size_t)e.B, s));
  PULSAR_CHECK_HIP(hipMemsetAsync(e.seen, 0, 4 * (size_t)e.B * (e.V / 32), s));
  set_seen_kernel<<<(BT + 255) / 256, 256, 0, s>>>(e.p_ids, e.seen, T, e.V, BT);
  PULSAR_LAUNCH_CHECK();
  const StepCtl* lctl = e.p_ctl + (e.P - 1);
  SampleArgs sa{};
  sa.ctl = lctl;
  sa.logits = e.plogits;
  sa.lrow_seq = e.lrow_seq;
  sa.lrow_extra = e.lrow_extra;
  sa.extra_stride = 1;
  sa.n_extra = 0;
  sa.seen = e.seen;
  sa.state = e.state;
  sa.V = e.V;
  sa.greedy = e.cfg.temperature <= 1e-4f;
  sa.temperature = std::max(e.cfg.temperature, 1e-5f);
  sa.top_p = e.cfg.top_p;
  sa.rep_penalty = e.cfg.repetition_penalty;
  sa.seed = e.d_seed;
  sa.out_argmax = e.argmax;
  sa.out_draw = e.draw;
  std::vector<int32_t> lseq(e.max_rows, 0), lext(e.max_rows, -1);
  for (int b = 0; b < e.B; ++b) lseq[b] = b;
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.lrow_seq, lseq.data(), 4 * lseq.size(), hipMemcpyHostToDevice, s));
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.lrow_extra, lext.data(), 4 * lext.size(), hipMemcpyHostToDevice, s));
  PULSAR_TRY(launch_sample(sa, e.dtype, e.B, s));
  ControllerArgs co{};
  co.last_ctl = e.last_ctl;
  co.last_rows = e.last_rows;
  co.ctl = e.ctl;
  co.state = e.state;
  co.rows = e.rows;
  co.units = e.units;
  co.lrow_seq = e.lrow_seq;
  co.lrow_extra = e.lrow_extra;
  co.lrow_ctr = e.lrow_ctr;
  co.draft_len = e.G;
  co.seen = e.seen;
  co.out_tokens = e.tokens;
  co.out_kinds = e.kinds;
  co.argmax = e.argmax;
  co.draw = e.draw;
  co.stop_ids = e.stop_ids;
  co.n_stop = e.cfg.n_stop;
  co.B = e.B;
  co.V = e.V;
  co.n_pulses = e.P;
  co.max_new = e.cfg.max_new;
  co.speculative = e.cfg.speculative;
  co.all_logits = e.cfg.all_logits;
  co.init = 1;
  co.prompt_len = T;
  co.early_exit = e.cfg.early_exit;
  co.maxprob = e.maxprob;
  co.exit_counts = e.exit_counts;
  co.exit_thr = e.cfg.early_exit_threshold;
  co.page_table = e.page_table;
  co.page_count = e.page_count;
  co.pool = e.pool;
  co.pool_pages = e.pool_pages;
  co.max_pages = e.max_pages;
  co.max_lrows = e.max_rows;
  PULSAR_TRY(launch_controller(co, s));
  // host vectors above are read by the async copies: finish before they go out of scope
  PULSAR_CHECK_HIP(hipStreamSynchronize(s));
  return PULSAR_OK;
}

constexpr int kWidePromptLen = 128;

int prefill(Engine& e, const int32_t* host_ids, int Bq, int T, hipStream_t s) {
  const PulsarModelDesc& m = e.m;
  PULSAR_REQUIRE(Bq == e.B, "prefill batch must equal max_batch");
  PULSAR_REQUIRE(T >= 1 && T <= e.cfg.max_prompt, "prompt length out of range");
  const int D = e.D, dt = e.dtype, P = e.P;
  const int BT = Bq * T;
  for (int i = 0; i < BT; ++i)
    PULSAR_REQUIRE(host_ids[i] >= 0 && host_ids[i] < e.V, "prompt id out of vocabulary");
  // from here on the cache and the saved prefill state are being replaced: a prefill that
  // fails part way leaves nothing to step, rewind or verify
  e.prefilled = false;
  e.kv_ready = false;
  e.v_n = 0;
  PULSAR_TRY(assign_prompt_pages(e, T, s));
  e.prompt_len = T;
  // graph of a previous generation refers to the same buffers; it stays valid.
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.p_ids, host_ids, 4 * (size_t)BT, hipMemcpyHostToDevice, s));
  std::vector<RowDesc> rows((size_t)P * BT);
  std::vector<StepCtl> ctls(P);
  for (int k = 0; k < P; ++k) {
    for (int b = 0; b < Bq; ++b)
      for (int t = 0; t < T; ++t) {
        const int lrow = (k == P - 1 && t == T - 1) ? b : -1;
        rows[(size_t)k * BT + b * T + t] = RowDesc{b, 0, k, t, host_ids[b * T + t], lrow, -1, 0};
      }
    StepCtl c{};
    c.n_rows = BT;
    c.n_lrows = (k == P - 1) ? Bq : 0;
    c.pulse_start[k] = 0;
    c.pulse_count[k] = BT;
    ctls[k] = c;
  }
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.p_rows, rows.data(), sizeof(RowDesc) * rows.size(),
                                  hipMemcpyHostToDevice, s));
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.p_ctl, ctls.data(), sizeof(StepCtl) * P,
                                  hipMemcpyHostToDevice, s));
  PULSAR_CHECK_HIP(hipMemsetAsync(e.ctl, 0, sizeof(StepCtl), s));

  PULSAR_TRY(launch_prefill_stem(e.p_ids, m.tok_emb, m.anchor_norm, m.conv_w, e.xn, e.e_state,
                                 Bq, T, D, m.rms_eps, dt, s));
  const int64_t lstride = (int64_t)e.R * e.K;
  // Wide-tile GEMMs for prompts of kWidePromptLen tokens or more. The choice depends on the
  // prompt length only, so a sequence gets the same arithmetic alone or in a batch.
  const bool wide = T >= kWidePromptLen;
  auto gemm_rows = [&](const GemmArgs& g, int epi, int groups, int rows) {
    return wide ? launch_gemm_wide(g, dt, epi, groups, rows, s)
                : launch_gemm(g, dt, epi, groups, rows, s);
  };
  for (int k = 0; k < P; ++k) {
    const StepCtl* ctl = e.p_ctl + k;
    const RowDesc* prow = e.p_rows + (size_t)k * BT;
    PulseInputArgs pi{};
    pi.ctl = ctl;
    pi.rows = prow;
    pi.D = D;
    pi.rank = m.reinject_rank;
    pi.prefill = 1;
    pi.prefill_T = T;
    pi.eps = m.rms_eps;
    pi.tok_emb = m.tok_emb;
    pi.anchor_norm = m.anchor_norm;
    pi.conv_w = m.conv_w;
    pi.state_norm = m.state_norm;
    pi.step_emb = m.step_emb;
    pi.reinject_down = m.reinject_down;
    pi.reinject_up = m.reinject_up;
    pi.reinject_bias = m.reinject_bias;
    pi.e_state = e.e_state;
    pi.hout_state = e.hout_state;
    pi.h_in = e.h_in;
    pi.h = e.h;
    PULSAR_TRY(launch_pulse_input(pi, dt, BT, s));
    for (int l = 0; l < e.L; ++l) {
      const bool loc = (m.local_mask >> l) & 1u;
      NormArgs na{};
      na.ctl = ctl;
      na.rows = prow;
      na.x = e.h;
      na.ldx = D;
      na.w = m.attn_norm[l];
      na.w_pulse_stride = D;
      na.y = e.xn;
      na.D = D;
      na.eps = m.rms_eps;
      PULSAR_TRY(launch_norm_rows(na, dt, BT, s));
      GemmArgs g = gemm_base(e);
      g.A = e.xn;
      g.lda = D;
      g.W = m.wqkvg[l];
      g.w_group_stride = (int64_t)e.qkvg * D;
      g.ldw = D;
      g.C = e.qkvbuf;
      g.ldc = e.qkv;
      g.K = D;
      g.N = e.qkvg;
      g.n_main = e.qkv;
      g.row_mode = ROWS_PULSE;
      g.group_offset = k;
      g.ctl = ctl;
      g.C2 = e.gate;
      g.ldc2 = e.H;
      g.bias = m.gate_bias[l];
      g.bias_group_stride = e.H;
      PULSAR_TRY(gemm_rows(g, EPI_QKVG, 1, BT));
      QKPostArgs qa{};
      qa.ctl = ctl;
      qa.rows = prow;
      qa.qkv = e.qkvbuf;
      qa.ldq = e.qkv;
      qa.H = e.H;
      qa.Hkv = e.Hkv;
      qa.layer = l;
      qa.is_local = loc;
      qa.prefill = 1;
      qa.prefill_T = T;
      qa.window = m.window;
      qa.base_seq_len = m.base_seq_len;
      qa.eps = m.rms_eps;
      qa.q_norm = m.q_norm[l];
      qa.k_norm = m.k_norm[l];
      qa.v_lambda = m.v_lambda[l];
      qa.v_first = e.v_first;
      qa.cos = loc ? m.rope_cos_local : m.rope_cos_global;
      qa.sin = loc ? m.rope_sin_local : m.rope_sin_global;
      qa.kv = e.kv;
      PULSAR_TRY(launch_qk_post(qa, dt, BT, s));
      AttnArgs aa{};
      aa.ctl = ctl;
      aa.rows = prow;
      aa.qkv = e.qkvbuf;
      aa.ldq = e.qkv;
      aa.gate = e.gate;
      aa.out = e.attn_out;
      aa.H = e.H;
      aa.Hkv = e.Hkv;
      aa.layer = l;
      aa.is_local = loc;
      aa.window = m.window;
      aa.prefill_T = T;
      aa.scale = 0.125f;
      aa.kv = e.kv;
      PULSAR_TRY(launch_attn_prefill(aa, dt, Bq, s));
      g = gemm_base(e);
      g.A = e.attn_out;
      g.lda = (int64_t)e.H * kHeadDim;
      g.W = m.wo[l];
      g.w_group_stride = (int64_t)D * e.H * kHeadDim;
      g.ldw = (int64_t)e.H * kHeadDim;
      g.C = e.h;
      g.ldc = D;
      g.K = e.H * kHeadDim;
      g.N = D;
      g.row_mode = ROWS_PULSE;
      g.group_offset = k;
      g.ctl = ctl;
      PULSAR_TRY(gemm_rows(g, EPI_RESID, 1, BT));
      na.w = m.mlp_norm[l];
      PULSAR_TRY(launch_norm_rows(na, dt, BT, s));
      RouterArgs ra{};
      ra.x = e.xn;
      ra.w = m.router[l];
      ra.bias = m.expert_bias[l];
      ra.E = e.E;
      ra.K = e.K;
      ra.D = D;
      ra.pulse = k;
      ra.m_fixed = BT;
      ra.topk_idx = e.topk_idx;
      ra.topk_w = e.topk_w;
      PULSAR_TRY(launch_router_prefill(ra, dt, s));
      // capacity of a reference prefill call: N = T tokens of one sequence (src/model.py:1339-1342)
      const double avg = (double)T * e.K / e.E;
      const long raw = (long)std::ceil(avg * 1.25);
      const int C = (int)std::max<long>(32, ((raw + 31) / 32) * 32);
      // an expert keeps at most C tokens of each sequence
      const int list_max = (int)std::min<long>(BT, (long)Bq * C);
      PULSAR_CHECK_HIP(hipMemsetAsync(e.p_lcount, 0, 4 * (size_t)e.E, s));
      PULSAR_TRY(launch_prefill_capacity(e.topk_idx, e.topk_w, e.keep, e.p_lists, e.p_lcount,
                                         lstride, Bq, T, e.K, e.E, C, s));
      g = gemm_base(e);
      g.A = e.xn;
      g.lda = D;
      g.W = m.shared_gu[l];
      g.ldw = D;
      g.C = e.act_s;
      g.ldc = e.ds;
      g.K = D;
      g.N = e.ds;
      g.row_mode = ROWS_ALL;
      g.m_fixed = BT;
      PULSAR_TRY(gemm_rows(g, EPI_SWIGLU, 1, BT));
      g = gemm_base(e);
      g.A = e.xn;
      g.lda = D;
      g.W = m.routed_gu[l];
      g.w_group_stride = (int64_t)2 * e.de * D;
      g.ldw = D;
      g.C = e.act_r;
      g.ldc = e.de;
      g.K = D;
      g.N = e.de;
      g.row_mode = ROWS_LIST;
      g.list = e.p_lists;
      g.list_count = e.p_lcount;
      g.list_stride = lstride;
      g.a_div = e.K;
      PULSAR_TRY(gemm_rows(g, EPI_SWIGLU, e.E, list_max));
      g = gemm_base(e);
      g.A = e.act_s;
      g.lda = e.ds;
      g.W = m.shared_down[l];
      g.ldw = e.ds;
      g.C = e.out_s;
      g.ldc = D;
      g.K = e.ds;
      g.N = D;
      g.row_mode = ROWS_ALL;
      g.m_fixed = BT;
      PULSAR_TRY(gemm_rows(g, EPI_STORE, 1, BT));
      g = gemm_base(e);
      g.A = e.act_r;
      g.lda = e.de;
      g.W = m.routed_down[l];
      g.w_group_stride = (int64_t)D * e.de;
      g.ldw = e.de;
      g.C = e.out_r;
      g.ldc = D;
      g.K = e.de;
      g.N = D;
      g.row_mode = ROWS_LIST;
      g.list = e.p_lists;
      g.list_count = e.p_lcount;
      g.list_stride = lstride;
      g.a_div = 1;
      g.bias = reinterpret_cast<const char*>(m.routed_scale[l]) + (size_t)k * D * e.es;
      PULSAR_TRY(gemm_rows(g, EPI_SCALE, e.E, list_max));
      CombineArgs ca{};
      ca.m_fixed = BT;
      ca.pulse = k;
      ca.prefill = 1;
      ca.K = e.K;
      ca.D = D;
      ca.shared = e.out_s;
      ca.routed = e.out_r;
      ca.topk_w = e.topk_w;
      ca.keep = e.keep;
      ca.routed_scale = m.routed_scale[l];
      ca.h = e.h;
      PULSAR_TRY(launch_moe_combine(ca, dt, BT, s));
    }
    PulseOutputArgs po{};
    po.ctl = ctl;
    po.rows = prow;
    po.D = D;
    po.prefill = 1;
    po.prefill_T = T;
    po.eps = m.rms_eps;
    po.h_in = e.h_in;
    po.h = e.h;
    po.res_scale = m.res_scale;
    po.hout_state = e.hout_state;
    po.final_norm = m.final_norm;
    po.xn_final = e.xn_final;
    PULSAR_TRY(launch_pulse_output(po, dt, BT, s));
  }
  const StepCtl* lctl = e.p_ctl + (P - 1);
  GemmArgs g = gemm_base(e);
  g.A = e.xn_final;
  g.lda = D;
  g.W = m.lm_head ? m.lm_head : m.tok_emb;
  g.ldw = D;
  g.C = e.plogits;
  g.ldc = e.V;
  g.K = D;
  g.N = e.V;
  g.row_mode = ROWS_LOGITS;
  g.ctl = lctl;
  PULSAR_TRY(launch_gemm(g, dt, EPI_LOGITS_RAW, 1, Bq, s));
  // the prefill logits are also the readable "last logits" until the first step runs
  PULSAR_CHECK_HIP(hipMemcpyAsync(e.logits, e.plogits, 4 * (size_t)Bq * e.V,
                                  hipMemcpyDeviceToDevice, s));
  PULSAR_TRY(save_rings(e, s, false));
  PULSAR_TRY(first_token(e, e.cfg.seed, s));
  PULSAR_CHECK_HIP(hipStreamSynchronize(s));
  e.prefilled = true;
  e.kv_ready = true;
  return PULSAR_OK;
}

// Synthetic cache contents: every key and value element of every layer ~ N(0, 1), from a
// counter-based generator (SplitMix64 finaliser of (seed, layer, K/V, element), Box-Muller).
__host__ __device__ __forceinline__ uint64_t fill_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename T>
__global__ void __launch_bounds__(256) fill_normal_kernel(T* p, int64_t n, uint64_t seed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t h = fill_mix64(seed + 0x9E3779B97F4A7C15ull * (uint64_t)(i + 1));
    const float u1 = (float)((h >> 40) + 1) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    p[i] = from_f<T>(sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2));
  }
}

// Global layers: the value of element `inner` of sequence b's page p is keyed by its
// position in a per-sequence layout, ((b * max_pages + p) * page_elems + inner), whichever
// pool page holds it (fill_kv assigns sequence b the pool pages [b * need, (b + 1) * need)).
template <typename T>
__global__ void __launch_bounds__(256) fill_pages_kernel(T* p, int64_t n, int need,
                                                         int max_pages, int64_t page_elems,
                                                         uint64_t seed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t pool_page = i / page_elems, inner = i % page_elems;
    const int64_t b = pool_page / need, pg = pool_page % need;
    const int64_t key = (b * max_pages + pg) * page_elems + inner;
    const uint64_t h = fill_mix64(seed + 0x9E3779B97F4A7C15ull * (uint64_t)(key + 1));
    const float u1 = (float)((h >> 40) + 1) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    p[i] = from_f<T>(sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2));
  }
}

int fill_kv(Engine& e, int ctx, uint64_t seed, hipStream_t s) {
  PULSAR_REQUIRE(ctx >= 1 && ctx + 1 <= e.cfg.max_ctx, "engine_fill_kv: 1 <= ctx < max_ctx");
  e.prefilled = false;
  e.kv_ready = false;
  e.v_n = 0;
  PULSAR_TRY(assign_prompt_pages(e, ctx, s));
  const int need = (ctx + kPage - 1) / kPage;
  const int64_t page_elems = (int64_t)e.Hkv * kPage * kHeadDim;
  const size_t local_elems = (size_t)e.B * e.Hkv * e.lcap * kHeadDim;
  for (int l = 0; l < e.L; ++l) {
    const bool loc = (e.m.local_mask >> l) & 1u;
    const int64_t n = loc ? (int64_t)local_elems : (int64_t)e.B * need * page_elems;
    for (int kvi = 0; kvi < 2; ++kvi) {
      void* p = kvi == 0 ? e.kv.k[l] : e.kv.v[l];
      const uint64_t sd = fill_mix64(seed ^ (uint64_t)(2 * l + kvi + 1));
      const unsigned grid = (unsigned)std::min<int64_t>(8192, (n + 255) / 256);
      if (loc) {
        if (e.dtype == PULSAR_BF16)
          fill_normal_kernel<bf16><<<grid, 256, 0, s>>>(reinterpret_cast<bf16*>(p), n, sd);
        else
          fill_normal_kernel<float><<<grid, 256, 0, s>>>(reinterpret_cast<float*>(p), n, sd);
      } else if (e.dtype == PULSAR_BF16) {
        fill_pages_kernel<bf16><<<grid, 256, 0, s>>>(reinterpret_cast<bf16*>(p), n, need,
                                                     e.max_pages, page_elems, sd);
      } else {
        fill_pages_kernel<float><<<grid, 256, 0, s>>>(reinterpret_cast<float*>(p), n, need,
                                                      e.max_pages, page_elems, sd);
      }
      PULSAR_LAUNCH_CHECK();
    }
  }
  PULSAR_CHECK_HIP(hipStreamSynchronize(s));
  e.prompt_len = ctx;
  e.kv_ready = true;
  e.prefilled = false;  // no prefill logits: decoding needs a prefill
  e.v_n = 0;
  return PULSAR_OK;
}

// Block verify (draft-block mode's verify, and the verify microbenchmark): n tokens per
// sequence at positions prompt_len .. prompt_len + n - 1 run every pulse, pulse k as one
// pass over the B*n rows (row b*n + i = token i of sequence b, state slot i); a row
// attends the cache and the block's pulse-k keys at positions <= its own. The last pass
// computes logits for every row (readable as the step logits, row b*n + i). The
// controller state is not touched; the keys/values of the block positions are
// overwritten. host_tokens == nullptr re-runs the last uploaded block.
int verify(Engine& e, const int32_t* host_tokens, int n, int use_graph, hipStream_t s) {
  PULSAR_REQUIRE(e.kv_ready, "engine_verify: prefill or fill_kv first");
  const int P = e.P, B = e.B, MR = e.max_rows;
  // re-running needs a block uploaded since the last prefill / fill_kv: the row, control
  // and unit buffers are uninitialised (or describe other positions) until then
  PULSAR_REQUIRE(host_tokens || e.v_n > 0,
                 "engine_verify: no block uploaded since the last prefill or fill_kv");
  PULSAR_REQUIRE(host_tokens || e.prompt_len + e.v_n <= e.cfg.max_ctx,
                 "engine_verify: block past max_ctx");
  if (host_tokens) {
    PULSAR_REQUIRE(n >= 1 && n <= e.S,
                   "engine_verify: 1 <= n <= rows per sequence (draft_len + 1, or 2)");
    PULSAR_REQUIRE(e.prompt_len + n <= e.cfg.max_ctx, "engine_verify: block past max_ctx");
    for (int i = 0; i < B * n; ++i)
      PULSAR_REQUIRE(host_tokens[i] >= 0 && host_tokens[i] < e.V,
                     "engine_verify: token id out of vocabulary");
    {
      // the block's global-layer pages must come from the pool: a block the pool cannot hold
      // fails here rather than attending and writing the spare page
      std::vector<int32_t> have(B);
      int32_t pool[2] = {0, 0};
      PULSAR_CHECK_HIP(hipMemcpyAsync(have.data(), e.page_count, 4 * (size_t)B,
                                      hipMemcpyDeviceToHost, s));
      PULSAR_CHECK_HIP(hipMemcpyAsync(pool, e.pool, 8, hipMemcpyDeviceToHost, s));
      PULSAR_CHECK_HIP(hipStreamSynchronize(s));
      const int need = (e.prompt_len + n - 1) / kPage + 1;
      int64_t more = 0;
      for (int b = 0; b < B; ++b) more += std::max(0, need - have[b]);
      PULSAR_REQUIRE(pool[0] + more <= e.pool_pages,
                     "engine_verify: KV page pool too small for the block: " +
                         std::to_string(more) + " more pages needed, " +
                         std::to_string(std::max(0, e.pool_pages - pool[0])) + " left");
    }
    const int pos = e.prompt_len, BN = B * n;
    std::vector<RowDesc> rows((size_t)P * MR, RowDesc{0, 0, 0, 0, 0, -1, -1, 0});
    std::vector<StepCtl> ctls(P);
    std::vector<AttnUnit> units((size_t)P * B);
    for (int k = 0; k < P; ++k) {
      for (int b = 0; b < B; ++b) {
        AttnUnit un{};
        un.seq = b;
        un.n = n;
        un.pos0 = pos;
        for (int i = 0; i < kMaxBlock; ++i) un.row[i] = i < n ? b * n + i : -1;
        for (int i = 0; i < n; ++i) {
          const int r = b * n + i;
          rows[(size_t)k * MR + r] =
              RowDesc{b, i, k, pos + i, host_tokens[r], k == P - 1 ? r : -1, -1, i};
        }
        units[(size_t)k * B + b] = un;
      }
      StepCtl c{};
      c.n_rows = BN;
      c.n_lrows = k == P - 1 ? BN : 0;
      c.pulse_start[k] = 0;
      c.pulse_count[k] = BN;
      c.n_units = B;
      c.active = B;
      ctls[k] = c;
    }
    PULSAR_CHECK_HIP(hipMemcpyAsync(e.v_rows, rows.data(), sizeof(RowDesc) * rows.size(),
                                    hipMemcpyHostToDevice, s));
    PULSAR_CHECK_HIP(hipMemcpyAsync(e.v_ctl, ctls.data(), sizeof(StepCtl) * P,
                                    hipMemcpyHostToDevice, s));
    PULSAR_CHECK_HIP(hipMemcpyAsync(e.v_units, units.data(), sizeof(AttnUnit) * units.size(),
                                    hipMemcpyHostToDevice, s));
    // the host vectors must outlive the copies
    PULSAR_CHECK_HIP(hipStreamSynchronize(s));
    e.v_n = n;
  }
  auto passes = [&](hipStream_t st) -> int {
    // pages for the block's positions (a no-op once taken)
    kv_ensure_pages_kernel<<<(B + 63) / 64, 64, 0, st>>>(e.v_units, e.page_table,
                                                         e.page_count, e.pool, e.pool_pages,
                                                         e.max_pages, B);
    PULSAR_LAUNCH_CHECK();
    for (int k = 0; k < P; ++k)
      PULSAR_TRY(enqueue_pass(e, e.v_ctl + k, e.v_rows + (size_t)k * MR, e.v_units + (size_t)k * B,
                              st, k == P - 1));  // logits rows: the last pulse's only
    return PULSAR_OK;
  };
  if (!use_graph || e.prof_on) {
    PULSAR_TRY(passes(s));
    return prof_collect(e, s);
  }
  if (!e.vexec) {
    hipStream_t cs = e.capture_stream;
    PULSAR_CHECK_HIP(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal));
    const int rc = passes(cs);
    hipGraph_t gr = nullptr;
    const hipError_t ce = hipStreamEndCapture(cs, &gr);
    if (rc != PULSAR_OK) {
      if (gr) hipGraphDestroy(gr);
      return rc;
    }
    if (ce != hipSuccess)
      return fail(PULSAR_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(ce));
    e.vgraph = gr;
    PULSAR_CHECK_HIP(hipGraphInstantiate(&e.vexec, gr, nullptr, nullptr, 0));
  }
  PULSAR_CHECK_HIP(hipGraphLaunch(e.vexec, s));
  return PULSAR_OK;
}

// Steps per graph launch of runs of steps. A step is about 70 kernel nodes; the host cost
// of launching a graph can approach the step's GPU time on a slow host, so runs of steps
// launch kGraphSteps of them per graph (the step's work is decided on the device, so
// consecutive steps capture into one graph unchanged).
constexpr int kGraphSteps = 4;

// Capture n_steps steps into a graph (on the engine's own stream; launched on the caller's).
int capture_step(Engine& e, int n_steps, hipGraph_t* graph, hipGraphExec_t* exec) {
  hipStream_t cs = e.capture_stream;
  PULSAR_CHECK_HIP(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal));
  int rc = PULSAR_OK;
  for (int i = 0; i < n_steps && rc == PULSAR_OK; ++i) rc = enqueue_step(e, cs);
  hipGraph_t gr = nullptr;
  const hipError_t ce = hipStreamEndCapture(cs, &gr);
  if (rc != PULSAR_OK) {
    if (gr) hipGraphDestroy(gr);
    return rc;
  }
  if (ce != hipSuccess)
    return fail(PULSAR_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(ce));
  *graph = gr;
  PULSAR_CHECK_HIP(hipGraphInstantiate(exec, gr, nullptr, nullptr, 0));
  return PULSAR_OK;
}

int step(Engine& e, int n, int use_graph, hipStream_t s) {
  PULSAR_REQUIRE(e.prefilled, "engine: prefill before stepping");
  if (!use_graph || e.prof_on) {
    for (int i = 0; i < n; ++i) {
      PULSAR_TRY(enqueue_step(e, s));
      PULSAR_TRY(prof_collect(e, s));
    }
    return PULSAR_OK;
  }
  if (!e.exec) PULSAR_TRY(capture_step(e, 1, &e.graph, &e.exec));
  int i = 0;
  if (n >= kGraphSteps) {
    if (!e.exec_multi) PULSAR_TRY(capture_step(e, kGraphSteps, &e.graph_multi, &e.exec_multi));
    for (; i + kGraphSteps <= n; i += kGraphSteps)
      PULSAR_CHECK_HIP(hipGraphLaunch(e.exec_multi, s));
  }
  for (; i < n; ++i) PULSAR_CHECK_HIP(hipGraphLaunch(e.exec, s));
  return PULSAR_OK;
}

}  // namespace

}  // namespace pulsar

using namespace pulsar;

extern "C" {

int pulsar_engine_create(const PulsarModelDesc* model, const PulsarEngineConfig* cfg,
                         void** handle) {
  PULSAR_REQUIRE(model && cfg && handle, "engine_create: null argument");
  Engine* e = nullptr;
  PULSAR_TRY(create(*model, *cfg, &e));
  *handle = e;
  return PULSAR_OK;
}

int pulsar_engine_destroy(void* handle) {
  delete reinterpret_cast<Engine*>(handle);
  return PULSAR_OK;
}

int pulsar_engine_prefill(void* handle, const int32_t* host_ids, int32_t B, int32_t T,
                          hipStream_t stream) {
  PULSAR_REQUIRE(handle && host_ids, "engine_prefill: null argument");
  return prefill(*reinterpret_cast<Engine*>(handle), host_ids, B, T, stream);
}

int pulsar_engine_step(void* handle, int32_t n_steps, int32_t use_graph, hipStream_t stream) {
  PULSAR_REQUIRE(handle, "engine_step: null handle");
  return step(*reinterpret_cast<Engine*>(handle), n_steps, use_graph, stream);
}

int pulsar_engine_generate(void* handle, int32_t max_steps, int32_t check_every,
                           hipStream_t stream, int32_t* steps_run) {
  PULSAR_REQUIRE(handle && check_every >= 1, "engine_generate: bad argument");
  Engine& e = *reinterpret_cast<Engine*>(handle);
  // Steps go out in batches of check_every. Each batch is followed by a copy of the control
  // block and the sequences' states into pinned host memory and an event. While the host
  // waits for one batch's readback, the next batch is already queued whenever that wait's
  // predecessor proved the work outlasts it, so the GPU does not idle between batches: with
  // no stop ids a live sequence still owes rem = max_new - produced tokens. In the
  // draft-block mode the round in flight can emit up to draft_len + 1 of them in one step
  // (a verify's last pulse), and every later round takes at least one step per token (a
  // round of g drafts is g + 2 or more steps for at most g + 1 tokens), so at least
  // max(1, rem - draft_len) steps remain; otherwise at least one step per two tokens. Near
  // the end, and with stop ids, each batch is checked before the next one goes out, so no
  // step runs past the last live sequence's batch.
  const size_t rb = sizeof(StepCtl) + sizeof(SeqState) * (size_t)e.B;
  if (!e.host_rb) {
    PULSAR_CHECK_HIP(hipHostMalloc(&e.host_rb, 2 * rb));
    for (hipEvent_t& ev : e.rb_ev) PULSAR_CHECK_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  }
  const int G = e.cfg.draft_len;
  int launched = 0, checked = 0, bound = 0;
  int q_n = 0, q_head = 0, q_steps[2] = {0, 0};  // queued readbacks, oldest first
  auto launch = [&](int n) -> int {
    PULSAR_TRY(step(e, n, 1, stream));
    launched += n;
    const int k = (q_head + q_n) & 1;
    char* dst = reinterpret_cast<char*>(e.host_rb) + k * rb;
    PULSAR_CHECK_HIP(hipMemcpyAsync(dst, e.ctl, sizeof(StepCtl), hipMemcpyDeviceToHost, stream));
    PULSAR_CHECK_HIP(hipMemcpyAsync(dst + sizeof(StepCtl), e.state, sizeof(SeqState) * e.B,
                                    hipMemcpyDeviceToHost, stream));
    PULSAR_CHECK_HIP(hipEventRecord(e.rb_ev[k], stream));
    q_steps[k] = launched;
    ++q_n;
    return PULSAR_OK;
  };
  if (max_steps > 0) PULSAR_TRY(launch(std::min(check_every, max_steps)));
  while (q_n > 0) {
    const int n = std::min(check_every, max_steps - launched);
    if (n > 0 && q_n < 2 && launched - checked + n <= bound) PULSAR_TRY(launch(n));
    const int k = q_head;
    PULSAR_CHECK_HIP(hipEventSynchronize(e.rb_ev[k]));
    q_head ^= 1;
    --q_n;
    checked = q_steps[k];
    const char* src = reinterpret_cast<const char*>(e.host_rb) + k * rb;
    const StepCtl* c = reinterpret_cast<const StepCtl*>(src);
    const SeqState* st = reinterpret_cast<const SeqState*>(src + sizeof(StepCtl));
    if (c->active == 0) break;
    int rem = 0;
    if (e.cfg.n_stop == 0)
      for (int b = 0; b < e.B; ++b)
        if (!st[b].done) rem = std::max(rem, st[b].max_new - st[b].produced);
    // steps that certainly still have a live sequence (see above)
    bound = G > 0 ? (rem > G ? rem - G : (rem > 0 ? 1 : 0)) : rem / 2;
    if (q_n == 0 && launched < max_steps) PULSAR_TRY(launch(std::min(check_every, max_steps - launched)));
  }
  // a batch queued behind the last readback (never, when the bound holds) finishes first
  if (q_n > 0) PULSAR_CHECK_HIP(hipEventSynchronize(e.rb_ev[(q_head + q_n - 1) & 1]));
  if (steps_run) *steps_run = launched;
  return PULSAR_OK;
}

int pulsar_engine_verify(void* handle, const int32_t* host_tokens, int32_t n, int32_t use_graph,
                         hipStream_t stream) {
  PULSAR_REQUIRE(handle, "engine_verify: null handle");
  return verify(*reinterpret_cast<Engine*>(handle), host_tokens, n, use_graph, stream);
}

int pulsar_engine_fill_kv(void* handle, int32_t ctx, uint64_t seed, hipStream_t stream) {
  PULSAR_REQUIRE(handle, "engine_fill_kv: null handle");
  return fill_kv(*reinterpret_cast<Engine*>(handle), ctx, seed, stream);
}

int pulsar_engine_rewind(void* handle, uint64_t seed, hipStream_t stream) {
  PULSAR_REQUIRE(handle, "engine_rewind: null handle");
  Engine& e = *reinterpret_cast<Engine*>(handle);
  PULSAR_REQUIRE(e.prefilled, "engine_rewind: prefill first");
  PULSAR_TRY(save_rings(e, stream, true));
  PULSAR_TRY(restore_pages(e, stream));
  return first_token(e, seed, stream);
}

int pulsar_engine_profile(void* handle, int32_t enable) {
  PULSAR_REQUIRE(handle, "engine_profile: null handle");
  Engine& e = *reinterpret_cast<Engine*>(handle);
  e.prof_on = enable != 0;
  if (e.prof_on) {
    for (int i = 0; i < PULSAR_PROF_CLASSES; ++i) {
      e.prof_ms[i] = 0.0;
      e.prof_n[i] = 0;
    }
    e.spans.clear();
    e.ev_used = 0;
  }
  return PULSAR_OK;
}

int pulsar_engine_profile_read(void* handle, double* host_ms, int64_t* host_launches) {
  PULSAR_REQUIRE(handle && host_ms && host_launches, "engine_profile_read: null argument");
  Engine& e = *reinterpret_cast<Engine*>(handle);
  for (int i = 0; i < PULSAR_PROF_CLASSES; ++i) {
    host_ms[i] = e.prof_ms[i];
    host_launches[i] = e.prof_n[i];
  }
  return PULSAR_OK;
}

int pulsar_engine_read(void* handle, int32_t what, void* host_dst, int64_t bytes,
                       hipStream_t stream) {
  PULSAR_REQUIRE(handle && host_dst && bytes >= 0, "engine_read: bad argument");
  Engine& e = *reinterpret_cast<Engine*>(handle);
  const void* src = nullptr;
  int64_t cap = 0;
  switch (what) {
    case PULSAR_BUF_TOKENS:
      src = e.tokens;
      cap = 4ll * e.B * std::max(1, e.cfg.max_new);
      break;
    case PULSAR_BUF_SEQSTATE:
      src = e.state;
      cap = (int64_t)sizeof(SeqState) * e.B;
      break;
    case PULSAR_BUF_LOGITS:
      src = e.logits;
      cap = 4ll * std::max(e.max_rows, e.B) * e.V;
      break;
    case PULSAR_BUF_ROWS:
      src = e.rows;
      cap = (int64_t)sizeof(RowDesc) * e.max_rows;
      break;
    case PULSAR_BUF_CTL:
      src = e.ctl;
      cap = sizeof(StepCtl);
      break;
    case PULSAR_BUF_LAST_ROWS:
      src = e.last_rows;
      cap = (int64_t)sizeof(RowDesc) * e.max_rows;
      break;
    case PULSAR_BUF_LAST_CTL:
      src = e.last_ctl;
      cap = sizeof(StepCtl);
      break;
    case PULSAR_BUF_EXPERT_COUNTS:
      src = e.list_count;
      cap = 4ll * e.L * e.E;
      break;
    case PULSAR_BUF_EXIT_COUNTS:
      src = e.exit_counts;
      cap = 16ll * e.B;
      break;
    case PULSAR_BUF_KV_LAYOUT: {
      const int32_t layout[4] = {e.lcap, e.max_pages, kPage, e.Hkv};
      PULSAR_REQUIRE(bytes <= (int64_t)sizeof(layout), "engine_read: more bytes than the buffer holds");
      std::memcpy(host_dst, layout, bytes);
      return PULSAR_OK;
    }
    case PULSAR_BUF_KV_PAGES: {
      int32_t pool[2] = {0, 0};
      PULSAR_CHECK_HIP(hipMemcpyAsync(pool, e.pool, 8, hipMemcpyDeviceToHost, stream));
      PULSAR_CHECK_HIP(hipStreamSynchronize(stream));
      const int32_t info[3] = {e.pool_pages, std::min(pool[0], e.pool_pages), pool[1]};
      PULSAR_REQUIRE(bytes <= (int64_t)sizeof(info), "engine_read: more bytes than the buffer holds");
      std::memcpy(host_dst, info, bytes);
      return PULSAR_OK;
    }
    case PULSAR_BUF_TOKEN_KINDS:
      src = e.kinds;
      cap = 4ll * e.B * std::max(1, e.cfg.max_new);
      break;
    case PULSAR_BUF_TOPK_IDX:
      src = e.dec_topk;
      cap = 4ll * e.L * e.max_rows * e.K;
      break;
    default:
      return fail(PULSAR_ERR_INVALID, "engine_read: unknown buffer");
  }
  PULSAR_REQUIRE(bytes <= cap, "engine_read: more bytes than the buffer holds");
  PULSAR_CHECK_HIP(hipMemcpyAsync(host_dst, src, bytes, hipMemcpyDeviceToHost, stream));
  PULSAR_CHECK_HIP(hipStreamSynchronize(stream));
  return PULSAR_OK;
}

int64_t pulsar_sample_workspace_bytes(int32_t n_seq) {
  return n_seq < 0 ? -1 : (int64_t)sample_workspace_bytes(n_seq);
}

int pulsar_sample_rows(const float* logits, int32_t n_rows, int32_t V, int32_t dtype,
                       const uint32_t* seen, const int32_t* row_seq, const int32_t* row_extra,
                       const uint32_t* seq_ctr, int32_t n_seq, uint64_t seed, float temperature,
                       float top_p, float repetition_penalty, int32_t greedy, int32_t* out_argmax,
                       int32_t* out_draw, void* workspace, hipStream_t stream) {
  PULSAR_REQUIRE(logits && seen && row_seq && row_extra && seq_ctr && out_argmax && out_draw &&
                     workspace,
                 "sample_rows: null argument");
  PULSAR_REQUIRE(n_rows >= 0 && n_seq >= 1, "sample_rows: n_rows >= 0 and n_seq >= 1");
  PULSAR_REQUIRE(dtype == PULSAR_BF16 || dtype == PULSAR_F32, "sample_rows: dtype");
  PULSAR_REQUIRE(temperature > 0.f && top_p > 0.f && top_p <= 1.f && repetition_penalty > 0.f,
                 "sample_rows: temperature > 0, 0 < top_p <= 1, repetition_penalty > 0");
  if (n_rows == 0) return PULSAR_OK;
  return launch_sample_rows(logits, n_rows, V, dtype, seen, row_seq, row_extra, seq_ctr, n_seq,
                            seed, temperature, top_p, repetition_penalty, greedy, out_argmax,
                            out_draw, workspace, stream);
}

}  // extern "C"
