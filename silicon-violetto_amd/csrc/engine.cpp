// engine.cpp — the host side of libsv_verify: the C ABI of include/sv_verify.h.
//
// Kernel-level calls wrap the launchers. The engine mirrors the reference's Engine
// (engine/src/engine.rs), its planner (engine/src/engine/plan.rs), page pool (kv.rs),
// buffers (buffers.rs) and encoder (encode.rs): it owns the KV cache and the GPU-resident
// sequence state, lays out a step, encodes it on its HIP stream (or captures it once into a
// HIP graph and replays it), and reads back what a synchronous step returns.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "layers.h"
#include "sv_internal.h"

namespace sv {

static thread_local std::string g_error;

sv_status fail(sv_status code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

sv_status check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return SV_OK;
  return fail(SV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

sv_status check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

}  // namespace sv

using namespace sv;

#define SV_TRY(x)                  \
  do {                             \
    const sv_status st_ = (x);     \
    if (st_ != SV_OK) return st_;  \
  } while (0)
#define SV_HIP(x, what) SV_TRY(check_hip((x), (what)))

extern "C" const char* sv_last_error(void) { return g_error.c_str(); }

// ---------------------------------------------------------------- kernel level

extern "C" sv_status sv_embed(void* stream, const sv_shape* shape, const uint16_t* d_table, uint32_t* d_tokens,
                              float* d_out, const uint32_t* d_tin, uint32_t* d_meta, const uint32_t* d_lens,
                              const uint32_t* d_feed, const uint32_t* d_tree, uint32_t* d_vis, uint32_t n) {
  return embed_launch((hipStream_t)stream, shape, d_table, d_tokens, d_tokens, d_out, d_tin, d_meta, d_lens, d_feed,
                      d_tree, d_vis, n);
}

extern "C" sv_status sv_rmsnorm_rows(void* stream, const float* d_in, const uint32_t* d_rows, float* d_out, uint32_t n,
                                     uint32_t hidden) {
  if (hidden == 0) return fail(SV_ERR_ARG, "rmsnorm_rows: hidden 0");
  return rmsnorm_rows_launch((hipStream_t)stream, d_in, d_rows, d_out, n, hidden);
}

extern "C" size_t sv_matmul_workspace_bytes(uint32_t n, uint32_t m, uint32_t k) { return matmul_ws_bytes(n, m, k); }

extern "C" sv_status sv_matmul(void* stream, const sv_matrix* w, const float* d_x, const uint32_t* d_x_rows,
                               float* d_y, const float* d_base, float* d_aux, const sv_mat_args* a, void* d_workspace,
                               size_t workspace_bytes) {
  return matmul_launch((hipStream_t)stream, w, d_x, d_x_rows, d_y, d_base, d_aux, a, d_workspace, workspace_bytes);
}

extern "C" sv_status sv_pack_matrix(void* stream, const sv_matrix* src, void* d_dst, sv_matrix* out) {
  return pack_matrix((hipStream_t)stream, src, d_dst, out);
}

extern "C" size_t sv_attn_workspace_bytes(const sv_shape* shape, uint32_t n_runs, uint32_t max_splits,
                                          uint32_t max_run) {
  if (!shape) return 0;
  return attn_ws_bytes(shape, n_runs, max_splits, max_run);
}

extern "C" sv_status sv_attn_verify(void* stream, const sv_shape* shape, const float* d_qkv, const uint32_t* d_meta,
                                    uint16_t* d_k_cache, uint16_t* d_v_cache, const uint32_t* d_page_table,
                                    const float* d_rope, const sv_kv_args* kv, const sv_attn_args* args,
                                    const uint32_t* d_runs, uint32_t n_runs, uint32_t max_run, const uint32_t* d_vis,
                                    float* d_out, void* d_workspace, size_t workspace_bytes,
                                    const sv_attn_extras* extras) {
  return attn_launch((hipStream_t)stream, shape, d_qkv, d_meta, d_k_cache, d_v_cache, d_page_table, d_rope, kv, args,
                     d_runs, n_runs, max_run, d_vis, d_out, d_workspace, workspace_bytes, 3, nullptr, true, extras);
}

extern "C" sv_status sv_mudd(void* stream, const float* d_cur, const float* d_tap0, const float* d_tap1,
                             const float* d_dense1, const float* d_mix, float* d_out_attn, float* d_out_base, uint32_t n,
                             uint32_t hidden) {
  return mudd_launch((hipStream_t)stream, d_cur, d_tap0, d_tap1, d_dense1, d_mix, d_out_attn, d_out_base, n, hidden);
}

extern "C" size_t sv_attn_noalloc_max_bytes(void) { return attn_scratch_bytes(); }

extern "C" sv_status sv_attn_verify_noalloc(void* stream, const sv_shape* shape, const float* d_qkv,
                                            const uint32_t* d_meta, uint16_t* d_k_cache, uint16_t* d_v_cache,
                                            const uint32_t* d_page_table, const float* d_rope, const sv_kv_args* kv,
                                            const sv_attn_args* args, const uint32_t* d_runs, uint32_t n_runs,
                                            uint32_t max_run, const uint32_t* d_vis, float* d_out) {
  return attn_launch_noalloc((hipStream_t)stream, shape, d_qkv, d_meta, d_k_cache, d_v_cache, d_page_table, d_rope, kv,
                             args, d_runs, n_runs, max_run, d_vis, d_out);
}

extern "C" sv_status sv_sample(void* stream, const float* d_logits, const sv_sample_row* d_rows, uint32_t* d_out,
                               const uint32_t* d_meta, uint32_t n_rows, uint32_t vocab) {
  return sample_launch((hipStream_t)stream, d_logits, d_rows, d_out, d_meta, n_rows, vocab);
}

extern "C" sv_status sv_accept(void* stream, const sv_run_in* d_runs, const uint32_t* d_tokens, uint32_t* d_out,
                               uint32_t* d_lens, uint32_t* d_feed, sv_gen_state* d_gen, uint32_t* d_emitted,
                               uint32_t nruns, const uint32_t* d_tree, uint32_t* d_path, uint32_t* d_path_len,
                               uint32_t* d_on_path) {
  return accept_launch((hipStream_t)stream, d_runs, d_tokens, d_out, d_lens, d_feed, d_gen, d_emitted, nruns, d_tree,
                       d_path, d_path_len, d_on_path);
}

extern "C" sv_status sv_kv_compact(void* stream, const sv_shape* shape, const sv_run_in* d_runs, uint32_t nruns,
                                   const uint32_t* d_path, const uint32_t* d_path_len, const uint32_t* d_lens,
                                   uint16_t* d_k_cache, uint16_t* d_v_cache, const uint32_t* d_page_table,
                                   const sv_kv_args* kv) {
  return kv_compact_launch((hipStream_t)stream, shape, d_runs, nruns, d_path, d_path_len, d_lens, d_k_cache, d_v_cache,
                           d_page_table, kv);
}

extern "C" sv_status sv_draft_top(void* stream, const float* d_logits, const uint32_t* d_vocab, const uint32_t* d_tin,
                                  uint32_t* d_cand, float* d_cand_q, uint32_t n_rows, uint32_t nv, float inv_t,
                                  uint32_t ncand) {
  return draft_top_launch((hipStream_t)stream, d_logits, d_vocab, d_tin, d_cand, d_cand_q, n_rows, nv, inv_t, ncand);
}

extern "C" sv_status sv_draft_tree(void* stream, const uint32_t* d_blocks, uint32_t nblocks, const uint32_t* d_tin,
                                   const uint32_t* d_cand, const float* d_cand_q, uint32_t* d_feed, uint32_t* d_tree,
                                   uint32_t ncand) {
  return draft_tree_launch((hipStream_t)stream, d_blocks, nblocks, d_tin, d_cand, d_cand_q, d_feed, d_tree, ncand);
}

extern "C" sv_status sv_tap_rows(void* stream, const float* d_in, float* d_out, uint32_t n, uint32_t hidden) {
  return tap_rows_launch((hipStream_t)stream, d_in, d_out, n, hidden);
}

extern "C" sv_status sv_draft_kv(void* stream, const sv_shape* shape, const float* d_kvp, const uint32_t* d_meta,
                                 const uint32_t* d_on_path, const float* d_rope, uint16_t* d_k_ring, uint16_t* d_v_ring,
                                 const uint32_t* d_page_table, const sv_kv_args* kv, uint32_t n, uint32_t n_layers) {
  return draft_kv_launch((hipStream_t)stream, shape, d_kvp, d_meta, d_on_path, d_rope, d_k_ring, d_v_ring, d_page_table,
                         kv, n, n_layers);
}

extern "C" sv_status sv_draft_ctx(void* stream, const float* d_ctx, const float* d_ctx_inv, const uint32_t* d_meta,
                                  const uint32_t* d_on_path, float* d_ring, uint32_t cr, uint32_t n, uint32_t hidden) {
  return draft_ctx_launch((hipStream_t)stream, d_ctx, d_ctx_inv, d_meta, d_on_path, d_ring, cr, n, hidden);
}

extern "C" sv_status sv_draft_embed(void* stream, const uint16_t* d_embed, const uint32_t* d_tin, const uint32_t* d_lens,
                                    const uint32_t* d_feed, const float* d_mask_emb, float* d_x, uint32_t* d_meta,
                                    uint32_t* d_tokens, const float* d_ring, float* d_last, uint32_t cr, uint32_t rows,
                                    uint32_t hidden) {
  return draft_embed_launch((hipStream_t)stream, d_embed, d_tin, d_lens, d_feed, d_mask_emb, d_x, d_meta, d_tokens, d_ring,
                            d_last, cr, rows, hidden);
}

extern "C" sv_status sv_draft_conv(void* stream, const float* d_x, const float* d_corr, uint32_t corr_w,
                                   const float* d_base, const uint32_t* d_tin, const float* d_resid, float* d_out,
                                   uint32_t rows, uint32_t hidden) {
  return draft_conv_launch((hipStream_t)stream, d_x, d_corr, corr_w, d_base, d_tin, d_resid, d_out, rows, hidden);
}

extern "C" sv_status sv_replay_draft(void* stream, const sv_run_in* d_runs, uint32_t nruns, const uint32_t* d_lens,
                                     uint32_t* d_feed, const uint32_t* d_trace, const uint32_t* d_trace_len,
                                     const sv_replay_args* ra, uint32_t* d_tree) {
  return replay_launch((hipStream_t)stream, d_runs, nruns, d_lens, d_feed, d_trace, d_trace_len, ra, d_tree);
}

// ---------------------------------------------------------------- the engine

namespace sv {
thread_local ProfEvents g_prof;
}

namespace {

// Attention split sizes considered (keys per workgroup: multiples of 128, one 32-key batch
// per wave and step of 128; at most 3968, the kernel's per-lane page-table prefetch).
constexpr uint32_t MIN_SPLIT = 128;
constexpr uint32_t MAX_SPLIT = 3968 / 128 * 128;

// Keys per split (plan.rs:156-164 decode_splits, re-derived for this device). The grid is
// max_splits x kv heads x runs; a run's splits past its context exit at once, so the work is
// the active workgroups: sum over runs of (its splits + the split of its new keys) x kv heads.
// Time model, fitted to measurements on MI355X (1-32 streams, 4k-64k keys, 5- and 16-row
// runs), in microseconds, with b = 32-key batches per wave (split / 128) and k = active
// workgroups per compute unit (rounded up):
//   one workgroup per compute unit: its dependent-load chain, 9.7 + 1.2 b;
//   more: they share the unit's throughput, k (F + 1.05 b), F = 5.3 (<= 32 columns per kv
//   head) or 19 (more: 4x the query, reduction and partial traffic per workgroup).
// The larger of the two; ties go to the smaller split. Contexts are counted at the plan's
// furthest replay (cached + extra keys).
uint32_t choose_split(const std::vector<uint32_t>& cached, uint32_t extra, uint32_t nkv, uint32_t max_run,
                      uint32_t group) {
  static const uint32_t cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256u;
    return (uint32_t)n;
  }();
  const double F = max_run * group <= 32 ? 5.3 : 19.0;
  uint32_t best = MIN_SPLIT;
  double best_t = 1e300;
  for (uint32_t split = MIN_SPLIT; split <= MAX_SPLIT; split += 128) {
    uint64_t active = 0;
    for (uint32_t c : cached) active += ((uint64_t)(c + extra + split - 1) / split + 1) * nkv;
    const double k = (double)((active + cus - 1) / cus), b = split / 128;
    const double t = std::max(9.7 + 1.2 * b, k * (F + 1.05 * b));
    if (t < best_t) best_t = t, best = split;
  }
  return best;
}

struct Plan {
  uint32_t n = 0, n_head = 0, n_runs = 0, branches = 0, max_run = 0, split = 0, max_splits = 0;
  uint32_t split_local = 0, max_splits_local = 0;  // sliding-window layers' splits
  uint32_t n_attn = 0;  // attention runs: each run's rows in runs of at most SV_MAX_RUN
  bool chunk = false;   // some run has more rows (a prompt chunk): new K/V are written first
  std::vector<uint32_t> slots;   // per run
  std::vector<uint32_t> counts;  // per run
  std::vector<uint32_t> verify;  // per run
  std::vector<uint32_t> inl;     // per attention run: first token, rows, slot (inline in the launch)
  // The drafter's blocks after the step (drafter.rs DraftRun): count, rows, longest, splits,
  // and per block (first row, rows, slot).
  uint32_t n_blocks = 0, d_rows = 0, d_max_run = 0, d_split = 0, d_max_splits = 0;
  std::vector<uint32_t> dinl;
  // Steps this plan may run (encodes, graph replays, profiled steps): each advances a run by at
  // most its row count, and every position it can reach has a reserved page.
  uint64_t budget = 0, issued = 0;
  // The persistent layer kernel runs the layers (layers.hip), with these parameters.
  bool persist = false;
  LayersParams lp{};
};

template <typename T>
sv_status dalloc(T** p, size_t count, const char* what) {
  *p = nullptr;
  if (count == 0) count = 1;
  SV_HIP(hipMalloc((void**)p, count * sizeof(T)), what);
  SV_HIP(hipMemset(*p, 0, count * sizeof(T)), what);
  return SV_OK;
}

}  // namespace

struct sv_engine {
  sv_engine_config cfg{};
  sv_shape sh{};
  hipStream_t stream = nullptr;
  const uint16_t* embed = nullptr;
  sv_matrix head_mat{};  // the head: the tied embedding or its own (tiled when the shape allows)
  bool own_head = false;
  // A head of its own in int8 groups under 64 (tools/convert.py's default, groups of 8): the
  // exact sum of two bf16 matrices, head_mat (hi) and head_lo; softcapped after both.
  sv_matrix head_lo{};
  void* head_lo_tiled = nullptr;
  std::vector<sv_layer> layers;  // as used: matrices repacked into the tiled layout where they fit it
  std::vector<bool> layer_set;
  std::vector<void*> packed;     // engine-owned tiled copies [layer * 4 + matrix]
  void* head_tiled = nullptr;    // tiled copy of the tied embedding for the head matmul
  uint32_t n_pages = 0, max_pages = 0, qkv_w = 0;
  // Rows per attention run: SV_MAX_COLS columns per kv head at most (16 rows up to 4 query
  // heads per kv head).
  uint32_t arun = SV_MAX_RUN;
  // Layer kinds (model.rs:116): each layer's index among the global or among the local layers.
  std::vector<uint8_t> is_local;
  std::vector<uint32_t> kv_index;
  uint32_t n_global = 0, n_local = 0, ring_pages = 0, n_lpages = 0;
  uint16_t* k_local = nullptr;
  uint16_t* v_local = nullptr;
  uint32_t* local_table = nullptr;  // cyclic: [slot][p] = slot ring_pages + p % ring_pages
  size_t local_elems = 0;
  // Model extras (value embeddings, MUDD) and the buffers MUDD routes the residual through.
  sv_model_extras extras{};
  float* h0 = nullptr;              // the embedding's rows (MUDD's first tap)
  float* tap[SV_MUDD_SITES] = {};   // outputs of the tap layers
  float* xattn = nullptr;           // MUDD's attention input
  float* rbase = nullptr;           // MUDD's residual base
  // sv_step_capture (engine.rs:318-355): the per-layer callback and the device buffers the
  // layers write their intermediates to (null: an ordinary step).
  struct Capture {
    sv_capture_fn fn = nullptr;
    void* user = nullptr;
    uint32_t* iota = nullptr;  // rows 0..n-1 for rmsnorm_rows
    float *resid_in = nullptr, *attn_in = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *sdpa = nullptr;
    float *attn_out = nullptr, *mlp_in = nullptr, *mlp_out = nullptr, *base = nullptr;
  };
  Capture* capture = nullptr;
  float* vdir = nullptr;            // XSA directions [n][NKV][D]
  // The drafter (drafter.rs): its matrices, the target's tapped rows, its rings (as the local
  // layers': pages behind a cyclic table) and its block rows' buffers.
  bool has_drafter = false;
  sv_drafter dr{};
  std::vector<sv_draft_layer> dlayers;
  float* tapbuf[SV_DRAFT_TAPS] = {};
  uint16_t* dk_ring = nullptr;
  uint16_t* dv_ring = nullptr;
  uint32_t* d_table = nullptr;
  uint32_t d_ring_pages = 0, d_n_pages = 0, d_max_pages = 0, d_cr = 0, d_rows_max = 0, d_corr_w = 0;
  float *d_ctx = nullptr, *d_ctx_inv = nullptr, *d_kvp = nullptr, *d_cring = nullptr, *d_last = nullptr,
        *d_x = nullptr, *d_qkv = nullptr, *d_inv = nullptr, *d_attn = nullptr, *d_mixed = nullptr, *d_act = nullptr,
        *d_cx = nullptr, *d_co = nullptr, *d_corr = nullptr, *d_corr_inv = nullptr, *d_logits = nullptr,
        *d_cand_q = nullptr;
  uint32_t *d_cand = nullptr, *d_meta = nullptr, *d_tokens = nullptr, *d_tin = nullptr, *d_vis = nullptr,
           *d_tiles = nullptr;
  std::vector<uint32_t> draft_rows;  // per slot: rows of its blocks (0: not drafted)
  std::vector<void*> d_packed;       // engine-owned tiled copies of the drafter's matrices
  sv_matrix d_head_lo{};             // with a head in small int8 groups: its lo part (d_w NULL: none)
  void free_drafter() {
    for (void* b : d_packed)
      if (b) (void)hipFree(b);
    d_packed.clear();
    d_head_lo = sv_matrix{};
    void* bufs[] = {dk_ring, dv_ring, d_table, d_ctx, d_ctx_inv, d_kvp, d_cring, d_last, d_x, d_qkv, d_inv, d_attn,
                    d_mixed, d_act, d_cx, d_co, d_corr, d_corr_inv, d_logits, d_cand_q, d_cand, d_meta, d_tokens,
                    d_tin, d_vis, d_tiles, tapbuf[0], tapbuf[1], tapbuf[2], tapbuf[3]};
    for (void* b : bufs)
      if (b) (void)hipFree(b);
    dk_ring = dv_ring = nullptr;
    d_table = d_cand = d_meta = d_tokens = d_tin = d_vis = d_tiles = nullptr;
    d_ctx = d_ctx_inv = d_kvp = d_cring = d_last = d_x = d_qkv = d_inv = d_attn = d_mixed = d_act = d_cx = d_co =
        d_corr = d_corr_inv = d_logits = d_cand_q = nullptr;
    for (auto& t : tapbuf) t = nullptr;
    has_drafter = false;
  }

  // device: KV and sequence state
  uint16_t* k_cache = nullptr;
  uint16_t* v_cache = nullptr;
  size_t kv_elems = 0;
  uint32_t* page_table = nullptr;
  float* rope = nullptr;
  float* rope_rows = nullptr;  // [max_step_tokens][32 pairs]: the table's row at each step row's position
  uint32_t *lens = nullptr, *feed = nullptr, *tree = nullptr, *trace = nullptr, *trace_len = nullptr;
  sv_gen_state* gen = nullptr;
  // device: one step set (plan.rs writes these per step)
  // tokens: the plan's ids (FEED_ROW + i kept, so a captured step can be replayed); tok_res:
  // the ids embed resolved, which accept compares.
  uint32_t *tokens = nullptr, *tok_res = nullptr, *tin = nullptr, *vis = nullptr, *head_rows = nullptr,
           *attn_runs = nullptr;
  sv_sample_row* sample_rows = nullptr;
  sv_run_in* runs = nullptr;
  uint32_t *out_ids = nullptr, *emitted = nullptr, *meta = nullptr, *path = nullptr, *path_len = nullptr,
           *on_path = nullptr;
  // device: activations (buffers.rs Scratch)
  float *h = nullptr, *qkv = nullptr, *attn = nullptr, *mixed = nullptr, *act = nullptr, *inv = nullptr,
        *logits = nullptr;
  void* ws = nullptr;  // attention split partials
  size_t ws_bytes = 0;
  void* mm_ws = nullptr;  // matmul split-k hand-off (counters stay zero between launches)
  size_t mm_ws_bytes = 0;

  // host: page pool (kv.rs) and sequences (engine.rs Seq)
  std::vector<uint32_t> free_pages;
  std::vector<std::vector<uint32_t>> pages;
  std::vector<uint32_t> seq_len;
  std::vector<bool> used;
  std::vector<sv_sample_row> sampling;

  // The persistent layer kernel's buffers: activation slices per layer (grown by plans that
  // use it), its per-layer parameters and attention parameters, and its counters (256 bytes
  // apart, never reset but after an abort), the epoch word embed increments and the abort word.
  float* pl_buf = nullptr;
  size_t pl_floats = 0;
  uint32_t* pl_sync = nullptr;
  size_t pl_sync_words = 0;

  Plan plan;
  bool planned = false;
  // sv_profile_step: an event pair around every kernel while `prof` is set.
  bool prof = false;
  std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> prof_events;

  // Each timed kernel's events are taken by sv::launch at the kernel's own start and end.
  sv_status mark_begin(hipEvent_t* ev) {
    if (!prof) return SV_OK;
    hipEvent_t stop;
    SV_HIP(hipEventCreate(ev), "event");
    SV_HIP(hipEventCreate(&stop), "event");
    g_prof.start = *ev;
    g_prof.stop = stop;
    g_prof.used = false;
    return SV_OK;
  }
  sv_status mark_end(int kind, hipEvent_t begin) {
    if (!prof) return SV_OK;
    const hipEvent_t stop = g_prof.stop;
    const bool used = g_prof.used;
    g_prof = ProfEvents{};
    if (!used) {  // nothing launched (an empty step part): no time
      SV_HIP(hipEventDestroy(begin), "event");
      SV_HIP(hipEventDestroy(stop), "event");
      return SV_OK;
    }
    prof_events.push_back({kind, {begin, stop}});
    return SV_OK;
  }
#define SV_TIMED(kind, call)          \
  do {                               \
    hipEvent_t ev_ = nullptr;        \
    SV_TRY(mark_begin(&ev_));        \
    SV_TRY(call);                    \
    SV_TRY(mark_end((kind), ev_));   \
  } while (0)
  sv_replay_args replay{0, 0, 0.0f, 0};
  hipGraphExec_t graph = nullptr;

  ~sv_engine() {
    if (graph) (void)hipGraphExecDestroy(graph);
    void* bufs[] = {k_cache, v_cache, page_table, rope, rope_rows, lens, feed, tree, trace, trace_len, gen, tokens, tok_res, tin, vis,
                    head_rows, attn_runs, sample_rows, runs, out_ids, emitted, meta, path, path_len, on_path, h, qkv,
                    attn, mixed, act, inv, logits, ws, mm_ws, k_local, v_local, local_table, h0, xattn, rbase, vdir};
    for (void* b : bufs)
      if (b) (void)hipFree(b);
    for (void* b : packed)
      if (b) (void)hipFree(b);
    for (void* b : {(void*)pl_buf, (void*)pl_sync})
      if (b) (void)hipFree(b);
    if (head_tiled) (void)hipFree(head_tiled);
    if (head_lo_tiled) (void)hipFree(head_lo_tiled);
    if (tap[0]) (void)hipFree(tap[0]);
    if (tap[1] && tap[1] != tap[0]) (void)hipFree(tap[1]);
    free_drafter();
    if (stream) (void)hipStreamDestroy(stream);
  }

  size_t kv_offset_layer() const { return (size_t)n_pages * sh.n_kv_heads * (1u << cfg.page_shift) * sh.head_dim; }

  // KvArgs of layer li (kv.rs:70-80 args): global layers page through the pool, local ones
  // through their cyclic rings.
  sv_kv_args kv_args(uint32_t li) const {
    sv_kv_args kv{};
    const bool local = is_local[li] != 0;
    kv.is_global = local ? 0u : 1u;
    kv.kv_layer = kv_index[li];
    kv.ring = local ? ring_pages << cfg.page_shift : 0u;
    kv.max_seqs = cfg.max_seqs;
    kv.page_shift = cfg.page_shift;
    kv.n_pages = local ? n_lpages : n_pages;
    kv.max_pages = max_pages;
    kv.window = local ? cfg.window : 0u;
    return kv;
  }
  uint16_t* kc_of(uint32_t li) const { return is_local[li] ? k_local : k_cache; }
  uint16_t* vc_of(uint32_t li) const { return is_local[li] ? v_local : v_cache; }
  const uint32_t* table_of(uint32_t li) const { return is_local[li] ? local_table : page_table; }
  // MUDD routing (encode.rs:107-122 resid_in / resid_out): the site of layer li, and the tap
  // buffer layer li writes (or -1).
  int mudd_site(uint32_t li) const {
    for (uint32_t s = 0; s < extras.n_mudd; s++)
      if (extras.mudd_layer[s] == li) return (int)s;
    return -1;
  }
  float* out_of(uint32_t li) const {
    for (uint32_t s = 0; s < extras.n_mudd; s++)
      if (extras.mudd_tap[s] == li) return tap[s];
    return h;
  }
  float* emb_out() const { return extras.n_mudd ? h0 : h; }
  float* in_of(uint32_t li) const { return li == 0 ? emb_out() : out_of(li - 1); }

  // kv.rs:49-56 reserve(): pages until the slot holds `len` positions; the page table
  // entry goes to the device at once.
  sv_status reserve(uint32_t slot, uint32_t len) {
    auto& pg = pages[slot];
    const size_t before = pg.size();
    while (((size_t)pg.size() << cfg.page_shift) < len) {
      if (free_pages.empty()) return fail(SV_ERR_CAPACITY, "global KV pool exhausted");
      if (pg.size() >= max_pages) return fail(SV_ERR_CAPACITY, "sequence needs more than %u pages", max_pages);
      pg.push_back(free_pages.back());
      free_pages.pop_back();
    }
    if (pg.size() > before) {
      SV_HIP(hipMemcpyAsync(page_table + (size_t)slot * max_pages + before, pg.data() + before,
                            (pg.size() - before) * 4, hipMemcpyHostToDevice, stream),
             "page table");
      SV_HIP(hipStreamSynchronize(stream), "page table");
    }
    return SV_OK;
  }

  sv_status ensure_ws(size_t bytes) {
    if (bytes <= ws_bytes) return SV_OK;
    if (graph) return fail(SV_ERR_STATE, "workspace must grow after a graph was captured");
    SV_HIP(hipStreamSynchronize(stream), "workspace");
    if (ws) SV_HIP(hipFree(ws), "workspace");
    ws = nullptr;
    ws_bytes = 0;
    SV_HIP(hipMalloc(&ws, bytes), "workspace");
    SV_HIP(hipMemset(ws, 0, bytes), "workspace");
    ws_bytes = bytes;
    return SV_OK;
  }

  // The matmuls' workspace (split-k partials, counters zero at rest), grown to `bytes`.
  sv_status ensure_mm_ws(size_t bytes) {
    if (bytes <= mm_ws_bytes) return SV_OK;
    SV_HIP(hipStreamSynchronize(stream), "matmul workspace");
    if (mm_ws) SV_HIP(hipFree(mm_ws), "matmul workspace");
    mm_ws = nullptr;
    mm_ws_bytes = 0;
    SV_HIP(hipMalloc(&mm_ws, bytes), "matmul workspace");
    SV_HIP(hipMemset(mm_ws, 0, bytes), "matmul workspace");
    mm_ws_bytes = bytes;
    return SV_OK;
  }

  sv_status upload(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return SV_OK;
    SV_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream), "upload");
    return SV_OK;
  }

  sv_status check_ready() const {
    if (!embed) return fail(SV_ERR_STATE, "no embedding set");
    for (uint32_t l = 0; l < sh.n_layers; l++)
      if (!layer_set[l]) return fail(SV_ERR_STATE, "layer %u not set", l);
    for (uint32_t l = 0; l < sh.n_layers; l++)
      if (layers[l].ve_gate && !extras.value_embed)
        return fail(SV_ERR_STATE, "layer %u has value embeddings but no table is set (sv_engine_set_extras)", l);
    return SV_OK;
  }

  sv_status matmul(const sv_matrix& w, uint32_t n, const float* x, const uint32_t* x_rows, float* y, uint32_t epi,
                   uint32_t flags, float scale, float ra, float rb, const float* base, float* aux) {
    sv_mat_args a{};
    a.n = n;
    a.k = w.k;
    a.m = w.m;
    a.epi = epi;
    a.flags = flags;
    a.vocab_real = sh.vocab_real;
    a.scale = scale;
    a.ra = ra;
    a.rb = rb;
    a.ksplit = 1;
    a.kchunk = w.k;
    a.gshift = w.gshift;
    return matmul_launch(stream, &w, x, x_rows, y, base, aux, &a, mm_ws, mm_ws_bytes);
  }

  // Whether the persistent layer kernel takes this plan, and its parameters if so: 1-8 rows,
  // no prompt chunk, global layers without extras or MUDD, no drafter, per-row int8 tiled
  // matrices at hidden 2048 / ffn 8192, head_dim 64, splits of at most 384 keys, and every
  // phase's workgroups within one set of the grid.
  sv_status plan_layers(Plan& P) {
    P.persist = false;
    const sv_shape& s = sh;
    if (!(cfg.options & SV_OPT_LAYERS_KERNEL) || P.n > 8 || P.chunk || n_local || has_drafter || extras.n_mudd)
      return SV_OK;
    if (s.hidden != 2048 || s.ffn != 8192 || s.head_dim != 64 || P.n_attn > 32 || P.split > 384)
      return SV_OK;
    for (uint32_t li = 0; li < s.n_layers; li++) {
      const sv_layer& L = layers[li];
      if (L.ve_gate || L.attn_gate || L.xsa) return SV_OK;
      for (const sv_matrix* m : {&L.qkv, &L.o, &L.gate_up, &L.down}) {
        const bool per_row = m->gshift >= 32 || (1ull << m->gshift) >= m->k;
        if (m->format != (SV_FMT_I8 | SV_FMT_TILED) || !per_row || !m->d_scales) return SV_OK;
      }
    }
    const int ns = layers_grid_per_set();
    const uint32_t G = s.n_heads / s.n_kv_heads, D = 64, maxcols = (P.max_run * G + 15) / 16 * 16;
    if (ns <= 0 || P.max_run * G > 32) return SV_OK;
    uint32_t mP = 1;
    while (mP < 64 && 8 * mP < P.max_splits) mP *= 2;
    const uint32_t G4 = 256 / mP, mz = (maxcols * D / 4 + G4 - 1) / G4;
    const uint32_t tq = qkv_w / 16, th = s.hidden / 16, tgu = (2 * s.ffn / 16 + 3) / 4;
    const uint32_t attn_items = P.n_attn * s.n_kv_heads * P.max_splits, merge_items = P.n_attn * s.n_kv_heads * mz;
    for (uint32_t c : {tq, th, tgu, attn_items, merge_items})
      if (c > (uint32_t)ns) return SV_OK;
    // buffers: h (L + 1 slices), qkv, attn, mixed, act and the split partials (L slices each)
    const uint32_t L = s.n_layers, NR = 8;
    LayersParams& lp = P.lp;
    lp = LayersParams{};
    lp.n_layers = L;
    lp.n = P.n;
    lp.H = s.hidden;
    lp.F = s.ffn;
    lp.qkv_m = qkv_w;
    lp.G = G;
    lp.h_stride = NR * s.hidden;
    lp.qkv_stride = NR * qkv_w;
    lp.attn_stride = NR * s.n_heads * D;
    lp.mixed_stride = NR * s.hidden;
    lp.act_stride = NR * s.ffn;
    size_t l_off = 0;
    const size_t part = attn_part_floats(&s, P.n_attn, P.max_splits, P.max_run, &l_off);
    const size_t per_layer = (size_t)lp.qkv_stride + lp.attn_stride + lp.mixed_stride + lp.act_stride + part;
    const size_t need = (size_t)(L + 1) * lp.h_stride + (size_t)L * per_layer;
    if (L > PL_MAX_LAYERS) return SV_OK;
    if (need > pl_floats) {
      if (graph) return fail(SV_ERR_STATE, "layer buffers must grow after a graph was captured");
      SV_HIP(hipStreamSynchronize(stream), "layers: buffers");
      if (pl_buf) SV_HIP(hipFree(pl_buf), "layers: buffers");
      pl_buf = nullptr;
      pl_floats = 0;
      SV_HIP(hipMalloc(&pl_buf, need * 4), "layers: buffers");
      SV_HIP(hipMemset(pl_buf, 0, need * 4), "layers: buffers");
      pl_floats = need;
    }
    if (!pl_sync) {
      pl_sync_words = (size_t)PL_MAX_LAYERS * 6 * 16 * 64 + 2;
      SV_HIP(hipMalloc(&pl_sync, pl_sync_words * 4), "layers: counters");
      SV_HIP(hipMemset(pl_sync, 0, pl_sync_words * 4), "layers: counters");
    }
    float* b = pl_buf;
    lp.h = b;
    b += (size_t)(L + 1) * lp.h_stride;
    lp.qkv = b;
    b += (size_t)L * lp.qkv_stride;
    lp.attn_out = b;
    b += (size_t)L * lp.attn_stride;
    lp.mixed = b;
    b += (size_t)L * lp.mixed_stride;
    lp.act = b;
    b += (size_t)L * lp.act_stride;
    lp.part = b;
    lp.part_stride = (uint32_t)part;
    lp.part_l_off = (uint32_t)l_off;
    sv_attn_args aa{};
    aa.scale_log2 = cfg.attn_scale * 1.44269504088896340736f;
    aa.split = P.split;
    aa.max_splits = P.max_splits;
    aa.rope = 1;
    lp.rope_mask = 0;
    for (uint32_t li = 0; li < L; li++) {
      const sv_layer& Ly = layers[li];
      const sv_matrix* mats[4] = {&Ly.qkv, &Ly.o, &Ly.gate_up, &Ly.down};
      for (int k = 0; k < 4; k++) {
        lp.layers[li].w[k] = (const uint8_t*)mats[k]->d_w;
        lp.layers[li].s[k] = mats[k]->d_scales;
      }
      lp.layers[li].qkv_scale = Ly.qkv_scale;
      lp.layers[li].o_scale = Ly.o_scale;
      lp.layers[li].ra_attn = Ly.resid_attn;
      lp.layers[li].rb_attn = Ly.post_attn;
      lp.layers[li].ra_mlp = Ly.resid_mlp;
      lp.layers[li].rb_mlp = Ly.post_mlp;
      if (Ly.rope) lp.rope_mask |= 1u << li;
    }
    // the shared attention parameters (layer 0's slices; the kernel replaces them per layer)
    const sv_kv_args kv0 = kv_args(0);
    SV_TRY(attn_params_fill(&lp.ap, &s, lp.qkv, meta, k_cache, v_cache, page_table, rope_rows, &kv0, &aa,
                            P.inl.data(), P.n_attn, P.max_run, vis, lp.attn_out, lp.part, lp.part + l_off));
    lp.attn_items = attn_items;
    lp.merge_items = merge_items;
    lp.merge_P = mP;
    lp.merge_z = mz;
    const uint32_t cnt[6] = {tq, attn_items, merge_items, th, tgu, th};
    for (int k = 0; k < 6; k++) lp.cnt[k] = cnt[k];
    // counters and epoch from zero for this plan (its phases' producer counts are its own)
    SV_HIP(hipMemsetAsync(pl_sync, 0, pl_sync_words * 4, stream), "layers: counters");
    lp.sync = pl_sync;
    lp.epoch = pl_sync + pl_sync_words - 2;
    lp.abort = pl_sync + pl_sync_words - 1;
    P.persist = true;
    return SV_OK;
  }

  // After a step that ran the layer kernel: an aborted launch (a wait that ran out) is an error;
  // its counters are cleared for the next one.
  sv_status check_layers() {
    if (!pl_sync) return SV_OK;
    uint32_t ab = 0;
    SV_HIP(hipMemcpy(&ab, pl_sync + pl_sync_words - 1, 4, hipMemcpyDeviceToHost), "layers: abort word");
    if (!ab) return SV_OK;
    SV_HIP(hipMemset(pl_sync, 0, pl_sync_words * 4), "layers: counters");
    return fail(SV_ERR_HIP, "the persistent layer kernel gave up waiting (not every workgroup was resident)");
  }

  // Counts `steps` more runs of the plan against its page reservation.
  sv_status issue(uint64_t steps) {
    if (!planned) return fail(SV_ERR_STATE, "no plan");
    if (plan.issued + steps > plan.budget)
      return fail(SV_ERR_CAPACITY,
                  "the plan's pages cover %llu steps (%llu run): plan again, with more extra_keys for replays",
                  (unsigned long long)plan.budget, (unsigned long long)plan.issued);
    plan.issued += steps;
    return SV_OK;
  }

  // encode.rs:99-126 encode_forward + :383-412 encode_tail.
  sv_status encode(uint32_t flags) {
    SV_TRY(check_ready());
    if (!planned) return fail(SV_ERR_STATE, "no plan");
    const Plan& P = plan;
    const uint32_t n = P.n, H = sh.hidden, F = sh.ffn, NQD = sh.n_heads * sh.head_dim;
    if (P.persist && !capture) {
      // embed into the first h slice (and the epoch the layer kernel's counters count in), every
      // layer in one launch, then the head on the last slice
      SV_TIMED(SV_KIND_EMBED, embed_launch(stream, &sh, embed, tokens, tok_res, P.lp.h, tin, meta, lens, feed, tree, vis,
                                           n, rope, rope_rows, cfg.max_seq_len + SV_FEED_W,
                                           pl_sync + pl_sync_words - 2));
      SV_TIMED(SV_KIND_LAYERS, layers_launch(stream, P.lp, P.max_run));
      return encode_tail(flags, P.lp.h + (size_t)sh.n_layers * P.lp.h_stride);
    }
    SV_TIMED(SV_KIND_EMBED,
             embed_launch(stream, &sh, embed, tokens, tok_res, emb_out(), tin, meta, lens, feed, tree, vis, n, rope,
                          rope_rows, cfg.max_seq_len + SV_FEED_W));
    sv_attn_args aa{};
    aa.scale_log2 = cfg.attn_scale * 1.44269504088896340736f;
    for (uint32_t li = 0; li < sh.n_layers; li++) {
      const sv_layer& L = layers[li];
      float* hin = in_of(li);
      float* hout = out_of(li);
      // MUDD (encode.rs:145-160): the attention input and residual base mixed from the taps.
      const float* x = hin;
      const float* resid = hin;
      const int site = mudd_site(li);
      if (site >= 0) {
        SV_TIMED(SV_KIND_MUDD, mudd_launch(stream, hin, h0, tap[site], extras.mudd_dense1,
                                           extras.mudd_mix + (size_t)site * 6 * (SV_MUDD_INNER + 1), xattn, rbase, n, H));
        x = xattn;
        resid = rbase;
      }
      Capture* cp = capture;
      if (cp) {
        SV_HIP(hipMemcpyAsync(cp->resid_in, hin, (size_t)n * H * 4, hipMemcpyDeviceToDevice, stream), "capture");
        SV_TRY(rmsnorm_rows_launch(stream, x, cp->iota, cp->attn_in, n, H));
        if (site >= 0)
          SV_HIP(hipMemcpyAsync(cp->base, rbase, (size_t)n * H * 4, hipMemcpyDeviceToDevice, stream), "capture");
        g_attn_capture = AttnCapture{cp->q, cp->k, cp->v, cp->sdpa};
      }
      SV_TIMED(SV_KIND_QKV,
               matmul(L.qkv, n, x, nullptr, qkv, SV_EPI_NORM, SV_FLAG_WRITE_INV, L.qkv_scale, 0, 0, nullptr, inv));
      aa.rope = L.rope;
      const bool local = is_local[li] != 0;
      aa.split = local ? P.split_local : P.split;
      aa.max_splits = local ? P.max_splits_local : P.max_splits;
      const sv_kv_args kv = kv_args(li);
      sv_attn_extras ex{x, inv, tok_res, extras.value_embed, L.ve_gate, L.attn_gate, L.xsa, vdir, H, 0};
      const sv_attn_extras* exp_ = (L.ve_gate || L.attn_gate || L.xsa) ? &ex : nullptr;
      uint16_t *kc = kc_of(li), *vc = vc_of(li);
      const uint32_t* tab = table_of(li);
      if (P.chunk)
        SV_TIMED(SV_KIND_KV_WRITE, attn_launch(stream, &sh, qkv, meta, kc, vc, tab, rope, &kv, &aa, attn_runs, P.n_attn,
                                               P.max_run, vis, attn, ws, ws_bytes, 4, P.inl.data(), true, exp_,
                                               rope_rows));
      SV_TIMED(SV_KIND_ATTN, attn_launch(stream, &sh, qkv, meta, kc, vc, tab, rope, &kv, &aa, attn_runs, P.n_attn,
                                         P.max_run, vis, attn, ws, ws_bytes, 1, P.inl.data(), true, exp_, rope_rows));
      SV_TIMED(SV_KIND_ATTN_MERGE, attn_launch(stream, &sh, qkv, meta, kc, vc, tab, rope, &kv, &aa, attn_runs, P.n_attn,
                                               P.max_run, vis, attn, ws, ws_bytes, 2, P.inl.data(), true, exp_,
                                               rope_rows));
      if (cp)  // the layer's queries, keys and values as the attention computed them
        SV_TRY(attn_launch(stream, &sh, qkv, meta, kc, vc, tab, rope, &kv, &aa, attn_runs, P.n_attn, P.max_run, vis,
                           attn, ws, ws_bytes, 8, P.inl.data(), true, exp_, rope_rows));
      g_attn_capture = AttnCapture{};
      const uint32_t raw = cp ? (uint32_t)SV_FLAG_WRITE_RAW : 0u;
      SV_TIMED(SV_KIND_O, matmul(L.o, n, attn, nullptr, mixed, SV_EPI_RESID, raw, L.o_scale, L.resid_attn, L.post_attn,
                                 resid, cp ? cp->attn_out : nullptr));
      if (cp) SV_TRY(rmsnorm_rows_launch(stream, mixed, cp->iota, cp->mlp_in, n, H));
      SV_TIMED(SV_KIND_GATE_UP, matmul(L.gate_up, n, mixed, nullptr, act, SV_EPI_SWIGLU, 0, 1.0f, 0, 0, nullptr, nullptr));
      SV_TIMED(SV_KIND_DOWN, matmul(L.down, n, act, nullptr, hout, SV_EPI_RESID, raw, 1.0f, L.resid_mlp, L.post_mlp,
                                    mixed, cp ? cp->mlp_out : nullptr));
      // the drafter's taps (encode.rs:186-190): this layer's output, normed, rounded to bf16
      for (uint32_t k = 0; has_drafter && k < dr.n_taps; k++)
        if (dr.taps[k] == li) SV_TIMED(SV_KIND_DRAFT, tap_rows_launch(stream, hout, tapbuf[k], n, H));
      if (cp) SV_TRY(capture_layer(li, site >= 0));
    }
    (void)F;
    (void)NQD;
    return encode_tail(flags, out_of(sh.n_layers - 1));
  }

  // sv_step_capture: wait for layer li, read its intermediates back and hand them to the
  // callback (q | k | v assembled per row as the qkv matmul lays them out).
  sv_status capture_layer(uint32_t li, bool mudd) {
    const Capture& c = *capture;
    const uint32_t n = plan.n, H = sh.hidden, D = sh.head_dim, NQD = sh.n_heads * D, NKD = sh.n_kv_heads * D;
    const uint32_t W = NQD + 2 * NKD;
    SV_HIP(hipStreamSynchronize(stream), "capture");
    std::vector<float> resid_in((size_t)n * H), attn_in((size_t)n * H), q((size_t)n * NQD), k((size_t)n * NKD),
        v((size_t)n * NKD), sdpa((size_t)n * NQD), attn_out((size_t)n * H), mlp_in((size_t)n * H),
        mlp_out((size_t)n * H), base(mudd ? (size_t)n * H : 0), qkv_rows((size_t)n * W);
    const std::pair<float*, const float*> reads[] = {{resid_in.data(), c.resid_in}, {attn_in.data(), c.attn_in},
                                                     {attn_out.data(), c.attn_out}, {mlp_in.data(), c.mlp_in},
                                                     {mlp_out.data(), c.mlp_out}};
    for (const auto& rd : reads) SV_HIP(hipMemcpy(rd.first, rd.second, (size_t)n * H * 4, hipMemcpyDeviceToHost), "capture");
    SV_HIP(hipMemcpy(sdpa.data(), c.sdpa, (size_t)n * NQD * 4, hipMemcpyDeviceToHost), "capture");
    SV_HIP(hipMemcpy(q.data(), c.q, (size_t)n * NQD * 4, hipMemcpyDeviceToHost), "capture");
    SV_HIP(hipMemcpy(k.data(), c.k, (size_t)n * NKD * 4, hipMemcpyDeviceToHost), "capture");
    SV_HIP(hipMemcpy(v.data(), c.v, (size_t)n * NKD * 4, hipMemcpyDeviceToHost), "capture");
    if (mudd) SV_HIP(hipMemcpy(base.data(), c.base, (size_t)n * H * 4, hipMemcpyDeviceToHost), "capture");
    for (uint32_t t = 0; t < n; t++) {
      memcpy(&qkv_rows[(size_t)t * W], &q[(size_t)t * NQD], NQD * 4);
      memcpy(&qkv_rows[(size_t)t * W + NQD], &k[(size_t)t * NKD], NKD * 4);
      memcpy(&qkv_rows[(size_t)t * W + NQD + NKD], &v[(size_t)t * NKD], NKD * 4);
    }
    sv_layer_capture lc{};
    lc.layer = li;
    lc.n = n;
    lc.hidden = H;
    lc.qkv_width = W;
    lc.sdpa_width = NQD;
    lc.resid_in = resid_in.data();
    lc.attn_in = attn_in.data();
    lc.qkv = qkv_rows.data();
    lc.sdpa_out = sdpa.data();
    lc.attn_out = attn_out.data();
    lc.mlp_in = mlp_in.data();
    lc.mlp_out = mlp_out.data();
    lc.resid_base = mudd ? base.data() : nullptr;
    c.fn(&lc, c.user);
    return SV_OK;
  }

  // The head, sampler and step tail after the layers; `last` holds the last layer's rows.
  sv_status encode_tail(uint32_t flags, const float* last) {
    const Plan& P = plan;
    if (P.n_head > 0) {
      // rmsnorm_rows + the tied head (encode.rs:390-393), the norm folded into the matmul.
      if (head_lo.d_w) {
        // hi + lo products (raw, the norm folded), then the softcap
        SV_TIMED(SV_KIND_HEAD, matmul(head_mat, P.n_head, last, head_rows, logits, SV_EPI_RAW, SV_FLAG_NORM_IN, 1.0f,
                                      0, 0, nullptr, nullptr));
        SV_TIMED(SV_KIND_HEAD, matmul(head_lo, P.n_head, last, head_rows, logits, SV_EPI_RESID, SV_FLAG_NORM_IN, 1.0f,
                                      1.0f, 1.0f, logits, nullptr));
        SV_TIMED(SV_KIND_HEAD, head_cap_launch(stream, logits, P.n_head, sh.vocab, sh.vocab_real));
      } else {
        SV_TIMED(SV_KIND_HEAD, matmul(head_mat, P.n_head, last, head_rows, logits, SV_EPI_HEAD,
                                      SV_FLAG_NORM_IN, 1.0f, 0, 0, nullptr, nullptr));
      }
      SV_TIMED(SV_KIND_SAMPLE, sample_launch(stream, logits, sample_rows, out_ids, meta, P.n_head, sh.vocab));
    }
    // accept + kv_compact + replay drafter (encode.rs:394-435, 439-451) as one launch.
    const bool compact = (flags & SV_STEP_COMPACT) || (P.branches && !(flags & SV_STEP_NO_COMPACT));
    sv_replay_args ra = replay;
    ra.stride = cfg.max_seq_len;
    ra.vocab = sh.vocab_real;
    const KvCacheRef caches[2] = {{k_cache, v_cache, page_table, n_global, n_pages},
                                  {k_local, v_local, local_table, n_local, n_lpages ? n_lpages : 1u}};
    SV_TIMED(SV_KIND_ACCEPT, step_tail_launch(stream, &sh, runs, P.n_runs, tok_res, out_ids, lens, feed, gen, emitted,
                                              tree, path, path_len, on_path, compact, caches, n_local ? 2u : 1u,
                                              cfg.page_shift, max_pages, (flags & SV_STEP_REPLAY) ? &ra : nullptr,
                                              trace, trace_len));
    if (has_drafter) SV_TRY(encode_draft((flags & SV_STEP_DRAFT) != 0));
    return SV_OK;
  }

  sv_kv_args draft_kv_args(uint32_t layer) const {
    sv_kv_args kv{};
    kv.is_global = 0;
    kv.kv_layer = layer;
    kv.ring = d_ring_pages << cfg.page_shift;
    kv.max_seqs = cfg.max_seqs;
    kv.page_shift = cfg.page_shift;
    kv.n_pages = d_n_pages;
    kv.max_pages = d_max_pages;
    kv.window = dr.window;
    return kv;
  }

  // drafter.rs:302-447 encode_drafter: the context of every token of the step, then the plan's
  // blocks through the drafter's layers, its head, draft_top and draft_tree (which write the
  // slots' next feed and tree).
  sv_status encode_draft(bool blocks) {
    const Plan& P = plan;
    const uint32_t n = P.n, H = sh.hidden, rows = P.d_rows;
    // 1. Context: sum over the taps of fc[k] tap_k, then every drafter layer's k | v of its norm.
    for (uint32_t k = 0; k < dr.n_taps; k++)
      SV_TIMED(SV_KIND_DRAFT, matmul(dr.fc[k], n, tapbuf[k], nullptr, d_ctx, k ? SV_EPI_RESID : SV_EPI_RAW, 0, 1.0f,
                                     1.0f, 1.0f, d_ctx, nullptr));
    SV_TIMED(SV_KIND_DRAFT,
             matmul(dr.kv_all, n, d_ctx, nullptr, d_kvp, SV_EPI_NORM, SV_FLAG_WRITE_INV, 1.0f, 0, 0, nullptr, d_ctx_inv));
    const sv_kv_args kv0 = draft_kv_args(0);
    SV_TIMED(SV_KIND_DRAFT, draft_kv_launch(stream, &sh, d_kvp, meta, on_path, rope, dk_ring, dv_ring, d_table, &kv0, n,
                                            dr.n_layers));
    const bool inject = dr.inject.d_w != nullptr;
    if (inject)
      SV_TIMED(SV_KIND_DRAFT, draft_ctx_launch(stream, d_ctx, d_ctx_inv, meta, on_path, d_cring, d_cr, n, H));
    if (!blocks || P.n_blocks == 0) return SV_OK;
    // 2. Block rows.
    SV_TIMED(SV_KIND_DRAFT, draft_embed_launch(stream, embed, d_tin, lens, feed, dr.mask_emb, d_x, d_meta, d_tokens,
                                               d_cring, d_last, inject ? d_cr : 0u, rows, H));
    if (inject)
      SV_TIMED(SV_KIND_DRAFT, matmul(dr.inject, rows, d_last, nullptr, d_x, SV_EPI_RESID, 0, 1.0f, 1.0f, 1.0f, d_x, nullptr));
    auto conv = [&](uint32_t li, int c, const float* x, const float* resid, float* out) -> sv_status {
      const sv_draft_layer& Ld = dlayers[li];
      SV_TIMED(SV_KIND_DRAFT, matmul(Ld.conv_corr[c], rows, x, nullptr, d_corr, SV_EPI_NORM, SV_FLAG_WRITE_INV, 1.0f, 0,
                                     0, nullptr, d_corr_inv));
      SV_TIMED(SV_KIND_DRAFT, draft_conv_launch(stream, x, d_corr, Ld.conv_corr[c].m, Ld.conv_base[c], d_tin, resid,
                                                out, rows, H));
      return SV_OK;
    };
    sv_attn_args aa{};
    aa.split = P.d_split;
    aa.max_splits = P.d_max_splits;
    aa.scale_log2 = cfg.attn_scale * 1.44269504088896340736f;
    aa.rope = 1;
    for (uint32_t li = 0; li < dr.n_layers; li++) {
      const sv_draft_layer& Ld = dlayers[li];
      const bool convs = Ld.conv_base[0] != nullptr;
      const float* xin = d_x;
      if (convs) {
        SV_TRY(conv(li, 0, d_x, nullptr, d_cx));
        xin = d_cx;
      }
      SV_TIMED(SV_KIND_DRAFT,
               matmul(Ld.qkv, rows, xin, nullptr, d_qkv, SV_EPI_NORM, SV_FLAG_WRITE_INV, 1.0f, 0, 0, nullptr, d_inv));
      const sv_kv_args kv = draft_kv_args(li);
      SV_TIMED(SV_KIND_DRAFT, attn_launch(stream, &sh, d_qkv, d_meta, dk_ring, dv_ring, d_table, rope, &kv, &aa, d_tiles,
                                          P.n_blocks, P.d_max_run, d_vis, d_attn, ws, ws_bytes, 1, P.dinl.data()));
      SV_TIMED(SV_KIND_DRAFT, attn_launch(stream, &sh, d_qkv, d_meta, dk_ring, dv_ring, d_table, rope, &kv, &aa, d_tiles,
                                          P.n_blocks, P.d_max_run, d_vis, d_attn, ws, ws_bytes, 2, P.dinl.data()));
      if (convs) {
        SV_TIMED(SV_KIND_DRAFT, matmul(Ld.o, rows, d_attn, nullptr, d_co, SV_EPI_RAW, 0, 1.0f, 0, 0, nullptr, nullptr));
        SV_TRY(conv(li, 1, d_co, d_x, d_mixed));
        SV_TRY(conv(li, 2, d_mixed, nullptr, d_cx));
        SV_TIMED(SV_KIND_DRAFT, matmul(Ld.gate_up, rows, d_cx, nullptr, d_act, SV_EPI_SWIGLU, 0, 1.0f, 0, 0, nullptr, nullptr));
        SV_TIMED(SV_KIND_DRAFT, matmul(Ld.down, rows, d_act, nullptr, d_co, SV_EPI_RAW, 0, 1.0f, 0, 0, nullptr, nullptr));
        SV_TRY(conv(li, 3, d_co, d_mixed, d_x));
      } else {
        SV_TIMED(SV_KIND_DRAFT, matmul(Ld.o, rows, d_attn, nullptr, d_mixed, SV_EPI_RESID, 0, 1.0f, 1.0f, 1.0f, d_x, nullptr));
        SV_TIMED(SV_KIND_DRAFT, matmul(Ld.gate_up, rows, d_mixed, nullptr, d_act, SV_EPI_SWIGLU, 0, 1.0f, 0, 0, nullptr, nullptr));
        SV_TIMED(SV_KIND_DRAFT, matmul(Ld.down, rows, d_act, nullptr, d_x, SV_EPI_RESID, 0, 1.0f, 1.0f, 1.0f, d_mixed, nullptr));
      }
    }
    // 3. The tree: raw logits of the normed rows (the norm folded into the head), candidates,
    // best-first trees into the slots' feed and tree.
    SV_TIMED(SV_KIND_DRAFT,
             matmul(dr.head, rows, d_x, nullptr, d_logits, SV_EPI_RAW, SV_FLAG_NORM_IN, 1.0f, 0, 0, nullptr, nullptr));
    if (d_head_lo.d_w)
      SV_TIMED(SV_KIND_DRAFT, matmul(d_head_lo, rows, d_x, nullptr, d_logits, SV_EPI_RESID, SV_FLAG_NORM_IN, 1.0f, 1.0f,
                                     1.0f, d_logits, nullptr));
    const uint32_t ncand = std::min(SV_DRAFT_CANDS, P.d_max_run - 1);
    if (ncand == 0) return SV_OK;  // blocks of one row: nothing to draft
    SV_TIMED(SV_KIND_DRAFT, draft_top_launch(stream, d_logits, dr.vocab, d_tin, d_cand, d_cand_q, rows, dr.v,
                                             dr.inv_temperature, ncand));
    SV_TIMED(SV_KIND_DRAFT, draft_tree_launch(stream, d_tiles, P.n_blocks, d_tin, d_cand, d_cand_q, feed, tree, ncand));
    return SV_OK;
  }
};

extern "C" sv_status sv_engine_create(const sv_engine_config* cfg, const float* rope_freq, sv_engine** out) {
  if (!cfg || !out || !rope_freq) return fail(SV_ERR_ARG, "engine_create: null pointer");
  *out = nullptr;
  const sv_shape& s = cfg->shape;
  if (s.hidden == 0 || s.hidden % 256 || s.ffn == 0 || s.ffn % 128 || s.n_kv_heads == 0 || s.n_heads % s.n_kv_heads ||
      (s.head_dim != 64 && s.head_dim != 128) || s.vocab == 0 || s.vocab % 16 || s.vocab_real > s.vocab ||
      s.n_layers == 0)
    return fail(SV_ERR_ARG, "engine_create: unsupported shape (hidden %u, heads %u/%u, dim %u, ffn %u, vocab %u)",
                s.hidden, s.n_heads, s.n_kv_heads, s.head_dim, s.ffn, s.vocab);
  if ((s.n_heads * s.head_dim) % 256 || ((s.n_heads + 2 * s.n_kv_heads) * s.head_dim) % 16)
    return fail(SV_ERR_ARG, "engine_create: heads x dim must be a multiple of 256");
  if (cfg->max_seqs == 0 || cfg->max_step_tokens == 0 || cfg->max_seq_len == 0 || cfg->max_head_rows == 0 ||
      cfg->kv_tokens == 0)
    return fail(SV_ERR_ARG, "engine_create: zero capacity");
  if (cfg->options & ~SV_OPT_LAYERS_KERNEL) return fail(SV_ERR_ARG, "engine_create: options %u", cfg->options);
  if (cfg->local) {
    bool any = false;
    for (uint32_t li = 0; li < s.n_layers; li++) any = any || cfg->local[li];
    if (any && (cfg->window == 0 || cfg->window > cfg->max_seq_len))
      return fail(SV_ERR_ARG, "engine_create: sliding-window layers need 0 < window <= max_seq_len (window %u)", cfg->window);
  }
  if (cfg->page_shift < 4 || cfg->page_shift > 16) return fail(SV_ERR_ARG, "engine_create: page_shift %u", cfg->page_shift);
  if (cfg->split_keys % 32 || cfg->split_keys > 3968)
    return fail(SV_ERR_ARG, "engine_create: split_keys %u (a multiple of 32, at most 3968)", cfg->split_keys);
  attn_init();
  matmul_init();
  sv_engine* e = new sv_engine();
  e->cfg = *cfg;
  e->sh = s;
  e->layers.resize(s.n_layers);
  e->layer_set.assign(s.n_layers, false);
  e->packed.assign((size_t)s.n_layers * 4, nullptr);
  const uint32_t page = 1u << cfg->page_shift;
  e->n_pages = (cfg->kv_tokens + page - 1) / page;
  e->max_pages = (cfg->max_seq_len + page - 1) / page;
  e->qkv_w = (s.n_heads + 2 * s.n_kv_heads) * s.head_dim;
  e->arun = std::min(SV_MAX_RUN, SV_MAX_COLS / (s.n_heads / s.n_kv_heads));
  e->is_local.assign(s.n_layers, 0);
  e->kv_index.assign(s.n_layers, 0);
  for (uint32_t li = 0; li < s.n_layers; li++) {
    e->is_local[li] = cfg->local && cfg->local[li] ? 1 : 0;
    e->kv_index[li] = e->is_local[li] ? e->n_local++ : e->n_global++;
  }
  if (e->n_local) {
    // A ring holds the window plus a whole step (kv.rs:26-28): a step's earlier queries still
    // need the keys its later rows overwrite.
    e->ring_pages = (cfg->window + cfg->max_step_tokens + page - 1) / page;
    e->n_lpages = cfg->max_seqs * e->ring_pages;
  }
  auto bad = [&](sv_status st) {
    delete e;
    return st;
  };
  if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) return bad(fail(SV_ERR_HIP, "stream"));
  const uint32_t n = cfg->max_step_tokens, S = cfg->max_seqs, R = cfg->max_head_rows;
  e->kv_elems = (size_t)e->n_global * e->kv_offset_layer();
  e->local_elems = (size_t)e->n_local * e->n_lpages * s.n_kv_heads * page * s.head_dim;
  sv_status st = SV_OK;
#define ALLOC(ptr, count)                                 \
  if ((st = dalloc(&e->ptr, (count), #ptr)) != SV_OK) return bad(st)
  ALLOC(k_cache, e->kv_elems);
  ALLOC(v_cache, e->kv_elems);
  ALLOC(page_table, (size_t)S * e->max_pages);
  if (e->n_local) {
    ALLOC(k_local, e->local_elems);
    ALLOC(v_local, e->local_elems);
    ALLOC(local_table, (size_t)S * e->max_pages);
  }
  ALLOC(vdir, (size_t)n * s.n_kv_heads * s.head_dim);
  ALLOC(rope, (size_t)(cfg->max_seq_len + SV_FEED_W) * SV_ROPE_PAIRS * 2);
  ALLOC(lens, S);
  ALLOC(feed, (size_t)S * SV_FEED_W);
  ALLOC(tree, (size_t)S * SV_FEED_W);
  ALLOC(trace, (size_t)S * cfg->max_seq_len);
  ALLOC(trace_len, S);
  ALLOC(gen, S);
  ALLOC(tokens, n);
  ALLOC(tok_res, n);
  ALLOC(tin, 2 * (size_t)n);
  ALLOC(vis, n);
  ALLOC(head_rows, n);
  ALLOC(attn_runs, 2 * ((size_t)n / e->arun + S));
  ALLOC(sample_rows, std::max(n, R));
  ALLOC(runs, S);
  ALLOC(out_ids, std::max(n, R));
  ALLOC(emitted, S);
  ALLOC(meta, 2 * (size_t)n);
  ALLOC(rope_rows, (size_t)n * SV_ROPE_PAIRS * 2);
  ALLOC(path, (size_t)S * SV_FEED_W);
  ALLOC(path_len, S);
  ALLOC(on_path, n);
  ALLOC(h, (size_t)n * s.hidden);
  ALLOC(qkv, (size_t)n * e->qkv_w);
  ALLOC(attn, (size_t)n * s.n_heads * s.head_dim);
  ALLOC(mixed, (size_t)n * s.hidden);
  ALLOC(act, (size_t)n * s.ffn);
  ALLOC(inv, n);
  ALLOC(logits, (size_t)std::max(n, R) * s.vocab);
#undef ALLOC
  // RoPE table (engine.rs:394-421): (bf16(cos), bf16(sin)) of float(pos) * freq[j].
  {
    const size_t npos = (size_t)cfg->max_seq_len + SV_FEED_W;
    std::vector<float> tab(npos * SV_ROPE_PAIRS * 2);
    auto rbf = [](float x) {
      uint32_t u;
      memcpy(&u, &x, 4);
      u += 0x7fffu + ((u >> 16) & 1u);
      u &= 0xffff0000u;
      float f;
      memcpy(&f, &u, 4);
      return f;
    };
    for (size_t pos = 0; pos < npos; pos++)
      for (uint32_t j = 0; j < SV_ROPE_PAIRS; j++) {
        const float th = (float)pos * rope_freq[j];
        tab[(pos * SV_ROPE_PAIRS + j) * 2] = rbf(cosf(th));
        tab[(pos * SV_ROPE_PAIRS + j) * 2 + 1] = rbf(sinf(th));
      }
    if (hipMemcpy(e->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bad(fail(SV_ERR_HIP, "rope table"));
  }
  // Chains in every slot's tree (buffers.rs:115-117), open generation state.
  {
    std::vector<uint32_t> chains((size_t)S * SV_FEED_W);
    for (size_t i = 0; i < chains.size(); i++) {
      const uint32_t row = (uint32_t)(i % SV_FEED_W);
      chains[i] = row | (row == 0 ? SV_NO_PARENT : row - 1) << 8 | ((2u << row) - 1u) << 16;
    }
    if (hipMemcpy(e->tree, chains.data(), chains.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bad(fail(SV_ERR_HIP, "tree"));
    std::vector<sv_gen_state> g(S);
    for (auto& x : g) {
      memset(&x, 0, sizeof x);
      x.remaining = 0xffffffffu;
    }
    if (hipMemcpy(e->gen, g.data(), g.size() * sizeof(sv_gen_state), hipMemcpyHostToDevice) != hipSuccess)
      return bad(fail(SV_ERR_HIP, "gen"));
  }
  if (e->n_local) {
    std::vector<uint32_t> lt((size_t)S * e->max_pages);
    for (uint32_t slot = 0; slot < S; slot++)
      for (uint32_t pg = 0; pg < e->max_pages; pg++) lt[(size_t)slot * e->max_pages + pg] = slot * e->ring_pages + pg % e->ring_pages;
    if (hipMemcpy(e->local_table, lt.data(), lt.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bad(fail(SV_ERR_HIP, "local page table"));
  }
  // kv.rs:40: free pages (0..n).rev(), popped 0, 1, 2, ...
  e->free_pages.resize(e->n_pages);
  for (uint32_t i = 0; i < e->n_pages; i++) e->free_pages[i] = e->n_pages - 1 - i;
  e->pages.resize(S);
  e->seq_len.assign(S, 0);
  e->used.assign(S, false);
  e->sampling.assign(S, sv_sample_row{0, 0, 0, 0.0f, 1.0f, SV_NO_TOK});
  // Workspace for the matmuls: the most any row count up to the step's (head: head rows) needs.
  size_t ws = 0;
  const uint32_t mk[][3] = {{e->qkv_w, s.hidden, n}, {s.hidden, s.n_heads * s.head_dim, n}, {2 * s.ffn, s.hidden, n},
                            {s.hidden, s.ffn, n}, {s.vocab, s.hidden, R}};
  for (auto& x : mk)
    for (uint32_t rows = 1; rows <= x[2]; rows++) ws = std::max(ws, matmul_ws_bytes(rows, x[0], x[1]));
  if (ws) {
    if (hipMalloc(&e->mm_ws, ws) != hipSuccess || hipMemset(e->mm_ws, 0, ws) != hipSuccess)
      return bad(fail(SV_ERR_HIP, "matmul workspace (%zu bytes)", ws));
    e->mm_ws_bytes = ws;
  }
  *out = e;
  return SV_OK;
}

extern "C" void sv_engine_destroy(sv_engine* e) {
  if (!e) return;
  (void)hipStreamSynchronize(e->stream);
  delete e;
}

extern "C" void* sv_engine_stream(sv_engine* e) { return e ? (void*)e->stream : nullptr; }

// A tiled copy of a row-major matrix in *slot (replacing what it held), as *out; a matrix that
// does not fit the tiled layout, or is tiled already, is used as given. The weight reads of a
// 1-16 row matmul are then contiguous kilobytes (measured on MI355X: head 31 -> 23 us, down
// 11.3 -> 9.1 us at 5 rows). Done once, at model load.
static sv_status pack_into(sv_engine* e, const sv_matrix& in, void** slot, sv_matrix* out) {
  *out = in;
  if ((in.format & SV_FMT_TILED) || in.m % 16 || in.k % 64) return SV_OK;
  const size_t bytes = (size_t)in.m * in.k * (in.format == SV_FMT_I8 ? 1 : 2);
  if (*slot) {
    SV_HIP(hipStreamSynchronize(e->stream), "pack: sync");
    SV_HIP(hipFree(*slot), "pack: free");
    *slot = nullptr;
  }
  SV_HIP(hipMalloc(slot, bytes), "pack: alloc");
  SV_TRY(pack_matrix(e->stream, &in, *slot, out));
  SV_HIP(hipStreamSynchronize(e->stream), "pack: sync");
  return SV_OK;
}

extern "C" sv_status sv_engine_set_embed(sv_engine* e, const uint16_t* d_embed) {
  if (!e || !d_embed) return fail(SV_ERR_ARG, "set_embed: null pointer");
  e->embed = d_embed;
  if (e->own_head) return SV_OK;
  const sv_matrix head{d_embed, nullptr, e->sh.vocab, e->sh.hidden, SV_FMT_BF16, 0};
  SV_TRY(pack_into(e, head, &e->head_tiled, &e->head_mat));
  return SV_OK;
}

static sv_status check_matrix(const sv_matrix& m, uint32_t rows, uint32_t cols, const char* name) {
  if (!m.d_w) return fail(SV_ERR_ARG, "%s: no weights", name);
  if (m.m != rows || m.k != cols) return fail(SV_ERR_ARG, "%s: [%u][%u], expected [%u][%u]", name, m.m, m.k, rows, cols);
  const uint32_t fmt = m.format & ~(uint32_t)SV_FMT_TILED;
  if (fmt == SV_FMT_I8 && !m.d_scales) return fail(SV_ERR_ARG, "%s: int8 without scales", name);
  if (fmt != SV_FMT_I8 && fmt != SV_FMT_BF16) return fail(SV_ERR_ARG, "%s: format %u", name, m.format);
  if ((m.format & SV_FMT_TILED) && (m.m % 16 || m.k % 64)) return fail(SV_ERR_ARG, "%s: tiled needs m %% 16, k %% 64", name);
  return SV_OK;
}

extern "C" sv_status sv_engine_set_layer(sv_engine* e, uint32_t layer, const sv_layer* l) {
  if (!e || !l) return fail(SV_ERR_ARG, "set_layer: null pointer");
  if (layer >= e->sh.n_layers) return fail(SV_ERR_ARG, "set_layer: layer %u of %u", layer, e->sh.n_layers);
  const sv_shape& s = e->sh;
  SV_TRY(check_matrix(l->qkv, e->qkv_w, s.hidden, "qkv"));
  SV_TRY(check_matrix(l->o, s.hidden, s.n_heads * s.head_dim, "o"));
  SV_TRY(check_matrix(l->gate_up, 2 * s.ffn, s.hidden, "gate_up"));
  SV_TRY(check_matrix(l->down, s.hidden, s.ffn, "down"));
  sv_layer used = *l;
  void** slots = &e->packed[(size_t)layer * 4];
  SV_TRY(pack_into(e, l->qkv, &slots[0], &used.qkv));
  SV_TRY(pack_into(e, l->o, &slots[1], &used.o));
  SV_TRY(pack_into(e, l->gate_up, &slots[2], &used.gate_up));
  SV_TRY(pack_into(e, l->down, &slots[3], &used.down));
  e->layers[layer] = used;
  e->layer_set[layer] = true;
  return SV_OK;
}

extern "C" sv_status sv_engine_set_head(sv_engine* e, const sv_matrix* head) {
  if (!e) return fail(SV_ERR_ARG, "set_head: null engine");
  if (e->graph) return fail(SV_ERR_STATE, "set_head: after a graph was captured");
  e->head_lo = sv_matrix{};
  if (!head) {
    e->own_head = false;
    if (!e->embed) return SV_OK;
    const sv_matrix tied{e->embed, nullptr, e->sh.vocab, e->sh.hidden, SV_FMT_BF16, 0};
    return pack_into(e, tied, &e->head_tiled, &e->head_mat);
  }
  SV_TRY(check_matrix(*head, e->sh.vocab, e->sh.hidden, "head"));
  const uint32_t fmt = head->format & ~(uint32_t)SV_FMT_TILED;
  const bool per_row = head->gshift >= 32 || (1ull << head->gshift) >= head->k;
  if (fmt == SV_FMT_I8 && !per_row && head->gshift < 6) {
    // groups of 8-32 (model.rs:98 accepts 8-256; the converter's head default is 8): a matrix
    // core step would mix several groups' scales, so the head runs as two bf16 matrices whose
    // sum is exactly q s (8 + 8 significant bits hold the 15 of the product)
    if (head->format & SV_FMT_TILED) return fail(SV_ERR_UNSUPPORTED, "set_head: a tiled head in groups under 64");
    const size_t elems = (size_t)head->m * head->k;
    uint16_t *hi = nullptr, *lo = nullptr;
    SV_TRY(dalloc(&hi, elems, "head hi"));
    sv_status st = dalloc(&lo, elems, "head lo");
    if (st == SV_OK) st = split_i8_launch(e->stream, head, hi, lo);
    if (st == SV_OK) st = check_hip(hipStreamSynchronize(e->stream), "head split");
    const sv_matrix mh{hi, nullptr, head->m, head->k, SV_FMT_BF16, 0}, ml{lo, nullptr, head->m, head->k, SV_FMT_BF16, 0};
    if (st == SV_OK) st = pack_into(e, mh, &e->head_tiled, &e->head_mat);
    if (st == SV_OK) st = pack_into(e, ml, &e->head_lo_tiled, &e->head_lo);
    (void)hipFree(hi);
    if (lo) (void)hipFree(lo);
    if (st != SV_OK) {
      e->head_lo = sv_matrix{};
      return st;
    }
    e->own_head = true;
    return SV_OK;
  }
  SV_TRY(pack_into(e, *head, &e->head_tiled, &e->head_mat));
  e->own_head = true;
  return SV_OK;
}

extern "C" sv_status sv_engine_set_extras(sv_engine* e, const sv_model_extras* x) {
  if (!e || !x) return fail(SV_ERR_ARG, "set_extras: null pointer");
  if (e->graph) return fail(SV_ERR_STATE, "set_extras: after a graph was captured");
  const sv_shape& s = e->sh;
  if (x->n_mudd > SV_MUDD_SITES) return fail(SV_ERR_ARG, "set_extras: %u MUDD sites (at most %u)", x->n_mudd, SV_MUDD_SITES);
  if (x->n_mudd && (!x->mudd_dense1 || !x->mudd_mix)) return fail(SV_ERR_ARG, "set_extras: MUDD without dense1 / mix");
  for (uint32_t i = 0; i < x->n_mudd; i++) {
    if (x->mudd_layer[i] >= s.n_layers || x->mudd_tap[i] >= x->mudd_layer[i])
      return fail(SV_ERR_ARG, "set_extras: MUDD site %u at layer %u with tap %u (needs tap < layer < %u)", i,
                  x->mudd_layer[i], x->mudd_tap[i], s.n_layers);
    for (uint32_t j = 0; j < i; j++)
      if (x->mudd_layer[j] == x->mudd_layer[i]) return fail(SV_ERR_ARG, "set_extras: two MUDD sites at layer %u", x->mudd_layer[i]);
  }
  SV_HIP(hipStreamSynchronize(e->stream), "set_extras");
  const size_t rows = (size_t)e->cfg.max_step_tokens * s.hidden;
  if (x->n_mudd) {
    float** bufs[] = {&e->h0, &e->xattn, &e->rbase};
    for (float** b : bufs)
      if (!*b) SV_TRY(dalloc(b, rows, "mudd buffers"));
    for (uint32_t i = 0; i < SV_MUDD_SITES; i++) {
      // one buffer per distinct tap layer
      if (i < x->n_mudd && i > 0 && x->mudd_tap[i] == x->mudd_tap[0]) {
        if (e->tap[i] && e->tap[i] != e->tap[0]) SV_HIP(hipFree(e->tap[i]), "mudd buffers");
        e->tap[i] = e->tap[0];
      } else if (i < x->n_mudd && (!e->tap[i] || (i > 0 && e->tap[i] == e->tap[0]))) {
        e->tap[i] = nullptr;
        SV_TRY(dalloc(&e->tap[i], rows, "mudd buffers"));
      }
    }
  }
  e->extras = *x;
  return SV_OK;
}

extern "C" sv_status sv_engine_get_buffers(sv_engine* e, sv_engine_buffers* o) {
  if (!e || !o) return fail(SV_ERR_ARG, "get_buffers: null pointer");
  o->d_k_cache = e->k_cache;
  o->d_v_cache = e->v_cache;
  o->d_page_table = e->page_table;
  o->d_lens = e->lens;
  o->d_feed = e->feed;
  o->d_tree = e->tree;
  o->d_gen = e->gen;
  o->d_trace = e->trace;
  o->d_trace_len = e->trace_len;
  o->d_logits = e->logits;
  o->d_rope = e->rope;
  o->d_out_ids = e->out_ids;
  o->d_emitted = e->emitted;
  o->d_path = e->path;
  o->d_path_len = e->path_len;
  o->n_pages = e->n_pages;
  o->max_pages = e->max_pages;
  o->kv_bytes = e->kv_elems * 2;
  o->d_k_local = e->k_local;
  o->d_v_local = e->v_local;
  o->d_local_table = e->local_table;
  o->n_local_pages = e->n_lpages;
  o->ring_pages = e->ring_pages;
  o->local_bytes = e->local_elems * 2;
  return SV_OK;
}

// drafter.rs:145-241 Drafter::load + :250-255 load_drafter: the matrices checked and tiled,
// the rings (cyclic pages, as the sliding-window layers'), the block rows' buffers.
extern "C" sv_status sv_engine_set_drafter(sv_engine* e, const sv_drafter* d) {
  if (!e || !d) return fail(SV_ERR_ARG, "set_drafter: null pointer");
  const sv_shape& s = e->sh;
  const uint32_t H = s.hidden, NKV = s.n_kv_heads, D = s.head_dim;
  if (d->n_layers == 0 || d->n_layers > SV_DRAFT_LAYERS || !d->layers)
    return fail(SV_ERR_ARG, "set_drafter: %u layers (1..%u)", d->n_layers, SV_DRAFT_LAYERS);
  if (d->n_taps == 0 || d->n_taps > SV_DRAFT_TAPS) return fail(SV_ERR_ARG, "set_drafter: %u taps (1..%u)", d->n_taps, SV_DRAFT_TAPS);
  for (uint32_t k = 0; k < d->n_taps; k++)
    if (d->taps[k] >= s.n_layers) return fail(SV_ERR_ARG, "set_drafter: tap %u at layer %u of %u", k, d->taps[k], s.n_layers);
  if (d->v < SV_DRAFT_CANDS || !d->vocab || !d->mask_emb) return fail(SV_ERR_ARG, "set_drafter: vocabulary of %u, or no ids / mask_emb", d->v);
  if (d->window == 0) return fail(SV_ERR_ARG, "set_drafter: window 0");
  if (!(d->inv_temperature > 0.0f) || !std::isfinite(d->inv_temperature))
    return fail(SV_ERR_ARG, "set_drafter: inverse temperature %g", d->inv_temperature);
  if (!e->embed) return fail(SV_ERR_STATE, "set_drafter: no embedding set (sv_engine_set_embed)");
  if (NKV * D / 4 > 256 || (D != 64 && D != 128)) return fail(SV_ERR_UNSUPPORTED, "set_drafter: %u kv heads x %u dims", NKV, D);
  SV_HIP(hipStreamSynchronize(e->stream), "set_drafter");
  // a captured step and the plan were laid out without this drafter: both go
  if (e->graph) {
    (void)hipGraphExecDestroy(e->graph);
    e->graph = nullptr;
  }
  e->planned = false;
  e->free_drafter();
  sv_drafter dr = *d;
  std::vector<sv_draft_layer> dl(d->layers, d->layers + d->n_layers);
  auto take = [&](sv_matrix& m, uint32_t rows, uint32_t cols, const char* name) -> sv_status {
    SV_TRY(check_matrix(m, rows, cols, name));
    const bool per_row = m.gshift >= 32 || (1ull << m.gshift) >= m.k;
    if ((m.format & ~(uint32_t)SV_FMT_TILED) == SV_FMT_I8 && !per_row && m.gshift < 6)
      return fail(SV_ERR_UNSUPPORTED, "set_drafter: %s in int8 groups of %u (64 or more, or one per row, are built)", name,
                  1u << m.gshift);
    e->d_packed.push_back(nullptr);
    return pack_into(e, m, &e->d_packed.back(), &m);
  };
  sv_status st = SV_OK;
  auto run = [&]() -> sv_status {
    for (uint32_t k = 0; k < d->n_taps; k++) SV_TRY(take(dr.fc[k], H, H, "drafter fc"));
    SV_TRY(take(dr.kv_all, d->n_layers * 2 * NKV * D, H, "drafter kv_all"));
    if (dr.inject.d_w) SV_TRY(take(dr.inject, H, H, "drafter inject"));
    // A head in int8 groups under 64 (export.py writes groups of 8) runs as the exact sum of
    // two bf16 matrices, hi + lo.
    const bool head_split = (dr.head.format & ~(uint32_t)SV_FMT_TILED) == SV_FMT_I8 && dr.head.gshift < 6 &&
                            (1ull << dr.head.gshift) < dr.head.k;
    if (head_split) {
      SV_TRY(check_matrix(dr.head, d->v, H, "drafter head"));
      if (dr.head.format & SV_FMT_TILED) return fail(SV_ERR_UNSUPPORTED, "set_drafter: a tiled head in groups under 64");
      uint16_t *hi = nullptr, *lo = nullptr;
      SV_TRY(dalloc(&hi, (size_t)d->v * H, "drafter head"));
      e->d_packed.push_back(hi);
      SV_TRY(dalloc(&lo, (size_t)d->v * H, "drafter head"));
      e->d_packed.push_back(lo);
      SV_TRY(split_i8_launch(e->stream, &dr.head, hi, lo));
      SV_HIP(hipStreamSynchronize(e->stream), "drafter head");
      dr.head = sv_matrix{hi, nullptr, d->v, H, SV_FMT_BF16, 0};
      e->d_head_lo = sv_matrix{lo, nullptr, d->v, H, SV_FMT_BF16, 0};
      SV_TRY(take(e->d_head_lo, d->v, H, "drafter head"));
    }
    SV_TRY(take(dr.head, d->v, H, "drafter head"));
    uint32_t corr_w = 0;
    for (uint32_t i = 0; i < d->n_layers; i++) {
      sv_draft_layer& L = dl[i];
      SV_TRY(take(L.qkv, e->qkv_w, H, "drafter qkv"));
      SV_TRY(take(L.o, H, s.n_heads * D, "drafter o"));
      SV_TRY(take(L.gate_up, 2 * s.ffn, H, "drafter gate_up"));
      SV_TRY(take(L.down, H, s.ffn, "drafter down"));
      const bool convs = L.conv_base[0] != nullptr;
      for (int c = 0; c < 4; c++) {
        if (!convs) continue;
        if (!L.conv_base[c]) return fail(SV_ERR_ARG, "set_drafter: layer %u has conv 0 but no conv %d", i, c);
        const uint32_t w = L.conv_corr[c].m;
        if (H % 16 || w < H / 8 || (corr_w && w != corr_w))
          return fail(SV_ERR_ARG, "set_drafter: conv corrections of %u rows for hidden %u", w, H);
        corr_w = w;
        SV_TRY(take(L.conv_corr[c], w, H, "drafter conv corr"));
      }
    }
    e->d_corr_w = corr_w;
    // Rings: every key a block row sees (the window before it) plus a step's or a block's new
    // positions, in whole pages.
    const uint32_t page = 1u << e->cfg.page_shift;
    const uint32_t span = d->window + std::max(e->cfg.max_step_tokens, e->arun);
    e->d_ring_pages = (span + page - 1) / page;
    e->d_n_pages = e->cfg.max_seqs * e->d_ring_pages;
    e->d_max_pages = (e->cfg.max_seq_len + e->arun + page - 1) / page;
    const size_t ring = (size_t)d->n_layers * e->d_n_pages * NKV * page * D;
    const size_t T = e->cfg.max_step_tokens, R = (size_t)e->cfg.max_seqs * e->arun, S = e->cfg.max_seqs;
    e->d_rows_max = (uint32_t)R;
    e->d_cr = dr.inject.d_w ? e->cfg.max_step_tokens : 0u;
    SV_TRY(dalloc(&e->dk_ring, ring, "drafter rings"));
    SV_TRY(dalloc(&e->dv_ring, ring, "drafter rings"));
    SV_TRY(dalloc(&e->d_table, S * e->d_max_pages, "drafter table"));
    for (uint32_t k = 0; k < d->n_taps; k++) SV_TRY(dalloc(&e->tapbuf[k], T * H, "drafter taps"));
    SV_TRY(dalloc(&e->d_ctx, T * H, "drafter context"));
    SV_TRY(dalloc(&e->d_ctx_inv, T, "drafter context"));
    SV_TRY(dalloc(&e->d_kvp, T * d->n_layers * 2 * NKV * D, "drafter context"));
    if (e->d_cr) SV_TRY(dalloc(&e->d_cring, S * e->d_cr * H, "drafter context ring"));
    SV_TRY(dalloc(&e->d_last, R * H, "drafter rows"));
    SV_TRY(dalloc(&e->d_x, R * H, "drafter rows"));
    SV_TRY(dalloc(&e->d_qkv, R * e->qkv_w, "drafter rows"));
    SV_TRY(dalloc(&e->d_inv, R, "drafter rows"));
    SV_TRY(dalloc(&e->d_attn, R * s.n_heads * D, "drafter rows"));
    SV_TRY(dalloc(&e->d_mixed, R * H, "drafter rows"));
    SV_TRY(dalloc(&e->d_act, R * s.ffn, "drafter rows"));
    SV_TRY(dalloc(&e->d_cx, R * H, "drafter rows"));
    SV_TRY(dalloc(&e->d_co, R * H, "drafter rows"));
    if (corr_w) SV_TRY(dalloc(&e->d_corr, R * corr_w, "drafter rows"));
    SV_TRY(dalloc(&e->d_corr_inv, R, "drafter rows"));
    SV_TRY(dalloc(&e->d_logits, R * d->v, "drafter logits"));
    SV_TRY(dalloc(&e->d_cand, R * SV_DRAFT_CANDS, "drafter candidates"));
    SV_TRY(dalloc(&e->d_cand_q, R * SV_DRAFT_CANDS, "drafter candidates"));
    SV_TRY(dalloc(&e->d_meta, 2 * R, "drafter rows"));
    SV_TRY(dalloc(&e->d_tokens, R, "drafter rows"));
    SV_TRY(dalloc(&e->d_tin, 2 * R, "drafter rows"));
    SV_TRY(dalloc(&e->d_vis, R, "drafter rows"));
    SV_TRY(dalloc(&e->d_tiles, 2 * S, "drafter rows"));
    // the matmul workspace covers the drafter's shapes: the context's at the step's rows, the
    // blocks' at their rows
    size_t mws = 0;
    const uint32_t ctx_mk[][2] = {{H, H}, {d->n_layers * 2 * NKV * D, H}};
    const uint32_t blk_mk[][2] = {{H, H}, {e->qkv_w, H}, {H, s.n_heads * D}, {2 * s.ffn, H}, {H, s.ffn}, {d->v, H},
                                  {corr_w ? corr_w : H, H}};
    for (auto& x : ctx_mk)
      for (uint32_t r = 1; r <= (uint32_t)T; r++) mws = std::max(mws, matmul_ws_bytes(r, x[0], x[1]));
    for (auto& x : blk_mk)
      for (uint32_t r = 1; r <= (uint32_t)R; r++) mws = std::max(mws, matmul_ws_bytes(r, x[0], x[1]));
    SV_TRY(e->ensure_mm_ws(mws));
    std::vector<uint32_t> tab(S * e->d_max_pages);
    for (size_t slot = 0; slot < S; slot++)
      for (uint32_t pg = 0; pg < e->d_max_pages; pg++)
        tab[slot * e->d_max_pages + pg] = (uint32_t)slot * e->d_ring_pages + pg % e->d_ring_pages;
    SV_HIP(hipMemcpy(e->d_table, tab.data(), tab.size() * 4, hipMemcpyHostToDevice), "drafter table");
    // the pools start at zero (a ring position no step has written reads as zeros, not NaN)
    SV_HIP(hipMemset(e->dk_ring, 0, ring * 2), "drafter rings");
    SV_HIP(hipMemset(e->dv_ring, 0, ring * 2), "drafter rings");
    return SV_OK;
  };
  if ((st = run()) != SV_OK) {
    e->free_drafter();
    return st;
  }
  dr.layers = nullptr;
  e->dr = dr;
  e->dlayers = std::move(dl);
  e->draft_rows.assign(e->cfg.max_seqs, 0u);
  e->has_drafter = true;
  return SV_OK;
}

extern "C" sv_status sv_set_draft_rows(sv_engine* e, uint32_t slot, uint32_t rows) {
  if (!e) return fail(SV_ERR_ARG, "set_draft_rows: null engine");
  if (!e->has_drafter) return fail(SV_ERR_STATE, "set_draft_rows: no drafter set");
  if (slot >= e->cfg.max_seqs) return fail(SV_ERR_ARG, "set_draft_rows: slot %u", slot);
  if (rows > e->arun) return fail(SV_ERR_CAPACITY, "set_draft_rows: %u rows (at most %u)", rows, e->arun);
  e->draft_rows[slot] = rows;
  return SV_OK;
}

extern "C" sv_status sv_engine_draft_buffers(sv_engine* e, sv_draft_buffers* o) {
  if (!e || !o) return fail(SV_ERR_ARG, "draft_buffers: null pointer");
  if (!e->has_drafter) return fail(SV_ERR_STATE, "draft_buffers: no drafter set");
  *o = sv_draft_buffers{};
  o->d_logits = e->d_logits;
  o->d_cand = e->d_cand;
  o->d_cand_q = e->d_cand_q;
  o->d_ctx = e->d_ctx;
  for (uint32_t k = 0; k < SV_DRAFT_TAPS; k++) o->d_taps[k] = e->tapbuf[k];
  o->d_k_ring = e->dk_ring;
  o->d_v_ring = e->dv_ring;
  o->d_table = e->d_table;
  o->ring_pages = e->d_ring_pages;
  o->n_pages = e->d_n_pages;
  o->max_pages = e->d_max_pages;
  return SV_OK;
}

static sv_status check_slot(sv_engine* e, uint32_t slot) {
  if (!e) return fail(SV_ERR_ARG, "null engine");
  if (slot >= e->cfg.max_seqs || !e->used[slot]) return fail(SV_ERR_STATE, "unknown sequence %u", slot);
  return SV_OK;
}

extern "C" sv_status sv_new_seq(sv_engine* e, uint32_t* slot) {
  if (!e || !slot) return fail(SV_ERR_ARG, "new_seq: null pointer");
  uint32_t s = 0;
  while (s < e->cfg.max_seqs && e->used[s]) s++;
  if (s == e->cfg.max_seqs) return fail(SV_ERR_CAPACITY, "no free sequence slot");
  e->used[s] = true;
  e->seq_len[s] = 0;
  e->pages[s].clear();
  e->sampling[s] = sv_sample_row{0, 0, 0, 0.0f, 1.0f, SV_NO_TOK};
  const uint32_t zero = 0;
  sv_gen_state g;
  memset(&g, 0, sizeof g);
  g.remaining = 0xffffffffu;
  SV_TRY(e->upload(e->lens + s, &zero, 4));
  SV_TRY(e->upload(e->trace_len + s, &zero, 4));
  SV_TRY(e->upload(e->gen + s, &g, sizeof g));
  SV_HIP(hipStreamSynchronize(e->stream), "new_seq");
  *slot = s;
  return SV_OK;
}

extern "C" sv_status sv_free_seq(sv_engine* e, uint32_t slot) {
  SV_TRY(check_slot(e, slot));
  // kv.rs:58-60 release(): pages pushed back in reverse.
  auto& pg = e->pages[slot];
  for (auto it = pg.rbegin(); it != pg.rend(); ++it) e->free_pages.push_back(*it);
  pg.clear();
  e->used[slot] = false;
  e->seq_len[slot] = 0;
  if (e->has_drafter) e->draft_rows[slot] = 0;
  return SV_OK;
}

extern "C" sv_status sv_seq_len(sv_engine* e, uint32_t slot, uint32_t* len) {
  SV_TRY(check_slot(e, slot));
  if (!len) return fail(SV_ERR_ARG, "seq_len: null pointer");
  *len = e->seq_len[slot];
  return SV_OK;
}

extern "C" sv_status sv_seq_pages(sv_engine* e, uint32_t slot, uint32_t* pages, uint32_t cap, uint32_t* n) {
  SV_TRY(check_slot(e, slot));
  const auto& pg = e->pages[slot];
  if (n) *n = (uint32_t)pg.size();
  if (pages)
    for (uint32_t i = 0; i < pg.size() && i < cap; i++) pages[i] = pg[i];
  return SV_OK;
}

extern "C" sv_status sv_set_sampling(sv_engine* e, uint32_t slot, float temperature, float top_p, uint64_t seed) {
  SV_TRY(check_slot(e, slot));
  // engine.rs:113-120 Sampling::check.
  const bool t_ok = temperature == 0.0f || (std::isnormal(temperature) && temperature > 0.0f);
  if (!t_ok || !(top_p > 0.0f && top_p <= 1.0f))
    return fail(SV_ERR_ARG, "sampling (T %g, top_p %g): needs T 0 or normal positive, 0 < top_p <= 1", temperature,
                top_p);
  e->sampling[slot] = sv_sample_row{(uint32_t)seed, (uint32_t)(seed >> 32), 0, temperature, top_p, SV_NO_TOK};
  return SV_OK;
}

extern "C" sv_status sv_set_gen(sv_engine* e, uint32_t slot, const sv_gen_state* g) {
  SV_TRY(check_slot(e, slot));
  if (!g || g->nstop > SV_MAX_STOP) return fail(SV_ERR_ARG, "set_gen: bad state");
  SV_TRY(e->upload(e->gen + slot, g, sizeof *g));
  SV_HIP(hipStreamSynchronize(e->stream), "set_gen");
  return SV_OK;
}

extern "C" sv_status sv_bench_fill(sv_engine* e, uint32_t slot, uint32_t len) {
  SV_TRY(check_slot(e, slot));
  const uint64_t nl = (uint64_t)e->seq_len[slot] + len;
  if (nl > e->cfg.max_seq_len) return fail(SV_ERR_CAPACITY, "sequence would reach %llu tokens", (unsigned long long)nl);
  SV_TRY(e->reserve(slot, (uint32_t)nl));
  e->seq_len[slot] = (uint32_t)nl;
  const uint32_t v = (uint32_t)nl;
  SV_TRY(e->upload(e->lens + slot, &v, 4));
  SV_HIP(hipStreamSynchronize(e->stream), "bench_fill");
  return SV_OK;
}

extern "C" sv_status sv_settle(sv_engine* e, uint32_t slot, uint32_t unused) {
  SV_TRY(check_slot(e, slot));
  if (unused > e->seq_len[slot]) return fail(SV_ERR_ARG, "settle: %u unused of %u", unused, e->seq_len[slot]);
  e->seq_len[slot] -= unused;
  return SV_OK;
}

extern "C" sv_status sv_set_feed(sv_engine* e, uint32_t slot, uint32_t len, uint32_t token) {
  SV_TRY(check_slot(e, slot));
  if (len > e->cfg.max_seq_len) return fail(SV_ERR_CAPACITY, "set_feed: length %u", len);
  if (token >= e->sh.vocab) return fail(SV_ERR_ARG, "set_feed: token %u", token);
  SV_TRY(e->reserve(slot, len));
  e->seq_len[slot] = len;
  SV_TRY(e->upload(e->lens + slot, &len, 4));
  SV_TRY(e->upload(e->feed + (size_t)slot * SV_FEED_W, &token, 4));
  SV_HIP(hipStreamSynchronize(e->stream), "set_feed");
  return SV_OK;
}

extern "C" sv_status sv_set_replay(sv_engine* e, uint32_t seed, float rate) {
  if (!e) return fail(SV_ERR_ARG, "set_replay: null engine");
  e->replay.seed = seed;
  e->replay.rate = rate;
  return SV_OK;
}

// plan.rs:47-151 Engine::plan.
extern "C" sv_status sv_plan(sv_engine* e, const sv_run* runs_in, uint32_t n_runs, uint32_t extra_keys,
                             sv_plan_info* info) {
  if (!e || (!runs_in && n_runs)) return fail(SV_ERR_ARG, "plan: null pointer");
  if (n_runs == 0) return fail(SV_ERR_ARG, "plan: no runs");
  if (n_runs > e->cfg.max_seqs) return fail(SV_ERR_CAPACITY, "plan: %u runs", n_runs);
  if (e->graph) {
    (void)hipGraphExecDestroy(e->graph);
    e->graph = nullptr;
  }
  SV_HIP(hipStreamSynchronize(e->stream), "plan");
  uint32_t n = 0;
  for (uint32_t ri = 0; ri < n_runs; ri++) n += runs_in[ri].count;
  if (n == 0 || n > e->cfg.max_step_tokens)
    return fail(SV_ERR_CAPACITY, "step has %u tokens (max %u)", n, e->cfg.max_step_tokens);
  std::vector<uint32_t> tokens, tin, vis, head_rows, attn_runs;
  std::vector<sv_sample_row> samples;
  std::vector<sv_run_in> run_in;
  Plan P;
  uint32_t max_cached = 0;
  std::vector<uint32_t> run_cached;
  for (uint32_t ri = 0; ri < n_runs; ri++) {
    const sv_run& r = runs_in[ri];
    SV_TRY(check_slot(e, r.slot));
    if (r.count == 0 || (r.verify && r.count > e->arun))
      return fail(SV_ERR_CAPACITY, "%u tokens for one sequence in a verify step (max %u)", r.count, e->arun);
    if (!r.tokens) return fail(SV_ERR_ARG, "plan: run %u has no tokens", ri);
    for (uint32_t j = 0; j < ri; j++)
      if (runs_in[j].slot == r.slot) return fail(SV_ERR_ARG, "a sequence appears twice in one step");
    for (uint32_t i = 0; i < r.count; i++) {
      const uint32_t t = r.tokens[i];
      if (t >= SV_FEED_ROW ? t - SV_FEED_ROW >= SV_FEED_W : t >= e->sh.vocab)
        return fail(SV_ERR_ARG, "token id %u out of range", t);
    }
    const uint64_t new_len = (uint64_t)e->seq_len[r.slot] + r.count;
    if (new_len > e->cfg.max_seq_len)
      return fail(SV_ERR_CAPACITY, "sequence would reach %llu tokens (max %u)", (unsigned long long)new_len,
                  e->cfg.max_seq_len);
  }
  // Pages for every position a replay of this plan can reach: the step's own rows plus
  // `extra_keys` more (capped at the sequence limit). A replay reads no host state, so the
  // number of steps the plan may run is bounded by the run with the least headroom.
  uint64_t budget = UINT64_MAX;
  for (uint32_t ri = 0; ri < n_runs; ri++) {
    const sv_run& r = runs_in[ri];
    const uint64_t want = std::min<uint64_t>((uint64_t)e->seq_len[r.slot] + r.count + extra_keys, e->cfg.max_seq_len);
    budget = std::min<uint64_t>(budget, (want - e->seq_len[r.slot]) / r.count);
  }
  for (uint32_t ri = 0; ri < n_runs; ri++) {
    const sv_run& r = runs_in[ri];
    const uint32_t slot = r.slot, count = r.count;
    const uint32_t want = (uint32_t)std::min<uint64_t>((uint64_t)e->seq_len[slot] + count + extra_keys,
                                                       e->cfg.max_seq_len);
    SV_TRY(e->reserve(slot, want));
    const uint32_t first_row = (uint32_t)tokens.size();
    for (uint32_t row = 0; row < count; row++) {
      tokens.push_back(r.tokens[row]);
      tin.push_back(slot);
      tin.push_back(row);
      vis.push_back(0xffffffffu >> (31 - row % e->arun));  // causal within its attention run (plan.rs:81)
    }
    const uint32_t first_head = (uint32_t)head_rows.size();
    if (r.verify)
      for (uint32_t x = first_row; x < first_row + count; x++) head_rows.push_back(x);
    else if (r.head)
      head_rows.push_back(first_row + count - 1);
    for (uint32_t hx = first_head; hx < head_rows.size(); hx++) {
      sv_sample_row s = e->sampling[slot];  // engine.rs:134-137 row_of
      s.pos = 0;
      s.tok = head_rows[hx];
      samples.push_back(s);
    }
    run_in.push_back(sv_run_in{slot, first_row, count, first_head, (uint32_t)head_rows.size() - first_head,
                               r.verify ? 1u : 0u});
    // Attention runs of at most arun rows: a prompt chunk's later ones see its earlier rows as
    // cached keys (plan.rs:99-104 tiles the chunk path the same way, in 8s).
    for (uint32_t j = 0; j < count; j += e->arun) {
      const uint32_t c = std::min(e->arun, count - j);
      attn_runs.push_back(first_row + j);
      attn_runs.push_back(c);
      P.inl.insert(P.inl.end(), {first_row + j, c, slot});
      max_cached = std::max(max_cached, e->seq_len[slot] + j);
      run_cached.push_back(e->seq_len[slot] + j);
    }
    P.max_run = std::max(P.max_run, std::min(count, e->arun));
    P.chunk = P.chunk || count > e->arun;
    P.branches |= (r.verify && count > 2) ? 1u : 0u;
    P.slots.push_back(slot);
    P.counts.push_back(count);
    P.verify.push_back(r.verify ? 1u : 0u);
    e->seq_len[slot] += count;
  }
  if (head_rows.size() > e->cfg.max_head_rows)
    return fail(SV_ERR_CAPACITY, "%zu head rows (max %u)", head_rows.size(), e->cfg.max_head_rows);
  P.n = n;
  P.n_attn = (uint32_t)attn_runs.size() / 2;
  P.budget = budget;
  P.n_head = (uint32_t)head_rows.size();
  P.n_runs = n_runs;
  // Attention splits: the cached keys of each run in splits of `split`, plus a split of its
  // own for the new keys; `extra_keys` sizes the grid for replays at later positions.
  uint32_t split = e->cfg.split_keys;
  if (split == 0)
    split = choose_split(run_cached, extra_keys, e->sh.n_kv_heads, P.max_run, e->sh.n_heads / e->sh.n_kv_heads);
  P.split = split;
  P.max_splits = (max_cached + extra_keys + split - 1) / split + 1;
  // Sliding-window layers: a run's cached keys start at its window (rounded down to 32 keys),
  // so at most window + 31 of them at any replay.
  P.split_local = split;
  P.max_splits_local = P.max_splits;
  if (e->n_local) {
    const uint32_t span = e->cfg.window + 31;
    std::vector<uint32_t> lc;
    uint32_t max_lc = 0;
    for (uint32_t c : run_cached) {
      lc.push_back((uint32_t)std::min<uint64_t>((uint64_t)c + extra_keys, span));
      max_lc = std::max(max_lc, lc.back());
    }
    P.split_local = e->cfg.split_keys ? e->cfg.split_keys
                                      : choose_split(lc, 0, e->sh.n_kv_heads, P.max_run, e->sh.n_heads / e->sh.n_kv_heads);
    P.max_splits_local = (max_lc + P.split_local - 1) / P.split_local + 1;
  }
  // The drafter's blocks (generate.rs:406-411 draft_runs): one per run that draws a token this
  // step and whose slot has draft rows, its rows all seeing each other (drafter.rs:327-334).
  std::vector<uint32_t> dtin, dvis, dtiles;
  if (e->has_drafter) {
    std::vector<uint32_t> bc;
    uint32_t max_bc = 0;
    const uint32_t span = e->dr.window + 31;
    for (uint32_t ri = 0; ri < n_runs; ri++) {
      const sv_run& r = runs_in[ri];
      const uint32_t rows = e->draft_rows[r.slot];
      if (!rows || !(r.verify || r.head)) continue;
      const uint32_t first = (uint32_t)dvis.size();
      dtiles.insert(dtiles.end(), {first, rows});
      P.dinl.insert(P.dinl.end(), {first, rows, r.slot});
      for (uint32_t i = 0; i < rows; i++) {
        dtin.insert(dtin.end(), {r.slot, i});
        dvis.push_back((1u << rows) - 1u);
      }
      P.d_max_run = std::max(P.d_max_run, rows);
      bc.push_back((uint32_t)std::min<uint64_t>((uint64_t)e->seq_len[r.slot] + extra_keys, span));
      max_bc = std::max(max_bc, bc.back());
    }
    P.n_blocks = (uint32_t)bc.size();
    P.d_rows = (uint32_t)dvis.size();
    if (P.n_blocks) {
      P.d_split = e->cfg.split_keys ? e->cfg.split_keys
                                    : choose_split(bc, 0, e->sh.n_kv_heads, P.d_max_run, e->sh.n_heads / e->sh.n_kv_heads);
      P.d_max_splits = (max_bc + P.d_split - 1) / P.d_split + 1;
    }
  }
  size_t need = attn_ws_bytes(&e->sh, P.n_attn, std::max(P.max_splits, P.max_splits_local), P.max_run);
  if (P.n_blocks) need = std::max(need, attn_ws_bytes(&e->sh, P.n_blocks, P.d_max_splits, P.d_max_run));
  SV_TRY(e->ensure_ws(need));
  if (P.n_blocks) {
    SV_TRY(e->upload(e->d_tin, dtin.data(), dtin.size() * 4));
    SV_TRY(e->upload(e->d_vis, dvis.data(), dvis.size() * 4));
    SV_TRY(e->upload(e->d_tiles, dtiles.data(), dtiles.size() * 4));
  }
  SV_TRY(e->upload(e->tokens, tokens.data(), tokens.size() * 4));
  SV_TRY(e->upload(e->tin, tin.data(), tin.size() * 4));
  SV_TRY(e->upload(e->vis, vis.data(), vis.size() * 4));
  SV_TRY(e->upload(e->head_rows, head_rows.data(), head_rows.size() * 4));
  SV_TRY(e->upload(e->sample_rows, samples.data(), samples.size() * sizeof(sv_sample_row)));
  SV_TRY(e->upload(e->runs, run_in.data(), run_in.size() * sizeof(sv_run_in)));
  SV_TRY(e->upload(e->attn_runs, attn_runs.data(), attn_runs.size() * 4));
  SV_TRY(e->plan_layers(P));
  SV_HIP(hipStreamSynchronize(e->stream), "plan upload");
  e->plan = P;
  e->planned = true;
  if (info) {
    info->n_tokens = P.n;
    info->n_head = P.n_head;
    info->n_runs = P.n_runs;
    info->branches = P.branches;
    info->max_run = P.max_run;
    info->split = P.split;
    info->max_splits = P.max_splits;
  }
  return SV_OK;
}

extern "C" sv_status sv_encode(sv_engine* e, uint32_t flags) {
  if (!e) return fail(SV_ERR_ARG, "encode: null engine");
  SV_TRY(e->issue(1));
  return e->encode(flags);
}

extern "C" sv_status sv_graph_capture(sv_engine* e, uint32_t flags) {
  if (!e) return fail(SV_ERR_ARG, "graph_capture: null engine");
  SV_TRY(e->check_ready());
  if (!e->planned) return fail(SV_ERR_STATE, "graph_capture: no plan");
  if (e->graph) {
    (void)hipGraphExecDestroy(e->graph);
    e->graph = nullptr;
  }
  SV_HIP(hipStreamSynchronize(e->stream), "graph_capture");
  SV_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal), "begin capture");
  const sv_status st = e->encode(flags);
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(e->stream, &g);
  if (st != SV_OK) {
    if (g) (void)hipGraphDestroy(g);
    return st;
  }
  SV_HIP(ec, "end capture");
  const hipError_t ei = hipGraphInstantiate(&e->graph, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  SV_HIP(ei, "graph instantiate");
  return SV_OK;
}

extern "C" sv_status sv_graph_replay(sv_engine* e, uint32_t count) {
  if (!e || !e->graph) return fail(SV_ERR_STATE, "graph_replay: no graph");
  SV_TRY(e->issue(count));
  for (uint32_t i = 0; i < count; i++) SV_HIP(hipGraphLaunch(e->graph, e->stream), "graph launch");
  return SV_OK;
}

extern "C" sv_status sv_sync(sv_engine* e) {
  if (!e) return fail(SV_ERR_ARG, "sync: null engine");
  SV_HIP(hipStreamSynchronize(e->stream), "sync");
  return e->check_layers();
}

// engine.rs:310-314 step, with generate.rs:446-463 collect: plan, encode, wait, read the
// head rows' ids (and logits), the tokens each run emitted, and give back a verify run's
// unused positions (settle).
// sv_step after its plan: encode, wait, read the outputs, roll back the rejected rows' lengths.
static sv_status step_planned(sv_engine* e, const sv_run* runs, uint32_t n_runs, uint32_t flags, uint32_t* ids,
                              float* logits, uint32_t* emitted, const sv_plan_info& pi) {
  SV_TRY(e->issue(1));
  SV_TRY(e->encode(flags));
  SV_HIP(hipStreamSynchronize(e->stream), "step");
  SV_TRY(e->check_layers());
  std::vector<uint32_t> em(n_runs);
  SV_HIP(hipMemcpy(em.data(), e->emitted, n_runs * 4, hipMemcpyDeviceToHost), "step emitted");
  if (ids && pi.n_head) SV_HIP(hipMemcpy(ids, e->out_ids, pi.n_head * 4, hipMemcpyDeviceToHost), "step ids");
  if (logits && pi.n_head)
    SV_HIP(hipMemcpy(logits, e->logits, (size_t)pi.n_head * e->sh.vocab * 4, hipMemcpyDeviceToHost), "step logits");
  if (emitted) memcpy(emitted, em.data(), n_runs * 4);
  for (uint32_t ri = 0; ri < n_runs; ri++)
    if (runs[ri].verify) {
      const uint32_t slot = runs[ri].slot;
      e->seq_len[slot] -= runs[ri].count - std::min(em[ri], runs[ri].count);
    }
  return SV_OK;
}

extern "C" sv_status sv_step(sv_engine* e, const sv_run* runs, uint32_t n_runs, uint32_t flags, uint32_t* ids,
                             float* logits, uint32_t* emitted, sv_plan_info* info) {
  sv_plan_info pi;
  SV_TRY(sv_plan(e, runs, n_runs, 0, &pi));
  if (info) *info = pi;
  return step_planned(e, runs, n_runs, flags, ids, logits, emitted, pi);
}

// engine.rs:318-355 step_capture: the step's layers one at a time, each layer's intermediates
// written to buffers of this call and handed to fn after the layer.
extern "C" sv_status sv_step_capture(sv_engine* e, const sv_run* runs, uint32_t n_runs, uint32_t flags,
                                     sv_capture_fn fn, void* user, uint32_t* ids, float* logits, uint32_t* emitted,
                                     sv_plan_info* info) {
  if (!e || !fn) return fail(SV_ERR_ARG, "step_capture: null engine or callback");
  sv_plan_info pi;
  SV_TRY(sv_plan(e, runs, n_runs, 0, &pi));
  if (info) *info = pi;
  const uint32_t n = e->plan.n, H = e->sh.hidden, NQD = e->sh.n_heads * e->sh.head_dim;
  const uint32_t NKD = e->sh.n_kv_heads * e->sh.head_dim;
  sv_engine::Capture c;
  c.fn = fn;
  c.user = user;
  std::vector<void*> bufs;
  sv_status st = SV_OK;
  auto alloc = [&](float** p, size_t floats) {
    if (st != SV_OK) return;
    if (hipMalloc((void**)p, floats * 4) != hipSuccess) {
      st = fail(SV_ERR_HIP, "step_capture: %zu bytes of capture buffers", floats * 4);
      return;
    }
    bufs.push_back(*p);
  };
  alloc((float**)&c.iota, n);
  for (float** p : {&c.resid_in, &c.attn_in, &c.attn_out, &c.mlp_in, &c.mlp_out, &c.base}) alloc(p, (size_t)n * H);
  for (float** p : {&c.q, &c.sdpa}) alloc(p, (size_t)n * NQD);
  for (float** p : {&c.k, &c.v}) alloc(p, (size_t)n * NKD);
  std::vector<uint32_t> iota(n);  // outlives the asynchronous upload (the step waits for it)
  for (uint32_t i = 0; i < n; i++) iota[i] = i;
  if (st == SV_OK) st = e->upload(c.iota, iota.data(), n * 4);
  if (st == SV_OK) {
    e->capture = &c;
    st = step_planned(e, runs, n_runs, flags, ids, logits, emitted, pi);
    e->capture = nullptr;
    g_attn_capture = AttnCapture{};
  }
  (void)hipStreamSynchronize(e->stream);
  for (void* b : bufs) (void)hipFree(b);
  return st;
}

extern "C" sv_status sv_profile_step(sv_engine* e, uint32_t flags, uint32_t reps, float* ms, uint32_t* launches) {
  if (!e || !ms || !launches) return fail(SV_ERR_ARG, "profile_step: null pointer");
  SV_HIP(hipStreamSynchronize(e->stream), "profile_step");
  SV_TRY(e->issue(reps));
  e->prof = true;
  e->prof_events.clear();
  sv_status st = SV_OK;
  for (uint32_t r = 0; r < reps && st == SV_OK; r++) st = e->encode(flags);
  e->prof = false;
  const hipError_t sync = hipStreamSynchronize(e->stream);
  for (auto& pe : e->prof_events) {
    float t = 0.0f;
    if (st == SV_OK && sync == hipSuccess && hipEventElapsedTime(&t, pe.second.first, pe.second.second) == hipSuccess &&
        pe.first >= 0 && pe.first < SV_KIND_COUNT) {
      ms[pe.first] += t;
      launches[pe.first] += 1;
    }
    (void)hipEventDestroy(pe.second.first);
    (void)hipEventDestroy(pe.second.second);
  }
  e->prof_events.clear();
  SV_TRY(st);
  SV_HIP(sync, "profile_step");
  return SV_OK;
}

// hooks.rs:41-55 sample_logits.
extern "C" sv_status sv_sample_logits(sv_engine* e, const float* logits, uint32_t rows, const float* temperature,
                                      const float* top_p, const uint64_t* seed, const uint32_t* pos, uint32_t* ids) {
  if (!e || !logits || !temperature || !top_p || !seed || !pos || !ids) return fail(SV_ERR_ARG, "sample_logits: null");
  if (rows == 0 || rows > std::max(e->cfg.max_head_rows, e->cfg.max_step_tokens))
    return fail(SV_ERR_CAPACITY, "%u rows of logits", rows);
  std::vector<sv_sample_row> s(rows);
  for (uint32_t r = 0; r < rows; r++) {
    const float t = temperature[r], p = top_p[r];
    if (!(t == 0.0f || (std::isnormal(t) && t > 0.0f)) || !(p > 0.0f && p <= 1.0f))
      return fail(SV_ERR_ARG, "row %u: T %g top_p %g", r, t, p);
    s[r] = sv_sample_row{(uint32_t)seed[r], (uint32_t)(seed[r] >> 32), pos[r], t, p, SV_NO_TOK};
  }
  SV_HIP(hipStreamSynchronize(e->stream), "sample_logits");
  SV_TRY(e->upload(e->logits, logits, (size_t)rows * e->sh.vocab * 4));
  SV_TRY(e->upload(e->sample_rows, s.data(), rows * sizeof(sv_sample_row)));
  SV_TRY(sample_launch(e->stream, e->logits, e->sample_rows, e->out_ids, e->meta, rows, e->sh.vocab));
  SV_HIP(hipStreamSynchronize(e->stream), "sample_logits");
  SV_HIP(hipMemcpy(ids, e->out_ids, rows * 4, hipMemcpyDeviceToHost), "sample_logits ids");
  e->planned = false;
  return SV_OK;
}
