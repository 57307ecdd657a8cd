// sv_internal.h — host-side declarations shared by the translation units of libsv_verify.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/sv_verify.h"

namespace sv {

// Per-kernel timing (sv_profile_step): when `start` is set, the next launch through sv::launch
// records the pair at the kernel's own start and end (hipExtLaunchKernelGGL), so the elapsed
// time is the kernel's execution as a profiler sees it, without the dispatch around it.
struct ProfEvents {
  hipEvent_t start = nullptr, stop = nullptr;
  bool used = false;
};
extern thread_local ProfEvents g_prof;

template <typename K, typename... A>
inline void launch(K kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t stream, A... args) {
  if (g_prof.start && !g_prof.used) {
    hipExtLaunchKernelGGL(kernel, grid, block, shm, stream, g_prof.start, g_prof.stop, 0, args...);
    g_prof.used = true;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shm, stream, args...);
  }
}


// Record a thread-local error message and return `code` (sv_last_error reads it).
sv_status fail(sv_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// SV_OK, or SV_ERR_HIP with the launch error of the last kernel.
sv_status check_launch(const char* what);
// SV_OK, or SV_ERR_HIP with the message of `e`.
sv_status check_hip(hipError_t e, const char* what);

size_t matmul_ws_bytes(uint32_t n, uint32_t m, uint32_t k);
// Launch-shape override for the skinny matmul (row tiles, waves, k splits; zero: built-in)
// and the path for more than 16 rows (0: built-in, 1: skinny, 2: GEMM).
struct SkinnyTune {
  int rt, w, s, path, splits;
};
// The variant of the last matmul launched on this process (1 skinny, 2 GEMM, 3 one-shot): tests.
extern int g_mm_variant;
// GEMM launch-shape override (row tiles per wave, token tiles, k splits, chunks in flight;
// zero: built-in).
struct GemmTune {
  int rtw, nt, s, d, mf, nw, cpi;  // mf: MFMA tile (16 or 32); nw: waves (4); cpi: chunks per barrier (1)
};
// The capture buffers attn_launch passes to the kernels (the engine's sv_step_capture sets
// them around a layer's attention launches on its thread; null: no capture).
struct AttnCapture {
  float* q = nullptr;
  float* k = nullptr;
  float* v = nullptr;
  float* sdpa = nullptr;
};
extern thread_local AttnCapture g_attn_capture;
extern GemmTune g_gemm_tune;
extern int g_gemm_order;  // tests: the GEMMs' work order (-1: modelled choice; 0 legacy; g: groups of g row blocks)
extern SkinnyTune g_skinny_tune;  // path 3: the one-shot 1-16 row kernel with (rt, w, s = chunks per wave, splits)
sv_status pack_matrix(hipStream_t stream, const sv_matrix* src, void* dst, sv_matrix* out);
sv_status matmul_launch(hipStream_t stream, const sv_matrix* w, const float* x, const uint32_t* x_rows, float* y,
                        const float* base, float* aux, const sv_mat_args* a, void* ws, size_t ws_bytes);

void attn_init();
void matmul_init();  // kernel attributes; call outside stream capture
size_t attn_ws_bytes(const sv_shape* sh, uint32_t n_runs, uint32_t max_splits, uint32_t max_run);
sv_status attn_launch(hipStream_t stream, const sv_shape* sh, const float* qkv, const uint32_t* meta,
                      uint16_t* k_cache, uint16_t* v_cache, const uint32_t* page_table, const float* rope,
                      const sv_kv_args* kv, const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs,
                      uint32_t max_run, const uint32_t* vis, float* out, void* ws, size_t ws_bytes,
                      uint32_t parts = 3,  // bits: 1 attention, 2 split merge, 4 new K/V first, 8 capture q/k/v
                      const uint32_t* host_runs = nullptr,  // (first token, rows, slot) per run, if known
                      bool may_fuse = true,  // the counted last-split merge may be used (tests select it)
                      const sv_attn_extras* ex = nullptr,   // the layer's extras (null: none)
                      // the step's rope words by token (embed_launch writes them); inline runs need them
                      const float* rope_rows = nullptr);
// attn_launch with the split partials in the library's per-device static scratch array.
sv_status attn_launch_noalloc(hipStream_t stream, const sv_shape* sh, const float* qkv, const uint32_t* meta,
                              uint16_t* k_cache, uint16_t* v_cache, const uint32_t* page_table, const float* rope,
                              const sv_kv_args* kv, const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs,
                              uint32_t max_run, const uint32_t* vis, float* out);
size_t attn_scratch_bytes();

// Fills `out` (an AttnParams) as attn_launch would for these arguments (the inline runs given),
// for the persistent layer kernel's attention and merge phases.
sv_status attn_params_fill(void* out, const sv_shape* sh, const float* qkv, const uint32_t* meta, uint16_t* k_cache,
                           uint16_t* v_cache, const uint32_t* page_table, const float* rope_rows,
                           const sv_kv_args* kv, const sv_attn_args* args, const uint32_t* host_runs,
                           uint32_t n_runs, uint32_t max_run, const uint32_t* vis, float* o, float* part_o,
                           float* part_l);
size_t attn_part_floats(const sv_shape* sh, uint32_t n_runs, uint32_t max_splits, uint32_t max_run, size_t* l_off);

// tokens_out may equal tokens (resolution in place, as the reference's embed).
sv_status embed_launch(hipStream_t stream, const sv_shape* sh, const uint16_t* table, const uint32_t* tokens,
                       uint32_t* tokens_out, float* out, const uint32_t* tin, uint32_t* meta, const uint32_t* lens,
                       const uint32_t* feed, const uint32_t* tree, uint32_t* vis, uint32_t n,
                       const float* rope = nullptr,  // with rope_rows: the table's row at each token's position
                       float* rope_rows = nullptr, uint32_t rope_n = 0,  // rope_n: the table's rows
                       uint32_t* epoch = nullptr);  // incremented once (the persistent kernel's step count)
sv_status head_cap_launch(hipStream_t stream, float* logits, uint32_t rows, uint32_t vocab, uint32_t vocab_real);
sv_status rmsnorm_rows_launch(hipStream_t stream, const float* in, const uint32_t* rows, float* out, uint32_t n,
                              uint32_t hidden);
sv_status sample_launch(hipStream_t stream, const float* logits, const sv_sample_row* rows, uint32_t* out,
                        const uint32_t* meta, uint32_t n_rows, uint32_t vocab);
sv_status accept_launch(hipStream_t stream, const sv_run_in* runs, const uint32_t* tokens, uint32_t* out,
                        uint32_t* lens, uint32_t* feed, sv_gen_state* gen, uint32_t* emitted, uint32_t nruns,
                        const uint32_t* tree, uint32_t* path, uint32_t* path_len, uint32_t* on_path);
sv_status kv_compact_launch(hipStream_t stream, const sv_shape* sh, const sv_run_in* runs, uint32_t nruns,
                            const uint32_t* path, const uint32_t* path_len, const uint32_t* lens, uint16_t* k_cache,
                            uint16_t* v_cache, const uint32_t* page_table, const sv_kv_args* kv);
sv_status draft_top_launch(hipStream_t stream, const float* logits, const uint32_t* vocab, const uint32_t* tin,
                           uint32_t* cand, float* cand_q, uint32_t n_rows, uint32_t nv, float inv_t, uint32_t ncand);
sv_status draft_tree_launch(hipStream_t stream, const uint32_t* blocks, uint32_t nblocks, const uint32_t* tin,
                            const uint32_t* cand, const float* cand_q, uint32_t* feed, uint32_t* tree, uint32_t ncand);
sv_status replay_launch(hipStream_t stream, const sv_run_in* runs, uint32_t nruns, const uint32_t* lens,
                        uint32_t* feed, const uint32_t* trace, const uint32_t* trace_len, const sv_replay_args* ra,
                        uint32_t* tree);

sv_status tap_rows_launch(hipStream_t stream, const float* in, float* out, uint32_t n, uint32_t hidden);
sv_status draft_kv_launch(hipStream_t stream, const sv_shape* sh, const float* kvp, const uint32_t* meta,
                          const uint32_t* on_path, const float* rope, uint16_t* kc, uint16_t* vc, const uint32_t* table,
                          const sv_kv_args* kv, uint32_t n, uint32_t n_layers);
sv_status draft_ctx_launch(hipStream_t stream, const float* ctx, const float* ctx_inv, const uint32_t* meta,
                           const uint32_t* on_path, float* ring, uint32_t cr, uint32_t n, uint32_t hidden);
sv_status draft_embed_launch(hipStream_t stream, const uint16_t* embed, const uint32_t* tin, const uint32_t* lens,
                             const uint32_t* feed, const float* mask_emb, float* x, uint32_t* meta, uint32_t* tokens,
                             const float* ring, float* last, uint32_t cr, uint32_t rows, uint32_t hidden);
sv_status split_i8_launch(hipStream_t stream, const sv_matrix* w, uint16_t* hi, uint16_t* lo);
sv_status draft_conv_launch(hipStream_t stream, const float* x, const float* corr, uint32_t corr_w, const float* base,
                            const uint32_t* tin, const float* resid, float* out, uint32_t rows, uint32_t hidden);
sv_status mudd_launch(hipStream_t stream, const float* cur, const float* tap0, const float* tap1, const float* dense1,
                      const float* mix, float* out_attn, float* out_base, uint32_t n, uint32_t hidden);

// A paged K/V cache kv_compact moves rows in: n_layers layers of n_pages pages through `table`.
struct KvCacheRef {
  uint16_t* kc;
  uint16_t* vc;
  const uint32_t* table;
  uint32_t n_layers, n_pages;
};
// accept, then (optionally) kv_compact over caches[0..n_caches) and the replay drafter, one
// workgroup per run.
sv_status step_tail_launch(hipStream_t stream, const sv_shape* sh, const sv_run_in* runs, uint32_t nruns,
                           const uint32_t* tokens, uint32_t* out, uint32_t* lens, uint32_t* feed, sv_gen_state* gen,
                           uint32_t* emitted, uint32_t* tree, uint32_t* path, uint32_t* path_len, uint32_t* on_path,
                           bool compact, const KvCacheRef* caches, uint32_t n_caches, uint32_t page_shift,
                           uint32_t max_pages, const sv_replay_args* ra, const uint32_t* trace,
                           const uint32_t* trace_len);


}  // namespace sv
