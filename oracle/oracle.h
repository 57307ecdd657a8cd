/*
 * oracle.h — CPU restatement of the reference's verify path, for TESTS ONLY.
 *
 * This is test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker (or the timed CPU baseline).
 * The product path (libsv_verify.so) never calls it.
 *
 * Each function cites the reference file:line whose semantics it restates. Matmuls and
 * attention accumulate in double (the reference's exact-arithmetic result; its own fp32
 * order differs between its GEMV, streaming-GEMM and GEMM variants, kernels.metal:211-690),
 * the sampler and every integer routine mirror the reference's operation order exactly.
 *
 * Pinning (what checks each function independently of its own formula) is listed in the
 * header comment of oracle.c.
 */
#ifndef SV_ORACLE_H
#define SV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/sv_verify.h"

#ifdef __cplusplus
extern "C" {
#endif

/* scalars */
float orc_bf(uint16_t u);
uint16_t orc_to_bf(float f);
float orc_round_bf16(float x);
void orc_philox(uint32_t ctr[4], const uint32_t key[2]);
float orc_uniform01(uint32_t seed_lo, uint32_t seed_hi, uint32_t pos, uint32_t round);
float orc_exp2(float x);
void orc_draft_top(const float* logits, const uint32_t* vocab, const uint32_t* tin, uint32_t* cand, float* cand_q,
                   uint32_t n_rows, uint32_t nv, float inv_t, uint32_t ncand);
void orc_draft_tree(const uint32_t* blocks, uint32_t nblocks, const uint32_t* tin, const uint32_t* cand,
                    const float* cand_q, uint32_t* feed, uint32_t* tree, uint32_t ncand);
void orc_to_bf_array(const float* x, uint16_t* out, size_t n);
void orc_exp2_array(const float* x, float* out, size_t n);

/* data formats */
void orc_quantize(const float* w, uint32_t m, uint32_t k, uint32_t group, int8_t* q, uint16_t* s);
void orc_rope_table(const float* freq, uint32_t n_pos, float* tab);

/* kernels */
void orc_embed(const sv_shape* sh, const uint16_t* table, uint32_t* tokens, float* out, const uint32_t* tin,
               uint32_t* meta, const uint32_t* lens, const uint32_t* feed, const uint32_t* tree, uint32_t* vis,
               uint32_t n);
void orc_rmsnorm_rows(const float* in, const uint32_t* rows, float* out, uint32_t n, uint32_t hidden);
void orc_matmul(const sv_matrix* w, const float* x, const uint32_t* x_rows, float* y, const float* base, float* aux,
                const sv_mat_args* a);
void orc_attn_verify(const sv_shape* sh, const float* qkv, const uint32_t* meta, uint16_t* k_cache,
                     uint16_t* v_cache, const uint32_t* page_table, const float* rope, const sv_kv_args* kv,
                     const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs, const uint32_t* vis,
                     float* out, const sv_attn_extras* ex);
void orc_mudd(const float* cur, const float* tap0, const float* tap1, const float* dense1, const float* mix,
              float* out_attn, float* out_base, uint32_t n, uint32_t hidden);
void orc_sample(const float* logits, const sv_sample_row* rows, uint32_t* out, const uint32_t* meta,
                uint32_t n_rows, uint32_t vocab);
void orc_accept(const sv_run_in* runs, const uint32_t* tokens, uint32_t* out, uint32_t* lens, uint32_t* feed,
                sv_gen_state* gen, uint32_t* emitted, uint32_t nruns, const uint32_t* tree, uint32_t* path,
                uint32_t* path_len, uint32_t* on_path);
void orc_kv_compact(const sv_shape* sh, const sv_run_in* runs, uint32_t nruns, const uint32_t* path,
                    const uint32_t* path_len, const uint32_t* lens, uint16_t* k_cache, uint16_t* v_cache,
                    const uint32_t* page_table, const sv_kv_args* kv);
void orc_replay_draft(const sv_run_in* runs, uint32_t nruns, const uint32_t* lens, uint32_t* feed,
                      const uint32_t* trace, const uint32_t* trace_len, const sv_replay_args* ra, uint32_t* tree);

/* page pool (kv.rs:40-60): LIFO free list initialised (0..n).rev() */
typedef struct orc_pool {
  uint32_t* free_list; /* [n_pages] */
  uint32_t n_free, n_pages, max_pages, page_shift;
  uint32_t* page_table; /* [max_seqs][max_pages] */
  uint32_t* seq_pages;  /* [max_seqs] pages held  */
} orc_pool;
void orc_pool_init(orc_pool* p, uint32_t n_pages, uint32_t max_seqs, uint32_t max_pages, uint32_t page_shift,
                   uint32_t* free_list, uint32_t* page_table, uint32_t* seq_pages);
int orc_pool_reserve(orc_pool* p, uint32_t slot, uint32_t len); /* 0 ok, -1 exhausted */
void orc_pool_release(orc_pool* p, uint32_t slot);

/* A step plan (plan.rs:47-151, without the split sizing). in_runs: (slot, count, verify,
 * head) per run, in_tokens: the runs' tokens back to back. Outputs sized by the caller:
 * tokens[n], tin[2n], vis[n], head_rows[n], samples[n], run_in[n_runs]. seq_len[] is the
 * host-side length per slot, advanced by each run (optimistically, as the reference).
 * Returns n_head, or -1 on a rejected plan. */
int orc_plan(const uint32_t* in_runs, uint32_t n_runs, const uint32_t* in_tokens, uint32_t* seq_len,
             const sv_sample_row* sampling_per_slot, uint32_t* tokens, uint32_t* tin, uint32_t* vis,
             uint32_t* head_rows, sv_sample_row* samples, sv_run_in* run_in, uint32_t arun);

/* The whole verify step on host memory (encode.rs:99-126 encode_forward + encode_tail
 * 383-412). Weights in `layers` and `embed` are host pointers. */
typedef struct orc_step_io {
  /* plan */
  uint32_t n, n_head, n_runs;
  uint32_t* tokens;          /* [n], resolved in place          */
  const uint32_t* tin;       /* [n][2]                           */
  uint32_t* vis;             /* [n]                              */
  const uint32_t* head_rows; /* [n_head]                         */
  const sv_sample_row* samples;
  const sv_run_in* runs;
  const uint32_t* attn_runs; /* [n_attn][2] (first, count <= 16) */
  uint32_t compact;          /* run kv_compact                   */
  /* device-resident state in the reference */
  uint32_t* lens, *feed, *tree;
  sv_gen_state* gen;
  uint16_t* k_cache, *v_cache;
  const uint32_t* page_table;
  sv_kv_args kv;
  const float* rope;
  /* outputs */
  uint32_t* meta;  /* [n][2]          */
  float* logits;   /* [n_head][vocab] */
  uint32_t* out;   /* [n_head]        */
  uint32_t* emitted, *path, *path_len, *on_path;
  float* hidden;   /* [n][H] final residual, may be NULL */
  uint32_t n_attn; /* attention runs: each run's rows in runs of 16 (0: n_runs) */
  /* the Limite extras: value-embedding table and MUDD (host pointers; NULL: none), the
   * sliding-window layers ([n_layers], NULL: all global) and their cache */
  const sv_model_extras* extras;
  const uint8_t* local;
  uint16_t* k_local, *v_local;
  const uint32_t* local_table;
  sv_kv_args kv_local;
  const sv_matrix* head; /* its own head (model.rs:93-95, host), NULL: the tied embedding */
  /* the drafter's taps (encode.rs:186-190): tap_out[k] [n][H] from layer tap_layers[k] */
  uint32_t n_taps;
  const uint32_t* tap_layers;
  float* const* tap_out;
  /* Engine::step_capture (engine.rs:318-355; NULL: off): per layer, [n] rows each of the input
   * residual [H], rms_norm of the attention input [H], q | k | v after the norms, RoPE and value
   * embeddings [W], the attention output before XSA and the gate [NQ D], o's and down's products
   * before the residual with rms_norm of the MLP input between them [H] x 3, and MUDD's
   * residual base [H] (zeros on other layers); layer blocks in order. */
  float* cap;
} orc_step_io;

int orc_step(const sv_shape* sh, const uint16_t* embed, const sv_layer* layers, float attn_scale,
             orc_step_io* io);
/* orc_attn_verify that also writes, where non-NULL, each token's queries after the norm and RoPE
 * [n][NQ D], keys after the norm and RoPE and values after the value embedding [n][NKV D], and
 * the attention output before XSA and the gate [n][NQ D] (fp32). */
void orc_attn_verify_cap(const sv_shape* sh, const float* qkv, const uint32_t* meta, uint16_t* k_cache,
                         uint16_t* v_cache, const uint32_t* page_table, const float* rope, const sv_kv_args* kv,
                         const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs, const uint32_t* vis,
                         float* out, const sv_attn_extras* ex, float* cap_q, float* cap_k, float* cap_v,
                         float* cap_sdpa);

/* The drafter (drafter.rs:278-447, kernels.metal:135-148, 1725-1934); host pointers. */
void orc_tap_rows(const float* in, float* out, uint32_t n, uint32_t hidden);
void orc_draft_kv(const sv_shape* sh, const float* kvp, const uint32_t* meta, const uint32_t* on_path,
                  const float* rope, uint16_t* k_ring, uint16_t* v_ring, const uint32_t* table, const sv_kv_args* kv,
                  uint32_t n, uint32_t n_layers);
void orc_draft_ctx(const float* ctx, const float* ctx_inv, const uint32_t* meta, const uint32_t* on_path, float* ring,
                   uint32_t cr, uint32_t n, uint32_t hidden);
void orc_draft_embed(const uint16_t* table, const uint32_t* tin, const uint32_t* lens, const uint32_t* feed,
                     const float* mask_emb, float* x, uint32_t* meta, uint32_t* tokens, const float* ring, float* last,
                     uint32_t cr, uint32_t rows, uint32_t hidden);
void orc_draft_conv(const float* x, const float* corr, uint32_t corr_w, const float* base, const uint32_t* tin,
                    const float* resid, float* out, uint32_t rows, uint32_t hidden);
typedef struct orc_draft_io {
  /* the step's tokens: their taps [n_taps][n][H], meta (slot, position), on_path */
  uint32_t n;
  const float* const* taps;
  const uint32_t* meta;
  const uint32_t* on_path;
  const float* rope;
  /* rings (cyclic page table, kv: is_global 0, window) and the context ring [slots][cr][H] */
  uint16_t* k_ring, *v_ring;
  const uint32_t* table;
  sv_kv_args kv;
  float* ctx_ring;
  uint32_t cr;
  /* blocks: (first row, rows) each, rows' (slot, i) and visibility; state after accept */
  uint32_t n_blocks, rows;
  const uint32_t* blocks, *tin, *vis;
  const uint32_t* lens;
  uint32_t* feed, *tree;
  /* outputs: raw logits [rows][v]; the context [n][H] (may be NULL) */
  float* logits;
  float* ctx;
} orc_draft_io;
int orc_draft(const sv_shape* sh, const uint16_t* embed, const sv_drafter* d, float attn_scale, orc_draft_io* io);

#ifdef __cplusplus
}
#endif
#endif
