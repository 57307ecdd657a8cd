/*
 * sv_verify.h — C ABI of the MI355X speculative-decoding verify path.
 *
 * This is the drop-in boundary for the kernel-dispatch surface of the reference engine
 * (Belluxx/silicon-violetto): the Metal pipelines that `Engine::encode_*` binds and
 * dispatches (engine/src/gpu.rs:158-194, engine/src/engine/encode.rs:99-573) become plain
 * `extern "C"` calls on a HIP stream, and `Engine::{new_seq, step, sample_logits,
 * bench_fill, settle}` (engine/src/engine.rs:267-379, engine/src/engine/hooks.rs:31-55)
 * become the sv_engine_* calls.
 *
 * Conventions (mirroring the reference's, engine/src/gpu.rs:158-167):
 *   - every call returns an sv_status; SV_OK is 0. On failure sv_last_error() returns a
 *     thread-local message (the reference's Result<_, String>);
 *   - pointers named d_* are device pointers (HBM); everything else is host memory;
 *   - kernels never allocate. Callers own buffers and keep them alive while work that uses
 *     them is in flight on the stream; calls on one stream run in order;
 *   - a `workspace` is caller-owned device memory of at least the size the matching
 *     *_workspace_bytes call returns, ZERO-FILLED ONCE before first use. The kernels keep
 *     its counters at zero between calls, so one workspace serves any number of calls that
 *     run in stream order (two calls that overlap in time must not share one).
 *
 * The #[repr(C)] argument structs of engine/src/engine/kernels.rs:36-136 are mirrored
 * field for field (sv_mat_args, sv_kv_args, sv_attn_args, sv_sample_row, sv_run_in,
 * sv_gen_state, sv_replay_args).
 */
#ifndef SV_VERIFY_H
#define SV_VERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ constants */
#define SV_FEED_ROW 0xffff0000u /* input token FEED_ROW + i is feed[slot][i] (kernels.rs:17) */
#define SV_FEED_W 16u           /* GPU-fed tokens per slot (kernels.rs:19) */
#define SV_NO_TOK 0xffffffffu   /* SampleRow.tok: not a token of the step (kernels.rs:28) */
#define SV_NO_PARENT 0xffu      /* tree node without a parent (kernels.metal:66) */
#define SV_MAX_STOP 8u          /* stop ids per slot (kernels.rs:32) */
/* Tokens per run the fused verify attention takes. The reference stops at VERIFY_T = 8
 * (kernels.rs:30) and sends longer runs to attn_mma, whose tree mask only holds within
 * tiles of 8 (kernels.metal:1240-1241); here a run of up to FEED_W rows keeps one full
 * 16-bit ancestry mask. */
#define SV_MAX_RUN 16u
#define SV_SAMPLE_THREADS 1024u /* the sampler's fixed summation order (kernels.rs:13) */
#define SV_SAMPLE_ROUNDS 8u     /* top-p rejection rounds (kernels.metal:1413) */
#define SV_RMS_EPS 1.1920928955078125e-07f /* 2^-23 (kernels.metal:13) */
#define SV_ROPE_PAIRS 32u       /* RoPE pairs per head: dims 0..63 (kernels.metal:727-736) */
#define SV_DRAFT_CANDS 4u       /* drafter candidates per block row, at most (kernels.metal:1845) */
#define SV_VE_GATE_W 12u        /* value-embedding gate inputs: rms_norm(x)[:12] (kernels.metal:738-747) */
#define SV_MUDD_INNER 32u       /* MUDD inner width (kernels.metal:1367-1372, model.rs:97) */
#define SV_MUDD_SITES 2u        /* MUDD sites, at most (model.rs:21) */
/* Attention columns per kv head: a run's rows x (n_heads / n_kv_heads) stay within this. With
 * n_heads / n_kv_heads = g, attention runs hold min(SV_MAX_RUN, SV_MAX_COLS / g) rows. */
#define SV_MAX_COLS 64u

/* Matmul epilogues and flags (kernels.metal:151-152, kernels.rs:4-10). */
enum {
  SV_EPI_NORM = 1,   /* y = scale * acc / rms(x)                                   */
  SV_EPI_RESID = 2,  /* y = ra * base + rb * scale * acc                           */
  SV_EPI_SWIGLU = 3, /* y[row/2] = silu(g) * u over interleaved (gate, up) rows, norm folded */
  SV_EPI_HEAD = 4,   /* y = 23 sigmoid((acc + 5) / 7.5), -inf at rows >= vocab_real */
  SV_EPI_RAW = 5     /* y = acc                                                     */
};
enum {
  SV_FLAG_WRITE_INV = 1, /* aux[t] = 1 / rms(x[t]) (EPI_NORM)                   */
  SV_FLAG_WRITE_RAW = 2, /* aux = scale * acc (EPI_RESID)                      */
  /* Extension: acc *= 1/rms(x) for EPI_HEAD/EPI_RAW/EPI_RESID, i.e. the reference's
   * rmsnorm_rows (kernels.metal:117-131) folded into the matmul that follows it. */
  SV_FLAG_NORM_IN = 4
};
enum {
  SV_FMT_BF16 = 0,
  SV_FMT_I8 = 1,
  /* Layout flag, or-ed into a format: weights in 16-row tiles, each tile's 64-k blocks stored
   * as one contiguous 1 KB (int8) or 2 KB (bf16) in the matrix-core lane order (written by
   * sv_pack_matrix). Not in the reference: its weights stay row-major (model.rs:22-47). */
  SV_FMT_TILED = 0x10
};

typedef enum sv_status {
  SV_OK = 0,
  SV_ERR_ARG = 1,         /* a bad argument (shape, size, null pointer)          */
  SV_ERR_HIP = 2,         /* a HIP runtime call failed                           */
  SV_ERR_CAPACITY = 3,    /* a capacity of the engine would be exceeded          */
  SV_ERR_UNSUPPORTED = 4, /* valid in the reference, not built here              */
  SV_ERR_STATE = 5        /* call out of order (unknown sequence, no weights...) */
} sv_status;

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* sv_last_error(void);

/* ------------------------------------------------------------- model shapes */
/* The reference hard-codes these (engine/src/model.rs:6-18); here they are runtime values.
 * Supported: head_dim 64 or 128, hidden and ffn multiples of 256, n_heads a multiple of
 * n_kv_heads, n_heads / n_kv_heads <= 8. */
typedef struct sv_shape {
  uint32_t hidden;     /* H                                    */
  uint32_t n_heads;    /* NQ                                   */
  uint32_t n_kv_heads; /* NKV                                  */
  uint32_t head_dim;   /* D                                    */
  uint32_t ffn;        /* F (gate_up has 2F interleaved rows)  */
  uint32_t vocab;      /* embedding rows                       */
  uint32_t vocab_real; /* ids from here on are masked padding  */
  uint32_t n_layers;   /* L                                    */
} sv_shape;

/* A weight matrix [m][k] row-major (model.rs:22-47): bf16, or int8 with one bf16 scale per
 * group of 2^gshift consecutive k in scales [m][k >> gshift]. int8 groups of 256 or more are
 * built; gshift >= log2(k) (e.g. 31) means one scale per output row, scales [m][1]. */
typedef struct sv_matrix {
  const void* d_w;
  const uint16_t* d_scales; /* NULL for bf16 */
  uint32_t m, k;
  uint32_t format; /* SV_FMT_* */
  uint32_t gshift;
} sv_matrix;

/* MatArgs (kernels.rs:36-50, kernels.metal:157-165). ksplit/kchunk are ignored: the split
 * of k is the implementation's. */
typedef struct sv_mat_args {
  uint32_t n, k, m;
  uint32_t epi, flags;
  uint32_t vocab_real;
  float scale;
  float ra, rb;
  uint32_t ksplit, kchunk;
  uint32_t gshift;
} sv_mat_args;

/* KvArgs (kernels.rs:53-63, kernels.metal:692-700). Cache layout per tensor (K and V):
 * bf16 [layers][n_pages][NKV][page][D], page = 1 << page_shift, through the page table
 * [max_seqs][max_pages]. is_global 0 is a sliding-window layer (kernels.metal:808-811): a
 * query at position pos sees the cached keys from pos - window on (window > 0). Its ring
 * (kv.rs:26-32, [layer][seq][NKV][ring][D] in the reference) is laid out here as pages too: a
 * sequence's ring of R pages is pages seq R .. seq R + R - 1 and its page-table row is
 * cyclic (entry p = seq R + p % R), so one addressing serves both kinds; `ring` is unused. */
typedef struct sv_kv_args {
  uint32_t is_global, kv_layer;
  uint32_t ring, max_seqs;
  uint32_t page_shift, n_pages, max_pages;
  uint32_t window;
} sv_kv_args;

/* AttnArgs (kernels.rs:72-83, kernels.metal:813-823). Used here: split (cached keys per
 * split, a multiple of 32, at most 3968), max_splits (grid size, at least the most splits any run needs,
 * counting the split of its new keys), scale_log2 (softmax scale * log2 e), rope. ve,
 * capture, fixed_splits, col_sets and one_round are ignored. */
typedef struct sv_attn_args {
  uint32_t split, max_splits;
  float scale_log2;
  uint32_t rope, ve, capture;
  uint32_t fixed_splits, col_sets, one_round;
} sv_attn_args;

/* SampleRow (kernels.rs:86-99, kernels.metal:1454-1461). */
typedef struct sv_sample_row {
  uint32_t seed_lo, seed_hi;
  uint32_t pos; /* position of the drawn token if tok == SV_NO_TOK */
  float temperature;
  float top_p;
  uint32_t tok; /* the step's token whose head row this is: draw at its position + 1 */
} sv_sample_row;

/* RunIn (kernels.rs:103-111, kernels.metal:1591-1595). */
typedef struct sv_run_in {
  uint32_t slot, first, count;
  uint32_t head0, nhead;
  uint32_t verify;
} sv_run_in;

/* GenState (kernels.rs:115-127, kernels.metal:1597-1603). */
typedef struct sv_gen_state {
  uint32_t remaining;
  uint32_t done;
  uint32_t nstop;
  uint32_t pad;
  uint32_t stop[SV_MAX_STOP];
} sv_gen_state;

/* ReplayArgs (kernels.rs:129-136, kernels.metal:1698-1703). */
typedef struct sv_replay_args {
  uint32_t stride, seed;
  float rate;
  uint32_t vocab;
} sv_replay_args;

/* ======================================================= kernel-level calls
 * One call per Metal pipeline group the forward pass dispatches. */

/* embed (kernels.metal:82-114, encode.rs:128-140): resolves GPU-fed tokens in place,
 * meta[t] = (slot, lens[slot] + depth), vis from the draft tree, and
 * d_out[t] = rms_norm(embedding row). d_tin and d_meta are uint2 per token. */
sv_status sv_embed(void* stream, const sv_shape* shape, const uint16_t* d_table, uint32_t* d_tokens,
                   float* d_out, const uint32_t* d_tin, uint32_t* d_meta, const uint32_t* d_lens,
                   const uint32_t* d_feed, const uint32_t* d_tree, uint32_t* d_vis, uint32_t n);

/* rmsnorm_rows (kernels.metal:117-131): d_out[r] = rms_norm(d_in[d_rows[r]]). */
sv_status sv_rmsnorm_rows(void* stream, const float* d_in, const uint32_t* d_rows, float* d_out, uint32_t n,
                          uint32_t hidden);

/* The matmul group (encode.rs:488-572 Engine::matmul_in; kernels.metal:151-690 gemv_*,
 * gemms_*, gemm_*, gemm_splitk_reduce): d_y[t][row] = epilogue(W[row] . x[t]) for
 * t < a->n, with x[t] = d_x[d_x_rows ? d_x_rows[t] : t] (rows of k floats). d_base is
 * [n][m] for EPI_RESID; d_aux is [n] (WRITE_INV) or [n][m] (WRITE_RAW). The kernel variant
 * is chosen from n (the reference's Matmul::for_tokens, encode.rs:33-44). The workspace
 * (sv_matmul_workspace_bytes; zero bytes needs none) carries split-k partials: zero-fill it
 * once; the kernels leave its counters at zero, so calls in stream order may share one, and
 * calls that overlap in time must not. */
size_t sv_matmul_workspace_bytes(uint32_t n, uint32_t m, uint32_t k);
sv_status sv_matmul(void* stream, const sv_matrix* w, const float* d_x, const uint32_t* d_x_rows, float* d_y,
                    const float* d_base, float* d_aux, const sv_mat_args* a, void* d_workspace,
                    size_t workspace_bytes);

/* Repacks a row-major matrix into the tiled layout (SV_FMT_TILED) for sv_matmul: d_dst gets
 * m * k bytes (int8) or 2 m k (bf16), *out the same matrix with format | SV_FMT_TILED and
 * src's scales. Needs m % 16 == 0 and k % 64 == 0. No counterpart in the reference (its
 * weights are used as loaded, model.rs:22-47); done once at model load. */
sv_status sv_pack_matrix(void* stream, const sv_matrix* src, void* d_dst, sv_matrix* out);

/* The Limite layer extras of the attention (kernels.metal:738-747 add_ve, 910-942 new_key,
 * 1316-1362 attn_dec_reduce; model.rs:49-67): any pointer may be NULL, which turns its part
 * off. With d_ve_gate, each new V row gets 2 sigmoid(rms_norm(x)[:12] . ve_gate[g]) *
 * value_embed[token][g D ..] before it is rounded and cached (needs d_x, d_inv, d_tokens,
 * d_value_embed). With d_attn_gate, output o of head h is scaled by 2 sigmoid(rms_norm(x)[:D] .
 * attn_gate[h]) (needs d_x, d_inv). With d_xsa (needs d_vdir), o - xsa[h] (o . v) v with v the
 * token's new value row of kv head h / g, normalised (|v| floored at 1e-4), before the gate. */
typedef struct sv_attn_extras {
  const float* d_x;              /* [n][hidden] the attention input before its norm    */
  const float* d_inv;            /* [n] 1 / rms(x) (the qkv matmul's SV_FLAG_WRITE_INV) */
  const uint32_t* d_tokens;      /* [n] the tokens' ids (resolved)                      */
  const uint16_t* d_value_embed; /* bf16 [vocab][NKV D]                                 */
  const float* d_ve_gate;        /* [NKV][SV_VE_GATE_W]                                 */
  const float* d_attn_gate;      /* [NQ][D]                                             */
  const float* d_xsa;            /* [NQ]                                                */
  float* d_vdir;                 /* [n][NKV][D] scratch the attention writes for XSA    */
  uint32_t hidden;               /* row stride of d_x                                   */
  uint32_t pad;
} sv_attn_extras;

/* Fused verify attention (kernels.metal:1008-1148 attn_verify + 1316-1362 attn_dec_reduce;
 * encode.rs:233-297): for each run (d_runs: uint2 (first token, count <= SV_MAX_RUN and
 * count x NQ / NKV <= SV_MAX_COLS)), q/k rms-norm + RoPE, the run's new K/V written bf16 to
 * the paged cache at p0 + row, attention over the cached keys [0, p0) (sliding-window layers:
 * from each query's pos - window) and the new keys in each token's vis mask, with split-KV
 * partials merged by plain sums. d_qkv is [n][(NQ + 2 NKV) D] fp32; d_out is [n][NQ D] fp32.
 * extras: NULL, or the layer's extras (sv_attn_extras). */
size_t sv_attn_workspace_bytes(const sv_shape* shape, uint32_t n_runs, uint32_t max_splits, uint32_t max_run);
sv_status sv_attn_verify(void* stream, const sv_shape* shape, const float* d_qkv, const uint32_t* d_meta,
                         uint16_t* d_k_cache, uint16_t* d_v_cache, const uint32_t* d_page_table,
                         const float* d_rope, const sv_kv_args* kv, const sv_attn_args* args,
                         const uint32_t* d_runs, uint32_t n_runs, uint32_t max_run, const uint32_t* d_vis,
                         float* d_out, void* d_workspace, size_t workspace_bytes, const sv_attn_extras* extras);

/* mudd (kernels.metal:1364-1407, encode.rs:145-160): per token, one inner projection of
 * rms_norm(cur) (inner = gelu(dense1 . x), dense1 [SV_MUDD_INNER][hidden]) feeds six mixes
 * w = mix[i][:32] . inner + mix[i][32] (mix [2][3][33]: attention input, residual base) of the
 * taps: out_attn = w0 tap0 + w1 tap1 + w2 cur, out_base = w3 tap0 + w4 tap1 + w5 cur. All
 * [n][hidden] fp32. gelu is the erf form, erf by Abramowitz & Stegun 7.1.26 as the
 * reference's (kernels.metal:30-37). */
sv_status sv_mudd(void* stream, const float* d_cur, const float* d_tap0, const float* d_tap1, const float* d_dense1,
                  const float* d_mix, float* d_out_attn, float* d_out_base, uint32_t n, uint32_t hidden);

/* No counterpart in the reference: sv_attn_verify for callers that cannot allocate (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). The same kernels and
 * results, with the split partials in a static array of the library, one per GPU, of
 * sv_attn_noalloc_max_bytes() bytes (32 MiB), held until the process ends; no allocation and no
 * library routine that allocates. A call whose partials (sv_attn_workspace_bytes) exceed it
 * returns SV_ERR_CAPACITY before anything runs. Calls on one GPU share the array: calls that
 * overlap on one GPU (different streams, or host threads) race and must be serialised. */
size_t sv_attn_noalloc_max_bytes(void);
sv_status sv_attn_verify_noalloc(void* stream, const sv_shape* shape, const float* d_qkv, const uint32_t* d_meta,
                                 uint16_t* d_k_cache, uint16_t* d_v_cache, const uint32_t* d_page_table,
                                 const float* d_rope, const sv_kv_args* kv, const sv_attn_args* args,
                                 const uint32_t* d_runs, uint32_t n_runs, uint32_t max_run, const uint32_t* d_vis,
                                 float* d_out);

/* sample (kernels.metal:1503-1576, with argmax_partial 1430-1451 folded in): one token
 * per row of d_logits [rows][vocab]: the argmax at temperature 0 (ties to the lowest id),
 * else the Philox-keyed inverse-CDF draw with top-p rounds. Bit-exact with the oracle. */
sv_status sv_sample(void* stream, const float* d_logits, const sv_sample_row* d_rows, uint32_t* d_out,
                    const uint32_t* d_meta, uint32_t n_rows, uint32_t vocab);

/* accept (kernels.metal:1578-1657). d_path is [nruns][SV_FEED_W]. */
sv_status sv_accept(void* stream, const sv_run_in* d_runs, const uint32_t* d_tokens, uint32_t* d_out,
                    uint32_t* d_lens, uint32_t* d_feed, sv_gen_state* d_gen, uint32_t* d_emitted, uint32_t nruns,
                    const uint32_t* d_tree, uint32_t* d_path, uint32_t* d_path_len, uint32_t* d_on_path);

/* kv_compact (kernels.metal:1659-1693): each verify run's accepted path's K/V rows to
 * p0 + j on every layer 0..n_layers-1. */
sv_status sv_kv_compact(void* stream, const sv_shape* shape, const sv_run_in* d_runs, uint32_t nruns,
                        const uint32_t* d_path, const uint32_t* d_path_len, const uint32_t* d_lens,
                        uint16_t* d_k_cache, uint16_t* d_v_cache, const uint32_t* d_page_table,
                        const sv_kv_args* kv);

/* draft_top (kernels.metal:1845-1891, dispatched by drafter.rs:427-436): for each drafted
 * block row r (d_tin[r] = (slot, row in block); rows with row 0, the bonus token's, are
 * skipped) the ncand (1..SV_DRAFT_CANDS) best drafter logits of d_logits [n_rows][nv], ties to
 * the lowest id, as target ids through d_vocab[nv] and their probabilities at temperature
 * 1 / inv_t, into d_cand / d_cand_q [n_rows][SV_DRAFT_CANDS]. A row without a candidate's
 * value (NaN or -inf logits) gets SV_NO_TOK and probability 0. */
sv_status sv_draft_top(void* stream, const float* d_logits, const uint32_t* d_vocab, const uint32_t* d_tin,
                       uint32_t* d_cand, float* d_cand_q, uint32_t n_rows, uint32_t nv, float inv_t, uint32_t ncand);
/* draft_tree (kernels.metal:1893-1934, drafter.rs:437-446): each block (d_blocks: uint2 (first
 * row, rows <= SV_FEED_W)) builds its DDTree best-first from its rows' candidates and writes
 * the nodes to d_feed / d_tree [slots][SV_FEED_W] entries 1.. of its slot, dead nodes after. */
sv_status sv_draft_tree(void* stream, const uint32_t* d_blocks, uint32_t nblocks, const uint32_t* d_tin,
                        const uint32_t* d_cand, const float* d_cand_q, uint32_t* d_feed, uint32_t* d_tree,
                        uint32_t ncand);

/* The drafter's own pieces (kernels.metal:135-148 tap_rows, 1725-1844 draft_kv, draft_ctx,
 * draft_embed, draft_conv), over [n][hidden] fp32 rows:
 *  - tap_rows: out[t] = bf16(rms_norm(in[t])) kept as float (a target layer's output tapped);
 *  - draft_kv: for the tokens on_path, kvp[t] = [layer][k | v][NKV][D] (the fused context through
 *    every drafter layer's k/v) is normed and roped (k) and written bf16 to the drafter's ring of
 *    each layer at the token's position (d_meta: (slot, position)); grid over (tokens, layers);
 *  - draft_ctx: for the tokens on_path, ring[slot][pos % cr] = ctx[t] * ctx_inv[t];
 *  - draft_embed: block row r (d_tin[r] = (slot, i)) at position lens[slot] + i: row 0 the slot's
 *    next input feed[slot][0] as rms_norm(embedding), later rows mask_emb; meta and tokens of
 *    the rows; with cr > 0, last[r] = ring[slot][(lens[slot] - 1) % cr];
 *  - draft_conv: out[r] = resid[r] (with resid) + (base[0] + corr[r][d / 16]) x[r] + (base[1] +
 *    corr[r][hidden / 16 + d / 16]) x[r - 1], the second term only for rows after a block's first
 *    (corr [n][corr_w]); out must not be x. */
sv_status sv_tap_rows(void* stream, const float* d_in, float* d_out, uint32_t n, uint32_t hidden);
sv_status sv_draft_kv(void* stream, const sv_shape* shape, const float* d_kvp, const uint32_t* d_meta,
                      const uint32_t* d_on_path, const float* d_rope, uint16_t* d_k_ring, uint16_t* d_v_ring,
                      const uint32_t* d_page_table, const sv_kv_args* kv, uint32_t n, uint32_t n_layers);
sv_status sv_draft_ctx(void* stream, const float* d_ctx, const float* d_ctx_inv, const uint32_t* d_meta,
                       const uint32_t* d_on_path, float* d_ring, uint32_t cr, uint32_t n, uint32_t hidden);
sv_status sv_draft_embed(void* stream, const uint16_t* d_embed, const uint32_t* d_tin, const uint32_t* d_lens,
                         const uint32_t* d_feed, const float* d_mask_emb, float* d_x, uint32_t* d_meta,
                         uint32_t* d_tokens, const float* d_ring, float* d_last, uint32_t cr, uint32_t rows,
                         uint32_t hidden);
sv_status sv_draft_conv(void* stream, const float* d_x, const float* d_corr, uint32_t corr_w, const float* d_base,
                        const uint32_t* d_tin, const float* d_resid, float* d_out, uint32_t rows, uint32_t hidden);

/* The weight file (engine/src/weights.rs:38-74; format tools/convert.py:117-150): header
 * "VIOLETTO", version 1, 128-byte records, 16 KiB-aligned data region. sv_weights_open reads and
 * checks the records on the host; sv_weights_upload copies every tensor into one device buffer;
 * sv_weights_matrix resolves a matrix as model.rs:80-103 does (bf16, or int8 with `<name>.scale`,
 * groups of 8..256 k, or one per row). Error strings follow the reference's. */
typedef struct sv_tensor_info {
  char name[64];
  uint32_t dtype; /* 0 f32, 1 bf16, 2 int8 */
  uint32_t ndim;
  uint32_t shape[4];
  uint64_t offset; /* bytes from the data region (device buffer) start */
  uint64_t nbytes;
} sv_tensor_info;
typedef struct sv_weights sv_weights;
sv_status sv_weights_open(const char* path, sv_weights** out);
uint32_t sv_weights_count(const sv_weights* w);
sv_status sv_weights_info(const sv_weights* w, uint32_t i, sv_tensor_info* out);
sv_status sv_weights_find(const sv_weights* w, const char* name, sv_tensor_info* out);
sv_status sv_weights_read(const sv_weights* w, const char* name, void* host, size_t bytes);
sv_status sv_weights_upload(sv_weights* w, void* stream);
sv_status sv_weights_device(const sv_weights* w, const char* name, void** d_ptr);
sv_status sv_weights_matrix(const sv_weights* w, const char* name, uint32_t m, uint32_t k, sv_matrix* out);
void sv_weights_close(sv_weights* w);

/* replay_draft (kernels.metal:1705-1724): the test drafter. */
sv_status sv_replay_draft(void* stream, const sv_run_in* d_runs, uint32_t nruns, const uint32_t* d_lens,
                          uint32_t* d_feed, const uint32_t* d_trace, const uint32_t* d_trace_len,
                          const sv_replay_args* ra, uint32_t* d_tree);

/* ========================================================= engine-level calls
 * The reference's Engine (engine/src/engine.rs): owns the KV cache, its page pool and
 * page table (kv.rs), the GPU-resident sequence state (buffers.rs:41-52), the scratch and
 * the RoPE table; the caller owns the weights (device pointers). */
typedef struct sv_engine sv_engine;

/* EngineConfig (engine.rs:32-57) plus the model's shape and constants. */
/* sv_engine_config.options. SV_OPT_LAYERS_KERNEL: steps of 1-8 rows whose layers the
 * persistent layer kernel takes (global attention, no extras, no drafter, per-row int8 matrices
 * at hidden 2048 / ffn 8192, splits of at most 384 keys that fit the grid) run all their layers
 * in one launch instead of one launch per matmul and attention. */
#define SV_OPT_LAYERS_KERNEL 1u

typedef struct sv_engine_config {
  sv_shape shape;
  uint32_t max_seqs;        /* sequence slots                                   */
  uint32_t max_step_tokens; /* tokens per step over all runs                    */
  uint32_t max_seq_len;     /* positions per sequence                           */
  uint32_t max_head_rows;   /* rows that go through the head in one step        */
  uint32_t kv_tokens;       /* page pool capacity, tokens, shared by all slots  */
  uint32_t page_shift;      /* log2 tokens per page (reference: 7; configs: 4)  */
  float attn_scale;         /* softmax scale (reference ATTN_SCALE, model.rs:19) */
  uint32_t split_keys;      /* cached keys per attention split, multiple of 32; 0: auto */
  uint32_t options;         /* SV_OPT_* bits                                     */
  /* Sliding-window layers (model.rs:16-17,116; kv.rs:26-32): keys a local query sees
   * besides itself, and which layers are local ([n_layers], 1 local; NULL: all global).
   * Local layers keep a ring of ceil((window + max_step_tokens) / page) pages per slot. */
  uint32_t window;
  uint32_t pad;
  const uint8_t* local;
} sv_engine_config;

/* One decoder layer (model.rs:49-67): matrices, scalars and the extras. rope: whether the
 * layer's q/k get RoPE (the reference ropes its local layers only, encode.rs:237). Device
 * pointers, NULL for a part the layer does not have: attn_gate [n_heads][head_dim] (NULL: gate
 * 1), ve_gate [n_kv_heads][SV_VE_GATE_W] (value embeddings; needs the model's table, set by
 * sv_engine_set_extras), xsa [n_heads] (NULL: 0). */
typedef struct sv_layer {
  sv_matrix qkv, o, gate_up, down;
  float qkv_scale, o_scale;
  float resid_attn, post_attn;
  float resid_mlp, post_mlp;
  uint32_t rope;
  uint32_t pad;
  const float* attn_gate;
  const float* ve_gate;
  const float* xsa;
} sv_layer;

/* The model's extras (model.rs:73-83, encode.rs:107-160). value_embed: bf16 [vocab][n_kv_heads
 * head_dim] for the layers with a ve_gate. MUDD: site s runs before layer mudd_layer[s] on its
 * input (cur), with taps the embedding's rows and the output of layer mudd_tap[s] <
 * mudd_layer[s] (the reference: sites 24 and 47, taps 11 and 22); dense1 [SV_MUDD_INNER][hidden],
 * mix [n_mudd][2][3][33]. */
typedef struct sv_model_extras {
  const uint16_t* value_embed;
  const float* mudd_dense1;
  const float* mudd_mix;
  uint32_t n_mudd;
  uint32_t mudd_layer[SV_MUDD_SITES];
  uint32_t mudd_tap[SV_MUDD_SITES];
  uint32_t pad;
} sv_model_extras;

/* rope_freq: host [SV_ROPE_PAIRS] frequencies (model.rs:81, tools/convert.py:59-61). */
sv_status sv_engine_create(const sv_engine_config* cfg, const float* rope_freq, sv_engine** out);
void sv_engine_destroy(sv_engine* e);
/* Tied bf16 embedding / head [vocab][hidden] (device), and the layers. */
sv_status sv_engine_set_embed(sv_engine* e, const uint16_t* d_embed);
sv_status sv_engine_set_layer(sv_engine* e, uint32_t layer, const sv_layer* l);
sv_status sv_engine_set_extras(sv_engine* e, const sv_model_extras* x);
/* A head of its own (model.rs:93-95: the weight file's quantized `head`), [vocab][hidden]: bf16,
 * or int8 with one scale per row or per group of 8 to 256 (groups under 64, such as the
 * reference converter's default of 8, run as two exact bf16 matrices hi + lo and a softcap
 * pass); NULL: the tied embedding again. */
sv_status sv_engine_set_head(sv_engine* e, const sv_matrix* head);
/* The HIP stream the engine runs on (a hipStream_t), created by the engine. */
void* sv_engine_stream(sv_engine* e);

/* Device buffers the engine owns, for tests and benchmarks to fill or read. */
typedef struct sv_engine_buffers {
  uint16_t* d_k_cache;      /* [L][n_pages][NKV][page][D] bf16      */
  uint16_t* d_v_cache;
  uint32_t* d_page_table;   /* [max_seqs][max_pages]                */
  uint32_t* d_lens;         /* [max_seqs]                           */
  uint32_t* d_feed;         /* [max_seqs][SV_FEED_W]                */
  uint32_t* d_tree;         /* [max_seqs][SV_FEED_W]                */
  sv_gen_state* d_gen;      /* [max_seqs]                           */
  uint32_t* d_trace;        /* [max_seqs][max_seq_len]  replay drafter */
  uint32_t* d_trace_len;    /* [max_seqs]                           */
  float* d_logits;          /* [max_head_rows][vocab]               */
  float* d_rope;            /* [max_seq_len + SV_FEED_W][32][2]     */
  uint32_t* d_out_ids;      /* [max_head_rows]                      */
  uint32_t* d_emitted;      /* [max_seqs]                           */
  uint32_t* d_path;         /* [max_seqs][SV_FEED_W]                */
  uint32_t* d_path_len;     /* [max_seqs]                           */
  uint32_t n_pages, max_pages;
  size_t kv_bytes;          /* bytes of each of K and V             */
  /* sliding-window layers (NULL without): [n_local][n_local_pages][NKV][page][D] bf16
   * with the cyclic page table [max_seqs][max_pages] (sv_kv_args) */
  uint16_t* d_k_local;
  uint16_t* d_v_local;
  uint32_t* d_local_table;
  uint32_t n_local_pages, ring_pages;
  size_t local_bytes;       /* bytes of each of K and V (local)     */
} sv_engine_buffers;
sv_status sv_engine_get_buffers(sv_engine* e, sv_engine_buffers* out);

/* Sequences (engine.rs:267-306). */
sv_status sv_new_seq(sv_engine* e, uint32_t* slot);
sv_status sv_free_seq(sv_engine* e, uint32_t slot);
sv_status sv_seq_len(sv_engine* e, uint32_t slot, uint32_t* len);
/* The slot's pages in order (its page-table row); *n is set to the count. */
sv_status sv_seq_pages(sv_engine* e, uint32_t slot, uint32_t* pages, uint32_t cap, uint32_t* n);
/* Sampling (engine.rs:104-138): temperature 0 (greedy) or normal positive, 0 < top_p <= 1. */
sv_status sv_set_sampling(sv_engine* e, uint32_t slot, float temperature, float top_p, uint64_t seed);
/* GenState of a slot (stop ids, budget) for accept; the default never stops. */
sv_status sv_set_gen(sv_engine* e, uint32_t slot, const sv_gen_state* g);
/* hooks.rs:31-37 bench_fill: advance a sequence by len positions without computing them
 * (reserving their pages); the caller fills the KV. */
sv_status sv_bench_fill(sv_engine* e, uint32_t slot, uint32_t len);
/* engine.rs:281-285 settle: give back `unused` positions of a speculative step. */
sv_status sv_settle(sv_engine* e, uint32_t slot, uint32_t unused);
/* Set a slot's device sequence position and GPU-fed input (the next input token). */
sv_status sv_set_feed(sv_engine* e, uint32_t slot, uint32_t len, uint32_t token);

/* One run of a step (plan.rs:8-18 PlanRun): tokens are ids or SV_FEED_ROW + i. */
typedef struct sv_run {
  uint32_t slot;
  uint32_t count;
  const uint32_t* tokens; /* host [count]                                 */
  uint32_t verify;        /* head on every row, rows 1.. are drafts       */
  uint32_t head;          /* non-verify runs: 0 no head row, 1 last row    */
} sv_run;

/* What a plan produced (plan.rs:20-36). */
typedef struct sv_plan_info {
  uint32_t n_tokens, n_head, n_runs;
  uint32_t branches;   /* some verify run has > 2 rows: kv_compact runs */
  uint32_t max_run;
  uint32_t split, max_splits;
} sv_plan_info;

enum {
  SV_STEP_REPLAY = 1,   /* after accept, the replay drafter writes the next drafts */
  SV_STEP_COMPACT = 2,  /* run kv_compact even if no run branches               */
  SV_STEP_NO_COMPACT = 4,
  SV_STEP_DRAFT = 8     /* after accept, the drafter's pass writes the next draft trees */
};

/* Engine::plan (plan.rs:47-151): lays out a step, reserves pages, advances the host-side
 * sequence lengths optimistically; `extra_keys` widens the attention grid for replays of
 * this plan at later positions (graph replays). */
sv_status sv_plan(sv_engine* e, const sv_run* runs, uint32_t n_runs, uint32_t extra_keys, sv_plan_info* info);
/* Encode the planned step (encode_forward + tail, encode.rs:99-126,383-412) on the
 * engine's stream: asynchronous, capturable. */
sv_status sv_encode(sv_engine* e, uint32_t flags);
/* Capture sv_encode(flags) of the current plan into a HIP graph; replay it `count` times. */
sv_status sv_graph_capture(sv_engine* e, uint32_t flags);
sv_status sv_graph_replay(sv_engine* e, uint32_t count);
sv_status sv_sync(sv_engine* e);
/* Replay-drafter settings (generate.rs:421-430). */
sv_status sv_set_replay(sv_engine* e, uint32_t seed, float rate);

/* The drafter (engine/src/engine/drafter.rs, its file written by tools/spec/export.py): a small
 * model of the target's shape that reads the target's tapped layers. Device pointers; matrices
 * as sv_matrix. conv_base[0] NULL: a layer without the two-tap convolutions; inject.d_w NULL:
 * none. vocab: the draft vocabulary's target ids [v]. The engine taps `taps` (their outputs,
 * normed and rounded to bf16) on every step once a drafter is set. */
#define SV_DRAFT_TAPS 4u
#define SV_DRAFT_LAYERS 8u
typedef struct sv_draft_layer {
  sv_matrix qkv, o, gate_up, down;
  const float* conv_base[4]; /* [2][hidden] each: before attention, after it, before the MLP, after it */
  sv_matrix conv_corr[4];    /* [corr_w][hidden] each, corr_w = hidden / 8 padded (export.py: 192) */
} sv_draft_layer;
typedef struct sv_drafter {
  uint32_t n_layers, n_taps, v;
  uint32_t taps[SV_DRAFT_TAPS];
  sv_matrix fc[SV_DRAFT_TAPS]; /* [hidden][hidden]: the context, sum over taps */
  sv_matrix kv_all;            /* [n_layers 2 NKV D][hidden]                  */
  sv_matrix inject;            /* [hidden][hidden] or d_w NULL                */
  sv_matrix head;              /* [v][hidden], raw logits                     */
  const float* mask_emb;       /* [hidden]                                    */
  const uint32_t* vocab;       /* [v]                                         */
  const sv_draft_layer* layers;/* host [n_layers]                             */
  float inv_temperature;       /* draft_top's 1 / T (drafter.rs: 1 / 0.6)      */
  uint32_t window;             /* the context positions a block row sees      */
} sv_drafter;
/* Drops a captured step and the current plan (plan again). */
sv_status sv_engine_set_drafter(sv_engine* e, const sv_drafter* d);
/* Draft rows per block (1 + drafts, at most the attention run length) of a slot's next steps
 * with SV_STEP_DRAFT; 0: the slot is not drafted. */
sv_status sv_set_draft_rows(sv_engine* e, uint32_t slot, uint32_t rows);
/* The drafter's device buffers (Engine::drafter_debug, drafter.rs:263-275), for tests to read:
 * the last pass's raw logits [rows][v] and candidates [rows][SV_DRAFT_CANDS], the context
 * [max_step_tokens][hidden], the taps [n_taps][max_step_tokens][hidden], the rings
 * [n_layers][n_pages][NKV][page][D] bf16 behind the cyclic table [max_seqs][max_pages]. */
typedef struct sv_draft_buffers {
  float* d_logits;
  uint32_t* d_cand;
  float* d_cand_q;
  float* d_ctx;
  float* d_taps[SV_DRAFT_TAPS];
  uint16_t* d_k_ring;
  uint16_t* d_v_ring;
  uint32_t* d_table;
  uint32_t ring_pages, n_pages, max_pages, pad;
} sv_draft_buffers;
sv_status sv_engine_draft_buffers(sv_engine* e, sv_draft_buffers* out);

/* A synchronous step (Engine::step, engine.rs:310-314): plan, encode, wait; read the head
 * rows' ids (ids[n_head]) and, if logits is non-null, their logits [n_head][vocab], and
 * per run the tokens emitted. */
sv_status sv_step(sv_engine* e, const sv_run* runs, uint32_t n_runs, uint32_t flags, uint32_t* ids,
                  float* logits, uint32_t* emitted, sv_plan_info* info);

/* One layer's intermediates over a capture step (LayerCapture, engine.rs:176-188): host
 * arrays of n rows each, valid for the duration of the callback. */
typedef struct sv_layer_capture {
  uint32_t layer, n;
  uint32_t hidden;         /* row width of resid_in, attn_in, attn_out, mlp_in, mlp_out, resid_base */
  uint32_t qkv_width;      /* (n_heads + 2 n_kv_heads) head_dim                                    */
  uint32_t sdpa_width;     /* n_heads head_dim                                                      */
  uint32_t pad;
  const float* resid_in;   /* the layer's input residual                                            */
  const float* attn_in;    /* rms_norm of the attention input (the MUDD mix on MUDD layers)         */
  const float* qkv;        /* q | k | v after the norms, RoPE and value embeddings                  */
  const float* sdpa_out;   /* the attention output before XSA and the gate                          */
  const float* attn_out;   /* the o projection's product, before the residual                       */
  const float* mlp_in;     /* rms_norm of the MLP input                                              */
  const float* mlp_out;    /* the down projection's product, before the residual                    */
  const float* resid_base; /* MUDD's residual base; null on other layers                            */
} sv_layer_capture;
typedef void (*sv_capture_fn)(const sv_layer_capture* cap, void* user);

/* Engine::step_capture (engine.rs:318-355), the parity hook: sv_step's step run layer by
 * layer, waiting after each layer and handing its intermediates to fn (layers in order), then
 * the head and tail; outputs as sv_step's. It runs the launch-per-kernel path (also with
 * SV_OPT_LAYERS_KERNEL) and is not captured into graphs. */
sv_status sv_step_capture(sv_engine* e, const sv_run* runs, uint32_t n_runs, uint32_t flags, sv_capture_fn fn,
                          void* user, uint32_t* ids, float* logits, uint32_t* emitted, sv_plan_info* info);

/* Per-kernel timing of one encoded step (the reference's profile/bench_matmul hooks,
 * hooks.rs:60-112, cli/src/profile.rs): encodes the planned step `reps` times on the engine's
 * stream with a hipEvent pair around every kernel, waits, and adds each kernel's elapsed
 * milliseconds and launch count into ms[kind] / launches[kind] (arrays of SV_KIND_COUNT).
 * The steps really run (sequence state advances). */
enum {
  SV_KIND_EMBED = 0,
  SV_KIND_QKV = 1,
  SV_KIND_ATTN = 2,
  SV_KIND_O = 3,
  SV_KIND_GATE_UP = 4,
  SV_KIND_DOWN = 5,
  SV_KIND_HEAD = 6,
  SV_KIND_SAMPLE = 7,
  SV_KIND_ACCEPT = 8,
  SV_KIND_COMPACT = 9,
  SV_KIND_REPLAY = 10,
  SV_KIND_ATTN_MERGE = 11, /* the attention split merge (its own launch) */
  SV_KIND_KV_WRITE = 12,   /* prompt chunks: the new K/V rows, before the attention */
  SV_KIND_MUDD = 13,
  SV_KIND_DRAFT = 14,      /* the drafter's pass (every launch of it) */
  SV_KIND_LAYERS = 15,     /* every layer of a 1-8 row step in one persistent launch */
  SV_KIND_COUNT = 16
};
sv_status sv_profile_step(sv_engine* e, uint32_t flags, uint32_t reps, float* ms, uint32_t* launches);

/* hooks.rs:41-55 sample_logits: the sampler on caller logits (host [rows][vocab]) with
 * per-row (temperature, top_p, seed, position). */
sv_status sv_sample_logits(sv_engine* e, const float* logits, uint32_t rows, const float* temperature,
                           const float* top_p, const uint64_t* seed, const uint32_t* pos, uint32_t* ids);

#ifdef __cplusplus
}
#endif
#endif /* SV_VERIFY_H */
