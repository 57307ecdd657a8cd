/*
 * oracle.c — CPU restatement of the reference's verify path. TEST INFRASTRUCTURE ONLY:
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
 * product library.
 *
 * Reference: Belluxx/silicon-violetto, engine/src/kernels.metal (Metal), engine/src/engine/
 * {plan,kv,encode}.rs, engine/src/engine.rs, tools/convert.py. Neither Metal nor Rust can be
 * built in this image, so this is a transcription of semantics, not a build of the
 * reference.
 *
 * How each function is pinned (tests/test_oracle.py), independently of its own formula:
 *   orc_to_bf / orc_round_bf16  exhaustive over all 2^32 bit patterns against numpy's
 *                               float32 -> bfloat16-by-rounding written from IEEE-754
 *                               (round to nearest, ties to even on the 16 dropped bits).
 *   orc_philox                  Random123 known-answer vectors for philox4x32-10.
 *   orc_exp2                    every float in [-126, 0] against double-precision exp2:
 *                               max error 2 ulp; exact at integers.
 *   orc_quantize                closed-form invariants: s = bf16(absmax/127), |q| <= 127,
 *                               |w - q s| <= s/2 (or the clamp's quarter step), exact ties
 *                               to even on constructed half-step inputs.
 *   orc_matmul                  numpy float64 matmul of the dequantised weights and each
 *                               epilogue's textbook form; identity / one-hot special cases.
 *   orc_attn_verify             numpy textbook softmax attention (with max subtraction)
 *                               over the same bf16 K/V; uniform-V and masked-key invariants.
 *   orc_sample                  T = 0 vs numpy argmax; T > 0 on tiny vocabularies against
 *                               an independent sort-based inverse-CDF sampler, enumerating
 *                               uniforms; top-p = 1 takes one round.
 *   orc_accept / orc_kv_compact brute force over all small trees and sample outcomes with an
 *                               independent longest-matching-path search.
 *   orc_pool_*                  LIFO order 0, 1, 2, ... and release/reuse order.
 *   orc_step                    the lossless-speculation invariant (bench_spec.rs:119-139):
 *                               greedy verify with replayed drafts emits the plain-decode
 *                               tokens.
 *   orc_rope_table              float64 cos/sin of the same float32 angle rounded to bf16 by
 *                               torch: equal except one bf16 step at rounding boundaries.
 *   orc_embed, orc_rmsnorm_rows a hand-built feed/tree resolution case; outputs collinear with
 *                               the input row, mean square 1 / (1 + eps / ms), constant-row
 *                               closed form.
 *   orc_replay_draft            rate 0 replays the trace, rate 1 shifts every id by one, runs
 *                               without head rows untouched, chain node encoding.
 *   orc_draft_top               numpy: the candidates are the top ids of a float64 sort
 *                               (value descending, id ascending); probabilities within 1e-6 of
 *                               the float64 softmax.
 *   orc_draft_tree              brute force over every candidate path of the block: the nodes
 *                               are the paths with the highest fp32 path products, in order.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define LOG2E_F 1.44269504088896340736f

/* ---------------------------------------------------------------- scalars */

/* kernels.metal:17 bf(): bf16 bits to float. */
float orc_bf(uint16_t u) {
  uint32_t b = (uint32_t)u << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* kernels.metal:23-27 to_bf(): round to nearest even (finite inputs). */
uint16_t orc_to_bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* plan.rs:176-179 round_bf16(). */
float orc_round_bf16(float x) { return orc_bf(orc_to_bf(x)); }

/* kernels.metal:1464-1472 philox(): Philox4x32-10 (Salmon et al. 2011), in place. */
void orc_philox(uint32_t c[4], const uint32_t key[2]) {
  uint32_t k0 = key[0], k1 = key[1];
  for (int i = 0; i < 10; i++) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

/* kernels.metal:1475-1477 uniform01(): (philox((pos, round, 0, 0); seed).x >> 8) 2^-24. */
float orc_uniform01(uint32_t seed_lo, uint32_t seed_hi, uint32_t pos, uint32_t round) {
  uint32_t c[4] = {pos, round, 0, 0};
  const uint32_t k[2] = {seed_lo, seed_hi};
  orc_philox(c, k);
  return (float)(c[0] >> 8) * 0x1p-24f;
}

/* exp2 for the sampler. The reference calls Metal's exp2 (kernels.metal:1536,1553), whose
 * bits are Apple's; both this oracle and the HIP sampler use this one function instead, so
 * their draws agree bit for bit. Method: Cody-Waite range reduction x = n + f with
 * n = rint(x), |f| <= 1/2 (exact), then 2^f by the degree-7 Taylor polynomial of e^(f ln 2)
 * in Horner form with fused multiply-adds, then an exact scaling by 2^n. Results below
 * 2^-125 flush to 0, so no step depends on subnormal handling. */
float orc_exp2(float x) {
  if (!(x >= -125.0f)) return 0.0f;
  if (x > 127.0f) return INFINITY;
  const float nf = rintf(x);
  const float f = x - nf;
  float p = 1.525273380405984e-05f;
  p = fmaf(p, f, 1.5403530393381608e-04f);
  p = fmaf(p, f, 1.3333558146428443e-03f);
  p = fmaf(p, f, 9.6181291076284772e-03f);
  p = fmaf(p, f, 5.5504108664821580e-02f);
  p = fmaf(p, f, 2.4022650695910071e-01f);
  p = fmaf(p, f, 6.9314718055994531e-01f);
  p = fmaf(p, f, 1.0f);
  const int n = (int)nf;
  uint32_t sb = (uint32_t)(n + 127) << 23;
  float s;
  memcpy(&s, &sb, 4);
  return p * s;
}

/* --------------------------------------------------------------- formats */

/* tools/convert.py:41-50 quantize(): symmetric int8 per group of `group` consecutive k;
 * s = bf16(absmax / 127) (fp32 division, RNE); q = clamp(round_half_even(w / s), +-127);
 * s = 0 gives q = 0. */
void orc_quantize(const float* w, uint32_t m, uint32_t k, uint32_t group, int8_t* q, uint16_t* s) {
  const uint32_t ng = k / group;
  for (uint32_t r = 0; r < m; r++) {
    for (uint32_t gi = 0; gi < ng; gi++) {
      const float* g = w + (size_t)r * k + (size_t)gi * group;
      float amax = 0.0f;
      for (uint32_t i = 0; i < group; i++) amax = fmaxf(amax, fabsf(g[i]));
      const uint16_t sb = orc_to_bf(amax / 127.0f);
      s[(size_t)r * ng + gi] = sb;
      const float sf = orc_bf(sb);
      for (uint32_t i = 0; i < group; i++) {
        float v = sf > 0.0f ? rintf(g[i] / sf) : 0.0f;
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        q[(size_t)r * k + (size_t)gi * group + i] = (int8_t)v;
      }
    }
  }
}

/* engine.rs:394-421 rope_table(): tab[pos][j] = (bf16(cos th), bf16(sin th)),
 * th = float(pos) * freq[j] in fp32, j < 32. */
void orc_rope_table(const float* freq, uint32_t n_pos, float* tab) {
  for (uint32_t pos = 0; pos < n_pos; pos++)
    for (uint32_t j = 0; j < SV_ROPE_PAIRS; j++) {
      const float th = (float)pos * freq[j];
      tab[((size_t)pos * SV_ROPE_PAIRS + j) * 2] = orc_round_bf16(cosf(th));
      tab[((size_t)pos * SV_ROPE_PAIRS + j) * 2 + 1] = orc_round_bf16(sinf(th));
    }
}

/* ---------------------------------------------------------------- kernels */

/* kernels.metal:64-72 tree nodes. */
static inline uint32_t node_depth(uint32_t n) { return n & 0xffu; }
static inline uint32_t node_parent(uint32_t n) { return (n >> 8) & 0xffu; }
static inline uint32_t node_sees(uint32_t n) { return n >> 16; }
static inline uint32_t chain_node(uint32_t row) {
  return row | (row == 0 ? SV_NO_PARENT : row - 1) << 8 | ((2u << row) - 1u) << 16;
}

/* kernels.metal:82-114 embed(). */
void orc_embed(const sv_shape* sh, const uint16_t* table, uint32_t* tokens, float* out, const uint32_t* tin,
               uint32_t* meta, const uint32_t* lens, const uint32_t* feed, const uint32_t* tree, uint32_t* vis,
               uint32_t n) {
  const uint32_t H = sh->hidden;
  for (uint32_t t = 0; t < n; t++) {
    const uint32_t slot = tin[2 * t];
    uint32_t tok = tokens[t], depth = tin[2 * t + 1];
    if (tok >= SV_FEED_ROW) {
      const uint32_t i = tok - SV_FEED_ROW, node = tree[slot * SV_FEED_W + i];
      tok = feed[slot * SV_FEED_W + i];
      depth = node_depth(node);
      vis[t] = node_sees(node);
    }
    const uint16_t* row = table + (size_t)tok * H;
    double ss = 0.0;
    for (uint32_t i = 0; i < H; i++) {
      const double v = orc_bf(row[i]);
      ss += v * v;
    }
    const double inv = 1.0 / sqrt(ss / H + (double)SV_RMS_EPS);
    for (uint32_t i = 0; i < H; i++) out[(size_t)t * H + i] = (float)(orc_bf(row[i]) * inv);
    tokens[t] = tok;
    meta[2 * t] = slot;
    meta[2 * t + 1] = lens[slot] + depth;
  }
}

/* kernels.metal:117-131 rmsnorm_rows(). */
void orc_rmsnorm_rows(const float* in, const uint32_t* rows, float* out, uint32_t n, uint32_t hidden) {
  for (uint32_t r = 0; r < n; r++) {
    const float* x = in + (size_t)rows[r] * hidden;
    double ss = 0.0;
    for (uint32_t i = 0; i < hidden; i++) ss += (double)x[i] * x[i];
    const double inv = 1.0 / sqrt(ss / hidden + (double)SV_RMS_EPS);
    for (uint32_t i = 0; i < hidden; i++) out[(size_t)r * hidden + i] = (float)(x[i] * inv);
  }
}

static inline double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

/* kernels.metal:151-209 (formats, epilogue, epilogue_swiglu) with the dot products of
 * gemv_impl/gemm_stream_impl/gemm_impl (:216-298, :524-674, :335-462): y[t][row] =
 * epilogue(sum_k w[row][k] x[t][k]), weights dequantised as q * scale[row][k >> gshift]. */
void orc_matmul(const sv_matrix* w, const float* x, const uint32_t* x_rows, float* y, const float* base, float* aux,
                const sv_mat_args* a) {
  const uint32_t n = a->n, k = a->k, m = a->m;
  double* inv = (double*)malloc(sizeof(double) * n);
  const float** xr = (const float**)malloc(sizeof(float*) * n);
  for (uint32_t t = 0; t < n; t++) {
    xr[t] = x + (size_t)(x_rows ? x_rows[t] : t) * k;
    double ss = 0.0;
    for (uint32_t i = 0; i < k; i++) ss += (double)xr[t][i] * xr[t][i];
    inv[t] = 1.0 / sqrt(ss / k + (double)SV_RMS_EPS);
    if ((a->flags & SV_FLAG_WRITE_INV) && a->epi == SV_EPI_NORM) aux[t] = (float)inv[t];
  }
  const int swiglu = a->epi == SV_EPI_SWIGLU;
  const int step = swiglu ? 2 : 1;
#pragma omp parallel
  {
    double* wr = (double*)malloc(sizeof(double) * k * 2);
#pragma omp for schedule(static)
    for (int64_t r0 = 0; r0 < (int64_t)m; r0 += step) {
      double acc[2][64];  /* [row of the pair][token], n <= 64 per pass */
      for (uint32_t t0 = 0; t0 < n; t0 += 64) {
        const uint32_t nt = n - t0 < 64 ? n - t0 : 64;
        for (int p = 0; p < step; p++) {
          const uint32_t row = (uint32_t)r0 + p;
          double* wrow = wr + (size_t)p * k;
          if (t0 == 0) {
            if (w->format == SV_FMT_I8) {
              /* one scale per row when the group covers k (per output channel) */
              const int per_row = a->gshift >= 32 || (1ull << a->gshift) >= k;
              const int8_t* q = (const int8_t*)w->d_w + (size_t)row * k;
              const uint16_t* sc = w->d_scales + (size_t)row * (per_row ? 1 : k >> a->gshift);
              for (uint32_t i = 0; i < k; i++) wrow[i] = (double)q[i] * orc_bf(sc[per_row ? 0 : i >> a->gshift]);
            } else {
              const uint16_t* b = (const uint16_t*)w->d_w + (size_t)row * k;
              for (uint32_t i = 0; i < k; i++) wrow[i] = orc_bf(b[i]);
            }
          }
          for (uint32_t tt = 0; tt < nt; tt++) {
            const float* xt = xr[t0 + tt];
            double s = 0.0;
            for (uint32_t i = 0; i < k; i++) s += wrow[i] * xt[i];
            acc[p][tt] = s;
          }
        }
        for (uint32_t tt = 0; tt < nt; tt++) {
          const uint32_t t = t0 + tt;
          if (swiglu) {
            const double g = acc[0][tt] * inv[t] * a->scale, u = acc[1][tt] * inv[t] * a->scale;
            y[(size_t)t * (m / 2) + r0 / 2] = (float)(g * sigmoid_d(g) * u);
            continue;
          }
          const uint32_t row = (uint32_t)r0;
          const size_t o = (size_t)t * m + row;
          double v = acc[0][tt];
          if ((a->flags & SV_FLAG_NORM_IN) && a->epi != SV_EPI_NORM) v *= inv[t];
          switch (a->epi) {
            case SV_EPI_NORM: y[o] = (float)(v * inv[t] * a->scale); break;
            case SV_EPI_RAW: y[o] = (float)v; break;
            case SV_EPI_RESID: {
              const double sv = a->scale * v;
              y[o] = (float)(a->ra * (double)base[o] + a->rb * sv);
              if (a->flags & SV_FLAG_WRITE_RAW) aux[o] = (float)sv;
              break;
            }
            case SV_EPI_HEAD:
              y[o] = row < a->vocab_real ? (float)(23.0 * sigmoid_d((v + 5.0) / 7.5)) : -INFINITY;
              break;
            default: break;
          }
        }
      }
    }
    free(wr);
  }
  free(xr);
  free(inv);
}

/* kernels.metal:704-711 kv_row_of(), global layers: element offset of the K (or V) row of
 * kv head g at cache position pos. */
static inline size_t kv_row(const sv_kv_args* kv, const uint32_t* page_table, uint32_t layer, uint32_t seq,
                            uint32_t g, uint32_t pos, uint32_t nkv, uint32_t D) {
  const uint32_t page = page_table[(size_t)seq * kv->max_pages + (pos >> kv->page_shift)];
  const uint32_t psize = 1u << kv->page_shift;
  return (((size_t)layer * kv->n_pages + page) * nkv + g) * psize * D + (size_t)(pos & (psize - 1)) * D;
}

/* kernels.metal:727-736 norm_rope(): rms-norm over the head (no gain), then RoPE on pairs
 * (2j, 2j+1), j < 32: (c a0 + s a1, c a1 - s a0). */
static void norm_rope_d(const float* v, double* o, uint32_t D, int rope, const float* cs) {
  double ss = 0.0;
  for (uint32_t d = 0; d < D; d++) ss += (double)v[d] * v[d];
  const double inv = 1.0 / sqrt(ss / D + (double)SV_RMS_EPS);
  for (uint32_t d = 0; d < D; d++) o[d] = v[d] * inv;
  if (rope)
    for (uint32_t j = 0; j < SV_ROPE_PAIRS && 2 * j + 1 < D; j++) {
      const double c = cs[2 * j], s = cs[2 * j + 1], a0 = o[2 * j], a1 = o[2 * j + 1];
      o[2 * j] = c * a0 + s * a1;
      o[2 * j + 1] = c * a1 - s * a0;
    }
}

/* kernels.metal:808-811 key_lo(): the first cached key a query at pos sees; a
 * sliding-window layer (is_global 0) sees `window` keys besides itself. */
static inline uint32_t key_lo(const sv_kv_args* kv, uint32_t pos) {
  return !kv->is_global && pos > kv->window ? pos - kv->window : 0u;
}

static inline double sigmoid2_d(double x) { return 2.0 / (1.0 + exp(-x)); }

/* sum over d < n of x[d] inv w[d]: a gate's input, rms_norm(x)[:n] . w (kernels.metal:738-747,
 * 936-941) */
static double gate_dot(const float* x, float inv, const float* w, uint32_t n) {
  double s = 0.0;
  for (uint32_t d = 0; d < n; d++) s += (double)x[d] * inv * w[d];
  return s;
}

/* kernels.metal:891-1148 attn_verify (new_key :910-942, verify_batches :963-1006) and
 * :1316-1362 attn_dec_reduce, as exact math: per run, the new keys are normed, roped,
 * rounded to bf16 and written at p0 + row (values first get their value embedding,
 * add_ve :738-747); each token's query (normed, roped, times scale_log2) attends to the cached
 * keys [key_lo(pos), p0) and the run's new keys in its vis mask, with p = 2^s and out =
 * sum p v / sum p (no running max: scores are bounded, :804-806); then XSA, out - xsa[h]
 * (out . v) v with v the token's value row of its kv head over max(|v|, 1e-4), and the gate
 * 2 sigmoid(rms_norm(x)[:D] . attn_gate[h]) (:1355-1361). ex NULL, or a NULL member: that part
 * off (xsa 0, gate 1). */
void orc_attn_verify(const sv_shape* sh, const float* qkv, const uint32_t* meta, uint16_t* k_cache,
                     uint16_t* v_cache, const uint32_t* page_table, const float* rope, const sv_kv_args* kv,
                     const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs, const uint32_t* vis,
                     float* out, const sv_attn_extras* ex) {
  orc_attn_verify_cap(sh, qkv, meta, k_cache, v_cache, page_table, rope, kv, args, runs, n_runs, vis, out, ex, NULL,
                      NULL, NULL, NULL);
}

void orc_attn_verify_cap(const sv_shape* sh, const float* qkv, const uint32_t* meta, uint16_t* k_cache,
                         uint16_t* v_cache, const uint32_t* page_table, const float* rope, const sv_kv_args* kv,
                         const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs, const uint32_t* vis,
                         float* out, const sv_attn_extras* ex, float* cap_q, float* cap_k, float* cap_v,
                         float* cap_sdpa) {
  const uint32_t D = sh->head_dim, NQ = sh->n_heads, NKV = sh->n_kv_heads, G = NQ / NKV;
  const uint32_t W = (NQ + 2 * NKV) * D, KOFF = NQ * D, VOFF = (NQ + NKV) * D;
  const uint32_t L = kv->kv_layer;
  const float* ve_gate = ex ? ex->d_ve_gate : NULL;
  const float* attn_gate = ex ? ex->d_attn_gate : NULL;
  const float* xsa = ex ? ex->d_xsa : NULL;
  for (uint32_t r = 0; r < n_runs; r++) {
    const uint32_t t0 = runs[2 * r], T = runs[2 * r + 1];
    const uint32_t seq = meta[2 * t0], p0 = meta[2 * t0 + 1];
    /* the new keys and values, bf16, and the values' directions */
    uint16_t* nk = (uint16_t*)malloc(sizeof(uint16_t) * T * NKV * D);
    uint16_t* nv = (uint16_t*)malloc(sizeof(uint16_t) * T * NKV * D);
    double* vdir = (double*)malloc(sizeof(double) * T * NKV * D);
    double* tmp = (double*)malloc(sizeof(double) * D);
    for (uint32_t i = 0; i < T; i++) {
      const uint32_t t = t0 + i, pos = meta[2 * t + 1];
      for (uint32_t g = 0; g < NKV; g++) {
        norm_rope_d(qkv + (size_t)t * W + KOFF + g * D, tmp, D, (int)args->rope, rope + (size_t)pos * 64);
        const size_t row = kv_row(kv, page_table, L, seq, g, p0 + i, NKV, D);
        double ve_g = 0.0;
        if (ve_gate)
          ve_g = sigmoid2_d(gate_dot(ex->d_x + (size_t)t * ex->hidden, ex->d_inv[t], ve_gate + g * SV_VE_GATE_W,
                                     SV_VE_GATE_W));
        double vs = 0.0;
        for (uint32_t d = 0; d < D; d++) {
          double v = qkv[(size_t)t * W + VOFF + g * D + d];
          if (ve_gate) v += ve_g * orc_bf(ex->d_value_embed[((size_t)ex->d_tokens[t] * NKV + g) * D + d]);
          vdir[((size_t)i * NKV + g) * D + d] = v;
          vs += v * v;
          if (cap_k) cap_k[((size_t)t * NKV + g) * D + d] = (float)tmp[d];
          if (cap_v) cap_v[((size_t)t * NKV + g) * D + d] = (float)v;
          const uint16_t kb = orc_to_bf((float)tmp[d]);
          const uint16_t vb = orc_to_bf((float)v);
          nk[((size_t)i * NKV + g) * D + d] = kb;
          nv[((size_t)i * NKV + g) * D + d] = vb;
          k_cache[row + d] = kb;
          v_cache[row + d] = vb;
        }
        const double den = fmax(sqrt(vs), 1e-4);
        for (uint32_t d = 0; d < D; d++) vdir[((size_t)i * NKV + g) * D + d] /= den;
      }
    }
    free(tmp);
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (uint32_t i = 0; i < T; i++) {
      for (uint32_t h = 0; h < NQ; h++) {
        const uint32_t t = t0 + i, pos = meta[2 * t + 1], g = h / G;
        double q[128], o[128];
        norm_rope_d(qkv + (size_t)t * W + h * D, q, D, (int)args->rope, rope + (size_t)pos * 64);
        for (uint32_t d = 0; d < D; d++) {
          if (cap_q) cap_q[(size_t)t * NQ * D + h * D + d] = (float)q[d];
          q[d] *= args->scale_log2;
          o[d] = 0.0;
        }
        double l = 0.0;
        for (uint32_t j = key_lo(kv, pos); j < p0; j++) {
          const size_t row = kv_row(kv, page_table, L, seq, g, j, NKV, D);
          double s = 0.0;
          for (uint32_t d = 0; d < D; d++) s += orc_bf(k_cache[row + d]) * q[d];
          const double p = exp2(s);
          l += p;
          for (uint32_t d = 0; d < D; d++) o[d] += p * orc_bf(v_cache[row + d]);
        }
        for (uint32_t j = 0; j < T; j++) {
          if (!((vis[t] >> j) & 1u)) continue;
          double s = 0.0;
          for (uint32_t d = 0; d < D; d++) s += orc_bf(nk[((size_t)j * NKV + g) * D + d]) * q[d];
          const double p = exp2(s);
          l += p;
          for (uint32_t d = 0; d < D; d++) o[d] += p * orc_bf(nv[((size_t)j * NKV + g) * D + d]);
        }
        for (uint32_t d = 0; d < D; d++) o[d] /= l;
        if (cap_sdpa)
          for (uint32_t d = 0; d < D; d++) cap_sdpa[(size_t)t * NQ * D + h * D + d] = (float)o[d];
        if (xsa) {
          const double* vd = vdir + ((size_t)i * NKV + g) * D;
          double dp = 0.0;
          for (uint32_t d = 0; d < D; d++) dp += o[d] * vd[d];
          for (uint32_t d = 0; d < D; d++) o[d] -= (double)xsa[h] * dp * vd[d];
        }
        const double gate =
            attn_gate ? sigmoid2_d(gate_dot(ex->d_x + (size_t)t * ex->hidden, ex->d_inv[t], attn_gate + (size_t)h * D, D))
                      : 1.0;
        for (uint32_t d = 0; d < D; d++) out[(size_t)t * NQ * D + h * D + d] = (float)(o[d] * gate);
      }
    }
    free(nk);
    free(nv);
    free(vdir);
  }
}

/* kernels.metal:1364-1407 mudd(), exact math: inner = gelu(dense1 . rms_norm(cur)) with the
 * erf form of gelu (C's erf: the reference's Abramowitz & Stegun 7.1.26 is within 1.5e-7 of it,
 * kernels.metal:30-37), w = mix . inner + bias, then the two mixes of (tap0, tap1, cur). */
void orc_mudd(const float* cur, const float* tap0, const float* tap1, const float* dense1, const float* mix,
              float* out_attn, float* out_base, uint32_t n, uint32_t hidden) {
#pragma omp parallel for schedule(static)
  for (uint32_t t = 0; t < n; t++) {
    const float* c = cur + (size_t)t * hidden;
    double ss = 0.0;
    for (uint32_t i = 0; i < hidden; i++) ss += (double)c[i] * c[i];
    const double inv = 1.0 / sqrt(ss / hidden + (double)SV_RMS_EPS);
    double inner[SV_MUDD_INNER], w[6];
    for (uint32_t j = 0; j < SV_MUDD_INNER; j++) {
      double s = 0.0;
      for (uint32_t i = 0; i < hidden; i++) s += (double)c[i] * inv * dense1[(size_t)j * hidden + i];
      inner[j] = 0.5 * s * (1.0 + erf(s * 0.70710678118654752440));
    }
    for (uint32_t k = 0; k < 6; k++) {
      const float* row = mix + k * (SV_MUDD_INNER + 1);
      double s = 0.0;
      for (uint32_t j = 0; j < SV_MUDD_INNER; j++) s += inner[j] * row[j];
      w[k] = s + row[SV_MUDD_INNER];
    }
    for (uint32_t i = 0; i < hidden; i++) {
      const size_t o = (size_t)t * hidden + i;
      out_attn[o] = (float)(w[0] * tap0[o] + w[1] * tap1[o] + w[2] * c[i]);
      out_base[o] = (float)(w[3] * tap0[o] + w[4] * tap1[o] + w[5] * c[i]);
    }
  }
}

/* kernels.metal:1418-1420 better(): larger value, ties to the lower id. */
static inline void better(float* bv, uint32_t* bi, float v, uint32_t i) {
  if (v > *bv || (v == *bv && i < *bi)) {
    *bv = v;
    *bi = i;
  }
}

/* kernels.metal:1484-1501 tg_scan(): ex[t] = sum of v over threads before t (32 serial runs
 * of 32, then their bases in order), ex[1024] = the total. */
static void tg_scan(const float* v, float* ex) {
  float base[32];
  for (uint32_t g = 0; g < 32; g++) {
    float acc = 0.0f;
    for (uint32_t i = 32 * g; i < 32 * g + 32; i++) {
      const float x = v[i];
      ex[i] = acc;
      acc += x;
    }
    base[g] = acc;
  }
  float acc = 0.0f;
  for (uint32_t g = 0; g < 32; g++) {
    const float x = base[g];
    base[g] = acc;
    acc += x;
  }
  ex[SV_SAMPLE_THREADS] = acc;
  for (uint32_t t = 0; t < SV_SAMPLE_THREADS; t++) ex[t] += base[t / 32];
}

/* kernels.metal:1845-1891 draft_top(): for each drafted block row (tin[r].y > 0; the
 * block's row 0 is the bonus token's and is skipped) the `ncand` best drafter logits, taken
 * one at a time as the best id not yet taken (ties to the lowest id), their target ids
 * through `vocab`, and their probabilities at temperature 1 / inv_t: exp((v_c - v_0) inv_t)
 * / z, z = the sum over the whole row. exp(y) is exp2(y log2 e) with this file's exp2; the
 * sum runs in the sampler's order (thread t of 1024 owns ids t, t + 1024, ...; tg_scan). */
void orc_draft_top(const float* logits, const uint32_t* vocab, const uint32_t* tin, uint32_t* cand, float* cand_q,
                   uint32_t n_rows, uint32_t nv, float inv_t, uint32_t ncand) {
  float* s = (float*)malloc(sizeof(float) * SV_SAMPLE_THREADS);
  float* ex = (float*)malloc(sizeof(float) * (SV_SAMPLE_THREADS + 1));
  const float c = inv_t * LOG2E_F;
  for (uint32_t r = 0; r < n_rows; r++) {
    if (tin[2 * r + 1] == 0) continue;
    const float* x = logits + (size_t)r * nv;
    float top_v[SV_DRAFT_CANDS];
    uint32_t top_i[SV_DRAFT_CANDS];
    for (uint32_t k = 0; k < ncand; k++) {
      float bv = -FLT_MAX;
      uint32_t bi = 0xffffffffu;
      for (uint32_t j = 0; j < nv; j++) {
        int taken = 0;
        for (uint32_t m = 0; m < k; m++) taken |= top_i[m] == j;
        if (!taken) better(&bv, &bi, x[j], j);
      }
      top_v[k] = bv;
      top_i[k] = bi;
    }
    for (uint32_t t = 0; t < SV_SAMPLE_THREADS; t++) {
      float a = 0.0f;
      for (uint32_t j = t; j < nv; j += SV_SAMPLE_THREADS) a += orc_exp2((x[j] - top_v[0]) * c);
      s[t] = a;
    }
    tg_scan(s, ex);
    const float z = ex[SV_SAMPLE_THREADS];
    for (uint32_t k = 0; k < ncand; k++) {  /* a row without k + 1 ordered values: no candidate */
      const int ok = top_i[k] < nv && top_i[0] < nv;
      cand[r * SV_DRAFT_CANDS + k] = ok ? vocab[top_i[k]] : SV_NO_TOK;
      cand_q[r * SV_DRAFT_CANDS + k] = ok ? orc_exp2((top_v[k] - top_v[0]) * c) / z : 0.0f;
    }
  }
  free(s);
  free(ex);
}

/* kernels.metal:1893-1934 draft_tree(): each block's draft tree, best-first (DDTree): the next
 * node is the best not-yet-taken candidate of any node so far, scored by the fp32 product of
 * q along its path; a node at depth d takes its children from block row d + 1's candidates
 * (rows are marginals); depth stays below the block's rows. Nodes go to feed/tree[slot][1..]
 * in the order taken (parents first, encoded depth | parent << 8 | sees << 16); the rest of
 * the slot's 16 entries become dead nodes (depth 1, no parent, seeing the root and itself).
 * A candidate draft_top could not fill (SV_NO_TOK) is never taken (the reference would read
 * its vocabulary out of range there). */
void orc_draft_tree(const uint32_t* blocks, uint32_t nblocks, const uint32_t* tin, const uint32_t* cand,
                    const float* cand_q, uint32_t* feed, uint32_t* tree, uint32_t ncand) {
  for (uint32_t b = 0; b < nblocks; b++) {
    const uint32_t first = blocks[2 * b], rows = blocks[2 * b + 1] < SV_FEED_W ? blocks[2 * b + 1] : SV_FEED_W;
    const uint32_t slot = tin[2 * first];
    float score[SV_FEED_W];
    uint32_t depth[SV_FEED_W], taken[SV_FEED_W], sees[SV_FEED_W];
    score[0] = 1.0f;
    depth[0] = taken[0] = 0;
    sees[0] = 1;
    uint32_t n = 1;
    for (; n < rows; n++) {
      float best = -1.0f;
      uint32_t p = 0;
      for (uint32_t i = 0; i < n; i++) {
        const uint32_t cc = (first + depth[i] + 1) * SV_DRAFT_CANDS + taken[i];
        if (depth[i] + 1 == rows || taken[i] == ncand || cand[cc] == SV_NO_TOK) continue;
        const float sc = score[i] * cand_q[cc];
        if (sc > best) {
          best = sc;
          p = i;
        }
      }
      if (best < 0.0f) break;
      const uint32_t d = depth[p] + 1;
      feed[slot * SV_FEED_W + n] = cand[(first + d) * SV_DRAFT_CANDS + taken[p]];
      taken[p]++;
      score[n] = best;
      depth[n] = d;
      taken[n] = 0;
      sees[n] = sees[p] | 1u << n;
      tree[slot * SV_FEED_W + n] = d | p << 8 | sees[n] << 16;
    }
    for (; n < SV_FEED_W; n++) tree[slot * SV_FEED_W + n] = 1u | SV_NO_PARENT << 8 | (1u | 1u << n) << 16;
  }
}

/* kernels.metal:1503-1576 sample() (with argmax_partial :1430-1451), thread by thread in
 * the kernel's summation order: thread t owns ids t, t + 1024, ... */
void orc_sample(const float* logits, const sv_sample_row* rows, uint32_t* out, const uint32_t* meta,
                uint32_t n_rows, uint32_t vocab) {
  float* s = (float*)malloc(sizeof(float) * SV_SAMPLE_THREADS);
  float* ex = (float*)malloc(sizeof(float) * (SV_SAMPLE_THREADS + 1));
  for (uint32_t r = 0; r < n_rows; r++) {
    const sv_sample_row row = rows[r];
    const uint32_t pos = row.tok == SV_NO_TOK ? row.pos : meta[2 * row.tok + 1] + 1;
    const float* x = logits + (size_t)r * vocab;
    float lmax = -FLT_MAX;
    uint32_t tok = 0xffffffffu;
    for (uint32_t i = 0; i < vocab; i++) better(&lmax, &tok, x[i], i);
    if (row.temperature > 0.0f) {
      const float c = LOG2E_F / row.temperature;
      for (uint32_t t = 0; t < SV_SAMPLE_THREADS; t++) {
        float a = 0.0f;
        for (uint32_t i = t; i < vocab; i += SV_SAMPLE_THREADS) a += orc_exp2((x[i] - lmax) * c);
        s[t] = a;
      }
      tg_scan(s, ex);
      const float z = ex[SV_SAMPLE_THREADS];
      float low = -INFINITY;
      for (uint32_t round = 0; round < SV_SAMPLE_ROUNDS; round++) {
        const float target = orc_uniform01(row.seed_lo, row.seed_hi, pos, round) * ex[SV_SAMPLE_THREADS];
        uint32_t pick = 0xffffffffu;
        for (uint32_t t = 0; t < SV_SAMPLE_THREADS; t++) {
          const float lo = ex[t];
          if (lo <= target && target < ex[t + 1]) {
            float acc = 0.0f;
            uint32_t j = 0xffffffffu;
            for (uint32_t i = t; i < vocab; i += SV_SAMPLE_THREADS) {
              const float xi = x[i];
              if (!(xi > low)) continue;
              const float e = orc_exp2((xi - lmax) * c);
              acc += e;
              if (e > 0.0f) j = i;
              if (target - lo < acc) break;
            }
            pick = j;
          }
        }
        const uint32_t j = pick;
        if (j == 0xffffffffu) break;
        const float xj = x[j];
        if (xj == lmax || row.top_p >= 1.0f) {
          tok = j;
          break;
        }
        for (uint32_t t = 0; t < SV_SAMPLE_THREADS; t++) {
          float q = 0.0f;
          for (uint32_t i = t; i < vocab; i += SV_SAMPLE_THREADS) {
            const float xi = x[i];
            if (xi > xj) q += orc_exp2((xi - lmax) * c);
          }
          s[t] = q;
        }
        tg_scan(s, ex);
        if (ex[SV_SAMPLE_THREADS] < row.top_p * z) {
          tok = j;
          break;
        }
        low = xj;
      }
    }
    out[r] = tok;
  }
  free(s);
  free(ex);
}

/* kernels.metal:1605-1657 accept(). One difference: a run that emits nothing (k = 0, only
 * possible with remaining = 0 on a slot not marked done) leaves feed alone, where the
 * reference would read out[first - 1]. */
void orc_accept(const sv_run_in* runs, const uint32_t* tokens, uint32_t* out, uint32_t* lens, uint32_t* feed,
                sv_gen_state* gen, uint32_t* emitted, uint32_t nruns, const uint32_t* tree, uint32_t* path,
                uint32_t* path_len, uint32_t* on_path) {
  for (uint32_t r = 0; r < nruns; r++) {
    const sv_run_in ru = runs[r];
    sv_gen_state* gs = &gen[ru.slot];
    path_len[r] = 0;
    for (uint32_t j = 0; j < ru.count; j++) on_path[ru.first + j] = !ru.verify && !gs->done;
    if (gs->done) {
      emitted[r] = 0;
      continue;
    }
    if (!ru.verify) lens[ru.slot] += ru.count;
    if (ru.nhead == 0) {
      emitted[r] = 0;
      continue;
    }
    uint32_t first = ru.head0 + ru.nhead - 1, e = 1;
    uint32_t walk[SV_FEED_W];
    walk[0] = 0;
    if (ru.verify) {
      const uint32_t* node = tree + (size_t)ru.slot * SV_FEED_W;
      for (uint32_t c = 1, at = 0; c < ru.count; c++) {
        if (node_parent(node[c]) == at && tokens[ru.first + c] == out[ru.head0 + at]) walk[e++] = at = c;
      }
      for (uint32_t j = 1; j < e; j++) out[ru.head0 + j] = out[ru.head0 + walk[j]];
      first = ru.head0;
    }
    int stop = 0;
    uint32_t k = 0;
    while (k < e && k < gs->remaining && !stop) {
      const uint32_t tok = out[first + k];
      for (uint32_t j = 0; j < gs->nstop; j++) stop = stop || tok == gs->stop[j];
      k++;
    }
    if (ru.verify) {
      lens[ru.slot] += k;
      path_len[r] = k;
      for (uint32_t j = 0; j < k; j++) {
        path[r * SV_FEED_W + j] = walk[j];
        on_path[ru.first + walk[j]] = 1;
      }
    }
    if (k > 0) feed[ru.slot * SV_FEED_W] = out[first + k - 1];
    gs->remaining -= k;
    if (stop || gs->remaining == 0) gs->done = 1;
    emitted[r] = k;
  }
}

/* kernels.metal:1659-1693 kv_compact(): per run and layer, rows p0 + path[j] -> p0 + j for
 * j = 1..k-1 in increasing j (path[j] >= j, increasing), p0 = lens[slot] - k. */
void orc_kv_compact(const sv_shape* sh, const sv_run_in* runs, uint32_t nruns, const uint32_t* path,
                    const uint32_t* path_len, const uint32_t* lens, uint16_t* k_cache, uint16_t* v_cache,
                    const uint32_t* page_table, const sv_kv_args* kv) {
  const uint32_t D = sh->head_dim, NKV = sh->n_kv_heads;
  for (uint32_t r = 0; r < nruns; r++) {
    const uint32_t k = path_len[r], slot = runs[r].slot, p0 = lens[slot] - k;
    for (uint32_t l = 0; l < sh->n_layers; l++)
      for (uint32_t g = 0; g < NKV; g++)
        for (uint32_t j = 1; j < k; j++) {
          const uint32_t from = path[r * SV_FEED_W + j];
          if (from == j) continue;
          const size_t src = kv_row(kv, page_table, l, slot, g, p0 + from, NKV, D);
          const size_t dst = kv_row(kv, page_table, l, slot, g, p0 + j, NKV, D);
          memmove(k_cache + dst, k_cache + src, D * 2);
          memmove(v_cache + dst, v_cache + src, D * 2);
        }
  }
}

/* kernels.metal:1705-1724 replay_draft(). */
void orc_replay_draft(const sv_run_in* runs, uint32_t nruns, const uint32_t* lens, uint32_t* feed,
                      const uint32_t* trace, const uint32_t* trace_len, const sv_replay_args* ra, uint32_t* tree) {
  for (uint32_t r = 0; r < nruns; r++) {
    if (runs[r].nhead == 0) continue;
    const uint32_t slot = runs[r].slot, n = trace_len[slot];
    if (n == 0) continue;
    for (uint32_t i = 1; i < SV_FEED_W; i++) {
      const uint32_t pos = lens[slot] + i;
      uint32_t tok = pos < n ? trace[(size_t)slot * ra->stride + pos] : 0u;
      uint32_t c[4] = {pos, 0x5eed, 0, 0};
      const uint32_t key[2] = {ra->seed, 0x0dd5u};
      orc_philox(c, key);
      if ((float)(c[0] >> 8) * 0x1p-24f < ra->rate) tok = (tok + 1) % ra->vocab;
      feed[slot * SV_FEED_W + i] = tok;
      tree[slot * SV_FEED_W + i] = chain_node(i);
    }
  }
}

/* ------------------------------------------------------------ page pool */

/* kv.rs:40: free pages (0..n).rev(), popped from the back: 0, 1, 2, ... */
void orc_pool_init(orc_pool* p, uint32_t n_pages, uint32_t max_seqs, uint32_t max_pages, uint32_t page_shift,
                   uint32_t* free_list, uint32_t* page_table, uint32_t* seq_pages) {
  p->free_list = free_list;
  p->n_pages = n_pages;
  p->n_free = n_pages;
  p->max_pages = max_pages;
  p->page_shift = page_shift;
  p->page_table = page_table;
  p->seq_pages = seq_pages;
  for (uint32_t i = 0; i < n_pages; i++) free_list[i] = n_pages - 1 - i;
  memset(page_table, 0, sizeof(uint32_t) * max_seqs * max_pages);
  memset(seq_pages, 0, sizeof(uint32_t) * max_seqs);
}

/* kv.rs:49-56 reserve(): pages until they hold len positions. */
int orc_pool_reserve(orc_pool* p, uint32_t slot, uint32_t len) {
  while ((p->seq_pages[slot] << p->page_shift) < len) {
    if (p->n_free == 0) return -1;
    const uint32_t page = p->free_list[--p->n_free];
    p->page_table[(size_t)slot * p->max_pages + p->seq_pages[slot]] = page;
    p->seq_pages[slot]++;
  }
  return 0;
}

/* kv.rs:58-60 release(): pages.iter().rev() pushed back. */
void orc_pool_release(orc_pool* p, uint32_t slot) {
  for (uint32_t i = p->seq_pages[slot]; i-- > 0;)
    p->free_list[p->n_free++] = p->page_table[(size_t)slot * p->max_pages + i];
  p->seq_pages[slot] = 0;
}

/* -------------------------------------------------------------- the plan */

/* plan.rs:47-151 Engine::plan(), the buffer layout part. Attention runs of up to arun rows
 * (0: SV_MAX_RUN) see the rows before them in their run (vis bits 0..row % arun); the
 * reference's bits restart every 8 rows (plan.rs:81), which only differs past row 7. */
int orc_plan(const uint32_t* in_runs, uint32_t n_runs, const uint32_t* in_tokens, uint32_t* seq_len,
             const sv_sample_row* sampling_per_slot, uint32_t* tokens, uint32_t* tin, uint32_t* vis,
             uint32_t* head_rows, sv_sample_row* samples, sv_run_in* run_in, uint32_t arun) {
  if (arun == 0 || arun > SV_MAX_RUN) arun = SV_MAX_RUN;
  uint32_t n = 0, n_head = 0;
  for (uint32_t ri = 0; ri < n_runs; ri++) {
    const uint32_t slot = in_runs[4 * ri], count = in_runs[4 * ri + 1], verify = in_runs[4 * ri + 2],
                   head = in_runs[4 * ri + 3];
    /* a verify run holds at most arun rows (its tree); other runs (prompt chunks) any */
    if (count == 0 || (verify && count > arun)) return -1;
    for (uint32_t j = 0; j < ri; j++)
      if (in_runs[4 * j] == slot) return -1;
    const uint32_t first_row = n;
    for (uint32_t row = 0; row < count; row++) {
      tokens[n] = in_tokens[n];
      tin[2 * n] = slot;
      tin[2 * n + 1] = row;
      vis[n] = 0xffffffffu >> (31 - row % arun); /* causal within its attention run */
      n++;
    }
    const uint32_t first_head = n_head;
    if (verify)
      for (uint32_t r = first_row; r < first_row + count; r++) head_rows[n_head++] = r;
    else if (head)
      head_rows[n_head++] = first_row + count - 1;
    for (uint32_t h = first_head; h < n_head; h++) {
      samples[h] = sampling_per_slot[slot];
      samples[h].pos = 0;
      samples[h].tok = head_rows[h];
    }
    run_in[ri].slot = slot;
    run_in[ri].first = first_row;
    run_in[ri].count = count;
    run_in[ri].head0 = first_head;
    run_in[ri].nhead = n_head - first_head;
    run_in[ri].verify = verify;
    seq_len[slot] += count;
  }
  return (int)n_head;
}

/* ------------------------------------------------------------- the step */

/* encode.rs:99-126 encode_forward, encode_layer :142-190 (MUDD at its sites with the taps
 * of resid_in / resid_out :107-122), encode_verify_attention :193-231 and encode_tail
 * :383-412. Sliding-window layers (io->local) use the local cache and io->kv_local; each
 * layer's KV index counts its own kind (model.rs:112-120). */
int orc_step(const sv_shape* sh, const uint16_t* embed, const sv_layer* layers, float attn_scale,
             orc_step_io* io) {
  const uint32_t n = io->n, H = sh->hidden, D = sh->head_dim, NQ = sh->n_heads, NKV = sh->n_kv_heads;
  const uint32_t W = (NQ + 2 * NKV) * D, F = sh->ffn;
  const sv_model_extras* mx = io->extras;
  const uint32_t n_mudd = mx ? mx->n_mudd : 0;
  float* h = (float*)malloc(sizeof(float) * n * H);
  float* qkv = (float*)malloc(sizeof(float) * n * W);
  float* attn = (float*)malloc(sizeof(float) * n * NQ * D);
  float* mixed = (float*)malloc(sizeof(float) * n * H);
  float* act = (float*)malloc(sizeof(float) * n * F);
  float* inv = (float*)malloc(sizeof(float) * n);
  float* hfin = (float*)malloc(sizeof(float) * (io->n_head ? io->n_head : 1) * H);
  float* h0 = (float*)malloc(sizeof(float) * n * H);
  float* taps = (float*)malloc(sizeof(float) * SV_MUDD_SITES * n * H);
  float* xattn = (float*)malloc(sizeof(float) * n * H);
  float* rbase = (float*)malloc(sizeof(float) * n * H);
  if (!h || !qkv || !attn || !mixed || !act || !inv || !hfin || !h0 || !taps || !xattn || !rbase) return -1;
  /* step_capture: per-layer blocks (orc_step_io.cap) and the attention's q, k, v before they
   * are interleaved into the block's qkv rows */
  const uint32_t NQD = NQ * D, NKD = NKV * D;
  const size_t cap_layer = (size_t)n * (6 * H + W + NQD);
  uint32_t* iota = NULL;
  float *cq = NULL, *ck = NULL, *cv = NULL;
  if (io->cap) {
    iota = (uint32_t*)malloc(sizeof(uint32_t) * n);
    cq = (float*)malloc(sizeof(float) * n * NQD);
    ck = (float*)malloc(sizeof(float) * n * NKD);
    cv = (float*)malloc(sizeof(float) * n * NKD);
    if (!iota || !cq || !ck || !cv) return -1;
    for (uint32_t t = 0; t < n; t++) iota[t] = t;
  }

  orc_embed(sh, embed, io->tokens, h, io->tin, io->meta, io->lens, io->feed, io->tree, io->vis, n);
  memcpy(h0, h, sizeof(float) * n * H);
  uint32_t n_global = 0, n_local = 0;
  for (uint32_t li = 0; li < sh->n_layers; li++) {
    const sv_layer* l = &layers[li];
    const int local = io->local && io->local[li];
    const uint32_t kv_index = local ? n_local++ : n_global++;
    const float* x = h;
    const float* resid = h;
    float* cb = io->cap ? io->cap + li * cap_layer : NULL;
    float *c_qkv = NULL, *c_sdpa = NULL, *c_attn_out = NULL, *c_mlp_in = NULL, *c_mlp_out = NULL;
    if (cb) {
      c_qkv = cb + 2 * (size_t)n * H;
      c_sdpa = c_qkv + (size_t)n * W;
      c_attn_out = c_sdpa + (size_t)n * NQD;
      c_mlp_in = c_attn_out + (size_t)n * H;
      c_mlp_out = c_mlp_in + (size_t)n * H;
      memcpy(cb, h, sizeof(float) * n * H);
      memset(c_mlp_out + (size_t)n * H, 0, sizeof(float) * n * H);
    }
    for (uint32_t site = 0; site < n_mudd; site++)
      if (mx->mudd_layer[site] == li) {
        orc_mudd(h, h0, taps + (size_t)site * n * H, mx->mudd_dense1,
                 mx->mudd_mix + (size_t)site * 6 * (SV_MUDD_INNER + 1), xattn, rbase, n, H);
        x = xattn;
        resid = rbase;
        if (cb) memcpy(c_mlp_out + (size_t)n * H, rbase, sizeof(float) * n * H);
      }
    if (cb) orc_rmsnorm_rows(x, iota, cb + (size_t)n * H, n, H);
    sv_mat_args a;
    memset(&a, 0, sizeof a);
    a.n = n;
    a.vocab_real = sh->vocab_real;
    a.scale = 1.0f;
    a.ksplit = 1;
    /* qkv: Norm (encode.rs:163-165) */
    a.k = H;
    a.m = W;
    a.epi = SV_EPI_NORM;
    a.flags = SV_FLAG_WRITE_INV;
    a.scale = l->qkv_scale;
    a.gshift = l->qkv.gshift;
    orc_matmul(&l->qkv, x, NULL, qkv, NULL, inv, &a);
    /* attention (encode.rs:166-170) */
    sv_attn_args aa;
    memset(&aa, 0, sizeof aa);
    aa.scale_log2 = attn_scale * LOG2E_F;
    aa.rope = l->rope;
    sv_kv_args kv = local ? io->kv_local : io->kv;
    kv.kv_layer = kv_index;
    sv_attn_extras ex = {x, inv, io->tokens, mx ? mx->value_embed : NULL, l->ve_gate, l->attn_gate, l->xsa, NULL, H, 0};
    orc_attn_verify_cap(sh, qkv, io->meta, local ? io->k_local : io->k_cache, local ? io->v_local : io->v_cache,
                        local ? io->local_table : io->page_table, io->rope, &kv, &aa, io->attn_runs,
                        io->n_attn ? io->n_attn : io->n_runs, io->vis, attn, &ex, cq, ck, cv, c_sdpa);
    if (cb)
      for (uint32_t t = 0; t < n; t++) {
        memcpy(c_qkv + (size_t)t * W, cq + (size_t)t * NQD, sizeof(float) * NQD);
        memcpy(c_qkv + (size_t)t * W + NQD, ck + (size_t)t * NKD, sizeof(float) * NKD);
        memcpy(c_qkv + (size_t)t * W + NQD + NKD, cv + (size_t)t * NKD, sizeof(float) * NKD);
      }
    /* o: Resid (encode.rs:172-175) */
    a.k = NQ * D;
    a.m = H;
    a.epi = SV_EPI_RESID;
    a.flags = cb ? SV_FLAG_WRITE_RAW : 0;
    a.scale = l->o_scale;
    a.ra = l->resid_attn;
    a.rb = l->post_attn;
    a.gshift = l->o.gshift;
    orc_matmul(&l->o, attn, NULL, mixed, resid, c_attn_out, &a);
    if (cb) orc_rmsnorm_rows(mixed, iota, c_mlp_in, n, H);
    a.flags = 0;
    /* gate_up: SwiGlu (encode.rs:179-181) */
    a.k = H;
    a.m = 2 * F;
    a.epi = SV_EPI_SWIGLU;
    a.scale = 1.0f;
    a.ra = a.rb = 0.0f;
    a.gshift = l->gate_up.gshift;
    orc_matmul(&l->gate_up, mixed, NULL, act, NULL, NULL, &a);
    /* down: Resid (encode.rs:182-185) */
    a.k = F;
    a.m = H;
    a.epi = SV_EPI_RESID;
    a.scale = 1.0f;
    a.ra = l->resid_mlp;
    a.rb = l->post_mlp;
    a.gshift = l->down.gshift;
    a.flags = cb ? SV_FLAG_WRITE_RAW : 0;
    orc_matmul(&l->down, act, NULL, h, mixed, c_mlp_out, &a);
    a.flags = 0;
    for (uint32_t site = 0; site < n_mudd; site++)
      if (mx->mudd_tap[site] == li) memcpy(taps + (size_t)site * n * H, h, sizeof(float) * n * H);
    for (uint32_t k = 0; k < io->n_taps; k++)
      if (io->tap_layers[k] == li) orc_tap_rows(h, io->tap_out[k], n, H);
  }
  if (io->hidden) memcpy(io->hidden, h, sizeof(float) * n * H);
  /* tail (encode.rs:383-412): final norm of the head rows, the head (tied, or its own), the sampler,
   * accept, kv_compact */
  if (io->n_head > 0) {
    orc_rmsnorm_rows(h, io->head_rows, hfin, io->n_head, H);
    sv_matrix head = {embed, NULL, sh->vocab, H, SV_FMT_BF16, 0};
    if (io->head) head = *io->head;
    sv_mat_args a;
    memset(&a, 0, sizeof a);
    a.n = io->n_head;
    a.k = H;
    a.m = sh->vocab;
    a.epi = SV_EPI_HEAD;
    a.vocab_real = sh->vocab_real;
    a.scale = 1.0f;
    a.gshift = head.gshift;
    orc_matmul(&head, hfin, NULL, io->logits, NULL, NULL, &a);
    orc_sample(io->logits, io->samples, io->out, io->meta, io->n_head, sh->vocab);
  }
  orc_accept(io->runs, io->tokens, io->out, io->lens, io->feed, io->gen, io->emitted, io->n_runs, io->tree,
             io->path, io->path_len, io->on_path);
  if (io->compact) {
    sv_shape part = *sh;
    part.n_layers = n_global;
    orc_kv_compact(&part, io->runs, io->n_runs, io->path, io->path_len, io->lens, io->k_cache, io->v_cache,
                   io->page_table, &io->kv);
    part.n_layers = n_local;
    if (n_local)
      orc_kv_compact(&part, io->runs, io->n_runs, io->path, io->path_len, io->lens, io->k_local, io->v_local,
                     io->local_table, &io->kv_local);
  }
  free(h0);
  free(taps);
  free(xattn);
  free(rbase);
  free(iota);
  free(cq);
  free(ck);
  free(cv);
  free(h);
  free(qkv);
  free(attn);
  free(mixed);
  free(act);
  free(inv);
  free(hfin);
  return 0;
}

/* ----------------------------------------------------------------- drafter */

/* kernels.metal:135-148 tap_rows(): out[t] = bf16(rms_norm(in[t])) as float. */
void orc_tap_rows(const float* in, float* out, uint32_t n, uint32_t hidden) {
  for (uint32_t t = 0; t < n; t++) {
    const float* x = in + (size_t)t * hidden;
    double ss = 0.0;
    for (uint32_t i = 0; i < hidden; i++) ss += (double)x[i] * x[i];
    const double inv = 1.0 / sqrt(ss / hidden + (double)SV_RMS_EPS);
    for (uint32_t i = 0; i < hidden; i++) out[(size_t)t * hidden + i] = orc_round_bf16((float)(x[i] * inv));
  }
}

/* kernels.metal:1734-1755 draft_kv(): for the tokens on_path, each drafter layer's k (normed,
 * roped) and v from kvp[t][layer][k | v][NKV][D], bf16 into the ring at the token's position. */
void orc_draft_kv(const sv_shape* sh, const float* kvp, const uint32_t* meta, const uint32_t* on_path,
                  const float* rope, uint16_t* k_ring, uint16_t* v_ring, const uint32_t* table, const sv_kv_args* kv,
                  uint32_t n, uint32_t n_layers) {
  const uint32_t D = sh->head_dim, NKV = sh->n_kv_heads;
  double* tmp = (double*)malloc(sizeof(double) * D);
  for (uint32_t t = 0; t < n; t++) {
    if (!on_path[t]) continue;
    const uint32_t seq = meta[2 * t], pos = meta[2 * t + 1];
    for (uint32_t l = 0; l < n_layers; l++) {
      const float* row = kvp + ((size_t)t * n_layers + l) * 2 * NKV * D;
      for (uint32_t g = 0; g < NKV; g++) {
        norm_rope_d(row + g * D, tmp, D, 1, rope + (size_t)pos * 64);
        const size_t at = kv_row(kv, table, l, seq, g, pos, NKV, D);
        for (uint32_t d = 0; d < D; d++) {
          k_ring[at + d] = orc_to_bf((float)tmp[d]);
          v_ring[at + d] = orc_to_bf(row[(NKV + g) * D + d]);
        }
      }
    }
  }
  free(tmp);
}

/* kernels.metal:1760-1772 draft_ctx(): ring[slot][pos % cr] = ctx[t] ctx_inv[t], tokens on_path. */
void orc_draft_ctx(const float* ctx, const float* ctx_inv, const uint32_t* meta, const uint32_t* on_path, float* ring,
                   uint32_t cr, uint32_t n, uint32_t hidden) {
  for (uint32_t t = 0; t < n; t++) {
    if (!on_path[t]) continue;
    float* dst = ring + ((size_t)meta[2 * t] * cr + meta[2 * t + 1] % cr) * hidden;
    for (uint32_t i = 0; i < hidden; i++) dst[i] = ctx[(size_t)t * hidden + i] * ctx_inv[t];
  }
}

/* kernels.metal:1778-1813 draft_embed(): block row r = (slot, i) at lens[slot] + i; row 0 the
 * rms-normed embedding of feed[slot][0], later rows mask_emb; with cr, the context before the block. */
void orc_draft_embed(const uint16_t* table, const uint32_t* tin, const uint32_t* lens, const uint32_t* feed,
                     const float* mask_emb, float* x, uint32_t* meta, uint32_t* tokens, const float* ring, float* last,
                     uint32_t cr, uint32_t rows, uint32_t hidden) {
  for (uint32_t r = 0; r < rows; r++) {
    const uint32_t slot = tin[2 * r], i = tin[2 * r + 1], tok = feed[slot * SV_FEED_W], len = lens[slot];
    meta[2 * r] = slot;
    meta[2 * r + 1] = len + i;
    tokens[r] = tok;
    if (cr) memcpy(last + (size_t)r * hidden, ring + ((size_t)slot * cr + (len - 1u) % cr) * hidden, sizeof(float) * hidden);
    float* xr = x + (size_t)r * hidden;
    if (i > 0) {
      memcpy(xr, mask_emb, sizeof(float) * hidden);
      continue;
    }
    const uint16_t* e = table + (size_t)tok * hidden;
    double ss = 0.0;
    for (uint32_t j = 0; j < hidden; j++) ss += (double)orc_bf(e[j]) * orc_bf(e[j]);
    const double inv = 1.0 / sqrt(ss / hidden + (double)SV_RMS_EPS);
    for (uint32_t j = 0; j < hidden; j++) xr[j] = (float)(orc_bf(e[j]) * inv);
  }
}

/* kernels.metal:1820-1836 draft_conv(): out = resid + (base[0] + corr[r][d/16]) x[r] +
 * (base[1] + corr[r][H/16 + d/16]) x[r - 1] (not for a block's first row). */
void orc_draft_conv(const float* x, const float* corr, uint32_t corr_w, const float* base, const uint32_t* tin,
                    const float* resid, float* out, uint32_t rows, uint32_t hidden) {
  for (uint32_t r = 0; r < rows; r++) {
    const float* c = corr + (size_t)r * corr_w;
    for (uint32_t d = 0; d < hidden; d++) {
      const size_t at = (size_t)r * hidden + d;
      double y = ((double)base[d] + c[d / 16]) * x[at];
      if (tin[2 * r + 1] > 0) y += ((double)base[hidden + d] + c[hidden / 16 + d / 16]) * x[at - hidden];
      out[at] = (float)(resid ? resid[at] + y : y);
    }
  }
}

static void draft_mm(const sv_matrix* w, uint32_t n, const float* x, float* y, uint32_t epi, uint32_t flags, float ra,
                     const float* base, float* aux) {
  sv_mat_args a;
  memset(&a, 0, sizeof a);
  a.n = n;
  a.k = w->k;
  a.m = w->m;
  a.epi = epi;
  a.flags = flags;
  a.scale = 1.0f;
  a.ra = ra;
  a.rb = 1.0f;
  a.ksplit = 1;
  a.gshift = w->gshift;
  orc_matmul(w, x, NULL, y, base, aux, &a);
}

/* drafter.rs:278-447 encode_drafter(): the step's context (taps -> fc -> kv_all -> the rings,
 * and the context ring with inject), then the blocks through the drafter's layers, the raw
 * head over the normed rows, draft_top and draft_tree into feed/tree. Host pointers. */
int orc_draft(const sv_shape* sh, const uint16_t* embed, const sv_drafter* d, float attn_scale, orc_draft_io* io) {
  const uint32_t n = io->n, H = sh->hidden, D = sh->head_dim, NQ = sh->n_heads, NKV = sh->n_kv_heads;
  const uint32_t W = (NQ + 2 * NKV) * D, F = sh->ffn, R = io->rows ? io->rows : 1;
  const uint32_t KVW = d->n_layers * 2 * NKV * D;
  float* ctx = (float*)calloc((size_t)(n ? n : 1) * H, sizeof(float));
  float* tmp = (float*)malloc(sizeof(float) * (n ? n : 1) * H);
  float* ctx_inv = (float*)malloc(sizeof(float) * (n ? n : 1));
  float* kvp = (float*)malloc(sizeof(float) * (n ? n : 1) * KVW);
  float* x = (float*)malloc(sizeof(float) * R * H);
  float* last = (float*)malloc(sizeof(float) * R * H);
  float* cx = (float*)malloc(sizeof(float) * R * H);
  float* co = (float*)malloc(sizeof(float) * R * H);
  float* mixed = (float*)malloc(sizeof(float) * R * H);
  float* qkv = (float*)malloc(sizeof(float) * R * W);
  float* inv = (float*)malloc(sizeof(float) * R);
  float* attn = (float*)malloc(sizeof(float) * R * NQ * D);
  float* act = (float*)malloc(sizeof(float) * R * F);
  uint32_t cw = 1;
  for (uint32_t li = 0; li < d->n_layers; li++)
    for (int c = 0; c < 4; c++) cw = d->layers[li].conv_corr[c].m > cw ? d->layers[li].conv_corr[c].m : cw;
  float* corr = (float*)malloc(sizeof(float) * R * cw);
  float* corr_inv = (float*)malloc(sizeof(float) * R);
  float* hfin = (float*)malloc(sizeof(float) * R * H);
  uint32_t* meta = (uint32_t*)malloc(sizeof(uint32_t) * 2 * R);
  uint32_t* tokens = (uint32_t*)malloc(sizeof(uint32_t) * R);
  uint32_t* iota = (uint32_t*)malloc(sizeof(uint32_t) * R);
  uint32_t* cand = (uint32_t*)malloc(sizeof(uint32_t) * R * SV_DRAFT_CANDS);
  float* cand_q = (float*)malloc(sizeof(float) * R * SV_DRAFT_CANDS);
  if (!ctx || !tmp || !ctx_inv || !kvp || !x || !last || !cx || !co || !mixed || !qkv || !inv || !attn || !act ||
      !corr || !corr_inv || !hfin || !meta || !tokens || !iota || !cand || !cand_q)
    return -1;
  /* 1. context */
  for (uint32_t k = 0; k < d->n_taps; k++) {
    draft_mm(&d->fc[k], n, io->taps[k], tmp, SV_EPI_RAW, 0, 0.0f, NULL, NULL);
    for (size_t i = 0; i < (size_t)n * H; i++) ctx[i] += tmp[i];
  }
  if (io->ctx) memcpy(io->ctx, ctx, sizeof(float) * n * H);
  draft_mm(&d->kv_all, n, ctx, kvp, SV_EPI_NORM, SV_FLAG_WRITE_INV, 0.0f, NULL, ctx_inv);
  sv_kv_args kv = io->kv;
  orc_draft_kv(sh, kvp, io->meta, io->on_path, io->rope, io->k_ring, io->v_ring, io->table, &kv, n, d->n_layers);
  const uint32_t cr = d->inject.d_w ? io->cr : 0u;
  if (cr) orc_draft_ctx(ctx, ctx_inv, io->meta, io->on_path, io->ctx_ring, cr, n, H);
  const uint32_t rows = io->rows;
  if (rows) {
    /* 2. block rows */
    orc_draft_embed(embed, io->tin, io->lens, io->feed, d->mask_emb, x, meta, tokens, io->ctx_ring, last, cr, rows, H);
    if (cr) draft_mm(&d->inject, rows, last, x, SV_EPI_RESID, 0, 1.0f, x, NULL);
    sv_attn_args aa;
    memset(&aa, 0, sizeof aa);
    aa.scale_log2 = attn_scale * LOG2E_F;
    aa.rope = 1;
    for (uint32_t li = 0; li < d->n_layers; li++) {
      const sv_draft_layer* L = &d->layers[li];
      const int convs = L->conv_base[0] != NULL;
#define CONV(c, in, res, out)                                                                               \
  do {                                                                                                      \
    draft_mm(&L->conv_corr[c], rows, in, corr, SV_EPI_NORM, SV_FLAG_WRITE_INV, 0.0f, NULL, corr_inv);      \
    orc_draft_conv(in, corr, L->conv_corr[c].m, L->conv_base[c], io->tin, res, out, rows, H);              \
  } while (0)
      const float* xin = x;
      if (convs) {
        CONV(0, x, NULL, cx);
        xin = cx;
      }
      draft_mm(&L->qkv, rows, xin, qkv, SV_EPI_NORM, SV_FLAG_WRITE_INV, 0.0f, NULL, inv);
      kv.kv_layer = li;
      orc_attn_verify(sh, qkv, meta, io->k_ring, io->v_ring, io->table, io->rope, &kv, &aa, io->blocks, io->n_blocks,
                      io->vis, attn, NULL);
      if (convs) {
        draft_mm(&L->o, rows, attn, co, SV_EPI_RAW, 0, 0.0f, NULL, NULL);
        CONV(1, co, x, mixed);
        CONV(2, mixed, NULL, cx);
        draft_mm(&L->gate_up, rows, cx, act, SV_EPI_SWIGLU, 0, 0.0f, NULL, NULL);
        draft_mm(&L->down, rows, act, co, SV_EPI_RAW, 0, 0.0f, NULL, NULL);
        CONV(3, co, mixed, x);
      } else {
        draft_mm(&L->o, rows, attn, mixed, SV_EPI_RESID, 0, 1.0f, x, NULL);
        draft_mm(&L->gate_up, rows, mixed, act, SV_EPI_SWIGLU, 0, 0.0f, NULL, NULL);
        draft_mm(&L->down, rows, act, x, SV_EPI_RESID, 0, 1.0f, mixed, NULL);
      }
#undef CONV
    }
    /* 3. tree */
    for (uint32_t r = 0; r < rows; r++) iota[r] = r;
    orc_rmsnorm_rows(x, iota, hfin, rows, H);
    draft_mm(&d->head, rows, hfin, io->logits, SV_EPI_RAW, 0, 0.0f, NULL, NULL);
    uint32_t max_run = 1;
    for (uint32_t b = 0; b < io->n_blocks; b++) max_run = io->blocks[2 * b + 1] > max_run ? io->blocks[2 * b + 1] : max_run;
    const uint32_t ncand = max_run - 1 < SV_DRAFT_CANDS ? max_run - 1 : SV_DRAFT_CANDS;
    if (ncand) {
      orc_draft_top(io->logits, d->vocab, io->tin, cand, cand_q, rows, d->v, d->inv_temperature, ncand);
      orc_draft_tree(io->blocks, io->n_blocks, io->tin, cand, cand_q, io->feed, io->tree, ncand);
    }
  }
  free(ctx); free(tmp); free(ctx_inv); free(kvp); free(x); free(last); free(cx); free(co); free(mixed); free(qkv);
  free(inv); free(attn); free(act); free(corr); free(corr_inv); free(hfin); free(meta); free(tokens); free(iota);
  free(cand); free(cand_q);
  return 0;
}

/* ------------------------------------------------- vectorised test helpers */

void orc_to_bf_array(const float* x, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_to_bf(x[i]);
}

void orc_exp2_array(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_exp2(x[i]);
}
