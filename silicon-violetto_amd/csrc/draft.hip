// draft.hip — the drafter's own kernels (engine/src/kernels.metal:135-148 tap_rows, 1725-1844
// draft_kv, draft_ctx, draft_embed, draft_conv; driven by engine/src/engine/drafter.rs). The
// drafter's matmuls, attention, head and tree run on the verify path's kernels; these move rows
// between them. Every kernel is a few loads and stores per row: latency, not bandwidth.
#include "sv_device.h"
#include "sv_internal.h"

namespace sv {

// Sum over a workgroup of 256 threads (4 waves), in a fixed order.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) red[wv] = v;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

// out[t] = bf16(rms_norm(in[t])), kept as float (a target layer's output, for the drafter).
__global__ __launch_bounds__(256) void tap_rows_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                       uint32_t H) {
  __shared__ float red[4];
  const uint32_t t = blockIdx.x;
  const float* x = in + (size_t)t * H;
  float ss = 0.0f;
  for (uint32_t i = threadIdx.x; i < H; i += 256) ss = __builtin_fmaf(x[i], x[i], ss);
  const float inv = 1.0f / __builtin_sqrtf(block_sum256(ss, red) / (float)H + SV_RMS_EPS);
  for (uint32_t i = threadIdx.x; i < H; i += 256) out[(size_t)t * H + i] = bf(to_bf(x[i] * inv));
}

struct DraftKvParams {
  const float* kvp;
  const uint32_t* meta;
  const uint32_t* on_path;
  const float* rope;
  uint16_t* kc;
  uint16_t* vc;
  const uint32_t* table;
  uint32_t NKV, D, page_shift, n_pages, max_pages, max_seqs;
};

// Token t's keys and values of drafter layer l (grid (tokens, layers)): D / 4 threads per kv
// head, four dims each (the rope pairs (2j, 2j + 1) within a thread); the head's sum of squares
// by lane exchange among its threads.
__global__ __launch_bounds__(256) void draft_kv_kernel(DraftKvParams p) {
  const uint32_t t = blockIdx.x, l = blockIdx.y, L = gridDim.y;
  if (!p.on_path[t]) return;
  const uint32_t per = p.D / 4, g = threadIdx.x / per, d0 = 4 * (threadIdx.x % per);
  if (g >= p.NKV) return;
  const uint32_t seq = p.meta[2 * t], pos = p.meta[2 * t + 1];
  const float* row = p.kvp + ((size_t)t * L + l) * (2 * p.NKV * p.D);
  const f32x4 k = *(const f32x4*)(row + g * p.D + d0);
  const f32x4 v = *(const f32x4*)(row + (p.NKV + g) * p.D + d0);
  float ss = ((k[0] * k[0] + k[1] * k[1]) + k[2] * k[2]) + k[3] * k[3];
  for (uint32_t m = 1; m < per; m <<= 1) ss += __shfl_xor(ss, m, WAVE);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)p.D + SV_RMS_EPS);
  float kk[4] = {k[0] * inv, k[1] * inv, k[2] * inv, k[3] * inv};
  if (d0 < 64) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const float2 cs = *(const float2*)(p.rope + ((size_t)pos * SV_ROPE_PAIRS + d0 / 2 + j) * 2);
      const float a0 = kk[2 * j], a1 = kk[2 * j + 1];
      kk[2 * j] = cs.x * a0 + cs.y * a1;
      kk[2 * j + 1] = cs.x * a1 - cs.y * a0;
    }
  }
  const uint32_t pi = min(pos >> p.page_shift, p.max_pages - 1);
  const uint32_t page = min(p.table[(size_t)seq * p.max_pages + pi], p.n_pages - 1);
  const size_t off = ((((size_t)l * p.n_pages + page) * p.NKV + g) << p.page_shift) * p.D +
                     (size_t)(pos & ((1u << p.page_shift) - 1u)) * p.D + d0;
  *(u32x2*)(p.kc + off) = u32x2{pack_bf2(kk[0], kk[1]), pack_bf2(kk[2], kk[3])};
  *(u32x2*)(p.vc + off) = u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
}

__global__ __launch_bounds__(256) void draft_ctx_kernel(const float* __restrict__ ctx, const float* __restrict__ ctx_inv,
                                                        const uint32_t* __restrict__ meta,
                                                        const uint32_t* __restrict__ on_path, float* __restrict__ ring,
                                                        uint32_t cr, uint32_t H) {
  const uint32_t t = blockIdx.x;
  if (!on_path[t]) return;
  const uint32_t seq = meta[2 * t], pos = meta[2 * t + 1];
  float* dst = ring + ((size_t)seq * cr + pos % cr) * H;
  const float inv = ctx_inv[t];
  for (uint32_t i = threadIdx.x; i < H; i += 256) dst[i] = ctx[(size_t)t * H + i] * inv;
}

__global__ __launch_bounds__(256) void draft_embed_kernel(const uint16_t* __restrict__ table,
                                                          const uint32_t* __restrict__ tin,
                                                          const uint32_t* __restrict__ lens,
                                                          const uint32_t* __restrict__ feed,
                                                          const float* __restrict__ mask_emb, float* __restrict__ x,
                                                          uint32_t* __restrict__ meta, uint32_t* __restrict__ tokens,
                                                          const float* __restrict__ ring, float* __restrict__ last,
                                                          uint32_t cr, uint32_t H) {
  __shared__ float red[4];
  const uint32_t r = blockIdx.x, slot = tin[2 * r], i = tin[2 * r + 1];
  const uint32_t tok = feed[slot * SV_FEED_W], len = lens[slot];
  if (threadIdx.x == 0) {
    meta[2 * r] = slot;
    meta[2 * r + 1] = len + i;
    tokens[r] = tok;
  }
  if (cr > 0) {
    const float* src = ring + ((size_t)slot * cr + (len - 1u) % cr) * H;
    for (uint32_t j = threadIdx.x; j < H; j += 256) last[(size_t)r * H + j] = src[j];
  }
  if (i > 0) {
    for (uint32_t j = threadIdx.x; j < H; j += 256) x[(size_t)r * H + j] = mask_emb[j];
    return;
  }
  const uint16_t* row = table + (size_t)tok * H;
  float ss = 0.0f;
  for (uint32_t j = threadIdx.x; j < H; j += 256) {
    const float v = bf(row[j]);
    ss = __builtin_fmaf(v, v, ss);
  }
  const float inv = 1.0f / __builtin_sqrtf(block_sum256(ss, red) / (float)H + SV_RMS_EPS);
  for (uint32_t j = threadIdx.x; j < H; j += 256) x[(size_t)r * H + j] = bf(row[j]) * inv;
}

__global__ __launch_bounds__(256) void draft_conv_kernel(const float* __restrict__ x, const float* __restrict__ corr,
                                                         uint32_t corr_w, const float* __restrict__ base,
                                                         const uint32_t* __restrict__ tin,
                                                         const float* __restrict__ resid, float* __restrict__ out,
                                                         uint32_t H) {
  const uint32_t r = blockIdx.x;
  const bool prev = tin[2 * r + 1] > 0;
  const float* c = corr + (size_t)r * corr_w;
  for (uint32_t d = threadIdx.x; d < H; d += 256) {
    const size_t at = (size_t)r * H + d;
    float y = (base[d] + c[d / 16]) * x[at];
    if (prev) y = __builtin_fmaf(base[H + d] + c[H / 16 + d / 16], x[at - H], y);
    out[at] = resid ? resid[at] + y : y;
  }
}

// w[r][c] = q[r][c] s[r][c >> gshift] exactly as hi + lo, two bf16 matrices: q (8 bits) times a
// bf16 scale (8 significant bits) has at most 16 significant bits, so hi = bf16(w) and lo =
// bf16(w - hi) (w - hi is exact in fp32 and fits 8 bits) sum back to w.
__global__ __launch_bounds__(256) void split_i8_kernel(const int8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                       uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                       uint32_t k, uint32_t gshift, size_t total) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const size_t r = i / k, c = i % k;
  const float w = (float)q[i] * bf(s[r * (k >> gshift) + (c >> gshift)]);
  const uint16_t h = (uint16_t)to_bf(w);
  hi[i] = h;
  lo[i] = (uint16_t)to_bf(w - bf(h));
}

sv_status split_i8_launch(hipStream_t stream, const sv_matrix* w, uint16_t* hi, uint16_t* lo) {
  if (!w || !w->d_w || !w->d_scales || !hi || !lo) return fail(SV_ERR_ARG, "split_i8: null pointer");
  if (w->gshift >= 32 || w->k % (1u << w->gshift)) return fail(SV_ERR_ARG, "split_i8: groups of 2^%u over k %u", w->gshift, w->k);
  const size_t total = (size_t)w->m * w->k;
  if (total == 0) return SV_OK;
  launch(split_i8_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, stream, (const int8_t*)w->d_w,
         w->d_scales, hi, lo, w->k, w->gshift, total);
  return check_launch("split_i8");
}

sv_status tap_rows_launch(hipStream_t stream, const float* in, float* out, uint32_t n, uint32_t hidden) {
  if (!in || !out || hidden == 0) return fail(SV_ERR_ARG, "tap_rows: null pointer or hidden 0");
  if (n == 0) return SV_OK;
  launch(tap_rows_kernel, dim3(n), dim3(256), 0, stream, in, out, hidden);
  return check_launch("tap_rows");
}

sv_status draft_kv_launch(hipStream_t stream, const sv_shape* sh, const float* kvp, const uint32_t* meta,
                          const uint32_t* on_path, const float* rope, uint16_t* kc, uint16_t* vc, const uint32_t* table,
                          const sv_kv_args* kv, uint32_t n, uint32_t n_layers) {
  if (!sh || !kvp || !meta || !on_path || !rope || !kc || !vc || !table || !kv) return fail(SV_ERR_ARG, "draft_kv: null pointer");
  // a head's D / 4 lanes sum its squares with xor shuffles (a power of two dividing 64) and
  // rope pairs (j, j + D / 2) from the 32-pair table: head_dim 64 or 128 only
  if ((sh->head_dim != 64 && sh->head_dim != 128) || sh->n_kv_heads * sh->head_dim / 4 > 256)
    return fail(SV_ERR_UNSUPPORTED, "draft_kv: %u kv heads x %u dims", sh->n_kv_heads, sh->head_dim);
  if (kv->page_shift < 4 || kv->page_shift > 16 || kv->n_pages == 0 || kv->max_pages == 0)
    return fail(SV_ERR_ARG, "draft_kv: pages of 2^%u, %u pages, %u per sequence", kv->page_shift, kv->n_pages, kv->max_pages);
  if (n == 0 || n_layers == 0) return SV_OK;
  DraftKvParams p{kvp, meta, on_path, rope, kc, vc, table, sh->n_kv_heads, sh->head_dim, kv->page_shift, kv->n_pages,
                  kv->max_pages, kv->max_seqs};
  launch(draft_kv_kernel, dim3(n, n_layers), dim3(256), 0, stream, p);
  return check_launch("draft_kv");
}

sv_status draft_ctx_launch(hipStream_t stream, const float* ctx, const float* ctx_inv, const uint32_t* meta,
                           const uint32_t* on_path, float* ring, uint32_t cr, uint32_t n, uint32_t hidden) {
  if (!ctx || !ctx_inv || !meta || !on_path || !ring || cr == 0 || hidden == 0)
    return fail(SV_ERR_ARG, "draft_ctx: null pointer or zero size");
  if (n == 0) return SV_OK;
  launch(draft_ctx_kernel, dim3(n), dim3(256), 0, stream, ctx, ctx_inv, meta, on_path, ring, cr, hidden);
  return check_launch("draft_ctx");
}

sv_status draft_embed_launch(hipStream_t stream, const uint16_t* embed, const uint32_t* tin, const uint32_t* lens,
                             const uint32_t* feed, const float* mask_emb, float* x, uint32_t* meta, uint32_t* tokens,
                             const float* ring, float* last, uint32_t cr, uint32_t rows, uint32_t hidden) {
  if (!embed || !tin || !lens || !feed || !mask_emb || !x || !meta || !tokens || (cr && (!ring || !last)) || hidden == 0)
    return fail(SV_ERR_ARG, "draft_embed: null pointer");
  if (rows == 0) return SV_OK;
  launch(draft_embed_kernel, dim3(rows), dim3(256), 0, stream, embed, tin, lens, feed, mask_emb, x, meta, tokens, ring,
         last, cr, hidden);
  return check_launch("draft_embed");
}

sv_status draft_conv_launch(hipStream_t stream, const float* x, const float* corr, uint32_t corr_w, const float* base,
                            const uint32_t* tin, const float* resid, float* out, uint32_t rows, uint32_t hidden) {
  if (!x || !corr || !base || !tin || !out) return fail(SV_ERR_ARG, "draft_conv: null pointer");
  if (out == x) return fail(SV_ERR_ARG, "draft_conv: out must not be x");
  if (hidden % 16 || corr_w < hidden / 8) return fail(SV_ERR_ARG, "draft_conv: corrections [%u] for hidden %u", corr_w, hidden);
  if (rows == 0) return SV_OK;
  launch(draft_conv_kernel, dim3(rows), dim3(256), 0, stream, x, corr, corr_w, base, tin, resid, out, hidden);
  return check_launch("draft_conv");
}

}  // namespace sv
