// tail.hip — the small kernels around the matmuls and attention: embed, rmsnorm_rows, the
// sampler, accept, kv_compact and the replay drafter (engine/src/kernels.metal:82-131,
// 1409-1724). The sampler's and accept's results are bit-exact with the oracle: this file is
// compiled with -ffp-contract=off, and the sampler sums in the reference's fixed order.
#include "sv_device.h"
#include "sv_internal.h"

#pragma clang fp contract(off)

namespace sv {

// Sum over a 256-thread workgroup, in a fixed order (waves 0..3).
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int wv = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wv] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

// embed (kernels.metal:82-114): one workgroup of 256 per token.
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* table, const uint32_t* tokens,
                                                    uint32_t* tokens_out, float* out,
                                                    const uint32_t* tin, uint32_t* meta, const uint32_t* lens,
                                                    const uint32_t* feed, const uint32_t* tree, uint32_t* vis,
                                                    uint32_t H, uint32_t vocab, const float* rope, float* rope_rows,
                                                    uint32_t rope_n, uint32_t* epoch) {
  __shared__ float red[4];
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  const uint32_t slot = tin[2 * t];
  uint32_t tok = tokens[t], depth = tin[2 * t + 1];
  if (epoch && t == 0 && tid == 0) *epoch += 1;
  if (tok >= SV_FEED_ROW) {
    const uint32_t i = tok - SV_FEED_ROW, node = tree[slot * SV_FEED_W + i];
    tok = feed[slot * SV_FEED_W + i];
    depth = node & 0xffu;
    if (tid == 0) vis[t] = node >> 16;
  }
  // An id past the table (only a corrupted feed can make one) reads row vocab - 1.
  const uint16_t* row = table + (size_t)min(tok, vocab - 1) * H;
  float ss = 0.0f;
  for (uint32_t i = tid; i < H; i += 256) {
    const float v = bf(row[i]);
    ss = __builtin_fmaf(v, v, ss);
  }
  const float inv = 1.0f / __builtin_sqrtf(block_sum256(ss, red) / (float)H + SV_RMS_EPS);
  if (tid == 0) {  // after block_sum256's barriers: every thread has read tokens[t]
    tokens_out[t] = tok;
    meta[2 * t] = slot;
    meta[2 * t + 1] = lens[slot] + depth;
  }
  // the rope table's row at this token's position, for the layers' attention (by token)
  if (rope_rows && tid < 2 * SV_ROPE_PAIRS)
    rope_rows[(size_t)t * 2 * SV_ROPE_PAIRS + tid] = rope[(size_t)min(lens[slot] + depth, rope_n - 1) * 2 * SV_ROPE_PAIRS + tid];
  for (uint32_t i = tid; i < H; i += 256) out[(size_t)t * H + i] = bf(row[i]) * inv;
}

// rmsnorm_rows (kernels.metal:117-131).
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* in, const uint32_t* rows, float* out,
                                                           uint32_t H) {
  __shared__ float red[4];
  const uint32_t r = blockIdx.x, tid = threadIdx.x;
  const float* x = in + (size_t)rows[r] * H;
  float ss = 0.0f;
  for (uint32_t i = tid; i < H; i += 256) ss = __builtin_fmaf(x[i], x[i], ss);
  const float inv = 1.0f / __builtin_sqrtf(block_sum256(ss, red) / (float)H + SV_RMS_EPS);
  for (uint32_t i = tid; i < H; i += 256) out[(size_t)r * H + i] = x[i] * inv;
}

// ------------------------------------------------------------------ sampler

// kernels.metal:1418-1420: the larger value, ties to the lower id.
__device__ __forceinline__ void better(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// kernels.metal:1484-1501 tg_scan: ex[t] = the sum of v over threads before t, in 32 serial
// runs of 32 then their bases in order; ex[1024] = the total.
__device__ __forceinline__ void scan1024(float v, float* ex, float* base, uint32_t tid) {
  ex[tid] = v;
  __syncthreads();
  if (tid < 32) {
    float acc = 0.0f;
    for (uint32_t i = 32 * tid; i < 32 * tid + 32; i++) {
      const float x = ex[i];
      ex[i] = acc;
      acc += x;
    }
    base[tid] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    float acc = 0.0f;
    for (uint32_t g = 0; g < 32; g++) {
      const float x = base[g];
      base[g] = acc;
      acc += x;
    }
    ex[SV_SAMPLE_THREADS] = acc;
  }
  __syncthreads();
  ex[tid] += base[tid / 32];
  __syncthreads();
}

// sample (kernels.metal:1503-1576), with argmax_partial (:1430-1451) folded in: one
// workgroup of 1024 per row. Thread t owns ids t, t + 1024, ...: the order of every sum.
__global__ __launch_bounds__(1024) void sample_kernel(const float* logits, const sv_sample_row* rows, uint32_t* out,
                                                      const uint32_t* meta, uint32_t vocab) {
  __shared__ float ex[SV_SAMPLE_THREADS + 1];
  __shared__ float base[32];
  __shared__ float bvs[16];
  __shared__ uint32_t bis[16];
  __shared__ uint32_t pick;
  const uint32_t r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const sv_sample_row row = rows[r];
  const uint32_t pos = row.tok == SV_NO_TOK ? row.pos : meta[2 * row.tok + 1] + 1;
  const float* x = logits + (size_t)r * vocab;

  // The first SAMPLE_CACHED logits of this thread (ids tid, tid + 1024, ...) are requested
  // together and kept in registers (one memory round trip, and the temperature pass below
  // reuses them); ids past that are read in the loop.
  constexpr int SAMPLE_CACHED = 32;
  float xc[SAMPLE_CACHED];
#pragma unroll
  for (int j = 0; j < SAMPLE_CACHED; j++) {
    const uint32_t i = tid + j * SV_SAMPLE_THREADS;
    xc[j] = i < vocab ? x[i] : 0.0f;
  }
  float lmax = -3.402823466e+38f;
  uint32_t tok = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < SAMPLE_CACHED; j++) {
    const uint32_t i = tid + j * SV_SAMPLE_THREADS;
    if (i < vocab) better(lmax, tok, xc[j], i);
  }
  for (uint32_t i = tid + SAMPLE_CACHED * SV_SAMPLE_THREADS; i < vocab; i += SV_SAMPLE_THREADS) better(lmax, tok, x[i], i);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(lmax, o, WAVE);
    const uint32_t i = __shfl_xor(tok, o, WAVE);
    better(lmax, tok, v, i);
  }
  if (lane == 0) {
    bvs[wv] = lmax;
    bis[wv] = tok;
  }
  __syncthreads();
  lmax = bvs[0];
  tok = bis[0];
  for (int w = 1; w < 16; w++) better(lmax, tok, bvs[w], bis[w]);

  if (row.temperature > 0.0f) {
    const float c = LOG2E_F / row.temperature;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < SAMPLE_CACHED; j++) {
      const uint32_t i = tid + j * SV_SAMPLE_THREADS;
      if (i < vocab) s += sv_exp2((xc[j] - lmax) * c);
    }
    for (uint32_t i = tid + SAMPLE_CACHED * SV_SAMPLE_THREADS; i < vocab; i += SV_SAMPLE_THREADS)
      s += sv_exp2((x[i] - lmax) * c);
    scan1024(s, ex, base, tid);
    const float z = ex[SV_SAMPLE_THREADS];
    float low = -__builtin_inff();
    for (uint32_t round = 0; round < SV_SAMPLE_ROUNDS; round++) {
      const u32x4 ph = philox(u32x4{pos, round, 0u, 0u}, row.seed_lo, row.seed_hi);
      const float target = (float)(ph[0] >> 8) * 0x1p-24f * ex[SV_SAMPLE_THREADS];
      if (tid == 0) pick = 0xffffffffu;
      __syncthreads();
      const float lo = ex[tid];
      if (lo <= target && target < ex[tid + 1]) {
        // Walk this thread's ids again, summing exactly as the scan did, until the sum
        // passes the target's offset into this thread's share. If fp32 rounding leaves the
        // offset beyond the re-sum, the thread's last nonzero term is the pick.
        float acc = 0.0f;
        uint32_t j = 0xffffffffu;
        for (uint32_t i = tid; i < vocab; i += SV_SAMPLE_THREADS) {
          const float xi = x[i];
          if (!(xi > low)) continue;
          const float e = sv_exp2((xi - lmax) * c);
          acc += e;
          if (e > 0.0f) j = i;
          if (target - lo < acc) break;
        }
        pick = j;
      }
      __syncthreads();
      const uint32_t j = pick;
      if (j == 0xffffffffu) break;
      const float xj = x[j];
      if (xj == lmax || row.top_p >= 1.0f) {
        tok = j;
        break;
      }
      float qs = 0.0f;
      for (uint32_t i = tid; i < vocab; i += SV_SAMPLE_THREADS) {
        const float xi = x[i];
        if (xi > xj) qs += sv_exp2((xi - lmax) * c);
      }
      scan1024(qs, ex, base, tid);
      if (ex[SV_SAMPLE_THREADS] < row.top_p * z) {
        tok = j;
        break;
      }
      low = xj;
    }
  }
  if (tid == 0) out[r] = tok;
}

// ---------------------------------------------------------------- accepting

// accept (kernels.metal:1605-1657): one thread per run. A run that emits nothing (only with
// remaining = 0 on a slot not marked done) leaves feed alone.
__global__ __launch_bounds__(64) void accept_kernel(const sv_run_in* runs, const uint32_t* tokens, uint32_t* out,
                                                    uint32_t* lens, uint32_t* feed, sv_gen_state* gen,
                                                    uint32_t* emitted, uint32_t nruns, const uint32_t* tree,
                                                    uint32_t* path, uint32_t* path_len, uint32_t* on_path) {
  const uint32_t r = blockIdx.x * 64 + threadIdx.x;
  if (r >= nruns) return;
  const sv_run_in ru = runs[r];
  sv_gen_state* gs = &gen[ru.slot];
  path_len[r] = 0;
  const uint32_t done = gs->done;
  for (uint32_t j = 0; j < ru.count; j++) on_path[ru.first + j] = !ru.verify && !done;
  if (done) {
    emitted[r] = 0;
    return;
  }
  if (!ru.verify) lens[ru.slot] += ru.count;
  if (ru.nhead == 0) {
    emitted[r] = 0;
    return;
  }
  uint32_t first = ru.head0 + ru.nhead - 1, e = 1;
  uint32_t walk[SV_FEED_W];
  walk[0] = 0;
  if (ru.verify) {
    const uint32_t* node = tree + (size_t)ru.slot * SV_FEED_W;
    for (uint32_t c = 1, at = 0; c < ru.count; c++) {
      if (((node[c] >> 8) & 0xffu) == at && tokens[ru.first + c] == out[ru.head0 + at]) walk[e++] = at = c;
    }
    for (uint32_t j = 1; j < e; j++) out[ru.head0 + j] = out[ru.head0 + walk[j]];
    first = ru.head0;
  }
  bool stop = false;
  uint32_t k = 0;
  const uint32_t remaining = gs->remaining, nstop = gs->nstop;
  while (k < e && k < remaining && !stop) {
    const uint32_t t = out[first + k];
    for (uint32_t j = 0; j < nstop && j < SV_MAX_STOP; j++) stop = stop || t == gs->stop[j];
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
  gs->remaining = remaining - k;
  if (stop || remaining - k == 0) gs->done = 1;
  emitted[r] = k;
}

// kv_compact (kernels.metal:1659-1693): grid (runs, layers); thread = (kv head, 4 dims).
// Rows p0 + path[j] -> p0 + j in increasing j: path[j] >= j and increases, so nothing is
// overwritten before it is read.
__global__ __launch_bounds__(256) void kv_compact_kernel(const sv_run_in* runs, const uint32_t* path,
                                                         const uint32_t* path_len, const uint32_t* lens,
                                                         uint16_t* kc, uint16_t* vc, const uint32_t* page_table,
                                                         uint32_t NKV, uint32_t D, uint32_t page_shift,
                                                         uint32_t n_pages, uint32_t max_pages) {
  const uint32_t r = blockIdx.x, l = blockIdx.y, tid = threadIdx.x;
  const uint32_t chunks = D / 4;
  if (tid >= NKV * chunks) return;
  const uint32_t g = tid / chunks, d0 = (tid % chunks) * 4;
  const uint32_t k = path_len[r], slot = runs[r].slot, p0 = lens[slot] - k;
  const uint32_t pmask = (1u << page_shift) - 1u;
  for (uint32_t j = 1; j < k; j++) {
    const uint32_t from = path[r * SV_FEED_W + j];
    if (from == j) continue;
    // (clamped to the pool: a page table entry never reserved cannot send the copy out of it)
    const uint32_t ps = min(page_table[(size_t)slot * max_pages + ((p0 + from) >> page_shift)], n_pages - 1);
    const uint32_t pd = min(page_table[(size_t)slot * max_pages + ((p0 + j) >> page_shift)], n_pages - 1);
    const size_t src = ((((size_t)l * n_pages + ps) * NKV + g) << page_shift) * D + (size_t)((p0 + from) & pmask) * D + d0;
    const size_t dst = ((((size_t)l * n_pages + pd) * NKV + g) << page_shift) * D + (size_t)((p0 + j) & pmask) * D + d0;
    *(u32x2*)(kc + dst) = *(const u32x2*)(kc + src);
    *(u32x2*)(vc + dst) = *(const u32x2*)(vc + src);
  }
}

// replay_draft (kernels.metal:1705-1724): grid runs, FEED_W threads.
__global__ __launch_bounds__(64) void replay_kernel(const sv_run_in* runs, uint32_t nruns, const uint32_t* lens,
                                                    uint32_t* feed, const uint32_t* trace, const uint32_t* trace_len,
                                                    sv_replay_args ra, uint32_t* tree) {
  const uint32_t r = blockIdx.x, i = threadIdx.x;
  if (i == 0 || i >= SV_FEED_W || r >= nruns || runs[r].nhead == 0) return;
  const uint32_t slot = runs[r].slot, n = trace_len[slot];
  if (n == 0) return;
  const uint32_t pos = lens[slot] + i;
  uint32_t tok = pos < n ? trace[(size_t)slot * ra.stride + pos] : 0u;
  const u32x4 h = philox(u32x4{pos, 0x5eedu, 0u, 0u}, ra.seed, 0x0dd5u);
  if ((float)(h[0] >> 8) * 0x1p-24f < ra.rate) tok = (tok + 1) % ra.vocab;
  feed[slot * SV_FEED_W + i] = tok;
  tree[slot * SV_FEED_W + i] = i | (i - 1) << 8 | ((2u << i) - 1u) << 16;
}

// accept (kernels.metal:1605-1657), then kv_compact (:1659-1693) and the replay drafter
// (:1705-1724) of the same run, in one workgroup per run: the engine's step tail as one
// launch. Thread 0 walks the tree exactly as accept_kernel; the path goes through LDS to
// the threads that move its K/V rows (all layers; element order per thread as kv_compact)
// and then write the next drafts.
struct TailParams {
  const sv_run_in* runs;
  const uint32_t* tokens;
  uint32_t* out;
  uint32_t* lens;
  uint32_t* feed;
  sv_gen_state* gen;
  uint32_t* emitted;
  const uint32_t* trace;
  const uint32_t* trace_len;
  uint32_t* tree;
  uint32_t* path;
  uint32_t* path_len;
  uint32_t* on_path;
  KvCacheRef cache[2];  // global (paged) layers, then sliding-window layers (cyclic table)
  uint32_t nruns, compact, replay;
  uint32_t NKV, D, page_shift, max_pages;
  sv_replay_args ra;
};

__global__ __launch_bounds__(256) void step_tail_kernel(TailParams p) {
  __shared__ uint32_t s_path[SV_FEED_W];
  __shared__ uint32_t s_k, s_len;
  const uint32_t r = blockIdx.x, tid = threadIdx.x;
  const sv_run_in ru = p.runs[r];
  if (tid == 0) {
    sv_gen_state* gs = &p.gen[ru.slot];
    p.path_len[r] = 0;
    const uint32_t done = gs->done;
    uint32_t k = 0;
    for (uint32_t j = 0; j < ru.count; j++) p.on_path[ru.first + j] = !ru.verify && !done;
    if (done) {
      p.emitted[r] = 0;
    } else {
      if (!ru.verify) p.lens[ru.slot] += ru.count;
      if (ru.nhead == 0) {
        p.emitted[r] = 0;
      } else {
        uint32_t first = ru.head0 + ru.nhead - 1, e = 1;
        uint32_t walk[SV_FEED_W];
        walk[0] = 0;
        if (ru.verify) {
          const uint32_t* node = p.tree + (size_t)ru.slot * SV_FEED_W;
          for (uint32_t c = 1, at = 0; c < ru.count; c++) {
            if (((node[c] >> 8) & 0xffu) == at && p.tokens[ru.first + c] == p.out[ru.head0 + at]) walk[e++] = at = c;
          }
          for (uint32_t j = 1; j < e; j++) p.out[ru.head0 + j] = p.out[ru.head0 + walk[j]];
          first = ru.head0;
        }
        bool stop = false;
        const uint32_t remaining = gs->remaining, nstop = gs->nstop;
        while (k < e && k < remaining && !stop) {
          const uint32_t t = p.out[first + k];
          for (uint32_t j = 0; j < nstop && j < SV_MAX_STOP; j++) stop = stop || t == gs->stop[j];
          k++;
        }
        if (ru.verify) {
          p.lens[ru.slot] += k;
          p.path_len[r] = k;
          for (uint32_t j = 0; j < k; j++) {
            p.path[r * SV_FEED_W + j] = walk[j];
            p.on_path[ru.first + walk[j]] = 1;
            s_path[j] = walk[j];
          }
        }
        if (k > 0) p.feed[ru.slot * SV_FEED_W] = p.out[first + k - 1];
        gs->remaining = remaining - k;
        if (stop || remaining - k == 0) gs->done = 1;
        p.emitted[r] = k;
      }
    }
    s_k = ru.verify ? k : 0;
    s_len = p.lens[ru.slot];
  }
  __syncthreads();
  const uint32_t k = s_k, len = s_len, slot = ru.slot;
  if (p.compact && k > 1) {
    const uint32_t chunks = p.D / 4, per_layer = p.NKV * chunks, p0 = len - k;
    const uint32_t pmask = (1u << p.page_shift) - 1u;
    const uint32_t n0 = p.cache[0].n_layers;
    for (uint32_t e = tid; e < (n0 + p.cache[1].n_layers) * per_layer; e += 256) {
      const uint32_t lx = e / per_layer, g = (e % per_layer) / chunks, d0 = (e % chunks) * 4;
      const KvCacheRef& c = lx < n0 ? p.cache[0] : p.cache[1];
      const uint32_t l = lx < n0 ? lx : lx - n0;
      for (uint32_t j = 1; j < k; j++) {
        const uint32_t from = s_path[j];
        if (from == j) continue;
        const uint32_t ps = min(c.table[(size_t)slot * p.max_pages + ((p0 + from) >> p.page_shift)], c.n_pages - 1);
        const uint32_t pd = min(c.table[(size_t)slot * p.max_pages + ((p0 + j) >> p.page_shift)], c.n_pages - 1);
        const size_t src = ((((size_t)l * c.n_pages + ps) * p.NKV + g) << p.page_shift) * p.D +
                           (size_t)((p0 + from) & pmask) * p.D + d0;
        const size_t dst = ((((size_t)l * c.n_pages + pd) * p.NKV + g) << p.page_shift) * p.D +
                           (size_t)((p0 + j) & pmask) * p.D + d0;
        *(u32x2*)(c.kc + dst) = *(const u32x2*)(c.kc + src);
        *(u32x2*)(c.vc + dst) = *(const u32x2*)(c.vc + src);
      }
    }
  }
  if (p.replay && tid > 0 && tid < SV_FEED_W && ru.nhead != 0) {
    const uint32_t n = p.trace_len[slot];
    if (n != 0) {
      const uint32_t i = tid, pos = len + i;
      uint32_t tok = pos < n ? p.trace[(size_t)slot * p.ra.stride + pos] : 0u;
      const u32x4 h = philox(u32x4{pos, 0x5eedu, 0u, 0u}, p.ra.seed, 0x0dd5u);
      if ((float)(h[0] >> 8) * 0x1p-24f < p.ra.rate) tok = (tok + 1) % p.ra.vocab;
      p.feed[slot * SV_FEED_W + i] = tok;
      p.tree[slot * SV_FEED_W + i] = i | (i - 1) << 8 | ((2u << i) - 1u) << 16;
    }
  }
}

// ---------------------------------------------------------------- launchers

sv_status embed_launch(hipStream_t stream, const sv_shape* sh, const uint16_t* table, const uint32_t* tokens,
                       uint32_t* tokens_out, float* out, const uint32_t* tin, uint32_t* meta, const uint32_t* lens,
                       const uint32_t* feed, const uint32_t* tree, uint32_t* vis, uint32_t n, const float* rope,
                       float* rope_rows, uint32_t rope_n, uint32_t* epoch) {
  if (!sh || !table || !tokens || !tokens_out || !out || !tin || !meta || !lens || !feed || !tree || !vis)
    return fail(SV_ERR_ARG, "embed: null pointer");
  if (rope_rows && (!rope || rope_n == 0)) return fail(SV_ERR_ARG, "embed: rope rows without the table");
  if (n == 0) return SV_OK;
  launch(embed_kernel, dim3(n), dim3(256), 0, stream, table, tokens, tokens_out, out, tin, meta, lens, feed,
                     tree, vis, sh->hidden, sh->vocab, rope, rope_rows, rope_n, epoch);
  return check_launch("embed");
}

// The head's softcap (kernels.metal:196-199) over logits a matmul left raw (a head in int8 groups
// under 64 runs as two bf16 products, hi + lo): y = 23 sigmoid((y + 5) / 7.5), -inf at ids >=
// vocab_real; the same expression as the matmul's head epilogue.
__global__ __launch_bounds__(256) void head_cap_kernel(float* logits, uint32_t vocab, uint32_t vocab_real, size_t total) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const uint32_t col = (uint32_t)(i % vocab);
  logits[i] = col < vocab_real ? 23.0f * (1.0f / (1.0f + __expf(-((logits[i] + 5.0f) / 7.5f)))) : -__builtin_inff();
}

sv_status head_cap_launch(hipStream_t stream, float* logits, uint32_t rows, uint32_t vocab, uint32_t vocab_real) {
  if (!logits || vocab == 0 || vocab_real > vocab) return fail(SV_ERR_ARG, "head_cap: arguments");
  const size_t total = (size_t)rows * vocab;
  if (total == 0) return SV_OK;
  launch(head_cap_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, stream, logits, vocab, vocab_real, total);
  return check_launch("head_cap");
}

sv_status rmsnorm_rows_launch(hipStream_t stream, const float* in, const uint32_t* rows, float* out, uint32_t n,
                              uint32_t hidden) {
  if (!in || !rows || !out) return fail(SV_ERR_ARG, "rmsnorm_rows: null pointer");
  if (n == 0) return SV_OK;
  launch(rmsnorm_rows_kernel, dim3(n), dim3(256), 0, stream, in, rows, out, hidden);
  return check_launch("rmsnorm_rows");
}

// ---------------------------------------------------------------- draft builder
// draft_top (kernels.metal:1845-1891): one workgroup of 1024 per drafted block row (the
// block's row 0, the bonus token's, is skipped). The ncand best ids in the order (value
// descending, id ascending) over the ids with a value above -FLT_MAX: every thread keeps its
// own sorted top ncand over ids t, t + 1024, ... in one pass (loads issued eight at a time),
// then ncand rounds of a workgroup argmax over the threads' list heads, the winner popping its
// head (the k-th pick of a strict total order is the same however the ids are dealt out).
// Then the row's sum of exp((x - x_top) inv_t) in the sampler's order (thread t adds ids t,
// t + 1024, ... in turn; 32 runs of 32 threads, then their bases) and each candidate's target
// id and probability.
__global__ __launch_bounds__(1024) void draft_top_kernel(const float* logits, const uint32_t* vocab, const uint32_t* tin,
                                                         uint32_t* cand, float* cand_q, uint32_t nv, float c,
                                                         uint32_t ncand) {
  __shared__ float part[SV_SAMPLE_THREADS];
  __shared__ float bvs[16];
  __shared__ uint32_t bis[16];
  __shared__ float top_v[SV_DRAFT_CANDS];
  __shared__ uint32_t top_i[SV_DRAFT_CANDS];
  __shared__ float total;
  const uint32_t r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tin[2 * r + 1] == 0) return;
  const float* x = logits + (size_t)r * nv;
  float lv[SV_DRAFT_CANDS];
  uint32_t li[SV_DRAFT_CANDS];
#pragma unroll
  for (uint32_t m = 0; m < SV_DRAFT_CANDS; m++) {
    lv[m] = -3.402823466e+38f;
    li[m] = 0xffffffffu;
  }
  // insert (v, j) into the sorted list if it beats the list's last entry
  auto insert = [&](float v, uint32_t j) {
    float cv = lv[SV_DRAFT_CANDS - 1];
    uint32_t ci = li[SV_DRAFT_CANDS - 1];
    better(cv, ci, v, j);
    if (ci != j) return;
#pragma unroll
    for (int m = SV_DRAFT_CANDS - 1; m >= 0; m--) {
      const bool above = m > 0 && (v > lv[m - 1] || (v == lv[m - 1] && j < li[m - 1]));
      if (above) {
        lv[m] = lv[m - 1];
        li[m] = li[m - 1];
      } else {
        lv[m] = v;
        li[m] = j;
        break;
      }
    }
  };
  // a row of up to 16 x 1024 ids is read once, every load in flight, and kept for the sum below
  constexpr int KEEP = 16;
  const bool kept = nv <= KEEP * SV_SAMPLE_THREADS;
  float keep[KEEP];
  uint32_t j = tid;
  if (kept) {
#pragma unroll
    for (int u = 0; u < KEEP; u++) keep[u] = j + u * SV_SAMPLE_THREADS < nv ? x[j + u * SV_SAMPLE_THREADS] : 0.0f;
#pragma unroll
    for (int u = 0; u < KEEP; u++)
      if (j + u * SV_SAMPLE_THREADS < nv) insert(keep[u], j + u * SV_SAMPLE_THREADS);
  } else {
    for (; j + 7 * SV_SAMPLE_THREADS < nv; j += 8 * SV_SAMPLE_THREADS) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = x[j + u * SV_SAMPLE_THREADS];
#pragma unroll
      for (int u = 0; u < 8; u++) insert(v[u], j + u * SV_SAMPLE_THREADS);
    }
    for (; j < nv; j += SV_SAMPLE_THREADS) insert(x[j], j);
  }
  uint32_t head = 0;
  for (uint32_t k = 0; k < ncand; k++) {
    float bv = -3.402823466e+38f;
    uint32_t bi = 0xffffffffu;
#pragma unroll
    for (uint32_t m = 0; m < SV_DRAFT_CANDS; m++)
      if (m == head) {
        bv = lv[m];
        bi = li[m];
      }
    const uint32_t mine = bi;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v = __shfl_xor(bv, o, WAVE);
      const uint32_t i = __shfl_xor(bi, o, WAVE);
      better(bv, bi, v, i);
    }
    if (lane == 0) {
      bvs[wv] = bv;
      bis[wv] = bi;
    }
    __syncthreads();
    bv = bvs[0];
    bi = bis[0];
    for (int w = 1; w < 16; w++) better(bv, bi, bvs[w], bis[w]);
    if (tid == 0) {
      top_v[k] = bv;
      top_i[k] = bi;
    }
    if (bi != 0xffffffffu && bi == mine) head++;  // this thread's head was picked
    __syncthreads();
  }
  const float t0 = top_v[0];
  float sum = 0.0f;
  j = tid;
  if (kept) {
#pragma unroll
    for (int u = 0; u < KEEP; u++)
      if (j + u * SV_SAMPLE_THREADS < nv) sum += sv_exp2((keep[u] - t0) * c);
    j = nv;
  }
  for (; j + 7 * SV_SAMPLE_THREADS < nv; j += 8 * SV_SAMPLE_THREADS) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = x[j + u * SV_SAMPLE_THREADS];
#pragma unroll
    for (int u = 0; u < 8; u++) sum += sv_exp2((v[u] - t0) * c);
  }
  for (; j < nv; j += SV_SAMPLE_THREADS) sum += sv_exp2((x[j] - t0) * c);
  // the sampler's scan order for the total: 32 serial runs of 32 threads, then the runs in order
  part[tid] = sum;
  __syncthreads();
  if (tid < 32) {
    float acc = 0.0f;
    for (uint32_t i = 32 * tid; i < 32 * tid + 32; i++) acc += part[i];
    part[32 * tid] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    float acc = 0.0f;
    for (uint32_t g = 0; g < 32; g++) acc += part[32 * g];
    total = acc;
  }
  __syncthreads();
  if (tid < ncand) {
    const bool ok = top_i[tid] < nv && top_i[0] < nv;  // a row without tid + 1 ordered values
    cand[r * SV_DRAFT_CANDS + tid] = ok ? vocab[top_i[tid]] : SV_NO_TOK;
    cand_q[r * SV_DRAFT_CANDS + tid] = ok ? sv_exp2((top_v[tid] - t0) * c) / total : 0.0f;
  }
}

// draft_tree (kernels.metal:1893-1934): a workgroup per block stages the block's candidates in
// LDS, then one thread builds its DDTree best-first: the next node is the not-yet-taken
// candidate of any node so far with the highest path product (first such node on ties), a node
// at depth d drawing children from block row d + 1's candidates; nodes go to feed/tree[slot][1..]
// parents first, the rest become dead nodes. A candidate draft_top could not fill (SV_NO_TOK) is
// never taken.
__global__ __launch_bounds__(64) void draft_tree_kernel(const uint32_t* blocks, uint32_t nblocks, const uint32_t* tin,
                                                        const uint32_t* cand, const float* cand_q, uint32_t* feed,
                                                        uint32_t* tree, uint32_t ncand) {
  __shared__ uint32_t sc_id[SV_FEED_W * SV_DRAFT_CANDS];
  __shared__ float sc_q[SV_FEED_W * SV_DRAFT_CANDS];
  __shared__ uint32_t out_feed[SV_FEED_W], out_tree[SV_FEED_W];
  const uint32_t b = blockIdx.x, tid = threadIdx.x;
  const uint32_t first = blocks[2 * b], rows = min(blocks[2 * b + 1], SV_FEED_W), slot = tin[2 * first];
  if (tid < rows * SV_DRAFT_CANDS) {
    sc_id[tid] = cand[first * SV_DRAFT_CANDS + tid];
    sc_q[tid] = cand_q[first * SV_DRAFT_CANDS + tid];
  }
  __syncthreads();
  if (tid == 0) {
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
        const uint32_t cc = (depth[i] + 1) * SV_DRAFT_CANDS + taken[i];
        if (depth[i] + 1 == rows || taken[i] == ncand || sc_id[cc] == SV_NO_TOK) continue;
        const float s = score[i] * sc_q[cc];
        if (s > best) {
          best = s;
          p = i;
        }
      }
      if (best < 0.0f) break;
      const uint32_t d = depth[p] + 1;
      out_feed[n] = sc_id[d * SV_DRAFT_CANDS + taken[p]];
      taken[p]++;
      score[n] = best;
      depth[n] = d;
      taken[n] = 0;
      sees[n] = sees[p] | 1u << n;
      out_tree[n] = d | p << 8 | sees[n] << 16;
    }
    for (uint32_t m = n; m < SV_FEED_W; m++) out_tree[m] = 1u | SV_NO_PARENT << 8 | (1u | 1u << m) << 16;
    out_feed[0] = n;  // the count of fed nodes, for the flush below
  }
  __syncthreads();
  const uint32_t n = out_feed[0];
  if (tid >= 1 && tid < SV_FEED_W) {
    if (tid < n) feed[slot * SV_FEED_W + tid] = out_feed[tid];
    tree[slot * SV_FEED_W + tid] = out_tree[tid];
  }
}

sv_status draft_top_launch(hipStream_t stream, const float* logits, const uint32_t* vocab, const uint32_t* tin,
                           uint32_t* cand, float* cand_q, uint32_t n_rows, uint32_t nv, float inv_t, uint32_t ncand) {
  if (!logits || !vocab || !tin || !cand || !cand_q) return fail(SV_ERR_ARG, "draft_top: null pointer");
  if (ncand == 0 || ncand > SV_DRAFT_CANDS) return fail(SV_ERR_ARG, "draft_top: %u candidates (1..%u)", ncand, SV_DRAFT_CANDS);
  if (nv < ncand) return fail(SV_ERR_ARG, "draft_top: %u ids for %u candidates", nv, ncand);
  if (!(inv_t > 0.0f) || !__builtin_isfinite(inv_t)) return fail(SV_ERR_ARG, "draft_top: inverse temperature %g", inv_t);
  if (n_rows == 0) return SV_OK;
  launch(draft_top_kernel, dim3(n_rows), dim3(SV_SAMPLE_THREADS), 0, stream, logits, vocab, tin, cand, cand_q, nv,
         inv_t * LOG2E_F, ncand);
  return check_launch("draft_top");
}

sv_status draft_tree_launch(hipStream_t stream, const uint32_t* blocks, uint32_t nblocks, const uint32_t* tin,
                            const uint32_t* cand, const float* cand_q, uint32_t* feed, uint32_t* tree, uint32_t ncand) {
  if (!blocks || !tin || !cand || !cand_q || !feed || !tree) return fail(SV_ERR_ARG, "draft_tree: null pointer");
  if (ncand == 0 || ncand > SV_DRAFT_CANDS) return fail(SV_ERR_ARG, "draft_tree: %u candidates (1..%u)", ncand, SV_DRAFT_CANDS);
  if (nblocks == 0) return SV_OK;
  launch(draft_tree_kernel, dim3(nblocks), dim3(64), 0, stream, blocks, nblocks, tin, cand, cand_q, feed,
         tree, ncand);
  return check_launch("draft_tree");
}

sv_status sample_launch(hipStream_t stream, const float* logits, const sv_sample_row* rows, uint32_t* out,
                        const uint32_t* meta, uint32_t n_rows, uint32_t vocab) {
  if (!logits || !rows || !out) return fail(SV_ERR_ARG, "sample: null pointer");
  if (n_rows == 0) return SV_OK;
  if (vocab == 0) return fail(SV_ERR_ARG, "sample: empty vocabulary");
  launch(sample_kernel, dim3(n_rows), dim3(SV_SAMPLE_THREADS), 0, stream, logits, rows, out, meta, vocab);
  return check_launch("sample");
}

sv_status accept_launch(hipStream_t stream, const sv_run_in* runs, const uint32_t* tokens, uint32_t* out,
                        uint32_t* lens, uint32_t* feed, sv_gen_state* gen, uint32_t* emitted, uint32_t nruns,
                        const uint32_t* tree, uint32_t* path, uint32_t* path_len, uint32_t* on_path) {
  if (!runs || !tokens || !out || !lens || !feed || !gen || !emitted || !tree || !path || !path_len || !on_path)
    return fail(SV_ERR_ARG, "accept: null pointer");
  if (nruns == 0) return SV_OK;
  launch(accept_kernel, dim3((nruns + 63) / 64), dim3(64), 0, stream, runs, tokens, out, lens, feed, gen,
                     emitted, nruns, tree, path, path_len, on_path);
  return check_launch("accept");
}

sv_status kv_compact_launch(hipStream_t stream, const sv_shape* sh, const sv_run_in* runs, uint32_t nruns,
                            const uint32_t* path, const uint32_t* path_len, const uint32_t* lens, uint16_t* k_cache,
                            uint16_t* v_cache, const uint32_t* page_table, const sv_kv_args* kv) {
  if (!sh || !runs || !path || !path_len || !lens || !k_cache || !v_cache || !page_table || !kv)
    return fail(SV_ERR_ARG, "kv_compact: null pointer");
  if (nruns == 0) return SV_OK;
  if (sh->n_kv_heads * sh->head_dim / 4 > 256 || sh->head_dim % 4)
    return fail(SV_ERR_UNSUPPORTED, "kv_compact: %u kv heads x %u dims", sh->n_kv_heads, sh->head_dim);
  launch(kv_compact_kernel, dim3(nruns, sh->n_layers), dim3(256), 0, stream, runs, path, path_len, lens,
                     k_cache, v_cache, page_table, sh->n_kv_heads, sh->head_dim, kv->page_shift, kv->n_pages,
                     kv->max_pages);
  return check_launch("kv_compact");
}

sv_status replay_launch(hipStream_t stream, const sv_run_in* runs, uint32_t nruns, const uint32_t* lens,
                        uint32_t* feed, const uint32_t* trace, const uint32_t* trace_len, const sv_replay_args* ra,
                        uint32_t* tree) {
  if (!runs || !lens || !feed || !trace || !trace_len || !ra || !tree) return fail(SV_ERR_ARG, "replay: null pointer");
  if (nruns == 0) return SV_OK;
  if (ra->vocab == 0) return fail(SV_ERR_ARG, "replay: vocab 0");
  launch(replay_kernel, dim3(nruns), dim3(64), 0, stream, runs, nruns, lens, feed, trace, trace_len, *ra,
                     tree);
  return check_launch("replay_draft");
}

}  // namespace sv

namespace sv {

sv_status step_tail_launch(hipStream_t stream, const sv_shape* sh, const sv_run_in* runs, uint32_t nruns,
                           const uint32_t* tokens, uint32_t* out, uint32_t* lens, uint32_t* feed, sv_gen_state* gen,
                           uint32_t* emitted, uint32_t* tree, uint32_t* path, uint32_t* path_len, uint32_t* on_path,
                           bool compact, const KvCacheRef* caches, uint32_t n_caches, uint32_t page_shift,
                           uint32_t max_pages, const sv_replay_args* ra, const uint32_t* trace,
                           const uint32_t* trace_len) {
  if (nruns == 0) return SV_OK;
  if (n_caches == 0 || n_caches > 2) return fail(SV_ERR_ARG, "step tail: %u caches", n_caches);
  TailParams p;
  p.runs = runs;
  p.tokens = tokens;
  p.out = out;
  p.lens = lens;
  p.feed = feed;
  p.gen = gen;
  p.emitted = emitted;
  p.trace = trace;
  p.trace_len = trace_len;
  p.tree = tree;
  p.path = path;
  p.path_len = path_len;
  p.on_path = on_path;
  p.cache[0] = caches[0];
  p.cache[1] = n_caches > 1 ? caches[1] : KvCacheRef{nullptr, nullptr, nullptr, 0u, 1u};
  p.nruns = nruns;
  p.compact = compact ? 1u : 0u;
  p.replay = ra ? 1u : 0u;
  p.NKV = sh->n_kv_heads;
  p.D = sh->head_dim;
  p.page_shift = page_shift;
  p.max_pages = max_pages;
  if (ra) {
    if (ra->vocab == 0) return fail(SV_ERR_ARG, "step tail: replay vocab 0");
    p.ra = *ra;
  } else {
    p.ra = sv_replay_args{0, 0, 0.0f, 1};
  }
  if (p.replay && (!trace || !trace_len)) return fail(SV_ERR_ARG, "step tail: replay without a trace");
  launch(step_tail_kernel, dim3(nruns), dim3(256), 0, stream, p);
  return check_launch("step tail");
}

}  // namespace sv
