// matmul.hip — Y = epilogue(W . X) for the verify step's rows (the reference's matmul
// group: engine/src/kernels.metal:151-690, chosen by Matmul::for_tokens, encode.rs:33-44).
//
// Skinny path (n <= 16 rows, the 1-5 row verify step): weight-streaming on the matrix cores.
//   - A workgroup of W = 4 or 8 waves owns RT tiles of 16 output rows over the whole of k;
//     wave w takes the k chunks of 256 numbered w, w + W, ... For each chunk, its X (16
//     tokens x 256 k, fp32) is loaded once, split into bf16 hi + lo (16 significant bits)
//     and held in registers as the MFMA B operands while the chunk's weights stream past:
//     16 rows x 16 bytes per lane per 64-k block, one dwordx4 each (int8) or two (bf16),
//     converted to bf16 in registers (int8 is exact in bf16); the next chunk's weights are
//     in flight during the products.
//   - Products run on v_mfma_f32_16x16x32_bf16 (fp32 accumulate); hi and lo each take one
//     MFMA, so the fp32 activations lose nothing the tolerance can see, and the VALU only
//     converts weights (about 1.5 ops per byte, where an fp32 FMA GEMV at 5 rows needs 6).
//   - The waves' partial sums meet in LDS and are added in wave order: no partial sum leaves
//     the workgroup, so there is no cross-workgroup synchronisation (on gfx950 an agent-scope
//     fence writes back and invalidates the XCD's whole L2) and results do not depend on
//     scheduling.
//   - The sum of squares of X for the folded rms-norm (EPI_NORM/SWIGLU, NORM_IN) rides
//     along the same path.
// int8 weights need one scale per k chunk: groups of 256 or more, or one scale per row
// (per-output-channel, any k).
#include "sv_device.h"
#include "sv_internal.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace sv {

struct MMParams {
  const uint8_t* w;
  const uint16_t* scales;
  const float* x;
  const uint32_t* x_rows;
  float* y;
  const float* base;
  float* aux;
  uint32_t n, k, m, epi, flags, vocab_real, gshift, chunks, per_row, tiled;
  float scale, ra, rb;
  // Split-k hand-off (skinny path with S > 1): counters per row group (zero at rest),
  // partial sums and sums of squares per (row group, split).
  uint32_t* counters;
  float* part;
  float* ssp;
  uint32_t splits, tgroups;  // skinny: k splits and 16-token groups
  // GEMM work order (gemm_item): 0 row block, split, token block (token block fastest); g > 0:
  // split, groups of g row blocks, token block, row block within the group.
  uint32_t order;
};

// The GEMMs' work item -> (token block, split, row block). Each XCD (workgroup id mod 8) takes a
// contiguous range of items, so the order decides which weights (row block, split) and which
// activations (token block, split) one XCD's L2 serves to several workgroups; the host picks the
// order with the least modelled HBM traffic (gemm_order).
__device__ __forceinline__ void gemm_item(uint32_t item, uint32_t n_tblk, uint32_t S, uint32_t nrb, uint32_t g,
                                          uint32_t& tblk, uint32_t& sp, uint32_t& rblk) {
  if (g == 0) {
    tblk = item % n_tblk;
    sp = (item / n_tblk) % S;
    rblk = item / (n_tblk * S);
    return;
  }
  const uint32_t per_sp = nrb * n_tblk, per_grp = g * n_tblk;
  sp = item / per_sp;
  const uint32_t rem = item % per_sp, r2 = rem % per_grp;
  tblk = r2 / g;
  rblk = (rem / per_grp) * g + r2 % g;
}


constexpr int KC = 256;  // k per chunk: one X chunk in registers, 4 blocks of 64
constexpr int NBLK = KC / 64;

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Epilogue of the skinny kernels (kernels.metal:183-209): lane (t, q) holds rows 4 q + 0..3
// of each of the workgroup's RT tiles for token tt; ss: the token's sum of squares over k.
template <int RT>
__device__ __forceinline__ void skinny_epilogue(const MMParams& p, const f32x4 (&acc)[RT], float ss, uint32_t xg, int q,
                                                uint32_t tt, const f32x4* base_pre = nullptr) {
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)p.k + SV_RMS_EPS);
  if ((p.flags & SV_FLAG_WRITE_INV) && p.epi == SV_EPI_NORM && xg == 0 && q == 0) p.aux[tt] = inv;
  const bool norm_in = (p.flags & SV_FLAG_NORM_IN) != 0;
#pragma unroll
  for (int rt = 0; rt < RT; rt++) {
    const uint32_t row0 = (xg * RT + rt) * 16 + 4 * q;
    f32x4 v = acc[rt];
    const size_t o = (size_t)tt * p.m + row0;
    switch (p.epi) {
      case SV_EPI_NORM:
        *(f32x4*)(p.y + o) = v * (inv * p.scale);
        break;
      case SV_EPI_RAW:
        if (norm_in) v *= inv;
        *(f32x4*)(p.y + o) = v;
        break;
      case SV_EPI_RESID: {
        if (norm_in) v *= inv;
        const f32x4 sv = v * p.scale;
        const f32x4 b = base_pre ? base_pre[rt] : *(const f32x4*)(p.base + o);
        *(f32x4*)(p.y + o) = b * p.ra + sv * p.rb;
        if (p.flags & SV_FLAG_WRITE_RAW) *(f32x4*)(p.aux + o) = sv;
        break;
      }
      case SV_EPI_HEAD: {
        if (norm_in) v *= inv;
        f32x4 l;
#pragma unroll
        for (int i = 0; i < 4; i++)
          l[i] = row0 + i < p.vocab_real ? 23.0f * sigmoidf_((v[i] + 5.0f) / 7.5f) : -__builtin_inff();
        *(f32x4*)(p.y + o) = l;
        break;
      }
      case SV_EPI_SWIGLU: {
        const float sc = inv * p.scale;
        const float g0 = v[0] * sc, u0 = v[1] * sc, g1 = v[2] * sc, u1 = v[3] * sc;
        float2 out;
        out.x = g0 * sigmoidf_(g0) * u0;
        out.y = g1 * sigmoidf_(g1) * u1;
        *(float2*)(p.y + (size_t)tt * (p.m / 2) + row0 / 2) = out;
        break;
      }
      default:
        break;
    }
  }
}

// One workgroup of W waves owns RT tiles of 16 output rows, one group of 16 tokens and a
// 1/S share of k: wave wv of split s takes k chunks s W + wv, + S W, ... The waves' sums meet
// in LDS in wave order; with S > 1 each split's sums go to the workspace with coherent stores
// and the last split of the (row group, token group) to arrive (relaxed agent-scope counter)
// adds them in split order and runs the epilogue: deterministic whatever the arrival order.
// Work items (row group, split, token group) are numbered token group fastest and dealt to
// the XCDs in contiguous blocks, so token groups that share weight rows share an L2.
template <int FMT, int RT, int W>
__global__ __launch_bounds__(64 * W) void mm_skinny(MMParams p) {
  constexpr int WV = FMT == SV_FMT_I8 ? 1 : 2;  // dwordx4 loads per lane per 64-k block
  constexpr int ESZ = FMT == SV_FMT_I8 ? 1 : 2;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int t = lane & 15, q = lane >> 4;
  const uint32_t S = p.splits, TG = p.tgroups, nwg = gridDim.x;
  uint32_t item = blockIdx.x;
  if (nwg % 8 == 0) item = (item % 8) * (nwg / 8) + item / 8;
  const uint32_t tg = item % TG, sp = (item / TG) % S, xg = item / (TG * S);
  const uint32_t tok0 = 16 * tg, n_loc = min(16u, p.n - tok0);

  __shared__ f32x4 red[W][RT][64];
  __shared__ float ssred[W][16];
  __shared__ uint32_t last_flag;

  f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ss = 0.0f;
  const bool tok = (uint32_t)t < n_loc;
  const uint32_t tt = tok0 + t;
  const float* xrow = p.x + (size_t)(tok ? (p.x_rows ? p.x_rows[tt] : tt) : 0u) * p.k + 16 * q;
  const uint32_t ng = p.per_row ? 1u : p.k >> p.gshift;
  const uint32_t stride = W * S;

  uint32_t c = sp * W + wv;
  u32x4 wr[RT][NBLK * WV];
  if (c < p.chunks) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
      for (int b = 0; b < NBLK; b++)
#pragma unroll
        for (int v = 0; v < WV; v++)
          wr[rt][b * WV + v] =
              ldg_nt(weight_word<ESZ>(p.w, p.k, p.tiled, xg * RT + rt, c * NBLK + b, v, lane));
  }
  for (; c < p.chunks; c += stride) {
    const uint32_t kbase = c * KC;
    // X chunk: token t, k = kbase + 64 b + 16 q + 0..15, as hi/lo bf16 B operands.
    bf16x8 xh[NBLK][2], xl[NBLK][2];
    if (tok) {
#pragma unroll
      for (int b = 0; b < NBLK; b++) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const f32x4 f = *(const f32x4*)(xrow + kbase + 64 * b + 4 * j);
          v[4 * j] = f[0];
          v[4 * j + 1] = f[1];
          v[4 * j + 2] = f[2];
          v[4 * j + 3] = f[3];
        }
#pragma unroll
        for (int j = 0; j < 16; j++) ss = __builtin_fmaf(v[j], v[j], ss);
        split8(v, xh[b][0], xl[b][0]);
        split8(v + 8, xh[b][1], xl[b][1]);
      }
    } else {
      const bf16x8 zero = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
      for (int b = 0; b < NBLK; b++) xh[b][0] = xh[b][1] = xl[b][0] = xl[b][1] = zero;
    }
    // Weights of this chunk (loaded), then the next chunk's in flight during the products.
    u32x4 cur[RT][NBLK * WV];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
      for (int i = 0; i < NBLK * WV; i++) cur[rt][i] = wr[rt][i];
    const uint32_t cn = c + stride;
    if (cn < p.chunks) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int b = 0; b < NBLK; b++)
#pragma unroll
          for (int v = 0; v < WV; v++)
            wr[rt][b * WV + v] =
                ldg_nt(weight_word<ESZ>(p.w, p.k, p.tiled, xg * RT + rt, cn * NBLK + b, v, lane));
    }
    f32x4 part[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) part[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NBLK; b++) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++) {
        bf16x8 a0, a1;
        if (FMT == SV_FMT_I8) {
          const u32x4 w = cur[rt][b];
          a0 = i8x8_to_bf(w[0], w[1]);
          a1 = i8x8_to_bf(w[2], w[3]);
        } else {
          a0 = __builtin_bit_cast(bf16x8, cur[rt][2 * b]);
          a1 = __builtin_bit_cast(bf16x8, cur[rt][2 * b + 1]);
        }
        part[rt] = mfma16(a0, xh[b][0], part[rt]);
        part[rt] = mfma16(a0, xl[b][0], part[rt]);
        part[rt] = mfma16(a1, xh[b][1], part[rt]);
        part[rt] = mfma16(a1, xl[b][1], part[rt]);
      }
    }
    if (FMT == SV_FMT_I8) {
      const uint32_t gi = p.per_row ? 0u : kbase >> p.gshift;
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const size_t row = (size_t)(xg * RT + rt) * 16 + 4 * q + i;
          part[rt][i] *= bf(p.scales[row * ng + gi]);
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; rt++) acc[rt] += part[rt];
  }
  ss += __shfl_xor(ss, 16, WAVE);
  ss += __shfl_xor(ss, 32, WAVE);
#pragma unroll
  for (int rt = 0; rt < RT; rt++) red[wv][rt][lane] = acc[rt];
  if (q == 0) ssred[wv][t] = ss;
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      f32x4 a = red[0][rt][lane];
#pragma unroll
      for (int w = 1; w < W; w++) a += red[w][rt][lane];
      acc[rt] = a;
    }
    ss = ssred[0][t];
#pragma unroll
    for (int w = 1; w < W; w++) ss += ssred[w][t];
  }
  if (S > 1) {
    // Split hand-off: partial [group][split][rt][lane] (f32x4), sums of squares [group][split][t].
    const size_t cell = (size_t)xg * TG + tg;
    float* part = p.part + (cell * S * RT) * 256;
    float* ssp = p.ssp + cell * S * 16;
    if (wv == 0) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) store_wt(part + ((size_t)sp * RT + rt) * 256 + 4 * lane + i, acc[rt][i]);
      if (q == 0) store_wt(ssp + sp * 16 + t, ss);
    }
    if (!arrive_last(p.counters + cell, S, &last_flag)) return;
    if (wv != 0) return;
    f32x4 tot[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) tot[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float sst = 0.0f;
    for (uint32_t s2 = 0; s2 < S; s2++) {
      if (s2 == sp) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) tot[rt] += acc[rt];
        sst += ss;
        continue;
      }
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) tot[rt][i] += load_wt(part + ((size_t)s2 * RT + rt) * 256 + 4 * lane + i);
      sst += load_wt(ssp + s2 * 16 + t);
    }
#pragma unroll
    for (int rt = 0; rt < RT; rt++) acc[rt] = tot[rt];
    ss = sst;
  } else if (wv != 0) {
    return;
  }

  // Epilogue (kernels.metal:183-209): lane (t, q) holds rows 4 q + 0..3 of each tile.
  if ((uint32_t)t >= n_loc) return;
  skinny_epilogue<RT>(p, acc, ss, xg, q, tt);
}

// ------------------------------------------------------------ 1-16 rows, one shot
// The verify step's matmuls at 1-16 rows: every wave requests everything it will read when
// it starts, so a launch costs about one memory round trip instead of one per dependency.
//   - A workgroup of W waves owns RT row tiles over the whole of k; wave wv takes the NCH
//     consecutive 256-k chunks from wv NCH, its weights held in registers.
//   - X is read densely (lane l: k 4 l .. 4 l + 3 of each token, a contiguous 1 KB per token
//     and chunk), XD chunks ahead (all of the wave's chunks when they fit in registers). Every
//     wave requests its first X chunks before any wave requests weights (an execution barrier,
//     no wait): a compute unit serves its waves' requests in order, and X is what every chunk
//     waits for first. The wave splits each chunk into bf16 hi + lo in its own LDS rows, from
//     which each lane reads its MFMA B operands (token slots >= n are zeros). LDS operations
//     of one wave execute in order: no barrier between the writes and the reads.
//   - Per-row int8 scales multiply the sums once at the end; grouped scales (>= 256) per chunk.
//   - Sums of squares (the folded rms-norm) by DPP row sums and four lane reads per token.
//   - The waves' sums meet in LDS in wave order; wave 0 runs the epilogue. No partial sum
//     leaves the workgroup: deterministic, no hand-off.
constexpr int XROW = KC + 8;  // bf16 per LDS row of one token's hi or lo (16 bytes of padding)

template <int CTRL>
__device__ __forceinline__ float mov_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
// Sum over a full wave, in a fixed order: within rows of 16 lanes by DPP (quad xor 1, xor 2,
// half-row mirror, row mirror), then the four row sums.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += mov_dpp<0xB1>(v);
  v += mov_dpp<0x4E>(v);
  v += mov_dpp<0x141>(v);
  v += mov_dpp<0x140>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// X chunks a wave keeps in flight: all NCH if NCH NT <= 24 (<= 96 registers), else fewer.
constexpr int x_depth(int nch, int nt) { return nch * nt <= 24 ? nch : (2 * nt <= 24 ? 2 : 1); }
// The one-shot kernel's int8 variant with scale groups of 64 or 128 k (the reference's default
// layer format, tools/convert.py:20): each group's products are summed on their own and scaled.
constexpr int FMT_I8_G64 = 16;

template <int FMT, int RT, int W, int NCH, int NT>
__global__ __launch_bounds__(64 * W) void mm_stream(MMParams p) {
  constexpr bool I8 = FMT != SV_FMT_BF16;
  constexpr bool SG = FMT == FMT_I8_G64;  // scale groups of 64 or 128 k
  constexpr int WV = I8 ? 1 : 2;
  constexpr int ESZ = I8 ? 1 : 2;
  constexpr int XD = x_depth(NCH, NT);
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_all[];  // [W][n][hi, lo][XROW]
  __shared__ f32x4 red[W][RT][64];
  __shared__ float ssred[W][NT];
  __shared__ uint32_t last_flag;
  const int lane = threadIdx.x & 63, t = lane & 15, q = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t n = p.n, nwg = gridDim.x, S = p.splits;
  uint32_t item = blockIdx.x;
  if (nwg % 8 == 0) item = (item % 8) * (nwg / 8) + item / 8;
  const uint32_t xg = item / S, sp = item % S;  // row group, k split (the splits of a group share an XCD)
  uint16_t* xs = xs_all + (size_t)wv * n * 2 * XROW;
  const uint32_t c0 = (sp * W + wv) * NCH;
  const bool grouped = I8 && !SG && !p.per_row;
  const uint32_t ng = p.per_row ? 1u : p.k >> p.gshift;
  // Loads go through buffer resources: one per-lane offset, a uniform offset per load.
  const __amdgpu_buffer_rsrc_t xrs = coherent_rsrc(p.x), wrs = coherent_rsrc(p.w);
  const uint32_t xv = 16 * lane;
  const uint32_t wvo = p.tiled ? 16u * lane : ((uint32_t)t * p.k + 16 * q) * ESZ;
  const uint32_t tile_bytes = 16 * p.k * ESZ, kb_bytes = p.tiled ? 1024 * ESZ : 64 * ESZ, v_bytes = p.tiled ? 1024 : 16;

  // Loads are unconditional (loads under branches would be waited for one by one): chunks
  // past k re-read the last chunk and are ignored; token slots past n take a lane offset past
  // the buffer's range, which the hardware answers with zeros without a memory access.
  const uint32_t nx = min(n, (uint32_t)NT);
  const uint32_t xv_none = 0x80000000u + xv;
  uint32_t xrow[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const uint32_t ii = (uint32_t)i < nx ? (uint32_t)i : 0u;
    xrow[i] = p.x_rows ? p.x_rows[ii] : ii;
  }
  auto load_x = [&](f32x4 (&dst)[NT], uint32_t c) {
    c = min(c, p.chunks - 1);
#pragma unroll
    for (int i = 0; i < NT; i++)
      dst[i] = __builtin_bit_cast(f32x4, buf_ld16(xrs, (uint32_t)i < nx ? xv : xv_none, (xrow[i] * p.k + c * KC) * 4));
  };
  auto load_gscale = [&](float (&dst)[RT][4], uint32_t c) {
    c = min(c, p.chunks - 1);
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
      for (int i = 0; i < 4; i++)
        dst[rt][i] = bf(ldg_u16(p.scales + ((size_t)(xg * RT + rt) * 16 + 4 * q + i) * ng + ((c * KC) >> p.gshift)));
  };

  // 1. X of the first XD chunks, the epilogue's operands; then (all waves) the weights.
  f32x4 xr[XD][NT];
#pragma unroll
  for (int d = 0; d < XD; d++) load_x(xr[d], c0 + d);
  // wave wv < RT finishes row tile wv: its per-row scales and residual base, requested now
  f32x4 base_pre[1];
  uint2 rsc = {0u, 0u};
  if (wv < RT) {
    const uint32_t row0 = (xg * RT + wv) * 16 + 4 * q;
    // four 16-bit loads: the scale array needs no alignment beyond its element's
    if (I8 && p.per_row)
      rsc = uint2{ldg_u16(p.scales + row0) | ((uint32_t)ldg_u16(p.scales + row0 + 1) << 16),
                  ldg_u16(p.scales + row0 + 2) | ((uint32_t)ldg_u16(p.scales + row0 + 3) << 16)};
    if (p.epi == SV_EPI_RESID && (uint32_t)t < n) base_pre[0] = *(const f32x4*)(p.base + (size_t)t * p.m + row0);
  }
  float gsc[RT][4];
  if (grouped) load_gscale(gsc, c0);
  // Groups of 64 (four per chunk) or 128 (two): each lane's four rows' scales of every chunk
  // it multiplies, requested with the weights (8 bytes per row and chunk).
  u32x2 sgw[SG ? NCH : 1][SG ? RT : 1][SG ? 4 : 1];
  if (SG) {
    const uint32_t gpc = KC >> p.gshift;
#pragma unroll
    for (int j = 0; j < NCH; j++)
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint16_t* sp_ = p.scales + ((size_t)(xg * RT + rt) * 16 + 4 * q + i) * ng + min(c0 + j, p.chunks - 1) * gpc;
          u32x2 v;
          v[0] = ldg_u32(sp_);
          v[1] = gpc == 4 ? ldg_u32(sp_ + 2) : 0u;
          sgw[SG ? j : 0][SG ? rt : 0][SG ? i : 0] = v;
        }
  }
  __builtin_amdgcn_s_barrier();
  u32x4 wr[NCH][RT][NBLK * WV];
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    const uint32_t cj = min(c0 + j, p.chunks - 1);
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
      for (int b = 0; b < NBLK; b++)
#pragma unroll
        for (int v = 0; v < WV; v++)
          wr[j][rt][b * WV + v] =
              buf_ld16_nt(wrs, wvo, (xg * RT + rt) * tile_bytes + (cj * NBLK + b) * kb_bytes + v * v_bytes);
  }

  // 2. chunks in order.
  f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ssl[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) ssl[i] = 0.0f;
  const bf16x8 zero = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    const uint32_t c = c0 + j;
    if (c >= p.chunks) break;
    // keep each chunk's conversions and products inside its iteration (register pressure)
    __builtin_amdgcn_sched_barrier(0);
    f32x4 (&xc)[NT] = xr[j % XD];
    // this chunk's X: sums of squares (token slots past n are zeros), hi/lo to the LDS rows
#pragma unroll
    for (int i = 0; i < NT; i++) {
      const f32x4 v = xc[i];
      ssl[i] = __builtin_fmaf(v[0], v[0], __builtin_fmaf(v[1], v[1], __builtin_fmaf(v[2], v[2], __builtin_fmaf(v[3], v[3], ssl[i]))));
    }
#pragma unroll
    for (int i = 0; i < NT; i++) {
      if ((uint32_t)i >= n) break;
      const f32x4 v = xc[i];
      const u32x2 s01 = split2(v[0], v[1]), s23 = split2(v[2], v[3]);
      const u32x2 hw = u32x2{s01[0], s23[0]}, lw = u32x2{s01[1], s23[1]};
      *(u32x2*)(xs + (2 * i) * XROW + 4 * lane) = hw;
      *(u32x2*)(xs + (2 * i + 1) * XROW + 4 * lane) = lw;
    }
    // the slot is free: the chunk XD ahead goes into it
    float gnext[RT][4];
    if (j + XD < NCH) load_x(xr[j % XD], c + XD);
    if (grouped && j + 1 < NCH) load_gscale(gnext, c + 1);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    f32x4 part[RT], gpart[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) part[rt] = gpart[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NBLK; b++) {
      bf16x8 xh0 = zero, xh1 = zero, xl0 = zero, xl1 = zero;
      if ((uint32_t)t < n) {
        const uint16_t* hp = xs + (2 * t) * XROW + 64 * b + 16 * q;
        xh0 = *(const bf16x8*)hp;
        xh1 = *(const bf16x8*)(hp + 8);
        xl0 = *(const bf16x8*)(hp + XROW);
        xl1 = *(const bf16x8*)(hp + XROW + 8);
      }
#pragma unroll
      for (int rt = 0; rt < RT; rt++) {
        bf16x8 a0, a1;
        if (I8) {
          const u32x4 w = wr[j][rt][b];
          a0 = i8x8_to_bf(w[0], w[1]);
          a1 = i8x8_to_bf(w[2], w[3]);
        } else {
          a0 = __builtin_bit_cast(bf16x8, wr[j][rt][2 * b]);
          a1 = __builtin_bit_cast(bf16x8, wr[j][rt][2 * b + 1]);
        }
        f32x4& pa = SG ? gpart[rt] : part[rt];
        pa = mfma16(a0, xh0, pa);
        pa = mfma16(a0, xl0, pa);
        pa = mfma16(a1, xh1, pa);
        pa = mfma16(a1, xl1, pa);
      }
      // a group of 64 ends with every block, one of 128 with every second: its sum, scaled
      if (SG && (p.gshift == 6 || (b & 1))) {
        const int g = p.gshift == 6 ? b : b >> 1;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const uint32_t w2 = sgw[SG ? j : 0][SG ? rt : 0][SG ? i : 0][g >> 1];
            part[rt][i] = __builtin_fmaf(bf(g & 1 ? w2 >> 16 : w2 & 0xffffu), gpart[rt][i], part[rt][i]);
          }
          gpart[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
    // the next chunk's LDS writes stay behind these reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      if (grouped) {
#pragma unroll
        for (int i = 0; i < 4; i++) part[rt][i] *= gsc[rt][i];
      }
      acc[rt] += part[rt];
    }
    if (grouped && j + 1 < NCH) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) gsc[rt][i] = gnext[rt][i];
    }
  }

  // 3. waves' sums: row tile rt's are added in wave order and finished by wave rt (the tiles'
  //    epilogues run in parallel); sums of squares per token.
  const bool need_ss = p.epi == SV_EPI_NORM || p.epi == SV_EPI_SWIGLU || (p.flags & SV_FLAG_NORM_IN);
  if (need_ss) {
#pragma unroll
    for (int i = 0; i < NT; i++) {
      const float v = wave_sum_dpp(ssl[i]);
      if (lane == 0) ssred[wv][i] = v;
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; rt++) red[wv][rt][lane] = acc[rt];
  __syncthreads();
  const bool mine = wv < RT;  // this wave finishes row tile wv
  const uint32_t rt0 = mine ? (uint32_t)wv : 0u;
  f32x4 tile = f32x4{0.f, 0.f, 0.f, 0.f};
  if (mine) {
    tile = red[0][rt0][lane];
#pragma unroll
    for (int w = 1; w < W; w++) tile += red[w][rt0][lane];
  }
  float ss = 0.0f;
  if (need_ss && (uint32_t)t < NT) {
    ss = ssred[0][t];
#pragma unroll
    for (int w = 1; w < W; w++) ss += ssred[w][t];
  }
  const uint32_t tg = xg * RT + rt0;  // this wave's row tile (of 16 rows)
  if (S > 1) {
    // k splits: each split's tile sums to the workspace (coherent stores), the last split of
    // the row group to arrive adds them in split order (each wave its own tile).
    const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(p.part), srs = coherent_rsrc(p.ssp);
    const uint32_t pbase = (xg * S) * RT * 1024, sbase = (xg * S) * 64;
    if (mine) store_wt4(prs, pbase + (sp * RT + rt0) * 1024 + 16 * lane, tile);
    if (wv == 0 && lane < 16) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ss), srs, sbase + sp * 64 + 4 * lane, 0, SV_CPOL_SC1);
    if (!arrive_last(p.counters + xg, S, &last_flag)) return;
    if (!mine) return;
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    float sst = 0.0f;
    for (uint32_t s2 = 0; s2 < S; s2++) {
      if (s2 == sp) {
        tot += tile;
        sst += ss;
      } else {
        tot += load_wt4(prs, pbase + (s2 * RT + rt0) * 1024 + 16 * lane);
        sst += __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, sbase + s2 * 64 + 4 * t, 0, SV_CPOL_SC1));
      }
    }
    tile = tot;
    ss = sst;
  }
  if (!mine) return;
  if (I8 && p.per_row) {
    tile[0] *= bf(rsc.x & 0xffffu);
    tile[1] *= bf(rsc.x >> 16);
    tile[2] *= bf(rsc.y & 0xffffu);
    tile[3] *= bf(rsc.y >> 16);
  }
  if ((uint32_t)t >= n) return;
  f32x4 one[1] = {tile};
  skinny_epilogue<1>(p, one, ss, tg, q, t, base_pre);
}

// Tiled copy of a row-major matrix (SV_FMT_TILED): one thread per 16-byte word of the
// output, in output order (the read side gathers 16-byte pieces of rows).
__global__ __launch_bounds__(256) void pack_tiled_kernel(const uint8_t* src, uint8_t* dst, uint32_t k, uint32_t esz,
                                                         size_t words) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= words) return;
  const uint32_t lane = i % 64;
  const size_t wi = i / 64;  // (tile, block, v)
  const uint32_t per_tile = k / 64 * esz;
  const uint32_t tile = wi / per_tile, bv = wi % per_tile, kb = bv / esz, v = bv % esz;
  const uint8_t* s = src + ((size_t)(tile * 16 + lane % 16) * k + 64 * kb + 16 * (lane / 16)) * esz + 16 * v;
  *(u32x4*)(dst + i * 16) = *(const u32x4*)s;
}

// ------------------------------------------------------------------- large n
// GEMM path (n > 16 rows: many streams, draft trees): a workgroup of 4 waves owns
// BM = 64 RTW output rows, BN = 16 NT tokens and a 1/S share of k (k splits when the tiles
// alone give too few workgroups); k goes in chunks of 64.
//   - Software pipeline D chunks deep: each wave's weights (16 bytes per lane per row tile
//     per chunk) and each thread's X pairs for chunk c + D are requested while chunk c is
//     multiplied. Every load is unconditional: chunks past the split's end and token slots
//     past n use offsets beyond the buffer's range, which the hardware answers with zeros
//     without a memory access, so no branch makes the compiler wait for a load early.
//   - X chunk [BN][64] fp32 is read once per workgroup (L2), split into bf16 hi + lo and
//     written to LDS in MFMA B-operand lane order (one 16-byte row per lane), so every
//     operand read is a conflict-free ds_read_b128; double-buffered, one barrier per chunk
//     (an LDS-only wait: weight and X loads stay in flight across it).
//   - Each wave converts its int8 weights to bf16 in registers (exact) and runs
//     RTW x NT x 2 k-steps x 2 (hi, lo) MFMAs per chunk.
//   - Workgroups that share weight rows (different token blocks) are mapped to the same XCD,
//     so all but the first read the rows from that XCD's L2.
//   - Sums of squares for the folded rms-norm: each thread owns fixed (token, 8-k group)
//     pairs for the whole k, added in a fixed order at the end.
//   - k splits: each split stores its sums (coherent stores) and the last split of the
//     (row block, token block) to arrive adds them in split order and runs the epilogue.
constexpr int GKC = 64;
// Split-k hand-off counters (skinny and GEMM paths): a region of fixed size at the front of the
// workspace, so every matmul sharing one workspace finds its counters at zero there, whatever
// its shape.
constexpr size_t COUNTER_SLOTS = 65536;

// Wait for this thread's LDS operations, then the workgroup barrier. Unlike __syncthreads()
// this leaves global loads in flight (no vmcnt wait).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Epilogue of the GEMM (kernels.metal:183-209) for one 16-token tile: lane (t16, q) holds rows
// 4 q + 0..3 of each of the wave's RTW row tiles (first row row0) for token t.
template <int RTW>
__device__ __forceinline__ void gemm_epilogue(const MMParams& p, const f32x4 (&acc)[RTW], uint32_t row0, int q,
                                              uint32_t t, float ss, bool write_inv) {
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)p.k + SV_RMS_EPS);
  if (write_inv && (p.flags & SV_FLAG_WRITE_INV) && p.epi == SV_EPI_NORM && q == 0) p.aux[t] = inv;
  const bool norm_in = (p.flags & SV_FLAG_NORM_IN) != 0;
#pragma unroll
  for (int r = 0; r < RTW; r++) {
    const uint32_t rowq = row0 + 16 * r + 4 * q;
    f32x4 v = acc[r];
    const size_t o = (size_t)t * p.m + rowq;
    switch (p.epi) {
      case SV_EPI_NORM:
        *(f32x4*)(p.y + o) = v * (inv * p.scale);
        break;
      case SV_EPI_RAW:
        if (norm_in) v *= inv;
        *(f32x4*)(p.y + o) = v;
        break;
      case SV_EPI_RESID: {
        if (norm_in) v *= inv;
        const f32x4 sv = v * p.scale;
        const f32x4 b = *(const f32x4*)(p.base + o);
        *(f32x4*)(p.y + o) = b * p.ra + sv * p.rb;
        if (p.flags & SV_FLAG_WRITE_RAW) *(f32x4*)(p.aux + o) = sv;
        break;
      }
      case SV_EPI_HEAD: {
        if (norm_in) v *= inv;
        f32x4 l;
#pragma unroll
        for (int i = 0; i < 4; i++)
          l[i] = rowq + i < p.vocab_real ? 23.0f * sigmoidf_((v[i] + 5.0f) / 7.5f) : -__builtin_inff();
        *(f32x4*)(p.y + o) = l;
        break;
      }
      case SV_EPI_SWIGLU: {
        const float sc = inv * p.scale;
        const float g0 = v[0] * sc, u0 = v[1] * sc, g1 = v[2] * sc, u1 = v[3] * sc;
        float2 out;
        out.x = g0 * sigmoidf_(g0) * u0;
        out.y = g1 * sigmoidf_(g1) * u1;
        *(float2*)(p.y + (size_t)t * (p.m / 2) + rowq / 2) = out;
        break;
      }
      default:
        break;
    }
  }
}

template <int FMT, int RTW, int NT, bool GROUPED, int GD>
__global__ __launch_bounds__(256) void mm_gemm(MMParams p, uint32_t n_tblk) {
  static_assert(GD % 2 == 0, "chunk parity = slot parity");
  constexpr int NTH = 256;
  constexpr int BN = 16 * NT;
  constexpr int ESZ = FMT == SV_FMT_I8 ? 1 : 2;
  constexpr int WL = FMT == SV_FMT_I8 ? 1 : 2;  // dwordx4 per lane per row tile per chunk
  constexpr int PAIRS = BN * 8;                 // (token, 8-k group) pairs per chunk
  constexpr int PPT = (PAIRS + NTH - 1) / NTH;  // pairs per thread
  // LDS: [2 buffers][NT][hi, lo][128 slots] of 16 bytes; lane (t, q) of k-step ks reads slot
  // 64 ks + 16 q + (t ^ (4 ks + q)). gfx950 serves a 16-byte read conflict-free when every
  // quarter-wave starts at a multiple of 16 slots and its lanes keep their slot mod 16 up to a
  // permutation within groups of 8 lanes (the XOR only flips the low three bits); a 16-byte
  // write, when each 8 consecutive lanes hit 8 different slots mod 8: the writers of one token
  // (8 lanes, k groups g = 2 q + ks) get t ^ (4 ks + q), 8 different values mod 8.
  __shared__ u32x4 xs[2][NT][2][128];
  __shared__ float ssp[BN][8];
  __shared__ uint32_t last_flag;
  const int tid = threadIdx.x, lane = tid & 63, t16 = lane & 15, q = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Work items (row block, split, token block), token block fastest; consecutive items go
  // to one XCD (workgroups are dealt to the 8 XCDs by id mod 8): XCD x takes a contiguous
  // range of nwg/8 items, one more for the first nwg%8 XCDs.
  const uint32_t nwg = gridDim.x, S = p.splits;
  const uint32_t xcd = blockIdx.x % 8, xq = nwg / 8;
  const uint32_t item = xcd * xq + min(xcd, nwg % 8) + blockIdx.x / 8;
  uint32_t tblk, sp, rblk;
  gemm_item(item, n_tblk, S, nwg / (n_tblk * S), p.order, tblk, sp, rblk);
  const uint32_t t0 = tblk * BN;
  const uint32_t row0 = (rblk * 4 + wv) * 16 * RTW;  // this wave's first row
  const uint32_t nc = __builtin_amdgcn_readfirstlane(p.k / GKC / S);
  const uint32_t cb = __builtin_amdgcn_readfirstlane(sp * nc);

  // Buffer resources (offsets below 2 GiB); an offset of 2^31 or more reads zeros.
  const __amdgpu_buffer_rsrc_t xrs = coherent_rsrc(p.x), wrs = coherent_rsrc(p.w);
  constexpr uint32_t OOB = 0x80000000u;
  // Weights: lane (t16, q) takes row t16 of each tile, bytes 16 q .. of each 64-k chunk.
  const uint32_t tile0 = row0 / 16;
  const uint32_t wv_lane = p.tiled ? 16u * lane : ((uint32_t)t16 * p.k + 16 * q) * ESZ;
  const uint32_t tile_bytes = 16 * p.k * ESZ, chunk_bytes = p.tiled ? 1024 * ESZ : 64 * ESZ,
                 v_bytes = p.tiled ? 1024 : 16;
  // X pairs of this thread: pair i -> token i / 8, k group i % 8 (k = 8 (i % 8) .. + 7).
  uint32_t xoff[PPT];
#pragma unroll
  for (int j = 0; j < PPT; j++) {
    const int i = tid + NTH * j;
    const uint32_t tt = t0 + i / 8;
    const bool v = i < PAIRS && tt < p.n;
    xoff[j] = v ? ((p.x_rows ? p.x_rows[tt] : tt) * p.k + 8 * (i % 8)) * 4 : OOB;
  }
  auto load_x = [&](uint32_t c, f32x4 (&xr)[PPT][2]) {
    // past the split's end: every lane's offset out of range (the range check covers the
    // per-lane offset)
    const uint32_t so = __builtin_amdgcn_readfirstlane((cb + min(c, nc - 1)) * GKC * 4);
#pragma unroll
    for (int j = 0; j < PPT; j++) {
      const uint32_t vo = c < nc ? xoff[j] : OOB;
      xr[j][0] = __builtin_bit_cast(f32x4, buf_ld16(xrs, vo, so));
      xr[j][1] = __builtin_bit_cast(f32x4, buf_ld16(xrs, vo + 16, so));
    }
  };
  auto load_w = [&](uint32_t c, u32x4 (&wr)[RTW][WL]) {
    const uint32_t cc = c < nc ? cb + c : 0u;
    const uint32_t vo = c < nc ? wv_lane : OOB;
#pragma unroll
    for (int r = 0; r < RTW; r++)
#pragma unroll
      for (int v = 0; v < WL; v++)
        wr[r][v] = buf_ld16(wrs, vo, __builtin_amdgcn_readfirstlane((tile0 + r) * tile_bytes + cc * chunk_bytes + v * v_bytes));
  };
  float ssacc[PPT];
#pragma unroll
  for (int j = 0; j < PPT; j++) ssacc[j] = 0.0f;
  auto store_x = [&](int buf, const f32x4 (&xr)[PPT][2]) {
#pragma unroll
    for (int j = 0; j < PPT; j++) {
      const int i = tid + NTH * j;
      if (i >= PAIRS) continue;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[e] = xr[j][0][e];
        v[4 + e] = xr[j][1][e];
      }
#pragma unroll
      for (int e = 0; e < 8; e++) ssacc[j] = __builtin_fmaf(v[e], v[e], ssacc[j]);
      bf16x8 h, l;
      split8(v, h, l);
      const int tok = i / 8, g8 = i % 8, qq = g8 >> 1, ks = g8 & 1;
      const int slot = 64 * ks + 16 * qq + ((tok & 15) ^ (4 * ks + qq));
      xs[buf][tok >> 4][0][slot] = __builtin_bit_cast(u32x4, h);
      xs[buf][tok >> 4][1][slot] = __builtin_bit_cast(u32x4, l);
    }
  };
  const uint32_t ng = p.per_row ? 1u : p.k >> p.gshift;

  f32x4 acc[RTW][NT];
  f32x4 grp[GROUPED ? RTW : 1][GROUPED ? NT : 1];
#pragma unroll
  for (int r = 0; r < RTW; r++)
#pragma unroll
    for (int n = 0; n < NT; n++) acc[r][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (GROUPED)
#pragma unroll
    for (int r = 0; r < RTW; r++)
#pragma unroll
      for (int n = 0; n < NT; n++) grp[GROUPED ? r : 0][GROUPED ? n : 0] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: chunks 0 .. D-1 requested; chunk 0's X to LDS.
  f32x4 xr[GD][PPT][2];
  u32x4 wr[GD][RTW][WL];
#pragma unroll
  for (int d = 0; d < GD; d++) {
    load_w(d, wr[d]);
    load_x(d, xr[d]);
  }
  store_x(0, xr[0]);
  load_x(GD, xr[0]);
  lds_barrier();

  // No branch inside the loop (a conditional load would make the compiler wait for every
  // load in flight): a last partial round of GD runs on zeros (weights and X past the split's
  // end read as zeros and add exactly nothing).
  for (uint32_t c0 = 0; c0 < nc; c0 += GD) {
#pragma unroll
    for (int d = 0; d < GD; d++) {
      const uint32_t c = c0 + d;
      const int buf = d & 1;  // GD is even: chunk parity
      u32x4 cur[RTW][WL];
#pragma unroll
      for (int r = 0; r < RTW; r++)
#pragma unroll
        for (int v = 0; v < WL; v++) cur[r][v] = wr[d][r][v];
      load_w(c + GD, wr[d]);
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        bf16x8 a[RTW];
#pragma unroll
        for (int r = 0; r < RTW; r++) {
          if (FMT == SV_FMT_I8) a[r] = i8x8_to_bf(cur[r][0][2 * ks], cur[r][0][2 * ks + 1]);
          else a[r] = __builtin_bit_cast(bf16x8, cur[r][ks]);
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
          const int slot = 64 * ks + 16 * q + (t16 ^ (4 * ks + q));
          const bf16x8 bh = __builtin_bit_cast(bf16x8, xs[buf][n][0][slot]);
          const bf16x8 bl = __builtin_bit_cast(bf16x8, xs[buf][n][1][slot]);
#pragma unroll
          for (int r = 0; r < RTW; r++) {
            f32x4& g = GROUPED ? grp[GROUPED ? r : 0][GROUPED ? n : 0] : acc[r][n];
            g = mfma16(a[r], bh, g);
            g = mfma16(a[r], bl, g);
          }
        }
      }
      // Close a scale group (int8 with groups < k): acc += scale * group sums; also at the
      // split's last chunk when a group straddles two splits (each part scaled: exact).
      if (GROUPED && c < nc && ((((cb + c) + 1) * GKC) % (1u << p.gshift) == 0 || c + 1 == nc)) {
        const uint32_t gi = ((cb + c) * GKC) >> p.gshift;
#pragma unroll
        for (int r = 0; r < RTW; r++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float sc = bf(ldg_u16(p.scales + (size_t)(row0 + 16 * r + 4 * q + i) * ng + gi));
#pragma unroll
            for (int n = 0; n < NT; n++) {
              acc[r][n][i] += sc * grp[GROUPED ? r : 0][GROUPED ? n : 0][i];
              grp[GROUPED ? r : 0][GROUPED ? n : 0][i] = 0.0f;
            }
          }
      }
      // Chunk c + 1's X (requested D - 1 chunks ago) to the other buffer, then chunk
      // c + 1 + D requested into its registers.
      const int dn = (d + 1) % GD;
      store_x(buf ^ 1, xr[dn]);
      load_x(c + 1 + GD, xr[dn]);
      lds_barrier();
    }
  }
  if (!GROUPED && FMT == SV_FMT_I8) {
#pragma unroll
    for (int r = 0; r < RTW; r++) {
      f32x4 sc;
#pragma unroll
      for (int i = 0; i < 4; i++) sc[i] = bf(ldg_u16(p.scales + (row0 + 16 * r + 4 * q + i)));
#pragma unroll
      for (int n = 0; n < NT; n++) acc[r][n] *= sc;
    }
  }
  // Sums of squares per token: the thread's pairs, then the 8 k groups in order.
#pragma unroll
  for (int j = 0; j < PPT; j++) {
    const int i = tid + NTH * j;
    if (i < PAIRS) ssp[i / 8][i % 8] = ssacc[j];
  }
  __syncthreads();
  float ssn[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) {
    const uint32_t tl = 16 * n + t16;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += ssp[tl][e];
    ssn[n] = ss;
  }

  if (S > 1) {
    // This split's sums to the workspace: [cell][split][256 threads][RTW NT] f32x4 and
    // [cell][split][BN] sums of squares; the last split of the cell adds them in split order.
    const uint32_t cell = rblk * n_tblk + tblk;
    const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(p.part), srs = coherent_rsrc(p.ssp);
    constexpr uint32_t PER = NTH * RTW * NT * 16;
    const uint32_t pb = (cell * S) * PER;
#pragma unroll
    for (int r = 0; r < RTW; r++)
#pragma unroll
      for (int n = 0; n < NT; n++) store_wt4(prs, pb + sp * PER + ((r * NT + n) * NTH + tid) * 16, acc[r][n]);
    for (int tt = tid; tt < BN; tt += NTH)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ssp[tt][0] + ssp[tt][1] + ssp[tt][2] + ssp[tt][3] +
                                                            ssp[tt][4] + ssp[tt][5] + ssp[tt][6] + ssp[tt][7]),
                                            srs, ((cell * S + sp) * BN + tt) * 4, 0, SV_CPOL_SC1);
    if (!arrive_last(p.counters + cell, S, &last_flag)) return;
#pragma unroll
    for (int r = 0; r < RTW; r++)
#pragma unroll
      for (int n = 0; n < NT; n++) acc[r][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < NT; n++) ssn[n] = 0.0f;
    for (uint32_t s2 = 0; s2 < S; s2++) {
#pragma unroll
      for (int r = 0; r < RTW; r++)
#pragma unroll
        for (int n = 0; n < NT; n++) acc[r][n] += load_wt4(prs, pb + s2 * PER + ((r * NT + n) * NTH + tid) * 16);
#pragma unroll
      for (int n = 0; n < NT; n++)
        ssn[n] += __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(srs, ((cell * S + s2) * BN + 16 * n + t16) * 4, 0, SV_CPOL_SC1));
    }
  }

  // Epilogue: lane (t16, q) holds rows 4 q + 0..3 of each row tile for token t0 + 16 n + t16.
#pragma unroll
  for (int n = 0; n < NT; n++) {
    const uint32_t t = t0 + 16 * n + t16;
    if (t >= p.n) continue;
    f32x4 col[RTW];
#pragma unroll
    for (int r = 0; r < RTW; r++) col[r] = acc[r][n];
    gemm_epilogue<RTW>(p, col, row0, q, t, ssn[n], rblk == 0 && wv == 0);
  }
}

// 32 x 32 x 16 GEMM (n > 16 rows). gfx950 runs v_mfma_f32_32x32x16_bf16 (32,768 flops) in
// about the time v_mfma_f32_16x16x32_bf16 (16,384 flops) takes when both stream back to back
// (measured: 2.2 vs 1.2 PFLOP/s), so the 32-wide tile halves the matrix-core time of the same
// product. Same structure as mm_gemm: NW waves (4 or 8), BM = 32 RT NW rows (RT 32-row tiles per wave),
// BN = 32 NT tokens, 1/S of k, chunks of 64 k in a software pipeline GD deep, X split once per
// workgroup into LDS, k splits merged by the last split to arrive.
//   - MFMA lane (c, h) = (lane % 32, lane / 32) supplies A row c and B column c with 8 k per
//     step; the chunk's k order is permuted (the same way for A and B): step ks, lane half h,
//     element e is k = 32 h + 8 ks + e. So a lane's weights for a chunk are 32 consecutive k of
//     its row: two 16-byte words (bf16: four) of the tiled layout, word q = 2 h + qq of the
//     lane's 16-row block.
//   - X in LDS as [hi, lo][4 steps][2 halves][32 columns] 16-byte slots, the column XOR-ed
//     with 4 h + ks (< 8): reads of a quarter-wave start at a multiple of 16 slots and keep the
//     slot order up to a permutation within 8 lanes, writes of a token's 8 k groups land on 8
//     different slots mod 8 (both conflict-free on gfx950).
//   - Lane (c, h) receives rows 8 j + 4 h + i (j, i = 0..3) of token c: f32x4 row groups, so
//     the epilogue (rms-norm fold, SwiGLU pairs, residual) is the 16-wide one per group.
typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <int FMT, int RT, int NT, int GD, int NW, int CPI>
__global__ __launch_bounds__(NW * 64) void mm_gemm32(MMParams p, uint32_t n_tblk) {
  static_assert(GD % (2 * CPI) == 0, "iteration parity = buffer parity");
  constexpr int BN = 32 * NT;
  constexpr int ESZ = FMT == SV_FMT_I8 ? 1 : 2;
  constexpr int WL = FMT == SV_FMT_I8 ? 1 : 2;  // 16-byte words per lane per 16 k
  constexpr int NTH = NW * 64;
  constexpr int PAIRS = BN * 8;                 // (token, 8-k group) pairs per chunk
  constexpr int PPT = (PAIRS + NTH - 1) / NTH;  // pairs per thread
  __shared__ u32x4 xs[2][CPI][NT][2][256];  // [buffer][chunk of the iteration]
  __shared__ float ssp[BN][8];
  __shared__ uint32_t last_flag;
  const int tid = threadIdx.x, lane = tid & 63, c32 = lane & 31, h = lane >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Work items dealt to XCDs as in mm_gemm (token block fastest within an XCD's range).
  const uint32_t nwg = gridDim.x, S = p.splits;
  const uint32_t xcd = blockIdx.x % 8, xq = nwg / 8;
  const uint32_t item = xcd * xq + min(xcd, nwg % 8) + blockIdx.x / 8;
  uint32_t tblk, sp, rblk;
  gemm_item(item, n_tblk, S, nwg / (n_tblk * S), p.order, tblk, sp, rblk);
  const uint32_t t0 = tblk * BN;
  const uint32_t row0 = (rblk * NW + wv) * 32 * RT;  // this wave's first row
  const uint32_t nc = __builtin_amdgcn_readfirstlane(p.k / GKC / S);
  const uint32_t cb = __builtin_amdgcn_readfirstlane(sp * nc);

  const __amdgpu_buffer_rsrc_t xrs = coherent_rsrc(p.x), wrs = coherent_rsrc(p.w);
  constexpr uint32_t OOB = 0x80000000u;
  // Weights: lane (c, h) takes row c of the wave's 32-row tile r (16-row block c / 16, row
  // c % 16), words q = 2 h, 2 h + 1 of each chunk.
  const uint32_t tile_bytes = 16 * p.k * ESZ;  // one 16-row block over all k
  const uint32_t wl = p.tiled ? (uint32_t)(c32 >> 4) * tile_bytes + (uint32_t)((c32 & 15) + 32 * h) * 16
                              : ((uint32_t)c32 * p.k + 32 * h) * ESZ;
  const uint32_t chunk_bytes = p.tiled ? 1024 * ESZ : 64 * ESZ, qq_bytes = p.tiled ? 256 : 16 * ESZ,
                 v_bytes = p.tiled ? 1024 : 16;
  uint32_t xoff[PPT];
#pragma unroll
  for (int j = 0; j < PPT; j++) {
    const int i = tid + NTH * j;
    const uint32_t tt = t0 + i / 8;
    xoff[j] = i < PAIRS && tt < p.n ? ((p.x_rows ? p.x_rows[tt] : tt) * p.k + 8 * (i % 8)) * 4 : OOB;
  }
  auto load_x = [&](uint32_t c, f32x4 (&xr)[PPT][2]) {
    const uint32_t so = __builtin_amdgcn_readfirstlane((cb + min(c, nc - 1)) * GKC * 4);
#pragma unroll
    for (int j = 0; j < PPT; j++) {
      const uint32_t vo = c < nc ? xoff[j] : OOB;
      xr[j][0] = __builtin_bit_cast(f32x4, buf_ld16(xrs, vo, so));
      xr[j][1] = __builtin_bit_cast(f32x4, buf_ld16(xrs, vo + 16, so));
    }
  };
  auto load_w = [&](uint32_t c, u32x4 (&wr)[RT][2 * WL]) {
    const uint32_t cc = c < nc ? cb + c : 0u;
    const uint32_t vo = c < nc ? wl : OOB;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int qq = 0; qq < 2; qq++)
#pragma unroll
        for (int v = 0; v < WL; v++) {
          const uint32_t rbase = p.tiled ? (row0 / 16 + 2 * r) * tile_bytes : (row0 + 32 * r) * p.k * ESZ;
          wr[r][qq * WL + v] =
              buf_ld16(wrs, vo, __builtin_amdgcn_readfirstlane(rbase + cc * chunk_bytes + qq * qq_bytes + v * v_bytes));
        }
  };
  float ssacc[PPT];
#pragma unroll
  for (int j = 0; j < PPT; j++) ssacc[j] = 0.0f;
  auto store_x = [&](int buf, int u, const f32x4 (&xr)[PPT][2]) {
#pragma unroll
    for (int j = 0; j < PPT; j++) {
      const int i = tid + NTH * j;
      if (PAIRS % NTH != 0 && i >= PAIRS) continue;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[e] = xr[j][0][e];
        v[4 + e] = xr[j][1][e];
      }
#pragma unroll
      for (int e = 0; e < 8; e++) ssacc[j] = __builtin_fmaf(v[e], v[e], ssacc[j]);
      bf16x8 hv, lv;
      split8(v, hv, lv);
      const int tok = i / 8, g8 = i % 8;  // k group g8 = 4 h + ks
      const int slot = 64 * (g8 & 3) + 32 * (g8 >> 2) + ((tok & 31) ^ g8);
      xs[buf][u][tok >> 5][0][slot] = __builtin_bit_cast(u32x4, hv);
      xs[buf][u][tok >> 5][1][slot] = __builtin_bit_cast(u32x4, lv);
    }
  };

  // One tile per wave: two accumulator sets (even and odd k-steps) halve the chain of
  // dependent products, and every B operand of an iteration is requested before the first
  // product (one LDS wait per iteration). Wider waves have independent tiles to interleave and
  // read each k-step's operands as they go (fewer registers).
  constexpr bool DUAL = RT * NT == 1, UPF = NT == 1;
  f32x16 acc[RT][NT], acc2[1][1];  // acc2: used when DUAL
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[r][n][e] = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; e++) acc2[0][0][e] = 0.0f;

  f32x4 xr[GD][PPT][2];
  u32x4 wr[GD][RT][2 * WL];
#pragma unroll
  for (int d = 0; d < GD; d++) {
    load_w(d, wr[d]);
    load_x(d, xr[d]);
  }
#pragma unroll
  for (int u = 0; u < CPI; u++) {
    store_x(0, u, xr[u]);
    load_x(GD + u, xr[u]);
  }
  lds_barrier();

  // CPI chunks per barrier: chunks c .. c + CPI - 1 multiplied from LDS buffer `buf` while
  // chunks c + CPI .. are split into the other.
  for (uint32_t c0 = 0; c0 < nc; c0 += GD) {
#pragma unroll
    for (int d = 0; d < GD; d += CPI) {
      const uint32_t c = c0 + d;
      const int buf = (d / CPI) & 1;
      u32x4 cur[CPI][RT][2 * WL];
#pragma unroll
      for (int u = 0; u < CPI; u++) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
          for (int v = 0; v < 2 * WL; v++) cur[u][r][v] = wr[d + u][r][v];
        load_w(c + u + GD, wr[d + u]);
      }
      auto read_b = [&](int u, int ks, bf16x8 (&bk)[NT][2]) {
        const int slot = 64 * ks + 32 * h + (c32 ^ (4 * h + ks));
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
          for (int hl = 0; hl < 2; hl++) bk[n][hl] = __builtin_bit_cast(bf16x8, xs[buf][u][n][hl][slot]);
      };
      bf16x8 bx[CPI][UPF ? 4 : 1][NT][2];
      if constexpr (UPF) {
#pragma unroll
        for (int u = 0; u < CPI; u++)
#pragma unroll
          for (int ks = 0; ks < 4; ks++) read_b(u, ks, bx[u][ks]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // The next iteration's X (requested GD - CPI chunks ago) to the other buffer while this
      // iteration's operands arrive, then the chunks GD further requested into its registers:
      // the split's VALU work overlaps the LDS reads' latency, and the products the writes'.
#pragma unroll
      for (int u = 0; u < CPI; u++) {
        const int dn = (d + CPI + u) % GD;
        store_x(buf ^ 1, u, xr[dn]);
        load_x(c + CPI + u + GD, xr[dn]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < CPI; u++)
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
          bf16x8 a[RT];
#pragma unroll
          for (int r = 0; r < RT; r++) {
            if (FMT == SV_FMT_I8) {
              const u32x4 w = cur[u][r][ks >> 1];
              a[r] = i8x8_to_bf(w[2 * (ks & 1)], w[2 * (ks & 1) + 1]);
            } else {
              a[r] = __builtin_bit_cast(bf16x8, cur[u][r][ks]);
            }
          }
          auto products = [&](const bf16x8 (&bk)[NT][2]) {
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
              for (int r = 0; r < RT; r++) {
                f32x16& g = (DUAL && (ks & 1)) ? acc2[0][0] : acc[r][n];
                g = mfma32(a[r], bk[n][0], g);
                g = mfma32(a[r], bk[n][1], g);
              }
          };
          if constexpr (UPF) {
            products(bx[u][ks]);
          } else {
            bf16x8 bk[NT][2];
            read_b(u, ks, bk);
            products(bk);
          }
        }
      lds_barrier();
    }
  }
  if constexpr (DUAL) acc[0][0] += acc2[0][0];
  // Per-row int8 scales: lane (c, h) holds rows 8 j + 4 h + i of each tile.
  if (FMT == SV_FMT_I8) {
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint16_t* sp4 = p.scales + row0 + 32 * r + 8 * j + 4 * h;  // any alignment
        const float s0 = bf(ldg_u16(sp4)), s1 = bf(ldg_u16(sp4 + 1)), s2 = bf(ldg_u16(sp4 + 2)),
                    s3 = bf(ldg_u16(sp4 + 3));
#pragma unroll
        for (int n = 0; n < NT; n++) {
          acc[r][n][4 * j + 0] *= s0;
          acc[r][n][4 * j + 1] *= s1;
          acc[r][n][4 * j + 2] *= s2;
          acc[r][n][4 * j + 3] *= s3;
        }
      }
  }
#pragma unroll
  for (int j = 0; j < PPT; j++) {
    const int i = tid + NTH * j;
    if (i < PAIRS) ssp[i / 8][i % 8] = ssacc[j];
  }
  __syncthreads();
  float ssn[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) {
    const uint32_t tl = 32 * n + c32;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += ssp[tl][e];
    ssn[n] = ss;
  }

  if (S > 1) {
    // [cell][split][NTH threads][RT NT 4] f32x4 and [cell][split][BN] sums of squares; the
    // last split of the cell adds them in split order.
    const uint32_t cell = rblk * n_tblk + tblk;
    const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(p.part), srs = coherent_rsrc(p.ssp);
    constexpr uint32_t PER = NTH * RT * NT * 64;
    const uint32_t pb = (cell * S) * PER;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int n = 0; n < NT; n++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          store_wt4(prs, pb + sp * PER + (((r * NT + n) * 4 + j) * NTH + tid) * 16,
                    f32x4{acc[r][n][4 * j], acc[r][n][4 * j + 1], acc[r][n][4 * j + 2], acc[r][n][4 * j + 3]});
    for (int tt = tid; tt < BN; tt += NTH)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ssp[tt][0] + ssp[tt][1] + ssp[tt][2] + ssp[tt][3] +
                                                            ssp[tt][4] + ssp[tt][5] + ssp[tt][6] + ssp[tt][7]),
                                            srs, ((cell * S + sp) * BN + tt) * 4, 0, SV_CPOL_SC1);
    if (!arrive_last(p.counters + cell, S, &last_flag)) return;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int n = 0; n < NT; n++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[r][n][e] = 0.0f;
#pragma unroll
    for (int n = 0; n < NT; n++) ssn[n] = 0.0f;
    for (uint32_t s2 = 0; s2 < S; s2++) {
#pragma unroll
      for (int r = 0; r < RT; r++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const f32x4 v = load_wt4(prs, pb + s2 * PER + (((r * NT + n) * 4 + j) * NTH + tid) * 16);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[r][n][4 * j + i] += v[i];
          }
#pragma unroll
      for (int n = 0; n < NT; n++)
        ssn[n] += __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(srs, ((cell * S + s2) * BN + 32 * n + c32) * 4, 0, SV_CPOL_SC1));
    }
  }

  // Epilogue: each (tile, token tile, j) is a group of 4 rows for token t0 + 32 n + c.
#pragma unroll
  for (int n = 0; n < NT; n++) {
    const uint32_t t = t0 + 32 * n + c32;
    if (t >= p.n) continue;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        f32x4 col[1] = {f32x4{acc[r][n][4 * j], acc[r][n][4 * j + 1], acc[r][n][4 * j + 2], acc[r][n][4 * j + 3]}};
        gemm_epilogue<1>(p, col, row0 + 32 * r + 8 * j + 4 * h, 0, t, ssn[n],
                         rblk == 0 && wv == 0 && r == 0 && j == 0 && h == 0);
      }
  }
}

// GEMM launch shape: RTW row tiles per wave (BM = 64 RTW), NT token tiles (BN = 16 NT),
// S k splits.
struct GemmCfg {
  int rtw, nt, s, d;  // d: chunks in flight (2, 4 or 8)
  int mf = 16;        // MFMA tile: 16 (mm_gemm, tiles of 16) or 32 (mm_gemm32, tiles of 32)
  int nw = 4;         // waves per workgroup (mm_gemm32: 4 or 8)
  int cpi = 1;        // mm_gemm32: chunks per barrier (1, or 2 with 4 chunks in flight)
  uint32_t bm() const { return (uint32_t)(nw * mf * rtw); }
  uint32_t bn() const { return (uint32_t)mf * nt; }
  uint32_t acc_bytes() const { return (uint32_t)(rtw * nt) * mf * mf / 16; }  // per thread
};
GemmTune g_gemm_tune;  // all zero: the built-in choice
int g_gemm_order = -1;  // tests: force a work order (-1: the modelled choice)

// Built-in choice, from measurements on MI355X at 40, 160 and 512 rows (qkv, o, gate_up, down
// int8, the bf16 head): int8 runs 32-token blocks (NT = 2) with two row tiles per wave and two
// k splits, four when that leaves fewer than 256 workgroups; bf16 (twice the weight bytes per
// row) runs the token block with the fewest padded tokens among NT = 3 and 5 and the fewest
// k splits (up to 8) that give 256 workgroups. Either way one row tile per wave when the
// splits alone cannot reach 256 workgroups, and with int8 scale groups shorter than k. At 384
// rows and more, matrices with 512 blocks of 256 rows x 64 tokens run those (four row tiles
// per wave, two chunks in flight), unsplit.
static GemmCfg pick_gemm(uint32_t fmt, bool grouped, uint32_t n, uint32_t m, uint32_t k) {
  if (g_gemm_tune.rtw)
    return GemmCfg{g_gemm_tune.rtw, g_gemm_tune.nt, std::max(1, g_gemm_tune.s), g_gemm_tune.d ? g_gemm_tune.d : 4,
                   g_gemm_tune.mf ? g_gemm_tune.mf : 16, g_gemm_tune.nw ? g_gemm_tune.nw : 4,
                   g_gemm_tune.cpi ? g_gemm_tune.cpi : 1};
  const uint32_t nch = k / GKC;
  // int8 at 96 rows and more: 32 x 32 tiles, 8 waves, four chunks in flight; one 32-row tile
  // per wave (256-row blocks) and 32 tokens, or for the widest matrices two tiles per wave
  // (512-row blocks) and 64 tokens from 384 rows; the fewest k splits that give 160
  // workgroups. Measured on MI355X against the 16-wide shapes below at 160 and 512 rows: qkv
  // 14.0 -> 13.4 and 23.6 -> 20.1 us, o 13.9 -> 13.1 and 20.5 -> 17.8, down 26.5 -> 23.9 and
  // 51.6 -> 44.1, gate_up 34.2 -> 31.6 and 73.5 -> 67.6.
  const bool wide = m >= 8192 && m % 512 == 0;
  if (fmt == SV_FMT_I8 && !grouped && n >= 96 && m % 256 == 0) {
    GemmCfg c{wide ? 2 : 1, wide && n >= 384 ? 2 : 1, 1, 4, 32, 8, 1};
    const uint32_t cells = m / c.bm() * ((n + c.bn() - 1) / c.bn());
    for (int s : {1, 2, 4, 8})
      if (nch % s == 0 && nch / s >= 4) {
        c.s = s;
        if (cells * s >= 160) break;
      }
    return c;
  }
  // Wide matrices at many rows: 256-row x 64-token blocks halve the operand traffic through
  // L2 (weights re-read per token block, X per row block) where they still fill the device.
  // Two chunks in flight (not four) keep that shape at two waves per SIMD.
  if (!grouped && n >= 384 && m % 256 == 0 && (uint64_t)(m / 256) * ((n + 63) / 64) >= 384) return GemmCfg{4, 4, 1, 2};
  // Weights too large to stay cached between token blocks (the 131 MB bf16 head) are re-read
  // from HBM by every token block: below that shape, the fewest token blocks (48 or 80 tokens,
  // whichever pads n least), no k splits, four chunks in flight for 48 tokens (measured with
  // the weights cold: 20-25 % faster than 32-token blocks or split k at 40 and 160 rows).
  if (!grouped && (uint64_t)m * k * (fmt == SV_FMT_I8 ? 1 : 2) > (96ull << 20)) {
    GemmCfg c{m % 128 ? 1 : 2, 3, 1, 4};
    uint32_t best = ~0u;
    for (int nt : {3, 5}) {
      const uint32_t pad = (n + 16 * nt - 1) / (16 * nt) * 16 * nt - n;
      if (pad < best || (pad == best && nt == 5)) best = pad, c.nt = nt;
    }
    if (c.nt == 5) c.d = 2;
    return c;
  }
  // Below that, 256-row x 32-token blocks without splits where they still make 512 workgroups
  // (measured on gate_up at 256 and 320 rows: 3-25% faster than 128-row blocks in splits).
  if (!grouped && m % 256 == 0 && (uint64_t)(m / 256) * ((n + 31) / 32) >= 512) return GemmCfg{4, 2, 1, 2};
  // Long reductions (k of 8192 or more): the largest row block (256, 128, 64 rows) that makes
  // 512 workgroups with four or eight k splits (measured on the down projection at 24-512
  // rows: up to 30 % faster than fewer splits or smaller blocks).
  if (nch >= 128) {
    for (int rtw : {4, 2, 1}) {
      if (rtw > 1 && (grouped || m % (64u * rtw))) continue;
      const uint32_t cells = m / (64u * rtw) * ((n + 31) / 32);
      for (int s : {4, 8})
        if (nch % s == 0 && cells * s >= 512) return GemmCfg{rtw, 2, s, 2};
    }
    for (int s : {8, 4, 2})
      if (nch % s == 0) return GemmCfg{1, 2, s, 2};
    return GemmCfg{1, 2, 1, 2};
  }
  // Otherwise 128-row x 32-token blocks, two chunks in flight (more waves per SIMD; measured as
  // fast or faster than 48- and 80-token blocks with four in flight for bf16 too).
  GemmCfg c{2, 2, 1, 2};
  const int s_first = 2, s_last = 4;
  if (grouped || m % 128) c.rtw = 1;
  const uint32_t n_tblk = (n + 16 * c.nt - 1) / (16 * c.nt);
  for (;;) {
    const uint32_t cells = m / (64 * c.rtw) * n_tblk;
    c.s = 1;
    for (int s = s_first; s <= s_last; s *= 2)
      if (nch % s == 0 && nch / s >= 4) {
        c.s = s;
        if (cells * s >= 256) break;
      }
    if (cells * c.s >= 256 || c.rtw == 1) break;
    c.rtw = 1;
  }
  return c;
}

static size_t gemm_ws_layout(uint32_t n, uint32_t m, const GemmCfg& c, size_t* ss_off, size_t* part_off) {
  if (c.s <= 1) return 0;
  const size_t n_tblk = (n + c.bn() - 1) / c.bn(), cells = m / c.bm() * n_tblk;
  size_t off = COUNTER_SLOTS * 4;
  *ss_off = off;
  off += (cells * c.s * c.bn() * 4 + 255) / 256 * 256;
  *part_off = off;
  off += cells * c.s * 64 * c.nw * c.acc_bytes();
  return off;
}

static bool gemm_shape_ok(uint32_t m, uint32_t k, const GemmCfg& c) {
  const bool nt_ok = c.nt == 2 || c.nt == 3 || c.nt == 4 || c.nt == 5 || c.nt == 8;
  // 32-wide tiles: one or two row tiles per wave, one to three token tiles.
  if (c.mf == 32)
    return (c.rtw == 1 || c.rtw == 2) && c.nt >= 1 && c.nt <= 3 && (c.d == 2 || c.d == 4) && (c.nw == 4 || c.nw == 8) &&
           (c.cpi == 1 || (c.cpi == 2 && c.d == 4)) &&
           c.s >= 1 && c.s <= 64 &&
           m % c.bm() == 0 && (k / GKC) % c.s == 0;
  return c.mf == 16 && c.nw == 4 && nt_ok && (c.rtw == 1 || c.rtw == 2 || (c.rtw == 4 && c.nt <= 5)) && (c.d == 2 || c.d == 4 || c.d == 8) && c.s >= 1 && c.s <= 64 && m % (64 * c.rtw) == 0 &&
         (k / GKC) % c.s == 0;
}

template <int FMT, int RTW, int NT, bool GR>
static void gemm_launch_one(hipStream_t stream, const MMParams& p, int d, uint32_t nwg, uint32_t n_tblk) {
  if (d == 8 && NT <= 3) launch((mm_gemm<FMT, RTW, NT, GR, (NT <= 3 ? 8 : 4)>), dim3(nwg), dim3(256), 0, stream, p, n_tblk);
  else if (d == 2) launch((mm_gemm<FMT, RTW, NT, GR, 2>), dim3(nwg), dim3(256), 0, stream, p, n_tblk);
  else launch((mm_gemm<FMT, RTW, NT, GR, 4>), dim3(nwg), dim3(256), 0, stream, p, n_tblk);
}

template <int FMT, int RTW, bool GR>
static void gemm_dispatch_nt(hipStream_t stream, const MMParams& p, int nt, int d, uint32_t nwg, uint32_t n_tblk) {
  switch (nt) {
    case 2: gemm_launch_one<FMT, RTW, 2, GR>(stream, p, d, nwg, n_tblk); break;
    case 3: gemm_launch_one<FMT, RTW, 3, GR>(stream, p, d, nwg, n_tblk); break;
    case 4: gemm_launch_one<FMT, RTW, 4, GR>(stream, p, d, nwg, n_tblk); break;
    case 5: gemm_launch_one<FMT, RTW, 5, GR>(stream, p, d, nwg, n_tblk); break;
    default: gemm_launch_one<FMT, RTW, (RTW == 4 ? 5 : 8), GR>(stream, p, d, nwg, n_tblk); break;
  }
}

static void gemm_dispatch32(hipStream_t stream, uint32_t fmt, const GemmCfg& c, const MMParams& p, uint32_t nwg,
                            uint32_t n_tblk) {
#define SV_G32W(F, R, N, D, C)                                                                 \
  (c.nw == 8 ? launch((mm_gemm32<F, R, N, D, 8, C>), dim3(nwg), dim3(512), 0, stream, p, n_tblk) \
             : launch((mm_gemm32<F, R, N, D, 4, C>), dim3(nwg), dim3(256), 0, stream, p, n_tblk))
#define SV_G32(F, R, N, D) (D == 4 && c.cpi == 2 ? SV_G32W(F, R, N, 4, 2) : SV_G32W(F, R, N, D, 1))
#define SV_G32_NT(F, R, D) (c.nt == 1 ? SV_G32(F, R, 1, D) : c.nt == 2 ? SV_G32(F, R, 2, D) : SV_G32(F, R, 3, D))
#define SV_G32_D(F, R) (c.d == 4 ? SV_G32_NT(F, R, 4) : SV_G32_NT(F, R, 2))
  if (fmt == SV_FMT_I8) c.rtw == 2 ? SV_G32_D(SV_FMT_I8, 2) : SV_G32_D(SV_FMT_I8, 1);
  else c.rtw == 2 ? SV_G32_D(SV_FMT_BF16, 2) : SV_G32_D(SV_FMT_BF16, 1);
#undef SV_G32_D
#undef SV_G32_NT
#undef SV_G32
#undef SV_G32W
}

// The work order for nrb row blocks x S splits x n_tblk token blocks with the least HBM traffic
// under a model where each XCD's L2 holds what its contiguous range of items shares: every
// distinct (row block, split) costs its weights once per XCD, every distinct (token block,
// split) its activations once per XCD. The activations are fp32, so at many rows and long k
// (down at 512 rows: 16.8 MB of weights, 16.8 MB of activations) dealing whole row blocks to
// an XCD re-reads the activations from every XCD.
static uint32_t gemm_order_model(uint32_t nrb, uint32_t n_tblk, uint32_t S, double w_bytes, double x_bytes) {
  const uint32_t nwg = nrb * n_tblk * S;
  uint32_t best = 0;
  double best_t = 0;
  std::vector<uint64_t> ws, xs;
  for (uint32_t g : {0u, 1u, 2u, 4u, 8u, 16u}) {
    if (g && (nrb % g || g > nrb)) continue;
    double t = 0;
    for (uint32_t x = 0; x < 8; x++) {
      const uint32_t q = nwg / 8, a = x * q + std::min(x, nwg % 8), cnt = q + (x < nwg % 8 ? 1 : 0);
      ws.clear();
      xs.clear();
      for (uint32_t i = a; i < a + cnt; i++) {
        uint32_t tb, sp, rb;
        if (g == 0) {
          tb = i % n_tblk, sp = (i / n_tblk) % S, rb = i / (n_tblk * S);
        } else {
          const uint32_t per_sp = nrb * n_tblk, per_grp = g * n_tblk, rem = i % per_sp, r2 = rem % per_grp;
          sp = i / per_sp, tb = r2 / g, rb = (rem / per_grp) * g + r2 % g;
        }
        ws.push_back((uint64_t)sp << 32 | rb);
        xs.push_back((uint64_t)sp << 32 | tb);
      }
      std::sort(ws.begin(), ws.end());
      std::sort(xs.begin(), xs.end());
      t += (double)(std::unique(ws.begin(), ws.end()) - ws.begin()) * w_bytes +
           (double)(std::unique(xs.begin(), xs.end()) - xs.begin()) * x_bytes;
    }
    if (g == 0 || t < best_t * 0.97) best_t = t, best = g;  // another order only where it saves 3 %
  }
  return best;
}

// The model sorts every item of the launch for each order: memoised per launch shape, since
// plans that are rebuilt per step (prompt chunks) launch the same few shapes many times.
static uint32_t gemm_order(uint32_t nrb, uint32_t n_tblk, uint32_t S, double w_bytes, double x_bytes) {
  struct Key {
    uint32_t nrb, n_tblk, S;
    double w, x;
    bool operator==(const Key& o) const {
      return nrb == o.nrb && n_tblk == o.n_tblk && S == o.S && w == o.w && x == o.x;
    }
  };
  static std::mutex mu;
  static std::vector<std::pair<Key, uint32_t>> memo;
  const Key key{nrb, n_tblk, S, w_bytes, x_bytes};
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& e : memo)
    if (e.first == key) return e.second;
  const uint32_t g = gemm_order_model(nrb, n_tblk, S, w_bytes, x_bytes);
  if (memo.size() < 4096) memo.push_back({key, g});
  return g;
}

static sv_status gemm_launch(hipStream_t stream, uint32_t fmt, MMParams& p, void* ws, size_t ws_bytes) {
  const bool grouped = fmt == SV_FMT_I8 && !p.per_row;
  const GemmCfg c = pick_gemm(fmt, grouped, p.n, p.m, p.k);
  if (!gemm_shape_ok(p.m, p.k, c) || (grouped && (c.rtw != 1 || c.mf != 16)))
    return fail(SV_ERR_ARG, "matmul (gemm): launch shape rtw %d, nt %d, splits %d for m %u, k %u", c.rtw, c.nt, c.s,
                p.m, p.k);
  if ((size_t)p.m * p.k * (fmt == SV_FMT_I8 ? 1 : 2) >= (1ull << 31) || (size_t)p.n * p.k * 4 >= (1ull << 31))
    return fail(SV_ERR_UNSUPPORTED, "matmul (gemm): operands of 2 GiB or more");
  const uint32_t n_tblk = (p.n + c.bn() - 1) / c.bn(), rb = p.m / c.bm();
  size_t ss_off = 0, part_off = 0;
  const size_t need = gemm_ws_layout(p.n, p.m, c, &ss_off, &part_off);
  if (need) {
    if ((size_t)rb * n_tblk > COUNTER_SLOTS) return fail(SV_ERR_UNSUPPORTED, "matmul (gemm): cells exceed the counters");
    if (!ws || ws_bytes < need)
      return fail(SV_ERR_ARG, "matmul: workspace %zu < %zu bytes (sv_matmul_workspace_bytes)", ws_bytes, need);
    p.counters = (uint32_t*)ws;
    p.ssp = (float*)((char*)ws + ss_off);
    p.part = (float*)((char*)ws + part_off);
  }
  p.splits = c.s;
  const uint32_t nwg = rb * n_tblk * c.s;
  {
    const double kk = (double)p.k / c.s;
    p.order = g_gemm_order >= 0 ? (uint32_t)g_gemm_order
                                : gemm_order(rb, n_tblk, c.s, c.bm() * kk * (fmt == SV_FMT_I8 ? 1 : 2), c.bn() * kk * 4);
    if (p.order && rb % p.order) p.order = 0;
  }
  if (c.mf == 32) {
    gemm_dispatch32(stream, fmt, c, p, nwg, n_tblk);
  } else if (fmt == SV_FMT_I8) {
    if (grouped) gemm_dispatch_nt<SV_FMT_I8, 1, true>(stream, p, c.nt, c.d, nwg, n_tblk);
    else if (c.rtw == 4) gemm_dispatch_nt<SV_FMT_I8, 4, false>(stream, p, c.nt, c.d, nwg, n_tblk);
    else if (c.rtw == 2) gemm_dispatch_nt<SV_FMT_I8, 2, false>(stream, p, c.nt, c.d, nwg, n_tblk);
    else gemm_dispatch_nt<SV_FMT_I8, 1, false>(stream, p, c.nt, c.d, nwg, n_tblk);
  } else {
    if (c.rtw == 4) gemm_dispatch_nt<SV_FMT_BF16, 4, false>(stream, p, c.nt, c.d, nwg, n_tblk);
    else if (c.rtw == 2) gemm_dispatch_nt<SV_FMT_BF16, 2, false>(stream, p, c.nt, c.d, nwg, n_tblk);
    else gemm_dispatch_nt<SV_FMT_BF16, 1, false>(stream, p, c.nt, c.d, nwg, n_tblk);
  }
  return check_launch("matmul (gemm)");
}

// Skinny launch shape: RT row tiles per workgroup, W waves, S splits of k.
struct SkinnyCfg {
  int rt, w, s;
};
SkinnyTune g_skinny_tune;  // all zero: the built-in choice
int g_mm_variant = -1;

// Beyond 16 rows the GEMM path runs; the skinny kernel (one workgroup per 16-token group,
// weights re-read from L2 per group) can still be forced for more rows (tests).

static bool use_skinny(uint32_t n, uint32_t m, uint32_t k) {
  if (m % 16 || k % KC) return false;
  if (g_skinny_tune.path) return g_skinny_tune.path != 2;
  return n <= 16;
}

// Measured on MI355X at 1-5 rows: about 128 KB of weights per workgroup and at least 256
// workgroups; with more token groups the X chunk dominates a wave's loads, so as many row
// tiles as possible share it. 8 waves for int8, 4 for bf16 (twice the registers per row);
// k splits only when the tiles give too few workgroups and every wave still has two chunks.
static SkinnyCfg pick_skinny(uint32_t fmt, uint32_t n, uint32_t m, uint32_t k) {
  const uint32_t tiles = m / 16, chunks = k / KC, esz = fmt == SV_FMT_I8 ? 1 : 2, tg = (n + 15) / 16;
  const size_t max_wg_bytes = tg > 1 ? ~(size_t)0 : (128u << 10);
  SkinnyCfg c{1, fmt == SV_FMT_I8 ? 8 : 4, 1};
  for (int rt = 4; rt > 1; rt /= 2)
    if (tiles % rt == 0 && (tg > 1 || tiles / rt >= 256) && (size_t)rt * 16 * k * esz <= max_wg_bytes) {
      c.rt = rt;
      break;
    }
  while (c.s < 8 && (tiles / c.rt) * c.s * tg < 256 && (uint32_t)(c.w * c.s * 2) <= chunks) c.s *= 2;
  if (g_skinny_tune.rt) {
    c.rt = g_skinny_tune.rt;
    c.w = g_skinny_tune.w;
    c.s = g_skinny_tune.s;
  }
  return c;
}

// Workspace layout (skinny, S > 1): the counters region at the front, then per cell (row
// group, token group) the sums of squares [cells][S][16] and partials [cells][S][RT][64][4]
// fp32.

static size_t skinny_ws_layout(uint32_t n, uint32_t m, const SkinnyCfg& c, size_t* ss_off, size_t* part_off) {
  if (c.s <= 1) return 0;
  const size_t tg = (n + 15) / 16, cells = (size_t)m / (16 * c.rt) * tg;
  size_t off = COUNTER_SLOTS * 4;
  *ss_off = off;
  off += (cells * c.s * 16 * 4 + 255) / 256 * 256;
  *part_off = off;
  off += cells * c.s * c.rt * 256 * 4;
  return off;
}

// One-shot launch shapes for 1-16 rows (RT row tiles, W waves, NCH chunks per wave, k split
// in S = 1 or 2), int8 and bf16; NT = 4, 5, 8 or 16 token slots. Measured on MI355X: the
// kernel is bound by its compute units' instruction work (weight conversion, X split, MFMA)
// as much as by memory, so it wants every compute unit busy (>= 256 workgroups), and a
// wave's weights <= 64 registers.
struct StreamCfg {
  int rt, w, nch, s;  // row tiles, waves, chunks per wave, k splits
};
constexpr StreamCfg STREAM_SHAPES[] = {{1, 8, 1}, {2, 8, 1}, {4, 8, 1}, {1, 8, 2}, {2, 8, 2},
                                       {1, 8, 4}, {1, 4, 1}, {1, 4, 2}};

static bool stream_shape_ok(uint32_t fmt, const StreamCfg& c, uint32_t n) {
  const int wv = fmt == SV_FMT_I8 ? 1 : 2;
  if (c.rt * c.nch * wv > 4) return false;  // weights <= 64 registers a wave
  const size_t lds = (size_t)c.w * n * 2 * XROW * 2 + (size_t)c.w * c.rt * 1024 + (size_t)c.w * 16 * 4;
  return lds <= 160 * 1024;
}

static bool stream_listed(const StreamCfg& c) {
  for (const StreamCfg& sh : STREAM_SHAPES)
    if (sh.rt == c.rt && sh.w == c.w && sh.nch == c.nch) return c.s == 1 || c.s == 2;
  return false;
}

// Built-in choice: at least 256 workgroups where the matrix allows (more row tiles per
// workgroup while that holds, else k split in two when each split keeps eight waves busy).
static bool pick_stream(uint32_t fmt, uint32_t n, uint32_t m, uint32_t k, StreamCfg* out) {
  const uint32_t tiles = m / 16, chunks = k / KC;
  if (g_skinny_tune.path == 3 && g_skinny_tune.rt) {
    *out = StreamCfg{g_skinny_tune.rt, g_skinny_tune.w, g_skinny_tune.s, std::max(1, g_skinny_tune.splits)};
    return tiles % out->rt == 0 && (uint32_t)(out->w * out->nch * out->s) >= chunks &&
           (uint32_t)(out->w * out->nch * (out->s - 1)) < chunks && stream_listed(*out) && stream_shape_ok(fmt, *out, n);
  }
  for (int s : {1, 2}) {
    if (s == 2 && chunks < 16) break;
    int nch = 1;
    while ((uint32_t)(nch * 8 * s) < chunks) nch *= 2;
    if (nch > 4) continue;
    for (int rt : {4, 2, 1}) {
      const StreamCfg c{rt, 8, nch, s};
      if (tiles % rt || (rt > 1 && tiles / rt < 256) || !stream_shape_ok(fmt, c, n) || !stream_listed(c)) continue;
      if (s == 1 && tiles / rt < 256 && chunks >= 16) break;  // too few workgroups: try two splits
      *out = c;
      return true;
    }
  }
  return false;
}

size_t matmul_ws_bytes(uint32_t n, uint32_t m, uint32_t k) {
  matmul_init();
  if (n == 0) return 0;
  if (!use_skinny(n, m, k)) {
    size_t a, b, need = 0;
    if (k % GKC) return 0;
    for (uint32_t fmt : {(uint32_t)SV_FMT_I8, (uint32_t)SV_FMT_BF16})
      for (bool grouped : {false, true})
        if (fmt == SV_FMT_I8 || !grouped) need = std::max(need, gemm_ws_layout(n, m, pick_gemm(fmt, grouped, n, m, k), &a, &b));
    return need;
  }
  size_t a, b;
  size_t need = std::max(skinny_ws_layout(n, m, pick_skinny(SV_FMT_I8, n, m, k), &a, &b),
                         skinny_ws_layout(n, m, pick_skinny(SV_FMT_BF16, n, m, k), &a, &b));
  StreamCfg c;
  for (uint32_t fmt : {(uint32_t)SV_FMT_I8, (uint32_t)SV_FMT_BF16})
    if (n <= 16 && m % 16 == 0 && pick_stream(fmt, n, m, k, &c))
      need = std::max(need, skinny_ws_layout(n, m, SkinnyCfg{c.rt, c.w, c.s}, &a, &b));
  return need;
}

template <int FMT, int RT, int W, int NCH, int NT>
static void stream_attr() {
  const size_t static_lds = (size_t)W * RT * 1024 + (size_t)W * NT * 4;
  const size_t dyn = std::min((size_t)W * NT * 2 * XROW * 2, (size_t)160 * 1024 - static_lds);
  (void)hipFuncSetAttribute((const void*)mm_stream<FMT, RT, W, NCH, NT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)dyn);
}

template <int FMT, int RT, int W, int NCH, int NT>
static void stream_launch_one(hipStream_t stream, const MMParams& p, uint32_t grid) {
  launch((mm_stream<FMT, RT, W, NCH, NT>), dim3(grid), dim3(64 * W), (size_t)W * p.n * 2 * XROW * 2, stream, p);
}

// Calls F<FMT, RT, W, NCH, NT> for the launch shape c (false if it is not built).
#define SV_STREAM_SHAPES(FMT, NT, CALL)                                        \
  SV_ST(FMT, NT, 1, 8, 1, CALL) SV_ST(FMT, NT, 2, 8, 1, CALL) SV_ST(FMT, NT, 1, 8, 2, CALL) \
  SV_ST(FMT, NT, 1, 4, 1, CALL) SV_ST(FMT, NT, 1, 4, 2, CALL)                                \
  if (FMT != SV_FMT_BF16) { SV_ST(FMT, NT, 4, 8, 1, CALL) SV_ST(FMT, NT, 2, 8, 2, CALL) SV_ST(FMT, NT, 1, 8, 4, CALL) }

template <int FMT, int NT>
static bool stream_dispatch(hipStream_t stream, const MMParams& p, const StreamCfg& c, uint32_t grid) {
#define SV_ST(F, N_, R, W_, C_, CALL)                       \
  if (c.rt == R && c.w == W_ && c.nch == C_) {              \
    stream_launch_one<F, R, W_, C_, N_>(stream, p, grid);   \
    return true;                                            \
  }
  SV_STREAM_SHAPES(FMT, NT, 0)
#undef SV_ST
  return false;
}

// Token slots NT: 4, 5 (the configs' k = 4 drafts + 1), 8 or 16.
template <int FMT>
static bool stream_dispatch_n(hipStream_t stream, const MMParams& p, const StreamCfg& c, uint32_t grid) {
  if (p.n <= 4) return stream_dispatch<FMT, 4>(stream, p, c, grid);
  if (p.n == 5) return stream_dispatch<FMT, 5>(stream, p, c, grid);
  if (p.n <= 8) return stream_dispatch<FMT, 8>(stream, p, c, grid);
  return stream_dispatch<FMT, 16>(stream, p, c, grid);
}

void matmul_init() {
  static bool done = false;
  if (done) return;
  done = true;
#define SV_ST(F, N_, R, W_, C_, CALL) stream_attr<F, R, W_, C_, N_>();
  SV_STREAM_SHAPES(SV_FMT_I8, 4, 0)
  SV_STREAM_SHAPES(SV_FMT_I8, 5, 0)
  SV_STREAM_SHAPES(SV_FMT_I8, 8, 0)
  SV_STREAM_SHAPES(SV_FMT_I8, 16, 0)
  SV_STREAM_SHAPES(SV_FMT_BF16, 4, 0)
  SV_STREAM_SHAPES(SV_FMT_BF16, 5, 0)
  SV_STREAM_SHAPES(SV_FMT_BF16, 8, 0)
  SV_STREAM_SHAPES(SV_FMT_BF16, 16, 0)
  SV_STREAM_SHAPES(FMT_I8_G64, 4, 0)
  SV_STREAM_SHAPES(FMT_I8_G64, 5, 0)
  SV_STREAM_SHAPES(FMT_I8_G64, 8, 0)
  SV_STREAM_SHAPES(FMT_I8_G64, 16, 0)
#undef SV_ST
  (void)hipGetLastError();  // an attribute the device refused is found by the launch check
}

sv_status matmul_launch(hipStream_t stream, const sv_matrix* w, const float* x, const uint32_t* x_rows, float* y,
                        const float* base, float* aux, const sv_mat_args* a, void* ws, size_t ws_bytes) {
  matmul_init();
  if (!w || !a || !x || !y || !w->d_w) return fail(SV_ERR_ARG, "matmul: null pointer");
  if (a->k != w->k || a->m != w->m) return fail(SV_ERR_ARG, "matmul: args (m %u, k %u) != matrix (%u, %u)", a->m, a->k, w->m, w->k);
  if (a->n == 0) return SV_OK;
  bool per_row = true;
  const uint32_t fmt = w->format & ~(uint32_t)SV_FMT_TILED;
  const bool tiled = (w->format & SV_FMT_TILED) != 0;
  if (tiled && (a->m % 16 || a->k % 64)) return fail(SV_ERR_ARG, "matmul: tiled layout needs m %% 16 == 0, k %% 64 == 0");
  if (fmt == SV_FMT_I8) {
    if (!w->d_scales) return fail(SV_ERR_ARG, "matmul: int8 without scales");
    per_row = a->gshift >= 32 || (1ull << a->gshift) >= a->k;
  } else if (fmt != SV_FMT_BF16) {
    return fail(SV_ERR_ARG, "matmul: format %u", w->format);
  }
  // The skinny kernels take int8 scales per row or per group of >= 256 (one per k chunk); the
  // one-shot kernel also groups of 64 and 128 (FMT_I8_G64).
  const bool small_groups = fmt == SV_FMT_I8 && !per_row && (a->gshift == 6 || a->gshift == 7);
  StreamCfg sc{};
  const bool stream_ok = a->n <= 16 && a->m % 16 == 0 && a->k % KC == 0 && g_skinny_tune.path != 1 &&
                         (per_row || a->gshift >= 6) && pick_stream(fmt, a->n, a->m, a->k, &sc);
  const bool skinny = use_skinny(a->n, a->m, a->k) && (per_row || a->gshift >= 8 || (small_groups && stream_ok));
  if (!skinny && (a->k % GKC != 0 || a->m % 64 != 0))
    return fail(SV_ERR_ARG, "matmul: k %u and m %u must be multiples of %d and 16 (or of %d and 64)", a->k, a->m, KC,
                GKC);
  if (a->epi == SV_EPI_SWIGLU && a->m % 2) return fail(SV_ERR_ARG, "matmul: swiglu needs even m");
  if (a->epi < SV_EPI_NORM || a->epi > SV_EPI_RAW) return fail(SV_ERR_ARG, "matmul: epilogue %u", a->epi);
  if (a->epi == SV_EPI_RESID && !base) return fail(SV_ERR_ARG, "matmul: resid needs base");
  if ((a->flags & (SV_FLAG_WRITE_INV | SV_FLAG_WRITE_RAW)) && !aux) return fail(SV_ERR_ARG, "matmul: flags need aux");
  if (!per_row) {
    const uint32_t min_shift = skinny && !stream_ok ? 8 : 6;
    if (a->gshift < min_shift || a->k % (1u << a->gshift) != 0)
      return fail(SV_ERR_UNSUPPORTED, "matmul: int8 group 2^%u: groups of at least %u (or one per row) are built",
                  a->gshift, 1u << min_shift);
  }
  MMParams p;
  p.w = (const uint8_t*)w->d_w;
  p.scales = w->d_scales;
  p.x = x;
  p.x_rows = x_rows;
  p.y = y;
  p.base = base;
  p.aux = aux;
  p.n = a->n;
  p.k = a->k;
  p.m = a->m;
  p.epi = a->epi;
  p.flags = a->flags;
  p.vocab_real = a->vocab_real;
  p.gshift = per_row ? 31 : a->gshift;
  p.per_row = per_row;
  p.tiled = tiled;
  p.scale = a->scale;
  p.ra = a->ra;
  p.rb = a->rb;
  p.chunks = a->k / KC;
  p.counters = nullptr;
  p.part = p.ssp = nullptr;
  if (!skinny) {
    g_mm_variant = 2;
    return gemm_launch(stream, fmt, p, ws, ws_bytes);
  }
  if (g_skinny_tune.path == 3 && !stream_ok) return fail(SV_ERR_ARG, "matmul: forced one-shot shape does not fit");
  if (stream_ok) {
    const uint32_t grid = a->m / 16 / sc.rt * sc.s;
    p.splits = sc.s;
    p.tgroups = 1;
    if (sc.s > 1) {
      size_t ss_off = 0, part_off = 0;
      const size_t need = skinny_ws_layout(a->n, a->m, SkinnyCfg{sc.rt, sc.w, sc.s}, &ss_off, &part_off);
      if (a->m / (16 * sc.rt) > COUNTER_SLOTS) return fail(SV_ERR_UNSUPPORTED, "matmul: row groups exceed the counters");
      if (!ws || ws_bytes < need)
        return fail(SV_ERR_ARG, "matmul: workspace %zu < %zu bytes (sv_matmul_workspace_bytes)", ws_bytes, need);
      p.counters = (uint32_t*)ws;
      p.ssp = (float*)((char*)ws + ss_off);
      p.part = (float*)((char*)ws + part_off);
    }
    const bool ok = fmt == SV_FMT_BF16 ? stream_dispatch_n<SV_FMT_BF16>(stream, p, sc, grid)
                    : small_groups     ? stream_dispatch_n<FMT_I8_G64>(stream, p, sc, grid)
                                       : stream_dispatch_n<SV_FMT_I8>(stream, p, sc, grid);
    if (!ok) return fail(SV_ERR_ARG, "matmul: launch shape rt %d, waves %d, chunks %d", sc.rt, sc.w, sc.nch);
    g_mm_variant = 3;
    return check_launch("matmul");
  }
  const SkinnyCfg cfg = pick_skinny(fmt, a->n, a->m, a->k);
  const int rt = cfg.rt, waves = cfg.w;
  if ((a->m / 16) % rt != 0 || (rt != 1 && rt != 2 && rt != 4) || (waves != 4 && waves != 8 && waves != 16) || (waves == 16 && rt == 4) ||
      cfg.s < 1)
    return fail(SV_ERR_ARG, "matmul: launch shape rt %d, waves %d, splits %d", rt, waves, cfg.s);
  size_t ss_off = 0, part_off = 0;
  const size_t need = skinny_ws_layout(a->n, a->m, cfg, &ss_off, &part_off);
  if (need && (size_t)a->m / (16 * rt) * ((a->n + 15) / 16) > COUNTER_SLOTS)
    return fail(SV_ERR_UNSUPPORTED, "matmul: %u row groups x token groups exceed the hand-off counters", a->m / (16 * rt));
  if (need > 0 && (!ws || ws_bytes < need))
    return fail(SV_ERR_ARG, "matmul: workspace %zu < %zu bytes (sv_matmul_workspace_bytes)", ws_bytes, need);
  p.counters = need ? (uint32_t*)ws : nullptr;
  p.ssp = need ? (float*)((char*)ws + ss_off) : nullptr;
  p.part = need ? (float*)((char*)ws + part_off) : nullptr;
  g_mm_variant = 1;
  p.splits = cfg.s;
  p.tgroups = (a->n + 15) / 16;
  dim3 grid(a->m / 16 / rt * cfg.s * p.tgroups);
#define SV_MM(F, R, W) launch((mm_skinny<F, R, W>), grid, dim3(64 * W), 0, stream, p)
#define SV_MM_W(F, R)                          \
  if (waves == 16 && R <= 2) SV_MM(F, R, 16);  \
  else if (waves == 8) SV_MM(F, R, 8);         \
  else SV_MM(F, R, 4)
  if (fmt == SV_FMT_I8) {
    if (rt == 4) { SV_MM_W(SV_FMT_I8, 4); }
    else if (rt == 2) { SV_MM_W(SV_FMT_I8, 2); }
    else { SV_MM_W(SV_FMT_I8, 1); }
  } else {
    if (rt == 4) { SV_MM_W(SV_FMT_BF16, 4); }
    else if (rt == 2) { SV_MM_W(SV_FMT_BF16, 2); }
    else { SV_MM_W(SV_FMT_BF16, 1); }
  }
#undef SV_MM_W
#undef SV_MM
  return check_launch("matmul");
}

sv_status pack_matrix(hipStream_t stream, const sv_matrix* src, void* dst, sv_matrix* out) {
  if (!src || !dst || !out || !src->d_w) return fail(SV_ERR_ARG, "pack_matrix: null pointer");
  const uint32_t fmt = src->format;
  if (fmt != SV_FMT_I8 && fmt != SV_FMT_BF16) return fail(SV_ERR_ARG, "pack_matrix: format %u (row-major int8 or bf16)", fmt);
  if (src->m % 16 || src->k % 64 || src->m == 0) return fail(SV_ERR_ARG, "pack_matrix: m %u, k %u (need m %% 16 == 0, k %% 64 == 0)", src->m, src->k);
  const uint32_t esz = fmt == SV_FMT_I8 ? 1 : 2;
  const size_t words = (size_t)src->m * src->k * esz / 16;
  launch(pack_tiled_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream, (const uint8_t*)src->d_w,
         (uint8_t*)dst, src->k, esz, words);
  *out = *src;
  out->d_w = dst;
  out->format = fmt | SV_FMT_TILED;
  return check_launch("pack_matrix");
}

}  // namespace sv
