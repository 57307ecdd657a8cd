// matmul.hip — Y = epilogue(W . X) for the verify step's rows (the reference's matmul
// group: engine/src/kernels.metal:151-690, chosen by Matmul::for_tokens, encode.rs:33-44).
//
// Skinny path (n <= 16 rows, the 1-5 row verify step): weight-streaming on the matrix cores.
//   - A workgroup is 4 waves; each wave owns one k-slice of KS = 256 and RT tiles of 16
//     output rows. Its X slice (16 tokens x 256 k, fp32) is loaded once, split into bf16
//     hi + lo (16 significant bits) and kept in registers as the MFMA B operands, while the
//     weights stream past: 16 rows x 16 bytes per lane per 64-k block, one dwordx4 each
//     (int8) or two (bf16), converted to bf16 in registers (int8 is exact in bf16).
//   - Products run on v_mfma_f32_16x16x32_bf16 (fp32 accumulate); hi and lo each take one
//     MFMA, so the fp32 activations lose nothing the tolerance can see, and the VALU only
//     converts weights (about 1.5 ops per byte, where an fp32 FMA GEMV at 5 rows needs 6).
//   - The 4 waves' partial sums meet in LDS in a fixed order. When k needs more than one
//     workgroup (kgroups > 1), each writes its partial to the workspace and the last to
//     arrive (an agent-scope counter per row group) adds them in workgroup order and runs
//     the epilogue, so results do not depend on scheduling.
//   - The sum of squares of X for the folded rms-norm (EPI_NORM/SWIGLU, NORM_IN) rides
//     along the same path.
// int8 weights need one scale per k-slice: groups of 256 or more, or one scale per row
// (per-output-channel, any k).
#include "sv_device.h"
#include "sv_internal.h"

namespace sv {

struct MMParams {
  const uint8_t* w;
  const uint16_t* scales;
  const float* x;
  const uint32_t* x_rows;
  float* y;
  const float* base;
  float* aux;
  float* part;
  uint32_t* counters;
  uint32_t n, k, m, epi, flags, vocab_real, gshift, kgroups, slices, per_row;
  float scale, ra, rb;
};

constexpr int KS = 256;  // k per wave
constexpr int NBLK = KS / 64;

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

template <int FMT, int RT>
__global__ __launch_bounds__(256) void mm_skinny(MMParams p) {
  constexpr int WV = FMT == SV_FMT_I8 ? 1 : 2;  // dwordx4 loads per lane per 64-k block
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int t = lane & 15, q = lane >> 4;
  const uint32_t xg = blockIdx.x, z = blockIdx.y;
  const uint32_t slice = z * 4 + wv;
  const bool active = slice < p.slices;

  __shared__ f32x4 red[4][RT][64];
  __shared__ float ssred[4][16];
  __shared__ uint32_t flag;

  f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ss = 0.0f;

  if (active) {
    const uint32_t kbase = slice * KS;
    // Weights: lane (t, q) takes row t of each tile, bytes 16 q.. of each 64-k block.
    u32x4 wr[RT][NBLK * WV];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      const size_t row = (size_t)(xg * RT + rt) * 16 + t;
      const uint8_t* wp = p.w + (row * p.k + kbase) * (FMT == SV_FMT_I8 ? 1 : 2);
#pragma unroll
      for (int b = 0; b < NBLK; b++)
#pragma unroll
        for (int v = 0; v < WV; v++)
          wr[rt][b * WV + v] = __builtin_nontemporal_load((const u32x4*)(wp + (64 * b + 16 * q) * WV + 16 * v));
    }
    // X: token t, k = kbase + 64 b + 16 q + 0..15, as hi/lo bf16 B operands.
    bf16x8 xh[NBLK][2], xl[NBLK][2];
    if ((uint32_t)t < p.n) {
      const float* xr = p.x + (size_t)(p.x_rows ? p.x_rows[t] : t) * p.k + kbase + 16 * q;
#pragma unroll
      for (int b = 0; b < NBLK; b++) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const f32x4 f = *(const f32x4*)(xr + 64 * b + 4 * j);
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
#pragma unroll
    for (int b = 0; b < NBLK; b++) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++) {
        bf16x8 a0, a1;
        if (FMT == SV_FMT_I8) {
          const u32x4 w = wr[rt][b];
          a0 = i8x8_to_bf(w[0], w[1]);
          a1 = i8x8_to_bf(w[2], w[3]);
        } else {
          a0 = __builtin_bit_cast(bf16x8, wr[rt][2 * b]);
          a1 = __builtin_bit_cast(bf16x8, wr[rt][2 * b + 1]);
        }
        acc[rt] = mfma16(a0, xh[b][0], acc[rt]);
        acc[rt] = mfma16(a0, xl[b][0], acc[rt]);
        acc[rt] = mfma16(a1, xh[b][1], acc[rt]);
        acc[rt] = mfma16(a1, xl[b][1], acc[rt]);
      }
    }
    if (FMT == SV_FMT_I8) {
      const uint32_t ng = p.per_row ? 1u : p.k >> p.gshift, gi = p.per_row ? 0u : kbase >> p.gshift;
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const size_t row = (size_t)(xg * RT + rt) * 16 + 4 * q + i;
          acc[rt][i] *= bf(p.scales[row * ng + gi]);
        }
    }
  }
  ss += __shfl_xor(ss, 16, WAVE);
  ss += __shfl_xor(ss, 32, WAVE);
#pragma unroll
  for (int rt = 0; rt < RT; rt++) red[wv][rt][lane] = acc[rt];
  if (q == 0) ssred[wv][t] = ss;
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) acc[rt] = ((red[0][rt][lane] + red[1][rt][lane]) + red[2][rt][lane]) + red[3][rt][lane];
    ss = ((ssred[0][t] + ssred[1][t]) + ssred[2][t]) + ssred[3][t];
  }
  if (p.kgroups > 1) {
    // Partials: [xg][z][rt][lane] f32x4, then sums of squares [xg][z][16].
    const size_t rec = ((size_t)xg * p.kgroups + z);
    f32x4* pp = (f32x4*)p.part + rec * RT * 64;
    float* ps = p.part + (size_t)gridDim.x * p.kgroups * RT * 256 + rec * 16;
    if (wv == 0) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++) pp[rt * 64 + lane] = acc[rt];
      if (q == 0) ps[t] = ss;
    }
    if (!arrive_last(&p.counters[xg], p.kgroups, &flag)) return;
    if (wv != 0) return;
    const f32x4* p0 = (const f32x4*)p.part + (size_t)xg * p.kgroups * RT * 64;
    const float* s0 = p.part + (size_t)gridDim.x * p.kgroups * RT * 256 + (size_t)xg * p.kgroups * 16;
#pragma unroll
    for (int rt = 0; rt < RT; rt++) acc[rt] = p0[rt * 64 + lane];
    ss = s0[t];
    for (uint32_t zz = 1; zz < p.kgroups; zz++) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++) acc[rt] += p0[(zz * RT + rt) * 64 + lane];
      ss += s0[zz * 16 + t];
    }
  } else if (wv != 0) {
    return;
  }

  // Epilogue (kernels.metal:183-209): lane (t, q) holds rows 4 q + 0..3 of each tile.
  if ((uint32_t)t >= p.n) return;
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)p.k + SV_RMS_EPS);
  if ((p.flags & SV_FLAG_WRITE_INV) && p.epi == SV_EPI_NORM && xg == 0 && q == 0) p.aux[t] = inv;
  const bool norm_in = (p.flags & SV_FLAG_NORM_IN) != 0;
#pragma unroll
  for (int rt = 0; rt < RT; rt++) {
    const uint32_t row0 = (xg * RT + rt) * 16 + 4 * q;
    f32x4 v = acc[rt];
    const size_t o = (size_t)t * p.m + row0;
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
        *(float2*)(p.y + (size_t)t * (p.m / 2) + row0 / 2) = out;
        break;
      }
      default:
        break;
    }
  }
}

// Row tiles per workgroup: the largest of 4, 2, 1 that divides the tiles and still gives at
// least 512 workgroups (2 per CU), else 1.
static int pick_rt(uint32_t tiles, uint32_t kgroups) {
  for (int rt = 4; rt > 1; rt /= 2)
    if (tiles % rt == 0 && (tiles / rt) * kgroups >= 512) return rt;
  return 1;
}

size_t matmul_ws_bytes(uint32_t n, uint32_t m, uint32_t k) {
  (void)n;
  const uint32_t slices = (k + KS - 1) / KS, kgroups = (slices + 3) / 4, tiles = m / 16;
  size_t b = WS_COUNTER_BYTES;                            // counters
  b += (size_t)tiles * kgroups * 256 * 4;                 // partial sums
  b += (size_t)tiles * kgroups * 16 * 4;                  // sums of squares (rt = 1 bound)
  return b;
}

sv_status matmul_launch(hipStream_t stream, const sv_matrix* w, const float* x, const uint32_t* x_rows, float* y,
                        const float* base, float* aux, const sv_mat_args* a, void* ws, size_t ws_bytes) {
  if (!w || !a || !x || !y || !w->d_w) return fail(SV_ERR_ARG, "matmul: null pointer");
  if (a->k != w->k || a->m != w->m) return fail(SV_ERR_ARG, "matmul: args (m %u, k %u) != matrix (%u, %u)", a->m, a->k, w->m, w->k);
  if (a->n == 0) return SV_OK;
  if (a->n > 16) return fail(SV_ERR_UNSUPPORTED, "matmul: %u rows: the skinny path takes at most 16", a->n);
  if (a->k % KS != 0 || a->m % 16 != 0)
    return fail(SV_ERR_ARG, "matmul: k %u must be a multiple of %d and m %u of 16", a->k, KS, a->m);
  if (a->epi == SV_EPI_SWIGLU && a->m % 2) return fail(SV_ERR_ARG, "matmul: swiglu needs even m");
  if (a->epi < SV_EPI_NORM || a->epi > SV_EPI_RAW) return fail(SV_ERR_ARG, "matmul: epilogue %u", a->epi);
  if (a->epi == SV_EPI_RESID && !base) return fail(SV_ERR_ARG, "matmul: resid needs base");
  if ((a->flags & (SV_FLAG_WRITE_INV | SV_FLAG_WRITE_RAW)) && !aux) return fail(SV_ERR_ARG, "matmul: flags need aux");
  bool per_row = true;
  if (w->format == SV_FMT_I8) {
    if (!w->d_scales) return fail(SV_ERR_ARG, "matmul: int8 without scales");
    per_row = a->gshift >= 32 || (1ull << a->gshift) >= a->k;
    if (!per_row && (a->gshift < 8 || a->k % (1u << a->gshift) != 0))
      return fail(SV_ERR_UNSUPPORTED, "matmul: int8 group 2^%u: groups of at least 256 (or one per row) are built",
                  a->gshift);
  } else if (w->format != SV_FMT_BF16) {
    return fail(SV_ERR_ARG, "matmul: format %u", w->format);
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
  p.scale = a->scale;
  p.ra = a->ra;
  p.rb = a->rb;
  p.slices = a->k / KS;
  p.kgroups = (p.slices + 3) / 4;
  const uint32_t tiles = a->m / 16;
  const int rt = pick_rt(tiles, p.kgroups);
  if (p.kgroups > 1) {
    const size_t need = matmul_ws_bytes(a->n, a->m, a->k);
    if (!ws || ws_bytes < need) return fail(SV_ERR_ARG, "matmul: workspace %zu < %zu bytes", ws_bytes, need);
    if ((size_t)tiles * 4 > WS_COUNTER_BYTES) return fail(SV_ERR_UNSUPPORTED, "matmul: %u row tiles", tiles);
    p.counters = (uint32_t*)ws;
    p.part = (float*)((char*)ws + WS_COUNTER_BYTES);
  } else {
    p.counters = nullptr;
    p.part = nullptr;
  }
  dim3 grid(tiles / rt, p.kgroups);
#define SV_MM(F, R) hipLaunchKernelGGL((mm_skinny<F, R>), grid, dim3(256), 0, stream, p)
  if (w->format == SV_FMT_I8) {
    if (rt == 4) SV_MM(SV_FMT_I8, 4);
    else if (rt == 2) SV_MM(SV_FMT_I8, 2);
    else SV_MM(SV_FMT_I8, 1);
  } else {
    if (rt == 4) SV_MM(SV_FMT_BF16, 4);
    else if (rt == 2) SV_MM(SV_FMT_BF16, 2);
    else SV_MM(SV_FMT_BF16, 1);
  }
#undef SV_MM
  return check_launch("matmul");
}

}  // namespace sv
