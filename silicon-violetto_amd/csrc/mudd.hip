// mudd.hip — the MUDD mix of the Limite model (engine/src/kernels.metal:1364-1407, encoded by
// encode.rs:145-160): at its sites, the layer's attention input and residual base are mixes of
// two earlier residual states (the taps) and the current one, with per-token weights from a
// small projection of the current state.
//
// One workgroup of 256 threads (4 waves) per token: rms over the row, the 32 inner dot products
// (wave w takes rows 8 w .. 8 w + 7, lanes stride the row by 4 floats), gelu, the six mix
// weights, then the two output rows. HBM-trivial: dense1 (32 x hidden fp32) is read from L2 by
// every token.
#include "sv_device.h"
#include "sv_internal.h"

namespace sv {

// erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), the method the reference names
// (kernels.metal:30-37): 1 - (a1 t + ... + a5 t^5) e^(-x^2), t = 1 / (1 + p |x|), odd in x.
__device__ __forceinline__ float erf_as(float x) {
  const float a = __builtin_fabsf(x);
  const float t = 1.0f / (1.0f + 0.3275911f * a);
  const float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
  const float y = 1.0f - poly * __builtin_amdgcn_exp2f(-a * a * LOG2E_F);
  return __builtin_copysignf(y, x);
}
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f)); }

__global__ __launch_bounds__(256) void mudd_kernel(const float* __restrict__ cur, const float* __restrict__ tap0,
                                                   const float* __restrict__ tap1, const float* __restrict__ dense1,
                                                   const float* __restrict__ mix, float* __restrict__ out_attn,
                                                   float* __restrict__ out_base, uint32_t H) {
  __shared__ float red[4];
  __shared__ float inner[SV_MUDD_INNER];
  __shared__ float w[6];
  const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float* c = cur + (size_t)t * H;
  float ss = 0.0f;
  for (uint32_t i = 4 * tid; i < H; i += 1024) {
    const f32x4 v = *(const f32x4*)(c + i);
    ss += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wv] = ss;
  __syncthreads();
  const float inv = 1.0f / __builtin_sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)H + SV_RMS_EPS);
  for (uint32_t j = 8 * wv; j < 8 * wv + 8; j++) {
    const float* dr = dense1 + (size_t)j * H;
    float s = 0.0f;
    for (uint32_t i = 4 * lane; i < H; i += 256) {
      const f32x4 v = *(const f32x4*)(c + i), d = *(const f32x4*)(dr + i);
#pragma unroll
      for (int e = 0; e < 4; e++) s = __builtin_fmaf(v[e] * inv, d[e], s);
    }
    s = wave_sum(s);
    if (lane == 0) inner[j] = gelu_erf(s);
  }
  __syncthreads();
  if (tid < 6) {
    const float* row = mix + tid * (SV_MUDD_INNER + 1);
    float s = 0.0f;
    for (uint32_t j = 0; j < SV_MUDD_INNER; j++) s = __builtin_fmaf(inner[j], row[j], s);
    w[tid] = s + row[SV_MUDD_INNER];
  }
  __syncthreads();
  const float w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4], w5 = w[5];
  for (uint32_t i = 4 * tid; i < H; i += 1024) {
    const size_t o = (size_t)t * H + i;
    const f32x4 a = *(const f32x4*)(tap0 + o), b = *(const f32x4*)(tap1 + o), x = *(const f32x4*)(c + i);
    f32x4 ya, yb;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      ya[e] = (w0 * a[e] + w1 * b[e]) + w2 * x[e];
      yb[e] = (w3 * a[e] + w4 * b[e]) + w5 * x[e];
    }
    *(f32x4*)(out_attn + o) = ya;
    *(f32x4*)(out_base + o) = yb;
  }
}

sv_status mudd_launch(hipStream_t stream, const float* cur, const float* tap0, const float* tap1, const float* dense1,
                      const float* mix, float* out_attn, float* out_base, uint32_t n, uint32_t hidden) {
  if (!cur || !tap0 || !tap1 || !dense1 || !mix || !out_attn || !out_base) return fail(SV_ERR_ARG, "mudd: null pointer");
  if (hidden == 0 || hidden % 4) return fail(SV_ERR_ARG, "mudd: hidden %u (a multiple of 4)", hidden);
  if (out_attn == cur || out_base == cur || out_attn == out_base)
    return fail(SV_ERR_ARG, "mudd: outputs must not alias the input or each other");
  if (n == 0) return SV_OK;
  launch(mudd_kernel, dim3(n), dim3(256), 0, stream, cur, tap0, tap1, dense1, mix, out_attn, out_base, hidden);
  return check_launch("mudd");
}

}  // namespace sv
