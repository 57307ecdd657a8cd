// sv_device.h — device-side helpers shared by the HIP kernels of libsv_verify (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sv_verify.h"

namespace sv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;
constexpr float LOG2E_F = 1.44269504088896340736f;

// bf16 bits -> float (kernels.metal:17).
__device__ __forceinline__ float bf(uint32_t u16) { return __uint_as_float(u16 << 16); }
// float -> bf16 bits, round to nearest even on the dropped 16 bits (kernels.metal:23-27).
__device__ __forceinline__ uint32_t to_bf(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// 16x16x32 bf16 matrix-core product, fp32 accumulate: c += a (16x32) * b (32x16).
// Lane l supplies a's row l % 16 and b's column l % 16, each with 8 consecutive k slots
// of k-group l / 16 (the same slots for a and b); lane l receives c's column l % 16,
// rows 4 (l / 16) + 0..3.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Two floats -> their bf16 bits in one word (lo in bits 0-15), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) { return to_bf(lo) | (to_bf(hi) << 16); }

// x = hi + lo, both bf16 (hi = x rounded to bf16, lo = the rest rounded): 16 significant
// bits of x for bf16 matrix-core products.
__device__ __forceinline__ void split_bf(float x, float& hi, float& lo) {
  hi = bf(to_bf(x));
  lo = x - hi;
}

// Two floats -> (hi, lo) bf16 pairs, one word each (element 0 in bits 0-15): hi = x rounded
// to bf16 (RNE), lo = x - hi rounded, the same values as split_bf. gfx950's packed convert
// (v_cvt_pk_bf16_f32) rounds two floats in one instruction: 3 VALU ops per element.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Returns (hi word, lo word).
__device__ __forceinline__ u32x2 split2(float a, float b) {
  const uint32_t hw = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
  const float ra = a - __uint_as_float(hw << 16), rb = b - __uint_as_float(hw & 0xffff0000u);
  return u32x2{hw, __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{ra, rb}), bf16x2))};
}

// Eight floats -> (hi, lo) bf16x8 operands.
__device__ __forceinline__ void split8(const float* v, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const u32x2 w = split2(v[2 * j], v[2 * j + 1]);
    h[j] = w[0];
    l[j] = w[1];
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

// Eight signed bytes (two words) -> bf16x8 (exact: |q| <= 128 fits bf16's 8 bits).
__device__ __forceinline__ bf16x8 i8x8_to_bf(uint32_t w0, uint32_t w1) {
  u32x4 r;
  const uint32_t w[2] = {w0, w1};
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const float f0 = (float)(int8_t)(w[j]), f1 = (float)(int8_t)(w[j] >> 8);
    const float f2 = (float)(int8_t)(w[j] >> 16), f3 = (float)(int8_t)(w[j] >> 24);
    r[2 * j] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    r[2 * j + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8, r);
}

// Loads through pointers the compiler cannot prove global (read from a struct in memory)
// would be FLAT loads, which also count against lgkmcnt: every LDS or scalar wait then
// waits for them too, which defeats loads issued ahead. These cast to the global space.
typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
typedef __attribute__((address_space(1))) const uint16_t g_u16;
__device__ __forceinline__ u32x4 ldg_nt(const void* p) { return __builtin_nontemporal_load((g_u32x4*)p); }
__device__ __forceinline__ uint16_t ldg_u16(const uint16_t* p) { return *(g_u16*)p; }
typedef __attribute__((address_space(1))) const uint32_t g_u32;
__device__ __forceinline__ uint32_t ldg_u32(const void* p) { return *(g_u32*)p; }

// Address of lane `lane`'s 16-byte weight word v (bf16: two per block) of 64-k block kb of
// row tile `tile` (16 rows): lane (t, q) = (lane % 16, lane / 16) takes row 16 tile + t, k
// 64 kb + 16 q .. + 15 (the MFMA A operand). Row-major [m][k], or tiled (SV_FMT_TILED): each
// tile's 64-k blocks stored as one contiguous 1 KB (int8) or 2 KB (bf16) in lane order, so
// a wave's load instruction reads one contiguous kilobyte.
template <int ESZ>
__device__ __forceinline__ const uint8_t* weight_word(const uint8_t* w, uint32_t k, bool tiled, uint32_t tile,
                                                      uint32_t kb, int v, int lane) {
  if (tiled) return w + (size_t)tile * 16 * k * ESZ + ((size_t)kb * ESZ + v) * 1024 + lane * 16;
  return w + ((size_t)(tile * 16 + (lane & 15)) * k + 64 * kb + 16 * (lane >> 4)) * ESZ + 16 * v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}

// The sampler's exp2, bit-identical to the oracle's orc_exp2: Cody-Waite reduction
// x = n + f, n = rint(x); 2^f by the degree-7 Taylor polynomial of e^(f ln 2) in Horner
// form with fused multiply-adds; exact scaling by 2^n; results below 2^-125 flush to 0.
__device__ __forceinline__ float sv_exp2(float x) {
  if (!(x >= -125.0f)) return 0.0f;
  if (x > 127.0f) return __builtin_inff();
  const float nf = __builtin_rintf(x);
  const float f = x - nf;
  float p = 1.525273380405984e-05f;
  p = __builtin_fmaf(p, f, 1.5403530393381608e-04f);
  p = __builtin_fmaf(p, f, 1.3333558146428443e-03f);
  p = __builtin_fmaf(p, f, 9.6181291076284772e-03f);
  p = __builtin_fmaf(p, f, 5.5504108664821580e-02f);
  p = __builtin_fmaf(p, f, 2.4022650695910071e-01f);
  p = __builtin_fmaf(p, f, 6.9314718055994531e-01f);
  p = __builtin_fmaf(p, f, 1.0f);
  const int n = (int)nf;
  return p * __uint_as_float((uint32_t)(n + 127) << 23);
}

// Philox4x32-10 (kernels.metal:1464-1472; Salmon et al. 2011).
__device__ __forceinline__ u32x4 philox(u32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; i++) {
    const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
    c = u32x4{hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// Cross-workgroup hand-off without agent-scope fences (on gfx950 such a fence writes back and
// invalidates the XCD's whole L2, microseconds per workgroup). The producer writes its partial
// with relaxed agent-scope atomic stores (global_store ... sc1: coherent across XCDs, and
// unlike volatile ones not serialised), waits for them (s_waitcnt vmcnt(0) in every thread),
// then counts its arrival with a relaxed agent-scope atomic; the last of `expected`
// arrivals reads every partial with relaxed agent-scope atomic loads (sc1, pipelined) and resets
// the counter for the next launch. All threads of the workgroup must call arrive_last.
//
// The ordering this relies on, instruction by instruction (not the HIP memory model's
// release/acquire, which would emit the L2 write-back and invalidate):
//   - An sc1 (device-scope) store is written through the XCD's L2 to memory, the level every
//     XCD's loads reach; its vmcnt decrement comes when that write is acknowledged, so after
//     s_waitcnt vmcnt(0) the data is visible to any device-scope load.
//   - s_waitcnt vmcnt(0) in every thread, then s_barrier, then the counter atomic from one
//     thread: the atomic issues after every thread's stores were acknowledged (the wait is an
//     instruction the hardware executes in order; the compiler does not move memory operations
//     across it or across the barrier).
//   - The consumer's device-scope atomic returns the count from memory; its partial loads are
//     sc1 loads issued after that return (their addresses do not depend on it, but the branch
//     on the count does: a wave does not issue an instruction after a branch before the branch
//     resolves, and the load is not hoisted above it: it sits behind the workgroup barrier that
//     publishes the count). They miss in any L2 line that could be stale: sc1 loads are served
//     at device scope.
// The split-k matmul and the counted attention merge are tested against the oracle (their
// partials cross XCDs in every launch), which is the regression check of this contract.
__device__ __forceinline__ void store_wt(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_wt(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte versions through a buffer resource (sc1 cache policy: the same agent-scope
// coherence as the relaxed atomics above, four words per access). `base` must be 16-byte
// aligned; byte offsets below 2 GiB.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}
constexpr int SV_CPOL_SC1 = 16;
__device__ __forceinline__ f32x4 load_wt4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, SV_CPOL_SC1));
}
__device__ __forceinline__ void store_wt4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, SV_CPOL_SC1);
}

// Plain and nontemporal 16-byte loads through a buffer resource (coherent_rsrc's descriptor:
// base + [0, 2 GB)): a per-lane offset in one register and a uniform offset in a scalar
// register, so a wave with many loads from one base spends no registers on addresses.
constexpr int SV_CPOL_NT = 2;
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
__device__ __forceinline__ u32x4 buf_ld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, SV_CPOL_NT);
}

// Wait until this thread's memory operations have completed (s_waitcnt vmcnt(0); the gfx9
// encoding leaves expcnt and lgkmcnt at their maxima). A workgroup-scope release fence does
// not wait for global stores (the workgroup shares one CU), so a cross-workgroup hand-off
// needs this before the workgroup barrier that precedes its counter update.
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected, uint32_t* lds_flag) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == expected - 1;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last;
  }
  __syncthreads();
  return *lds_flag != 0;
}

}  // namespace sv
