// layers.hip — every decoder layer of a 1-8 row verify step in one persistent launch (the
// reference's encode_forward layer loop, engine/src/encode.rs:99-190, at the GEMV regime of
// Matmul::for_tokens, encode.rs:33-44).
//
// Why: at 1-8 rows a layer is six dependent launches (qkv, attention, split merge, o, gate_up,
// down) of a few microseconds each, and every launch starts its weight (or K/V) stream only
// when it starts: each kernel pays a first round trip and streams its bytes on the critical
// path. A grid barrier costs about what a kernel boundary does (measured on MI355X: 1.7-1.9
// us against 1.6 us), so fusing only pays if the next phase's independent bytes are already
// in flight when its inputs are ready. This kernel does exactly that.
//
// Two sets of workgroups, one workgroup of each per compute unit (2 x CUs workgroups of 4
// waves, all resident: the host checks the occupancy), take the phases in turns:
//   set A: qkv(l) [then requests gate_up(l)'s weights] ... gate_up(l) [then qkv(l+1)'s]
//   set B: attention(l) [then o(l)'s weights], merge(l), o(l) [then down(l)'s weights],
//          down(l) [then the cached K/V of attention(l+1)]
// so every phase's weights, or its cached keys and values, are requested one or more phases
// before its inputs exist, by waves that have no stores left to wait for. Loads return to a
// wave in issue order and s_waitcnt vmcnt counts loads and stores together, so the set that
// signals a phase's completion never has prefetched loads outstanding behind its stores: a
// workgroup arrives (vmcnt(0), then its counter) before it requests anything for a later phase.
//
// Hand-offs (the memory-ordering contract): a phase's outputs are stored with the sc1 cache
// policy (global/buffer stores at device scope: written through this XCD's L2 to memory, the
// level every XCD's loads reach); each producing workgroup waits until those stores have
// completed (s_waitcnt vmcnt(0) in every thread, then s_barrier), then adds 1 to one of 16
// counters of the phase with a relaxed device-scope atomic. Consumers poll the 16 counters
// with device-scope (sc1) loads until they sum to epoch x producers. Every activation buffer
// is a slice of its own per layer that nothing in this launch reads before its phase's
// barrier, and the launch starts with the L2 invalidated (kernel boundary), so no L2 can hold
// a stale copy of a line a consumer reads: consumers use plain loads, which share each XCD's
// L2 among its workgroups. No fence instruction is used (a device-scope release or acquire on
// gfx950 writes back or invalidates the XCD's whole L2).
//
// Counters are never reset: embed increments an epoch word before each launch, and phase
// targets are epoch x producers. Every poll is bounded; a workgroup that waits too long sets
// the abort word (every poll reads it) and the whole grid drains without hanging; the host
// reports it and clears the counters.
#include "layers.h"

namespace sv {

constexpr int PL_SUB = 16;         // counters per phase (producers spread over them)
constexpr uint32_t PL_SPIN = 1u << 18;  // polls before a wait gives up (~0.3 s)
constexpr int PL_KC = 256;         // k per chunk
constexpr int PL_XROW = PL_KC + 8;  // bf16 per LDS row of one token's hi or lo
constexpr int PL_NBW = 3;           // cached-key batches per wave: splits of at most 384 keys

__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Probe stamps (null in production): the clock at a point of (set, workgroup, layer, phase):
// 0 after the phase's wait, 1 after its arrival, 2.. inside the phase.
__device__ __forceinline__ uint64_t* pl_rec(const LayersParams& p, uint32_t set, uint32_t j, uint32_t l, uint32_t ph) {
  return p.stamps ? p.stamps + ((((size_t)set * 256 + j) * p.n_layers + l) * 6 + ph) * 8 : nullptr;
}
__device__ __forceinline__ void st_at(uint64_t* rec, int which) {
  if (rec && threadIdx.x == 0) rec[which] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void pl_stamp(const LayersParams& p, uint32_t set, uint32_t j, uint32_t l, uint32_t ph,
                                         uint32_t which) {
  if (p.stamps && threadIdx.x == 0)
    p.stamps[((((size_t)set * 256 + j) * p.n_layers + l) * 6 + ph) * 8 + which] = __builtin_amdgcn_s_memrealtime();
}

// ------------------------------------------------------------------------------- sync
// Arrive at phase `ph`: every thread's stores have completed, then one counter increment.
__device__ __forceinline__ void pl_arrive(const LayersParams& p, uint32_t ph, uint32_t j) {
  wait_mem();
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(p.sync + ((size_t)ph * PL_SUB + j % PL_SUB) * 64, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_sched_barrier(0);
}

// Wait until phase ph's counters sum to `target`. Wave 0 polls (lanes 0..15 one counter each,
// lane 16 the abort word); false if the grid aborted.
__device__ __forceinline__ bool pl_wait(const LayersParams& p, uint32_t ph, uint32_t target, uint32_t* sflag) {
  __builtin_amdgcn_sched_barrier(0);
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const uint32_t* src = lane < PL_SUB ? p.sync + ((size_t)ph * PL_SUB + lane) * 64 : p.abort;
    uint32_t it = 0;
    bool ok = true;
    while (true) {
      const uint32_t v = lane <= PL_SUB ? ld_dev(src) : 0u;
      const uint32_t ab = __builtin_amdgcn_readlane(v, PL_SUB);
      uint32_t s = lane < PL_SUB ? v : 0u;
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      if (ab) {
        ok = false;
        break;
      }
      if (__builtin_amdgcn_readfirstlane(s) >= target) break;
      if (++it > p.spin) {
        if (lane == 0) __hip_atomic_fetch_or(p.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = false;
        break;
      }
    }
    if (lane == 0) *sflag = ok ? 1u : 0u;
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  return *sflag != 0;
}

// ----------------------------------------------------------------------------- matmul
// One workgroup: RT row tiles of 16 output rows over all of k; wave wv takes the NCH chunks of
// 256 k numbered wv NCH ... Weights (tiled int8, per-row bf16 scales) are held in registers
// from the prefetch on; X is read when the phase starts, split into bf16 hi + lo in the wave's
// LDS rows, and multiplied on v_mfma_f32_16x16x32_bf16 as in the one-shot matmul (matmul.hip).
template <int RT, int NCH>
struct MmW {
  u32x4 w[NCH][RT][4];
  uint32_t rs0, rs1;  // wave wv < RT: the scales of rows 16 (tile0 + wv) + 4 q + 0..3
};

// Every load is issued whether or not the workgroup has the tiles (`on` false: offsets past the
// buffer's range, answered with zeros without a memory access), so the registers are always
// written here and no earlier value stays live around the layer loop.
template <int RT, int NCH>
__device__ __forceinline__ void mm_prefetch(MmW<RT, NCH>& W, const uint8_t* w, const uint16_t* s, uint32_t k,
                                            uint32_t tile0, bool on, int wv, int lane) {
  const __amdgpu_buffer_rsrc_t wrs = coherent_rsrc(w);
  const uint32_t tile_bytes = 16 * k, vo = 16u * lane + (on ? 0u : 0x80000000u);
  if (!on) tile0 = 0;
#pragma unroll
  for (int j = 0; j < NCH; j++)
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
      for (int b = 0; b < 4; b++)
        W.w[j][rt][b] = buf_ld16_nt(wrs, vo, (tile0 + rt) * tile_bytes + ((wv * NCH + j) * 4 + b) * 1024);
  const uint16_t* sp = s + (size_t)(tile0 + (wv < RT ? wv : 0)) * 16 + 4 * (lane >> 4);
  W.rs0 = ldg_u16(sp) | ((uint32_t)ldg_u16(sp + 1) << 16);
  W.rs1 = ldg_u16(sp + 2) | ((uint32_t)ldg_u16(sp + 3) << 16);
}

enum { PL_NORM = 0, PL_RESID = 1, PL_SWIGLU = 2 };

// y = epilogue(W . X) for the workgroup's tiles. x: [n][k] (plain loads: its slice was written
// before the phase's barrier), y written through (sc1). NORM: y = acc scale / rms(x);
// RESID: y = ra base + rb scale acc; SWIGLU: y[row / 2] = silu(g) u of the norm-scaled pair.
template <int RT, int NCH, int NT, int EPI>
__device__ __forceinline__ void mm_compute(const MmW<RT, NCH>& W, const float* x, uint32_t n, uint32_t k, uint32_t m,
                                           uint32_t tile0, float* y, const float* base, float scale, float ra,
                                           float rb, char* smem, int wv, int lane, uint64_t* rec = nullptr) {
  constexpr int XD = NCH < 2 ? NCH : 2;  // X chunks in flight per wave
  uint16_t* xs = (uint16_t*)smem + (size_t)wv * NT * 2 * PL_XROW;
  f32x4* red = (f32x4*)(smem + 4 * NT * 2 * PL_XROW * 2);  // [4][RT][64]
  float* ssred = (float*)(red + 4 * RT * 64);              // [4][NT]
  const int t = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t xrs = coherent_rsrc(x);
  const uint32_t xv = 16u * lane, xv_none = 0x80000000u + xv;
  const uint32_t c0 = wv * NCH;
  auto load_x = [&](f32x4 (&dst)[NT], uint32_t c) {
#pragma unroll
    for (int i = 0; i < NT; i++)
      dst[i] = __builtin_bit_cast(f32x4, buf_ld16(xrs, (uint32_t)i < n ? xv : xv_none, ((uint32_t)i * k + c * PL_KC) * 4));
  };
  f32x4 xr[XD][NT];
#pragma unroll
  for (int d = 0; d < XD; d++) load_x(xr[d], c0 + d);
  f32x4 bpre = f32x4{0.f, 0.f, 0.f, 0.f};
  if (EPI == PL_RESID && wv < RT && (uint32_t)t < n)
    bpre = *(const f32x4*)(base + (size_t)t * m + (tile0 + wv) * 16 + 4 * q);

  f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ssl[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) ssl[i] = 0.0f;
  const bf16x8 zero = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    __builtin_amdgcn_sched_barrier(0);
    f32x4 (&xc)[NT] = xr[j % XD];
    if (j == 0) st_at(rec, 2);
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
      *(u32x2*)(xs + (2 * i) * PL_XROW + 4 * lane) = u32x2{s01[0], s23[0]};
      *(u32x2*)(xs + (2 * i + 1) * PL_XROW + 4 * lane) = u32x2{s01[1], s23[1]};
    }
    if (j + XD < NCH) load_x(xr[j % XD], c0 + j + XD);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int b = 0; b < 4; b++) {
      bf16x8 xh0 = zero, xh1 = zero, xl0 = zero, xl1 = zero;
      if ((uint32_t)t < n) {
        const uint16_t* hp = xs + (2 * t) * PL_XROW + 64 * b + 16 * q;
        xh0 = *(const bf16x8*)hp;
        xh1 = *(const bf16x8*)(hp + 8);
        xl0 = *(const bf16x8*)(hp + PL_XROW);
        xl1 = *(const bf16x8*)(hp + PL_XROW + 8);
      }
#pragma unroll
      for (int rt = 0; rt < RT; rt++) {
        const u32x4 w = W.w[j][rt][b];
        const bf16x8 a0 = i8x8_to_bf(w[0], w[1]), a1 = i8x8_to_bf(w[2], w[3]);
        acc[rt] = mfma16(a0, xh0, acc[rt]);
        acc[rt] = mfma16(a0, xl0, acc[rt]);
        acc[rt] = mfma16(a1, xh1, acc[rt]);
        acc[rt] = mfma16(a1, xl1, acc[rt]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  st_at(rec, 3);
  constexpr bool NEED_SS = EPI != PL_RESID;
  if (NEED_SS) {
#pragma unroll
    for (int i = 0; i < NT; i++) {
      float v = ssl[i];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      if (lane == 0) ssred[wv * NT + i] = v;
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; rt++) red[(wv * RT + rt) * 64 + lane] = acc[rt];
  __syncthreads();
  st_at(rec, 4);
  if (wv < RT && (uint32_t)t < n) {
    f32x4 tile = red[(0 * RT + wv) * 64 + lane];
#pragma unroll
    for (int w2 = 1; w2 < 4; w2++) tile += red[(w2 * RT + wv) * 64 + lane];
    tile[0] *= bf(W.rs0 & 0xffffu);
    tile[1] *= bf(W.rs0 >> 16);
    tile[2] *= bf(W.rs1 & 0xffffu);
    tile[3] *= bf(W.rs1 >> 16);
    const uint32_t row0 = (tile0 + wv) * 16 + 4 * q;
    const __amdgpu_buffer_rsrc_t yrs = coherent_rsrc(y);
    if (EPI == PL_RESID) {
      const f32x4 sv = tile * scale;
      store_wt4(yrs, ((uint32_t)t * m + row0) * 4, bpre * ra + sv * rb);
    } else {
      float ss = ((ssred[0 * NT + t] + ssred[1 * NT + t]) + ssred[2 * NT + t]) + ssred[3 * NT + t];
      const float inv = 1.0f / __builtin_sqrtf(ss / (float)k + SV_RMS_EPS);
      if (EPI == PL_NORM) {
        store_wt4(yrs, ((uint32_t)t * m + row0) * 4, tile * (inv * scale));
      } else {
        const float sc = inv * scale;
        const float g0 = tile[0] * sc, u0 = tile[1] * sc, g1 = tile[2] * sc, u1 = tile[3] * sc;
        const float o0 = g0 * (1.0f / (1.0f + __expf(-g0))) * u0, o1 = g1 * (1.0f / (1.0f + __expf(-g1))) * u1;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(o0), __float_as_uint(o1)}, yrs,
                                              ((uint32_t)t * (m / 2) + row0 / 2) * 4, 0, SV_CPOL_SC1);
      }
    }
  }
  st_at(rec, 5);
  __syncthreads();  // the LDS is the next phase's
}

// -------------------------------------------------------------------------- attention
// Work item i of a layer's attention: run r, kv head g, split s (the all-batches-in-flight
// variant of attn_verify_kernel: splits of at most 512 cached keys, the run's new keys in a
// split of their own after its cached ones). The cached keys' page-table words and batches are
// requested by prefetch (the cache below the run's first position does not change during the
// step); the queries, new keys and products run once the layer's qkv phase is done.
struct AttnItem {
  KvBatchT<64> bt[PL_NBW];
  uint32_t r, g, s, t0, T, seq, p0, nsplit;
  uint32_t active, newest;
};

// Every batch slot is written (slots the item does not need read nothing: offsets past the
// range), so no earlier batch stays live around the layer loop. item >= items: inactive.
__device__ __forceinline__ void attn_prefetch(const AttnParams& p, const uint32_t* inl, uint32_t item, uint32_t items,
                                              AttnItem& a, int wv, int lane) {
  a.active = item < items;
  if (!a.active) item = 0;
  const uint32_t per_run = p.NKV * p.max_splits;
  a.r = item / per_run;
  a.g = (item / p.max_splits) % p.NKV;
  a.s = item % p.max_splits;
  a.t0 = inl[3 * a.r];
  a.T = inl[3 * a.r + 1];
  a.seq = inl[3 * a.r + 2];
  const uint32_t kbeg = a.s * p.split;
  const uint32_t tpos = kbeg + 32 * (wv + 4 * (lane >> 1)) + 16 * (lane & 1);
  const uint32_t pword = p.page_table[(size_t)a.seq * p.max_pages + min(tpos >> p.page_shift, p.max_pages - 1)];
  a.p0 = p.meta[2 * a.t0 + 1];
  a.nsplit = (a.p0 + p.split - 1) / p.split + 1;
  a.newest = a.s == a.nsplit - 1;
  if (a.s >= a.nsplit) a.active = 0;
  const bool load = a.active && !a.newest && a.nsplit <= p.max_splits;
  const uint32_t nbw_full = load && p.split / 32 > (uint32_t)wv ? (p.split / 32 - wv + 3) / 4 : 0u;
  size_t tile_off = 0;
  if ((uint32_t)lane < 2 * nbw_full) {
    const uint32_t page = min(pword, p.n_pages - 1);
    tile_off = ((((size_t)p.layer * p.n_pages + page) * p.NKV + a.g) << p.page_shift) * 64 +
               (size_t)(tpos & ((1u << p.page_shift) - 1u)) * 64;
  }
#pragma unroll
  for (int i = 0; i < PL_NBW; i++) {
    const size_t toffs[2] = {readlane64(tile_off, 2 * i), readlane64(tile_off, 2 * i + 1)};
    load_batch_tiles_t<64>(p, toffs, a.bt[i], lane, (uint32_t)i < nbw_full ? 0u : 0x80000000u);
  }
}

template <int NCT>
__device__ __forceinline__ void attn_compute(const AttnParams& p, AttnItem& a, char* smem, int tid,
                                             uint64_t* rec = nullptr) {
  constexpr int D = 64, KST = 2, VE = 4, COLS = 16 * NCT;
  if (!a.active) return;
  const int lane = tid & 63, wv = tid >> 6, c16 = lane & 15, q = lane >> 4;
  float* ored = (float*)smem;                 // [4][COLS][D], the V stages at its front
  float* lred = ored + 4 * COLS * D;          // [4][COLS]
  uint16_t* nk = (uint16_t*)(lred + 4 * COLS);  // [SV_MAX_RUN][D]
  uint16_t* nv = nk + SV_MAX_RUN * D;
  uint32_t* svis = (uint32_t*)(nv + SV_MAX_RUN * D);
  uint16_t* stage = (uint16_t*)((char*)smem + (size_t)wv * stage_bytes<D>());
  const uint32_t t0 = a.t0, T = a.T, g = a.g, s = a.s, p0 = a.p0, ncols = T * p.G;
  if (a.nsplit > p.max_splits) {
    // too few splits for this context (the plan's budget is exceeded): NaN, never a partial
    if (s == 0) {
      const __amdgpu_buffer_rsrc_t ors = coherent_rsrc(p.out);
      for (uint32_t idx = tid; idx < ncols * D; idx += 256) {
        const uint32_t col = idx / D, i = col / p.G, h = g * p.G + col % p.G;
        __builtin_amdgcn_raw_buffer_store_b32(0x7fc00000u, ors, (((t0 + i) * p.NQ + h) * D + idx % D) * 4, 0, SV_CPOL_SC1);
      }
    }
    return;
  }
  if (rec) {
    wait_mem();
    if (tid == 0) rec[7] = __builtin_amdgcn_s_memrealtime();
  }
  // queries (rope words by token: the step's rows), visibility words
  QRaw<D, NCT> qr;
  float2 cs[NCT][KST][4];
  const __amdgpu_buffer_rsrc_t rrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.rope_rows), 0, p.rope_on ? 0x7fffffff : 0, 0x00020000);
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    const uint32_t c = min(16u * ct + c16, ncols - 1), i = c / p.G, h = g * p.G + c % p.G, t = t0 + i;
    const size_t qo = (size_t)t * p.W + h * D + 8 * q;
#pragma unroll
    for (int ks = 0; ks < KST; ks++) {
      const f32x4 x0 = *(const f32x4*)(p.qkv + qo + 32 * ks), x1 = *(const f32x4*)(p.qkv + qo + 32 * ks + 4);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        qr.v[ct][ks][e] = x0[e];
        qr.v[ct][ks][4 + e] = x1[e];
      }
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        const uint32_t jp = 16 * ks + 4 * q + jj;
        const bool on = p.rope_on && 32 * ks + 8 * q < 64;
        const uint32_t off = (t * SV_ROPE_PAIRS + jp) * 8 + (on ? 0u : 0x80000000u);
        cs[ct][ks][jj] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rrs, off, 0, 0));
      }
    }
  }
  const uint32_t visw = p.vis[t0 + min((uint32_t)tid, T - 1)];
  if ((uint32_t)tid < T) svis[tid] = visw;
  if (rec && tid == 0) {
    // probe: when the first query word is in (s_waitcnt on its use)
    float q0 = qr.v[0][0][0];
    asm volatile("" : "+v"(q0));
    rec[6] = __builtin_amdgcn_s_memrealtime() + (q0 == 12345.0f ? 1 : 0);
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ct++)
#pragma unroll
    for (int ks = 0; ks < KST; ks++)
#pragma unroll
      for (int jj = 0; jj < 4; jj++)
        if (!(p.rope_on && 32 * ks + 8 * q < 64)) cs[ct][ks][jj] = float2{1.0f, 0.0f};
#pragma unroll
  for (int ct = 0; ct < NCT; ct++)
    if (16u * ct + c16 >= ncols)
#pragma unroll
      for (int ks = 0; ks < KST; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) qr.v[ct][ks][e] = 0.0f;
  bf16x8 qh[NCT][KST], ql[NCT][KST];
  qfinish_cs<D, NCT>(p, ncols, qr, cs, qh, ql, lane);
  st_at(rec, 2);

  const bool newest = a.newest != 0;
  const uint32_t kbeg = s * p.split;
  const uint32_t kend = newest ? p0 : min(kbeg + p.split, p0);
  const uint32_t nb = newest ? 0u : (kend - kbeg + 31) / 32;
  if (newest) new_keys<D, false>(p, a.seq, g, t0, T, p0, nk, nv, tid, 256);
  __syncthreads();
  f32x4 O[VE][NCT];
  float lsum[NCT];
  uint32_t clo[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    lsum[ct] = 0.0f;
    clo[ct] = 0u;
#pragma unroll
    for (int dt = 0; dt < VE; dt++) O[dt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (newest) {
    if (wv == 0) {
      KvBatchT<D> nb0;
      load_batch_new_t<D>(nk, nv, p0, p0 + T, p0, nb0, lane);
      compute_batch_t<D, NCT, true>(p, nb0, p0, p0 + T, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo, svis);
    }
  } else {
#pragma unroll
    for (int i = 0; i < PL_NBW; i++) {
      const uint32_t b = wv + 4 * i, kb = kbeg + 32 * b;
      if (b < nb) {
        if (kb + 32 <= kend)
          compute_batch_t<D, NCT, false, true>(p, a.bt[i], kb, kend, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo);
        else
          compute_batch_t<D, NCT, false>(p, a.bt[i], kb, kend, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo);
      }
    }
  }
  st_at(rec, 3);
  __syncthreads();  // every wave's V stage read before the reduction buffer (over it) is written
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    float l = lsum[ct];
    l += __shfl_xor(l, 16, WAVE);
    l += __shfl_xor(l, 32, WAVE);
    const uint32_t col = 16 * ct + c16;
    float* od = ored + ((size_t)wv * COLS + col) * D;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int dt = 0; dt < VE; dt++) od[16 * dt + 4 * q + i] = O[dt][ct][i];
    if (q == 0) lred[wv * COLS + col] = l;
  }
  __syncthreads();
  st_at(rec, 4);
  const size_t rec_i = ((size_t)a.r * p.NKV + g) * p.max_splits + s;
  const uint32_t n4 = ncols * D / 4;
  const __amdgpu_buffer_rsrc_t po = coherent_rsrc(p.part_o + rec_i * p.maxcols * D);
  const uint32_t cs4 = COLS * D / 4;
  for (uint32_t i4 = tid; i4 < n4; i4 += 256) {
    const f32x4* o4 = (const f32x4*)ored;
    store_wt4(po, i4 * 16, ((o4[i4] + o4[cs4 + i4]) + o4[2 * cs4 + i4]) + o4[3 * cs4 + i4]);
  }
  float* pl = p.part_l + rec_i * p.maxcols;
  for (uint32_t idx = tid; idx < ncols; idx += 256)
    store_wt(pl + idx, ((lred[idx] + lred[COLS + idx]) + lred[2 * COLS + idx]) + lred[3 * COLS + idx]);
  st_at(rec, 5);
  __syncthreads();
}

// The split merge (attn_dec_reduce, kernels.metal:1316-1362) as attn_merge_kernel: item
// (run, kv head, z) with P parts of 256 / P float4 outputs each.
__device__ __forceinline__ void attn_merge_item(const AttnParams& p, const uint32_t* inl, uint32_t item, uint32_t P,
                                                uint32_t mz, char* smem,
                                                int tid) {
  constexpr int D = 64;
  f32x4* so = (f32x4*)smem;
  float* sl = (float*)(so + 256);
  const uint32_t G4 = 256 / P, part = tid / G4, gi = tid % G4;
  const uint32_t r = item / (p.NKV * mz), g = (item / mz) % p.NKV, z = item % mz;
  const uint32_t i4 = z * G4 + gi;
  const uint32_t t0 = inl[3 * r], T = inl[3 * r + 1];
  const uint32_t ncols = T * p.G;
  const bool live = 4 * i4 < ncols * D;
  const uint32_t col = live ? (4 * i4) / D : 0u, d = (4 * i4) % D;
  const uint32_t p0 = p.meta[2 * t0 + 1];
  const size_t rec0 = ((size_t)r * p.NKV + g) * p.max_splits;
  const size_t so_stride = (size_t)p.maxcols * D;
  const float* po = p.part_o + rec0 * so_stride + (size_t)col * D + d;
  const float* pl = p.part_l + rec0 * p.maxcols + col;
  const uint32_t nsplit = (p0 + p.split - 1) / p.split + 1;
  f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
  float l = 0.0f;
  for (uint32_t sp = part; sp < p.max_splits; sp += 8 * P) {
    f32x4 ov[8];
    float lv[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const uint32_t x = sp + u * P;
      const bool in = live && x < nsplit && x < p.max_splits;
      ov[u] = in ? *(const f32x4*)(po + x * so_stride) : f32x4{0.f, 0.f, 0.f, 0.f};
      lv[u] = in ? pl[x * p.maxcols] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      o += ov[u];
      l += lv[u];
    }
  }
  if (P > 1) {
    so[tid] = o;
    sl[tid] = l;
    __syncthreads();
    if (part == 0)
      for (uint32_t jj = 1; jj < P; jj++) {
        o += so[jj * G4 + gi];
        l += sl[jj * G4 + gi];
      }
  }
  if (part == 0 && live && nsplit <= p.max_splits) {
    const uint32_t i = col / p.G, h = g * p.G + col % p.G, t = t0 + i;
    store_wt4(coherent_rsrc(p.out), (((t * p.NQ) + h) * D + d) * 4, o / l);
  }
  __syncthreads();
}

// Layer l's attention: the shared parameters with its slices, its cache layer and its rope.
__device__ __forceinline__ AttnParams layer_attn(const LayersParams& p, uint32_t l) {
  AttnParams a = p.ap;
  a.qkv = p.qkv + (size_t)l * p.qkv_stride;
  a.out = p.attn_out + (size_t)l * p.attn_stride;
  a.part_o = p.part + (size_t)l * p.part_stride;
  a.part_l = a.part_o + p.part_l_off;
  a.layer = l;
  a.rope_on = (p.rope_mask >> l) & 1u;
  return a;
}

// ------------------------------------------------------------------------------ kernel
constexpr size_t PL_SMEM = 51200;

// Set A: qkv, then gate_up (its weights requested while attention, merge and o run).
template <int NT>
__device__ __forceinline__ void run_set_a(const LayersParams& p, uint32_t j, uint32_t epoch, char* smem,
                                                   uint32_t* sflag) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t H = p.H, F = p.F, n = p.n, L = p.n_layers;
  const uint32_t tq = p.qkv_m / 16, tgu = 2 * F / 16;
  MmW<1, 2> wq;
  MmW<4, 2> wg;
  mm_prefetch<1, 2>(wq, p.layers[0].w[0], p.layers[0].s[0], H, j, j < tq, wv, lane);
  for (uint32_t l = 0; l < L; l++) {
    const LayerW& lw = p.layers[l];
    if (l > 0 && !pl_wait(p, 6 * (l - 1) + 5, epoch * p.cnt[5], sflag)) return;
    pl_stamp(p, 0, j, l, 0, 0);
    if (j < tq) {
      mm_compute<1, 2, NT, PL_NORM>(wq, p.h + (size_t)l * p.h_stride, n, H, p.qkv_m, j,
                                    p.qkv + (size_t)l * p.qkv_stride, nullptr, lw.qkv_scale, 0.f, 0.f, smem, wv, lane,
                                    pl_rec(p, 0, j, l, 0));
      pl_arrive(p, 6 * l + 0, j);
      pl_stamp(p, 0, j, l, 0, 1);
    }
    mm_prefetch<4, 2>(wg, lw.w[2], lw.s[2], H, 4 * j, 4 * j < tgu, wv, lane);
    if (!pl_wait(p, 6 * l + 3, epoch * p.cnt[3], sflag)) return;
    pl_stamp(p, 0, j, l, 4, 0);
    if (4 * j < tgu) {
      mm_compute<4, 2, NT, PL_SWIGLU>(wg, p.mixed + (size_t)l * p.mixed_stride, n, H, 2 * F, 4 * j,
                                      p.act + (size_t)l * p.act_stride, nullptr, 1.0f, 0.f, 0.f, smem, wv, lane,
                                      pl_rec(p, 0, j, l, 4));
      pl_arrive(p, 6 * l + 4, j);
      pl_stamp(p, 0, j, l, 4, 1);
    }
    const uint32_t ln = l + 1 < L ? l + 1 : l;
    mm_prefetch<1, 2>(wq, p.layers[ln].w[0], p.layers[ln].s[0], H, j, l + 1 < L && j < tq, wv, lane);
  }
}

// Set B: attention (cached K/V requested during down of the layer before, or at entry), the
// split merge, o (weights requested after attention), down (weights requested after o).
template <int NT, int NCT>
__device__ __forceinline__ void run_set_b(const LayersParams& p, uint32_t j, uint32_t epoch, char* smem,
                                                   uint32_t* sflag) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t H = p.H, F = p.F, n = p.n, L = p.n_layers;
  const uint32_t th = H / 16;
  AttnItem ai;
  attn_prefetch(layer_attn(p, 0), p.ap.inl, j, p.attn_items, ai, wv, lane);
  for (uint32_t l = 0; l < L; l++) {
    const LayerW& lw = p.layers[l];
    const AttnParams ap = layer_attn(p, l);
    if (!pl_wait(p, 6 * l + 0, epoch * p.cnt[0], sflag)) return;
    pl_stamp(p, 1, j, l, 1, 0);
    if (j < p.attn_items) {
      attn_compute<NCT>(ap, ai, smem, tid, pl_rec(p, 1, j, l, 1));
      pl_arrive(p, 6 * l + 1, j);
      pl_stamp(p, 1, j, l, 1, 1);
    }
    {
      MmW<1, 2> wo;
      mm_prefetch<1, 2>(wo, lw.w[1], lw.s[1], H, j, j < th, wv, lane);
      if (!pl_wait(p, 6 * l + 1, epoch * p.cnt[1], sflag)) return;
      pl_stamp(p, 1, j, l, 2, 0);
      if (j < p.merge_items) {
        attn_merge_item(ap, p.ap.inl, j, p.merge_P, p.merge_z, smem, tid);
        pl_arrive(p, 6 * l + 2, j);
        pl_stamp(p, 1, j, l, 2, 1);
      }
      if (!pl_wait(p, 6 * l + 2, epoch * p.cnt[2], sflag)) return;
      pl_stamp(p, 1, j, l, 3, 0);
      if (j < th) {
        mm_compute<1, 2, NT, PL_RESID>(wo, p.attn_out + (size_t)l * p.attn_stride, n, H, H, j,
                                       p.mixed + (size_t)l * p.mixed_stride, p.h + (size_t)l * p.h_stride, lw.o_scale,
                                       lw.ra_attn, lw.rb_attn, smem, wv, lane, pl_rec(p, 1, j, l, 3));
        pl_arrive(p, 6 * l + 3, j);
        pl_stamp(p, 1, j, l, 3, 1);
      }
    }
    {
      MmW<1, 8> wd;
      mm_prefetch<1, 8>(wd, lw.w[3], lw.s[3], F, j, j < th, wv, lane);
      if (!pl_wait(p, 6 * l + 4, epoch * p.cnt[4], sflag)) return;
      pl_stamp(p, 1, j, l, 5, 0);
      if (j < th) {
        mm_compute<1, 8, NT, PL_RESID>(wd, p.act + (size_t)l * p.act_stride, n, F, H, j,
                                       p.h + (size_t)(l + 1) * p.h_stride, p.mixed + (size_t)l * p.mixed_stride, 1.0f,
                                       lw.ra_mlp, lw.rb_mlp, smem, wv, lane, pl_rec(p, 1, j, l, 5));
        pl_arrive(p, 6 * l + 5, j);
        pl_stamp(p, 1, j, l, 5, 1);
      }
    }
    const uint32_t ln = l + 1 < L ? l + 1 : l;
    attn_prefetch(layer_attn(p, ln), p.ap.inl, l + 1 < L ? j : p.attn_items, p.attn_items, ai, wv, lane);
  }
}

template <int NT, int NCT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void layers_kernel(LayersParams p) {
  __shared__ __attribute__((aligned(16))) char smem[PL_SMEM];
  __shared__ uint32_t sflag;
  // 16 consecutive workgroups: 8 of set A, then 8 of set B (workgroup b runs on XCD b % 8)
  const uint32_t set = (blockIdx.x >> 3) & 1u, j = ((blockIdx.x >> 4) << 3) | (blockIdx.x & 7u);
  const uint32_t epoch = *p.epoch;
  if (set == 0) run_set_a<NT>(p, j, epoch, smem, &sflag);
  else run_set_b<NT, NCT>(p, j, epoch, smem, &sflag);
}

// ------------------------------------------------------------------------------- host
int layers_grid_per_set() {
  static int ns = -1;
  if (ns >= 0) return ns;
  int dev = 0, cus = 0;
  ns = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return ns;
  const void* ks[] = {(const void*)layers_kernel<4, 1>, (const void*)layers_kernel<5, 2>, (const void*)layers_kernel<8, 1>,
                      (const void*)layers_kernel<8, 2>};
  int occ = 1 << 30;
  for (const void* k : ks) {
    int o = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, k, 256, 0) != hipSuccess) return ns;
    occ = std::min(occ, o);
  }
  // two workgroups per compute unit (one of each set), all resident; 16 per group of XCDs
  if (occ >= 2 && cus % 8 == 0) ns = cus;
  return ns;
}

uint32_t g_layers_spin = 0, g_layers_extra = 0;
uint64_t g_layers_stamps = 0;

sv_status layers_launch(hipStream_t stream, const LayersParams& pin, uint32_t max_run) {
  LayersParams p = pin;
  p.spin = g_layers_spin ? g_layers_spin : PL_SPIN;
  p.cnt[1] += g_layers_extra;
  p.stamps = (uint64_t*)g_layers_stamps;
  const int ns = layers_grid_per_set();
  if (ns <= 0) return fail(SV_ERR_UNSUPPORTED, "layers: the persistent kernel does not fit two workgroups per CU");
  if (p.n == 0 || p.n > 8) return fail(SV_ERR_UNSUPPORTED, "layers: %u rows (1-8)", p.n);
  const dim3 grid(2 * ns), block(256);
  const uint32_t cols = max_run * p.G;
  // token slots: the step's rows exactly at 5 (k = 4 chains), else 4 or 8; columns per kv head
  // in tiles of 16
  if (p.n <= 4 && cols <= 16) launch(layers_kernel<4, 1>, grid, block, 0, stream, p);
  else if (p.n == 5 && cols <= 32) launch(layers_kernel<5, 2>, grid, block, 0, stream, p);
  else if (cols <= 16) launch(layers_kernel<8, 1>, grid, block, 0, stream, p);
  else if (cols <= 32) launch(layers_kernel<8, 2>, grid, block, 0, stream, p);
  else return fail(SV_ERR_UNSUPPORTED, "layers: %u columns per kv head", cols);
  return check_launch("layers");
}

}  // namespace sv
