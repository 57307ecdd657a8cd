// step.hip — the persistent verify step: every layer of the step's forward pass (the
// reference's encode_forward, engine/src/encode.rs:99-126: qkv, attention, o, gate_up, down
// per layer) in ONE launch of one workgroup per CU, for steps of at most 16 rows.
//
// Why: on MI355X a kernel boundary costs ~1.6 us and the first dependent load after one
// another ~1 us (cold L2), so a 16-layer step of six launches per layer spent more time in
// boundaries than in HBM traffic. Here the phases are separated by a grid barrier and each
// phase's weights (or K/V) are requested while the barrier is awaited, into registers, so the weight
// stream overlaps the previous phase and the barrier.
//
//   - Grid barrier without fences: each workgroup waits for its own stores (s_waitcnt
//     vmcnt(0)), then stores the barrier generation to its flag word (coherent sc1 store);
//     workgroup 0 polls all flags, then stores the generation to eight release words that the
//     others poll. Generations continue across launches from an epoch word that workgroup 0
//     advances at the end. Every wait has a wall-clock limit; on expiry the kernel records
//     an error word, later waits end at once, and the launch runs to its end (results are
//     then invalid and the host reports the error: never a hang).
//   - Data written in the launch and read by other workgroups (h, qkv, attn, mixed, act,
//     attention partials) moves through coherent (sc1) stores and loads; weights, the
//     cache's older keys, rope and tables are plain loads.
//   - Matmul phases: workgroup g owns row tiles [g RT, g RT + RT) (RT = tiles / grid rounded
//     up, <= 4) over all of k; wave w takes k chunks w, w + 8, ...; partial sums meet in LDS in
//     wave order; wave j runs the epilogue of tile j. Same products as mm_skinny.
//   - Attention phase: each (run, kv head) pair gets grid / pairs workgroups; 32-key batches
//     are dealt to their waves (the newest batch, with the run's new keys, to the first wave);
//     each workgroup's partial (plain sums, no running max) goes to the workspace and the last
//     workgroup of the pair to arrive merges them in workgroup order.
#include <cstdlib>
#include <cstring>

#include "attn_device.h"
#include "sv_internal.h"

namespace sv {

constexpr int SW = 8;               // waves per workgroup
constexpr int ST = 64 * SW;         // threads per workgroup
constexpr int SPF = 16;             // prefetched weight words (u32x4) per lane
constexpr uint64_t SPIN_TICKS = 20000000;  // barrier wait limit: 0.2 s of the 100 MHz clock

struct StepParams {
  const StepLayerHost* layers;
  uint32_t n_layers, n, H, F;
  AttnParams ap;  // layer-independent attention fields; .layer set per layer
  uint32_t n_runs, pairs, wpp;  // (run, kv head) pairs, workgroups per pair
  // Activations: every (layer, buffer) has its own slice (rows of 16 tokens), written once
  // per launch with write-through stores before any workgroup reads it, so readers use
  // ordinary cached loads (an XCD's L2 can hold no older copy of a fresh slice; the L2s
  // are invalidated between launches). h: the input (embed) and the last layer's output;
  // hs[l - 1]: the residual stream entering layer l.
  float *h, *inv;
  float *hs, *qkv, *attn, *mixed, *act;
  uint32_t qkv_w;  // (NQ + 2 NKV) D
  uint32_t* counters;  // [pairs], zero at rest
  float* part_o;       // [pairs][wpp][maxcols][D]
  float* part_l;       // [pairs][wpp][maxcols]
  uint32_t* bar;       // flags [grid][16], release [8][16], epoch [16], error [16]
  uint64_t* stamps;    // optional (SV_STEP_STAMPS): workgroup 0's clock at each phase end / barrier exit
  uint32_t rc_off;        // byte offset of the RunConsts in LDS
  uint32_t* mm_counters;  // matmul k-split hand-off: counters [row groups] (zero at rest)
  float* mm_part;         // and partials [row groups][S][RT][64][4]
};

// ---------------------------------------------------------------- barrier
__device__ __forceinline__ uint32_t ld_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct BarWords {
  uint32_t* flags;
  uint32_t* rel;
  uint32_t* epoch;
  uint32_t* err;
};
__device__ __forceinline__ BarWords bar_words(uint32_t* bar, uint32_t grid) {
  BarWords b;
  b.flags = bar;
  b.rel = bar + (size_t)grid * 16;
  b.epoch = b.rel + 8 * 16;
  b.err = b.epoch + 16;
  return b;
}

__device__ __forceinline__ void stamp(uint64_t* st, uint32_t i) {
  if (st && blockIdx.x == 0 && threadIdx.x == 0) st[i] = wall_clock64();
}
// Sub-phase stamps (workgroup 0, wave 0) of one layer, for the same developer aid.
#define SUBSTAMP(i) stamp(sub, (i))

// `ahead` issues the next phase's weight (or K/V) loads: after this workgroup's stores have
// completed and it has arrived, so they overlap the wait instead of delaying the arrival
// (s_waitcnt vmcnt counts loads and stores together).
template <typename Ahead>
__device__ __forceinline__ void grid_barrier(const BarWords& b, uint32_t gen, uint64_t* st, uint32_t si, Ahead ahead) {
  stamp(st, 2 * si);
  wait_mem();
  __syncthreads();
  const uint32_t G = gridDim.x, tid = threadIdx.x;
  if (blockIdx.x == 0) {
    ahead();
    const uint64_t t0 = wall_clock64();
    for (uint32_t spins = 0;; spins++) {
      bool mine = true;
      for (uint32_t w = tid + 1; w < G; w += ST) mine = mine && (int)(ld_u32(b.flags + w * 16) - gen) >= 0;
      if (__syncthreads_and(mine)) break;
      if (spins > 64 && (wall_clock64() - t0 > SPIN_TICKS || ld_u32(b.err) != 0)) {
        if (tid == 0) st_u32(b.err, 1u);
        break;
      }
    }
    if (tid < 8) st_u32(b.rel + tid * 16, gen);
  } else {
    if (tid == 0) st_u32(b.flags + blockIdx.x * 16, gen);
    ahead();
    if (tid == 0) {
      const uint32_t* r = b.rel + (blockIdx.x % 8) * 16;
      const uint64_t t0 = wall_clock64();
      for (uint32_t spins = 0; (int)(ld_u32(r) - gen) < 0; spins++) {
        __builtin_amdgcn_s_sleep(1);
        if (spins > 64 && (wall_clock64() - t0 > SPIN_TICKS || ld_u32(b.err) != 0)) {
          st_u32(b.err, 1u);
          break;
        }
      }
    }
  }
  __syncthreads();
  stamp(st, 2 * si + 1);
}

// ---------------------------------------------------------------- matmul phase
struct MatJob {
  StepMat m;
  const float* x;  // [n][k], coherent
  float* y;
  const float* base;
  float* aux;
  uint32_t epi, write_inv;
  float scale, ra, rb;
};

constexpr int SKC = 256;      // k per chunk
constexpr int SNBLK = 4;      // 64-k blocks per chunk
constexpr int SRT = 4;        // most row tiles per workgroup
// (row tiles per workgroup, k splits) of qkv, o, gate_up, down
constexpr int QKV_RT = 1, QKV_S = 1, O_RT = 1, O_S = 1, GU_RT = 4, GU_S = 1, DN_RT = 2, DN_S = 4;

// One (tile j, chunk i) unit's weights for this lane: row (tile * 16 + t), bytes
// [c 256 + 64 b + 16 q, + 16) per block (int8) or twice that (bf16).
template <int FMT>
__device__ __forceinline__ void load_unit(const StepMat& M, uint32_t tile, uint32_t c, int lane, u32x4* dst) {
  constexpr int WV = FMT == SV_FMT_I8 ? 1 : 2, ESZ = FMT == SV_FMT_I8 ? 1 : 2;
#pragma unroll
  for (int b = 0; b < SNBLK; b++)
#pragma unroll
    for (int v = 0; v < WV; v++)
      dst[b * WV + v] = ldg_nt(weight_word<ESZ>((const uint8_t*)M.w, M.k, M.tiled, tile, c * SNBLK + b, v, lane));
}

// Per-phase work shapes (compile time): the matrix's row tiles go in groups of RT to a
// workgroup, its k in S splits; every wave takes one 256-k chunk of its split for all RT
// tiles (so k = S x 8 x 256), and its RT units of weights are requested a phase ahead into
// pre (slot j: tile j). step_supported() admits a model only if every matrix has this shape.
template <int RT>
__device__ __forceinline__ void mm_prefetch(const StepMat& M, int S, u32x4 (&pre)[SPF], uint32_t (&psc)[SRT * 4], int wv,
                                            int lane) {
  static_assert(RT * SNBLK <= SPF, "prefetch slots");
  const uint32_t groups = M.m / 16 / RT, g = blockIdx.x;
  const bool on = g < groups * S;
  const uint32_t tile0 = (g / S) * RT, c = (g % S) * SW + wv;
  const uint32_t ng = M.per_row ? 1u : M.k >> M.gshift, gi = M.per_row ? 0u : (c * SKC) >> M.gshift;
  const int q = lane >> 4;
  // Slots this phase does not use are written too, so no older contents stay live.
#pragma unroll
  for (int j = RT; j < SRT; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) psc[4 * j + e] = 0u;
#pragma unroll
  for (int i = RT * SNBLK; i < SPF; i++) pre[i] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < RT; j++) {
    if (on) {
      load_unit<SV_FMT_I8>(M, tile0 + j, c, lane, pre + j * SNBLK);
#pragma unroll
      for (int e = 0; e < 4; e++) psc[4 * j + e] = ldg_u16(M.scales + ((size_t)(tile0 + j) * 16 + 4 * q + e) * ng + gi);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) psc[4 * j + e] = 0u;
      // written either way, so the slots' older contents are dead here
#pragma unroll
      for (int b = 0; b < SNBLK; b++) pre[j * SNBLK + b] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

struct MMHandoff {  // split-k partials of the phases with S > 1 (zero at rest: counters)
  uint32_t* counters;  // [groups]
  float* part;         // [groups][S][RT][64][4]
};

// `ahead` requests the next phase's loads once this phase's weights are consumed (in every
// workgroup, including those without rows here).
template <int RT, int S, bool SS, typename Ahead>
__device__ __forceinline__ void mm_phase(const MatJob& J, uint32_t n, const u32x4 (&pre)[SPF], const uint32_t (&psc)[SRT * 4],
                                         float* lds, const MMHandoff& hs, int wv, int lane, Ahead ahead,
                                         uint64_t* sub = nullptr) {
  SUBSTAMP(0);
  const StepMat& M = J.m;
  const uint32_t g = blockIdx.x, groups = M.m / 16 / RT;
  if (g >= groups * S) {  // no rows here: straight to the barrier
    ahead();
    return;
  }
  const int t = lane & 15, q = lane >> 4;
  const uint32_t grp = g / S, sp = g % S, tile0 = grp * RT;
  const bool tok = (uint32_t)t < n;
  // The workgroup's X slice [n][8 x 256] (k from sp x 2048), converted once to the MFMA
  // operands (bf16 hi + lo: 16 significant bits) while it is staged to LDS: thread i takes
  // k words 4 i .. 4 i + 3 of every token row (one round trip for all loads). Rows are
  // padded by 16 bytes against bank conflicts. With SS, each token's sum of squares over
  // the slice (for the folded rms-norm) is added in thread order, then wave order.
  // The residual base of the tile whose epilogue this wave runs is requested meanwhile.
  constexpr uint32_t KS = SW * SKC, XROWB = KS + 8;  // bf16 elements per LDS row
  static_assert(KS / 4 == ST, "one 4-word group per thread and token");
  uint16_t* xh = (uint16_t*)lds;
  uint16_t* xl = xh + 16 * XROWB;
  float* ssw = (float*)(xl + 16 * XROWB);  // [SW][16]
  const size_t o = (size_t)t * M.m + (tile0 + (wv < RT ? wv : 0)) * 16 + 4 * q;
  f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};
  if (J.epi == SV_EPI_RESID && wv < RT && tok) bv = *(const f32x4*)(J.base + o);
  {
    const uint32_t k4 = threadIdx.x;
    // tokens in groups of 8: each group's loads all in flight, then converted
    for (uint32_t r0 = 0; r0 < n; r0 += 8) {
      f32x4 xv[8];
#pragma unroll
      for (int r = 0; r < 8; r++)
        if (r0 + r < n) xv[r] = *(const f32x4*)(J.x + (size_t)(r0 + r) * M.k + sp * KS + 4 * k4);
#pragma unroll
      for (int r = 0; r < 8; r++) {
        if (r0 + r >= n) continue;
        uint32_t hb[4], lb[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          hb[e] = to_bf(xv[r][e]);
          lb[e] = to_bf(xv[r][e] - bf(hb[e]));
        }
        *(u32x2*)(xh + (r0 + r) * XROWB + 4 * k4) = u32x2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
        *(u32x2*)(xl + (r0 + r) * XROWB + 4 * k4) = u32x2{lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16)};
        if (SS) {
          float ss = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; e++) ss = __builtin_fmaf(xv[r][e], xv[r][e], ss);
          ss = wave_sum(ss);
          if (lane == 0) ssw[wv * 16 + r0 + r] = ss;
        }
      }
    }
  }
  SUBSTAMP(1);
  __syncthreads();
  SUBSTAMP(2);

  f32x4 part[RT];
#pragma unroll
  for (int j = 0; j < RT; j++) part[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < SNBLK; b++) {
    // X block: token t, k = 256 wv + 64 b + 16 q + 0..15 of the slice.
    bf16x8 xh0, xh1, xl0, xl1;
    if (tok) {
      const uint32_t e0 = t * XROWB + wv * SKC + 64 * b + 16 * q;
      xh0 = *(const bf16x8*)(xh + e0);
      xh1 = *(const bf16x8*)(xh + e0 + 8);
      xl0 = *(const bf16x8*)(xl + e0);
      xl1 = *(const bf16x8*)(xl + e0 + 8);
    } else {
      xh0 = xh1 = xl0 = xl1 = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    }
#pragma unroll
    for (int j = 0; j < RT; j++) {
      const u32x4 w = pre[j * SNBLK + b];
      const bf16x8 a0 = i8x8_to_bf(w[0], w[1]), a1 = i8x8_to_bf(w[2], w[3]);
      part[j] = mfma16(a0, xh0, part[j]);
      part[j] = mfma16(a0, xl0, part[j]);
      part[j] = mfma16(a1, xh1, part[j]);
      part[j] = mfma16(a1, xl1, part[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < RT; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) part[j][e] *= bf(psc[4 * j + e]);
  ahead();
  float sst = 0.0f;
  if (SS && tok) {
#pragma unroll
    for (int w = 0; w < SW; w++) sst += ssw[w * 16 + t];
  }
  SUBSTAMP(3);
  __syncthreads();  // X is read: its LDS takes the partial sums
  f32x4* red = (f32x4*)lds;                        // [SW][SRT][64]
#pragma unroll
  for (int j = 0; j < RT; j++) red[(wv * SRT + j) * 64 + lane] = part[j];
  __syncthreads();
  // Wave j: tile j's sums in wave order.
  f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
  if (wv < RT) {
    v = red[wv * 64 + lane];
#pragma unroll
    for (int w = 1; w < SW; w++) v += red[(w * SRT + wv) * 64 + lane];
  }
  SUBSTAMP(4);
  if (S > 1) {
    // k splits: the group's last workgroup to arrive adds the partials in split order.
    float* pp = hs.part + ((size_t)grp * S * RT) * 256;
    if (wv < RT) store_wt4(coherent_rsrc(pp), (uint32_t)((((size_t)sp * RT + wv) * 64 + lane) * 16), v);
    __shared__ uint32_t flag;
    if (!arrive_last(hs.counters + grp, S, &flag)) return;
    if (wv >= RT) return;
    v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < S; s2++) v += load_wt4(coherent_rsrc(pp), (uint32_t)((((size_t)s2 * RT + wv) * 64 + lane) * 16));
  }
  if (wv >= RT || !tok) return;
  // Epilogue (kernels.metal:183-209): lane (t, q) holds rows 4 q + 0..3 of tile wv.
  const float inv = 1.0f / __builtin_sqrtf(sst / (float)M.k + SV_RMS_EPS);
  const uint32_t row0 = (tile0 + wv) * 16 + 4 * q;
  switch (J.epi) {
    case SV_EPI_NORM:
      if (J.write_inv && g == 0 && wv == 0 && q == 0) store_wt(J.aux + t, inv);
      store_wt4(coherent_rsrc(J.y), (uint32_t)(o * 4), v * (inv * J.scale));
      break;
    case SV_EPI_RESID:
      store_wt4(coherent_rsrc(J.y), (uint32_t)(o * 4), bv * J.ra + (v * J.scale) * J.rb);
      break;
    case SV_EPI_SWIGLU: {
      const float sc2 = inv * J.scale;
      const float g0 = v[0] * sc2, u0 = v[1] * sc2, g1 = v[2] * sc2, u1 = v[3] * sc2;
      float* yo = J.y + (size_t)t * (M.m / 2) + row0 / 2;
      store_wt(yo, g0 * (1.0f / (1.0f + __expf(-g0))) * u0);
      store_wt(yo + 1, g1 * (1.0f / (1.0f + __expf(-g1))) * u1);
      break;
    }
    default:
      break;
  }
  wait_mem();
  SUBSTAMP(5);
}

// ---------------------------------------------------------------- attention phase
// This workgroup's share of the (run, kv head) pair it serves: slots are (workgroup in the
// pair) x 8 + wave; the newest batch (new keys) goes to slot 0 and cached batch b to slot
// (b + 1) mod slots.
struct AttnJob {
  uint32_t pair, wslot, r, hg, t0, T, seq, p0, nb, slots, active;
  bool on;
};

__device__ __forceinline__ AttnJob attn_job(const StepParams& p) {
  AttnJob a;
  const uint32_t g = blockIdx.x;
  a.on = g < p.pairs * p.wpp;
  a.pair = a.on ? g / p.wpp : 0;
  a.wslot = g % p.wpp;
  a.r = a.pair / p.ap.NKV;
  a.hg = a.pair % p.ap.NKV;
  a.t0 = p.ap.runs[2 * a.r];
  a.T = p.ap.runs[2 * a.r + 1];
  a.seq = p.ap.meta[2 * a.t0];
  a.p0 = p.ap.meta[2 * a.t0 + 1];
  a.nb = (a.p0 + 31) / 32;
  a.slots = p.wpp * SW;
  const uint32_t used = min(a.nb + 1, a.slots);
  a.active = (used + SW - 1) / SW;
  a.on = a.on && a.wslot < a.active;
  return a;
}

// First cached batch of this wave (or none): batch index, or ~0u.
__device__ __forceinline__ uint32_t first_batch(const AttnJob& a, int wv) {
  const uint32_t s = a.wslot * SW + wv;
  const uint32_t b = s == 0 ? a.slots - 1 : s - 1;
  return b < a.nb ? b : ~0u;
}

__device__ __forceinline__ AttnJob uniform_job(const AttnJob& s) {
  AttnJob a;
  a.pair = __builtin_amdgcn_readfirstlane(s.pair);
  a.wslot = __builtin_amdgcn_readfirstlane(s.wslot);
  a.r = __builtin_amdgcn_readfirstlane(s.r);
  a.hg = __builtin_amdgcn_readfirstlane(s.hg);
  a.t0 = __builtin_amdgcn_readfirstlane(s.t0);
  a.T = __builtin_amdgcn_readfirstlane(s.T);
  a.seq = __builtin_amdgcn_readfirstlane(s.seq);
  a.p0 = __builtin_amdgcn_readfirstlane(s.p0);
  a.nb = __builtin_amdgcn_readfirstlane(s.nb);
  a.slots = __builtin_amdgcn_readfirstlane(s.slots);
  a.active = __builtin_amdgcn_readfirstlane(s.active);
  a.on = __builtin_amdgcn_readfirstlane(s.on ? 1u : 0u) != 0;
  return a;
}

// The layer's attention parameters: the launch's plus the per-layer fields.
__device__ __forceinline__ AttnParams layer_params(const StepParams& p, uint32_t l, uint32_t rope, const float* qkv,
                                                   float* out) {
  AttnParams ap = p.ap;
  ap.layer = l;
  ap.rope_on = rope;
  ap.qkv = qkv;
  ap.out = out;
  return ap;
}

template <int D>
__device__ __forceinline__ void kv_prefetch(const StepParams& p, uint32_t l, const AttnJob& sa, int wv, int lane,
                                            KvBatch<D>& kb, const RunConsts* rc) {
  const AttnJob a = uniform_job(sa);
  const AttnParams& ap = p.ap;
  const uint32_t b = a.on ? first_batch(a, wv) : ~0u;
  if (b != ~0u) {
    const size_t ls = (size_t)l * ap.n_pages * ap.NKV * ((size_t)D << ap.page_shift);
    const size_t toff[2] = {rc->kvt[wv][0] + ls, rc->kvt[wv][1] + ls};
    load_batch<D, false>(ap, a.seq, a.hg, 32 * b, a.p0, a.p0, nullptr, nullptr, kb, lane, toff);
  } else {
    // written either way, so the previous layer's batch is dead here
    kb = KvBatch<D>{};
  }
}

template <int D, int NCT, typename Ahead>
__device__ __forceinline__ void attn_phase(const StepParams& p, uint32_t l, uint32_t rope, const float* qkv, float* out,
                                           const AttnJob& sa, KvBatch<D>& cur, float* lds, const RunConsts* rc, int wv,
                                           int lane, Ahead ahead, uint64_t* sub = nullptr) {
  constexpr int VE = D / 16, COLS = 16 * NCT;
  const AttnJob a = uniform_job(sa);
  const AttnParams ap = layer_params(p, l, rope, qkv, out);
  if (!a.on) {
    ahead();
    return;
  }
  const int tid = threadIdx.x, c16 = lane & 15, q = lane >> 4;
  float* ored = lds;                       // [SW][COLS][D]
  float* lred = lds + SW * COLS * D;       // [SW][COLS]
  uint16_t* nk = (uint16_t*)(lred + SW * COLS);
  uint16_t* nv = nk + SV_MAX_RUN * D;
  const uint32_t ncols = a.T * ap.G;

  SUBSTAMP(0);
  // The run's new keys (normed, roped, to the cache and LDS) by all threads of the pair's
  // first workgroup, first: independent of the queries, so the two overlap.
  if (a.wslot == 0) new_keys<D, false>(ap, a.seq, a.hg, a.t0, a.T, a.p0, nk, nv, threadIdx.x, ST, rc);
  bf16x8 qh[NCT][D / 32], ql[NCT][D / 32];
  build_queries<D, NCT, false>(ap, a.t0, a.hg, ncols, qh, ql, lane, rc);
  SUBSTAMP(1);
  f32x4 O[VE][NCT];
  float lsum[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    lsum[ct] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < VE; dt++) O[dt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Cached batches: the first was requested before the barrier; later ones (contexts longer
  // than 32 keys x the pair's waves) load one at a time (registers are the limit here).
  uint32_t b = first_batch(a, wv);
  while (b != ~0u) {
    compute_batch<D, NCT, false>(ap, cur, 32 * b, a.p0, a.p0, ncols, a.t0, qh, ql, O, lsum, lane);
    b = b + a.slots < a.nb ? b + a.slots : ~0u;
    if (b != ~0u) load_batch<D, false>(ap, a.seq, a.hg, 32 * b, a.p0, a.p0, nullptr, nullptr, cur, lane);
  }
  SUBSTAMP(2);
  // The newest batch (slot 0) after this wave's cached ones, so their registers are free.
  if (a.wslot == 0) __syncthreads();  // the new keys are in LDS
  SUBSTAMP(6);
  if (a.wslot == 0 && wv == 0) {
    KvBatch<D> nb0;
    load_batch<D, true>(ap, a.seq, a.hg, a.p0, a.p0 + a.T, a.p0, nk, nv, nb0, lane);
    compute_batch<D, NCT, true>(ap, nb0, a.p0, a.p0 + a.T, a.p0, ncols, a.t0, qh, ql, O, lsum, lane, rc->vis);
  }
  SUBSTAMP(3);
  ahead();
  // The waves' (l, o) to LDS, then the workgroup's partial in wave order.
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
      for (int dt = 0; dt < VE; dt++) od[VE * (4 * q + i) + dt] = O[dt][ct][i];
    if (q == 0) lred[wv * COLS + col] = l;
  }
  __syncthreads();
  SUBSTAMP(4);
  const uint32_t n4 = ncols * D / 4;
  const size_t rec = (size_t)a.pair * p.wpp + a.wslot;
  {
    const __amdgpu_buffer_rsrc_t po = coherent_rsrc(p.part_o + rec * ap.maxcols * D);
    const f32x4* o4 = (const f32x4*)ored;
    const uint32_t cs = COLS * D / 4;
    for (uint32_t i4 = tid; i4 < n4; i4 += ST) {
      f32x4 o = o4[i4];
#pragma unroll
      for (int w = 1; w < SW; w++) o += o4[w * cs + i4];
      store_wt4(po, i4 * 16, o);
    }
  }
  float* pl = p.part_l + rec * ap.maxcols;
  for (uint32_t c = tid; c < ncols; c += ST) {
    float l = lred[c];
#pragma unroll
    for (int w = 1; w < SW; w++) l += lred[w * COLS + c];
    store_wt(pl + c, l);
  }
  // The pair's last workgroup to arrive merges the partials in workgroup order
  // (attn_dec_reduce, kernels.metal:1316-1362).
  __shared__ uint32_t flag;
  SUBSTAMP(5);
  if (!arrive_last(p.counters + a.pair, a.active, &flag)) return;
  const size_t rec0 = (size_t)a.pair * p.wpp;
  const uint32_t so = ap.maxcols * D * 4;
  const __amdgpu_buffer_rsrc_t po0 = coherent_rsrc(p.part_o + rec0 * ap.maxcols * D);
  const float* pl0 = p.part_l + rec0 * ap.maxcols;
  const __amdgpu_buffer_rsrc_t outr = coherent_rsrc(ap.out);
  for (uint32_t i4 = tid; i4 < n4; i4 += ST) {
    const uint32_t col = (4 * i4) / D, d = (4 * i4) % D;
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
    float l = 0.0f;
    uint32_t s = 0;
    for (; s + 8 <= a.active; s += 8) {
      f32x4 ov[8];
      float lv[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        ov[u] = load_wt4(po0, (s + u) * so + i4 * 16);
        lv[u] = load_wt(pl0 + (s + u) * ap.maxcols + col);
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        o += ov[u];
        l += lv[u];
      }
    }
    for (; s < a.active; s++) {
      o += load_wt4(po0, s * so + i4 * 16);
      l += load_wt(pl0 + s * ap.maxcols + col);
    }
    const uint32_t i = col / ap.G, h = a.hg * ap.G + col % ap.G;
    store_wt4(outr, (uint32_t)(((size_t)(a.t0 + i) * ap.NQ * D + h * D + d) * 4), o / l);
  }
  wait_mem();
  SUBSTAMP(7);
}

// ---------------------------------------------------------------- the kernel
template <int D, int NCT>
__global__ __launch_bounds__(ST) void step_kernel(StepParams p) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const BarWords bw = bar_words(p.bar, gridDim.x);
  const uint32_t epoch = ld_u32(bw.epoch);
  uint32_t gen = epoch;
  // This workgroup's attention job lives in LDS (written by thread 0); each phase that uses
  // it takes a scalar copy, so it holds no registers across the launch.
  __shared__ AttnJob s_aj;
  if (threadIdx.x == 0) s_aj = attn_job(p);
  __syncthreads();
  const AttnJob& aj = s_aj;
  const AttnParams& ap = p.ap;
  const MMHandoff hs{p.mm_counters, p.mm_part};
  // This workgroup's run's step constants, cached in LDS for every layer.
  RunConsts* rc = (RunConsts*)((char*)lds + p.rc_off);
  if (aj.on) {
    const uint32_t tid = threadIdx.x;
    if (tid < aj.T) {
      rc->pos[tid] = ap.meta[2 * (aj.t0 + tid) + 1];
      rc->vis[tid] = ap.vis[aj.t0 + tid];
      AttnParams a0 = ap;
      a0.layer = 0;
      rc->row0[tid] = kv_off<D>(a0, aj.seq, aj.hg, aj.p0 + tid);
    }
    const int wv0 = tid >> 6, l0 = tid & 63;
    if (l0 < 2) {
      const uint32_t b = first_batch(aj, wv0);
      AttnParams a0 = ap;
      a0.layer = 0;
      rc->kvt[wv0][l0] = b != ~0u ? kv_off<D>(a0, aj.seq, aj.hg, min(32 * b + 16 * l0, aj.p0 - 1)) : 0;
    }
    __syncthreads();
    if (tid < aj.T * SV_ROPE_PAIRS)
      rc->rope[tid / SV_ROPE_PAIRS][tid % SV_ROPE_PAIRS] =
          *(const float2*)(ap.rope + ((size_t)rc->pos[tid / SV_ROPE_PAIRS] * SV_ROPE_PAIRS + tid % SV_ROPE_PAIRS) * 2);
    __syncthreads();
  }

  stamp(p.stamps, 0);
  u32x4 pre[SPF];
  uint32_t psc[SRT * 4];  // raw bf16 scale bits (converted at use, so the loads are not waited on)
  KvBatch<D> kvb;
  mm_prefetch<QKV_RT>(p.layers[0].mat[0], QKV_S, pre, psc, wv, lane);
  for (uint32_t l = 0; l < p.n_layers; l++) {
    const StepLayerHost& L = p.layers[l];
    const size_t HS = 16 * (size_t)p.H;
    const float* h_in = l == 0 ? p.h : p.hs + (l - 1) * HS;
    float* h_out = l + 1 == p.n_layers ? p.h : p.hs + l * HS;
    float* qkv = p.qkv + l * 16 * (size_t)p.qkv_w;
    float* attn = p.attn + l * 16 * (size_t)(p.ap.NQ * 64);
    float* mixed = p.mixed + l * HS;
    float* act = p.act + l * 16 * (size_t)p.F;
    uint64_t* sub = p.stamps && l == 1 ? p.stamps + 10 * p.n_layers + 8 : nullptr;  // [5 phases][8]
    // qkv (EPI_NORM, inv written): h -> qkv; then the layer's first K/V batch is requested.
    auto none = [] {};
    {
      MatJob J{L.mat[0], h_in, qkv, nullptr, p.inv, SV_EPI_NORM, 1u, L.qkv_scale, 0.f, 0.f};
      mm_phase<QKV_RT, QKV_S, true>(J, p.n, pre, psc, lds, hs, wv, lane, none, sub);
    }
    ++gen;
    grid_barrier(bw, gen, p.stamps, gen - epoch, [&] { kv_prefetch<D>(p, l, aj, wv, lane, kvb, rc); });
    // attention: qkv -> attn; then o's weights.
    attn_phase<D, NCT>(p, l, L.rope, qkv, attn, aj, kvb, lds, rc, wv, lane, none, sub ? sub + 8 : nullptr);
    ++gen;
    grid_barrier(bw, gen, p.stamps, gen - epoch, [&] { mm_prefetch<O_RT>(L.mat[1], O_S, pre, psc, wv, lane); });
    // o (EPI_RESID, base h): attn -> mixed; then gate_up's weights.
    {
      MatJob J{L.mat[1], attn, mixed, h_in, nullptr, SV_EPI_RESID, 0u, L.o_scale, L.resid_attn, L.post_attn};
      mm_phase<O_RT, O_S, false>(J, p.n, pre, psc, lds, hs, wv, lane, none, sub ? sub + 16 : nullptr);
    }
    ++gen;
    grid_barrier(bw, gen, p.stamps, gen - epoch, [&] { mm_prefetch<GU_RT>(L.mat[2], GU_S, pre, psc, wv, lane); });
    // gate_up (EPI_SWIGLU): mixed -> act; then down's weights.
    {
      MatJob J{L.mat[2], mixed, act, nullptr, nullptr, SV_EPI_SWIGLU, 0u, 1.0f, 0.f, 0.f};
      mm_phase<GU_RT, GU_S, true>(J, p.n, pre, psc, lds, hs, wv, lane, none, sub ? sub + 24 : nullptr);
    }
    ++gen;
    grid_barrier(bw, gen, p.stamps, gen - epoch, [&] { mm_prefetch<DN_RT>(L.mat[3], DN_S, pre, psc, wv, lane); });
    // down (EPI_RESID, base mixed): act -> h; then the next layer's qkv weights.
    {
      MatJob J{L.mat[3], act, h_out, mixed, nullptr, SV_EPI_RESID, 0u, 1.0f, L.resid_mlp, L.post_mlp};
      const bool more = l + 1 < p.n_layers;
      mm_phase<DN_RT, DN_S, false>(J, p.n, pre, psc, lds, hs, wv, lane, none, sub ? sub + 32 : nullptr);
      if (more) {
        ++gen;
        grid_barrier(bw, gen, p.stamps, gen - epoch,
                     [&] { mm_prefetch<QKV_RT>(p.layers[l + 1].mat[0], QKV_S, pre, psc, wv, lane); });
      }
    }
  }
  stamp(p.stamps, 2 * (gen - epoch + 1));
  if (blockIdx.x == 0 && threadIdx.x == 0) st_u32(bw.epoch, gen);
}

// ---------------------------------------------------------------- host side
static uint32_t step_grid() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 0;
  }
  return (uint32_t)cus;
}

static size_t rc_offset(uint32_t D, uint32_t nct, uint32_t n);
static size_t step_lds_bytes(uint32_t D, uint32_t nct, uint32_t n) { return rc_offset(D, nct, n) + sizeof(RunConsts); }
static size_t rc_offset(uint32_t D, uint32_t nct, uint32_t n) {
  (void)n;
  const size_t xs = 2 * (size_t)16 * (SW * SKC + 8) * 2 + (size_t)SW * 16 * 4;
  const size_t red = (size_t)SW * SRT * 64 * 16 + (size_t)SW * 16 * 4;
  const size_t mm = xs > red ? xs : red;
  const size_t at = (size_t)SW * 16 * nct * D * 4 + (size_t)SW * 16 * nct * 4 + 2 * (size_t)SV_MAX_RUN * D * 2;
  return ((mm > at ? mm : at) + 15) / 16 * 16;
}

static const void* step_fn(uint32_t nct) {
  return nct == 1 ? (const void*)step_kernel<64, 1> : (const void*)step_kernel<64, 2>;
}

// Workspace: barrier words, then per (run, kv head) pair a counter and the workgroups' partials.
static void step_ws_layout(const sv_shape* sh, uint32_t n_runs, uint32_t max_run, size_t* cnt_off, size_t* po_off,
                           size_t* pl_off, size_t* mmc_off, size_t* mmp_off, size_t* total) {
  const uint32_t G = step_grid(), pairs = n_runs * sh->n_kv_heads, wpp = pairs ? G / pairs : 0;
  const size_t maxcols = (max_run * (sh->n_heads / sh->n_kv_heads) + 15) / 16 * 16;
  size_t off = (((size_t)G * 16 + 8 * 16 + 32) * 4 + 255) / 256 * 256;
  *cnt_off = off;
  off += ((size_t)pairs * 4 + 255) / 256 * 256;
  *po_off = off;
  off += (size_t)pairs * wpp * maxcols * sh->head_dim * 4;
  off = (off + 255) / 256 * 256;
  *pl_off = off;
  off += (size_t)pairs * wpp * maxcols * 4;
  off = (off + 255) / 256 * 256;
  *mmc_off = off;
  const size_t dn_groups = sh->hidden / 16 / DN_RT;
  off += (dn_groups * 4 + 255) / 256 * 256;
  *mmp_off = off;
  off += dn_groups * DN_S * DN_RT * 256 * 4;
  *total = off;
}

size_t step_acts_bytes(const sv_shape* sh) {
  const size_t L = sh->n_layers, H = sh->hidden, W = (size_t)(sh->n_heads + 2 * sh->n_kv_heads) * sh->head_dim;
  return ((L - 1) * H + L * W + L * (size_t)sh->n_heads * sh->head_dim + L * H + L * (size_t)sh->ffn) * 16 * 4;
}

size_t step_ws_bytes(const sv_shape* sh, uint32_t n_runs, uint32_t max_run) {
  size_t a, b, c, d, e, t;
  step_ws_layout(sh, n_runs, max_run, &a, &b, &c, &d, &e, &t);
  return t;
}

// int8 weights with scales per row or per group of >= 256, and the matrix in the phase's
// work shape: row tiles in groups of rt, k = splits x 8 waves x 256, groups x splits <= grid.
static bool mat_ok(const sv_matrix& m, uint32_t G, uint32_t rt, uint32_t splits) {
  if ((m.format & ~(uint32_t)SV_FMT_TILED) != SV_FMT_I8 || !m.d_scales || m.m % (16 * rt) || m.k != splits * SW * SKC || m.m / 16 / rt * splits > G)
    return false;
  const bool per_row = m.gshift >= 32 || (1ull << m.gshift) >= m.k;
  return per_row || (m.gshift >= 8 && m.k % (1u << m.gshift) == 0);
}

bool step_supported(const sv_shape* sh, const sv_layer* layers, uint32_t n, uint32_t n_runs, uint32_t max_run) {
  if (n == 0 || n > 16 || sh->head_dim != 64 || max_run == 0 || max_run > SV_MAX_RUN) return false;
  const uint32_t G = step_grid();
  const uint32_t nct = (max_run * (sh->n_heads / sh->n_kv_heads) + 15) / 16;
  if (G == 0 || nct > 2 || n_runs * sh->n_kv_heads > G) return false;
  for (uint32_t l = 0; l < sh->n_layers; l++)
    if (!mat_ok(layers[l].qkv, G, QKV_RT, QKV_S) || !mat_ok(layers[l].o, G, O_RT, O_S) ||
        !mat_ok(layers[l].gate_up, G, GU_RT, GU_S) || !mat_ok(layers[l].down, G, DN_RT, DN_S))
      return false;
  const void* fn = step_fn(nct);
  const size_t lds = step_lds_bytes(64, nct, 16);
  static bool attr_done[3] = {};
  if (!attr_done[nct]) {
    attr_done[nct] = true;
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, ST, lds) != hipSuccess || per_cu < 1) return false;
  return true;
}

void step_fill_layer(const sv_layer* l, StepLayerHost* out) {
  const sv_matrix* ms[4] = {&l->qkv, &l->o, &l->gate_up, &l->down};
  for (int i = 0; i < 4; i++) {
    const sv_matrix& m = *ms[i];
    out->mat[i].w = m.d_w;
    out->mat[i].scales = m.d_scales;
    out->mat[i].m = m.m;
    out->mat[i].k = m.k;
    const bool per_row = (m.format & ~(uint32_t)SV_FMT_TILED) != SV_FMT_I8 || m.gshift >= 32 || (1ull << m.gshift) >= m.k;
    out->mat[i].per_row = per_row;
    out->mat[i].tiled = (m.format & SV_FMT_TILED) != 0;
    out->mat[i].gshift = per_row ? 31 : m.gshift;
  }
  out->qkv_scale = l->qkv_scale;
  out->o_scale = l->o_scale;
  out->resid_attn = l->resid_attn;
  out->post_attn = l->post_attn;
  out->resid_mlp = l->resid_mlp;
  out->post_mlp = l->post_mlp;
  out->rope = l->rope;
}

sv_status step_launch(hipStream_t stream, const StepLaunch& a) {
  const sv_shape* sh = a.sh;
  const uint32_t G = step_grid(), D = sh->head_dim, NQ = sh->n_heads, NKV = sh->n_kv_heads;
  if (D != 64) return fail(SV_ERR_UNSUPPORTED, "step: head_dim %u", D);
  const uint32_t maxcols = (a.max_run * (NQ / NKV) + 15) / 16 * 16, nct = maxcols / 16;
  size_t cnt_off, po_off, pl_off, mmc_off, mmp_off, total;
  step_ws_layout(sh, a.n_runs, a.max_run, &cnt_off, &po_off, &pl_off, &mmc_off, &mmp_off, &total);
  if (!a.ws || a.ws_bytes < total) return fail(SV_ERR_ARG, "step: workspace %zu < %zu bytes", a.ws_bytes, total);
  StepParams p;
  p.layers = (const StepLayerHost*)a.layers;
  p.n_layers = sh->n_layers;
  p.n = a.n;
  p.H = sh->hidden;
  p.F = sh->ffn;
  AttnParams& ap = p.ap;
  ap.qkv = nullptr;  // per layer
  ap.meta = a.meta;
  ap.kc = a.kc;
  ap.vc = a.vc;
  ap.page_table = a.page_table;
  ap.rope = a.rope;
  ap.runs = a.runs;
  ap.vis = a.vis;
  ap.out = nullptr;  // per layer
  ap.part_o = ap.part_l = nullptr;
  ap.counters = nullptr;
  ap.NQ = NQ;
  ap.NKV = NKV;
  ap.G = NQ / NKV;
  ap.W = (NQ + 2 * NKV) * D;
  ap.KOFF = NQ * D;
  ap.VOFF = (NQ + NKV) * D;
  ap.split = 32;
  ap.max_splits = 0;
  ap.scale_log2 = a.scale_log2;
  ap.rope_on = 0;
  ap.page_shift = a.page_shift;
  ap.n_pages = a.n_pages;
  ap.max_pages = a.max_pages;
  ap.layer = 0;
  ap.maxcols = maxcols;
  ap.n_inline = 0;
  ap.newest_own = 1;  // this kernel's attention keeps the new keys apart (its own phases)
  p.n_runs = a.n_runs;
  p.pairs = a.n_runs * NKV;
  p.wpp = G / p.pairs;
  p.h = a.h;
  p.qkv_w = ap.W;
  {
    // activation slices: hs [L - 1][16][H], qkv [L][16][W], attn [L][16][NQ D], mixed
    // [L][16][H], act [L][16][F]
    float* b = (float*)a.acts;
    const size_t L = sh->n_layers, H = sh->hidden;
    p.hs = b;
    b += (L - 1) * 16 * H;
    p.qkv = b;
    b += L * 16 * (size_t)ap.W;
    p.attn = b;
    b += L * 16 * (size_t)NQ * D;
    p.mixed = b;
    b += L * 16 * H;
    p.act = b;
  }
  p.inv = a.inv;
  p.bar = (uint32_t*)a.ws;
  p.counters = (uint32_t*)((char*)a.ws + cnt_off);
  p.part_o = (float*)((char*)a.ws + po_off);
  p.part_l = (float*)((char*)a.ws + pl_off);
  p.stamps = (uint64_t*)a.stamps;
  p.rc_off = (uint32_t)rc_offset(D, nct, a.n);
  p.mm_counters = (uint32_t*)((char*)a.ws + mmc_off);
  p.mm_part = (float*)((char*)a.ws + mmp_off);
  const size_t lds = step_lds_bytes(D, nct, a.n);
  if (nct == 1) launch((step_kernel<64, 1>), dim3(G), dim3(ST), lds, stream, p);
  else launch((step_kernel<64, 2>), dim3(G), dim3(ST), lds, stream, p);
  return check_launch("step");
}

// The error word of the step workspace (non-zero: a barrier wait ran out of time).
size_t step_err_offset() { return ((size_t)step_grid() * 16 + 8 * 16 + 16) * 4; }

}  // namespace sv
