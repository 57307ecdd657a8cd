// attention.hip — fused verify attention over the paged KV cache (the reference's
// attn_verify + attn_dec_reduce, engine/src/kernels.metal:891-1148 and :1316-1362, encoded by
// encode.rs:233-297).
//
// One workgroup (4 waves) per (key split s, kv head g, run r):
//   - Columns are the run's T tokens x G query heads of kv head g (column c: token c / G,
//     head g G + c % G), in NCT tiles of 16. Each lane builds its columns' queries in
//     registers: rms-norm over the head (no gain), RoPE on pairs (2j, 2j+1), j < 32, times
//     softmax scale * log2 e, split into bf16 hi + lo MFMA operands.
//   - Splits own `split` cached keys each. The run's new keys (norm, RoPE, K and V rounded to
//     bf16, written to the cache at p0 + row and kept in LDS) go to a split of their own after
//     the cached ones (all-in-flight variant) or to the last cached split, after its batches
//     (streaming variant; without cached keys the one split holds only them).
//   - Keys go in batches of 32 (wave w takes batches w, w + 4, ..., the next one's K/V in
//     flight while the current one is multiplied; the first is issued before the queries
//     are built): S^T = K Q^T on
//     v_mfma_f32_16x16x32_bf16 (two 16-key tiles, hi and lo), p = 2^s for visible keys (no
//     running max: q and k are rms-normed, so scores are bounded, kernels.metal:804-806),
//     then O^T += V^T P^T with P (hi, lo) taken straight from the S^T accumulators' layout.
//     K rows are read as 16-byte slices; each V row is read whole by 16 lanes (8 bytes per
//     lane for D = 64), and the matrix-core operand takes one of its dims per tile.
//   - The 4 waves' (l, o) meet in LDS and the split's partial goes to the workspace with
//     coherent stores (sc1: write-through to the agent-coherent level). attn_merge_kernel,
//     the next launch, sums the partials of each (run, kv head) output in split order and
//     writes o / l. With g_attn_fused_merge set (tests; measured slower) the last split of
//     (run, kv head) to arrive (a relaxed agent-scope counter: no L2 write-back or invalidate)
//     does the same, in the same order (the same bits), with coherent 16-byte loads.
//   - The capture step (sv_step_capture) adds attn_capture_kernel after the merge: it repeats
//     the query and new-key device code into float buffers; the kernels above are unchanged.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "attn_device.h"
#include "sv_internal.h"

#define SV_TRY_LAUNCH(what)                        \
  do {                                             \
    const sv_status st_ = check_launch(what);      \
    if (st_ != SV_OK) return st_;                  \
  } while (0)

namespace sv {

// Batches per wave of the all-in-flight variant (splits of at most 128 x this many keys).
constexpr int SV_ATTN_NBW = 4;
// Batch slots per wave of the streaming variant: one batch is multiplied while the others are in
// flight. Up to 32 columns per kv head three slots at two waves per SIMD (measured 1-3 % faster
// than two slots at three waves per SIMD at 32 streams and 65536 x 8); wider runs two (a third
// does not fit two waves per SIMD, and at one wave per SIMD it measured no faster).
constexpr int attn_ring(int NCT) { return NCT <= 2 ? 3 : 2; }
// Waves per SIMD the register budget allows: two for D = 64 (64 columns fit in 228 registers
// without spills; 3 % faster than one wave per SIMD on the trees), one for D = 128.
constexpr int attn_waves(int D, int, int) { return D == 64 ? 2 : 1; }
// Whether a run's new keys get a split of their own. All-in-flight variant: yes (it runs beside
// the cached splits on an otherwise idle CU). Streaming variant up to 32 columns per kv head:
// no, the last cached split takes them (a split of new keys alone is a short workgroup that
// holds a resident slot and pushes cached splits into a later round: configs[2] attention 3 %
// faster). Wider runs: yes (their splits are bound by their own products, and the extra
// workgroup adds parallelism: the trees 2 % faster).
constexpr bool attn_newest_own(int NCT, int NBW) { return NBW > 0 || NCT >= 3; }

// NBW = 0: each wave keeps one batch in flight ahead of the one it multiplies (any split).
// NBW > 0 (splits of at most 128 NBW keys, grids of about one workgroup per CU): each wave
// requests all of its batches at once, after the queries, positions and page-table words (one
// round trip) and the rope words, and builds the queries while they arrive.
template <int D, int NCT, int NBW, bool INL, bool LOCAL = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(attn_waves(D, NCT, NBW)))) void attn_verify_kernel(AttnParams p) {
  constexpr int KST = D / 32, VE = D / 16, COLS = 16 * NCT;
  extern __shared__ __attribute__((aligned(16))) float lds[];  // [4][COLS][D] partial o, then [4][COLS] partial l
  __shared__ uint16_t nk[SV_MAX_RUN * D], nv[SV_MAX_RUN * D];
  float* ored = lds;
  float* lred = lds + 4 * COLS * D;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c16 = lane & 15, q = lane >> 4;
  // Streaming variant: workgroups are dispatched in linear order (x fastest) and take their
  // (split, kv head, run) split-major, so every run's first splits go out before any run's later
  // ones, and the workgroups past a run's last split (the grid is sized for the longest context;
  // they exit once the context length is in) come last, into the tail, instead of holding CU
  // slots between live ones (configs[2]: about half the grid). Within a split the kv head is the
  // fastest index (the run fastest measured 4 % slower per step at configs[2]). The all-in-flight
  // variant (about one workgroup per CU, few past the context) keeps split fastest: an XCD
  // (workgroup id mod 8) reads every kv head of its splits' pages (split-major measured 0.7 %
  // slower per step at configs[1], each XCD then reading one kv head's slice of every page).
  uint32_t s = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
  if constexpr (NBW == 0) {
    const uint32_t lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), per = gridDim.y * gridDim.z;
    s = lin / per;
    g = lin % per % gridDim.y;
    r = lin % per / gridDim.y;
  }
  uint32_t t0, T, seq;
  run_header<INL>(p, r, t0, T, seq);
  // The run's visibility masks (the newest split's masks): requested with the first loads and
  // put in LDS once those have arrived (before the barrier that precedes their use), so no
  // round trip is spent on them alone.
  __shared__ uint32_t svis[SV_MAX_RUN];
  const uint32_t visw = p.vis[t0 + min((uint32_t)tid, T - 1)];
  constexpr int R = attn_ring(NCT);
  KvBatchT<D> ring[NBW == 0 ? R : 1];
  // A sliding-window layer's splits start at its first query's window (its position first).
  uint32_t p0 = LOCAL ? p.meta[2 * t0 + 1] : 0u;
  const uint32_t kbeg = (LOCAL ? key_base_t<true>(p, p0) : 0u) + s * p.split;
  // this wave's V stage (2 tiles x 16 keys), at the front of the reduction buffer
  uint16_t* stage = (uint16_t*)((char*)lds + (size_t)wv * stage_bytes<D>());
  // Page-table lookups of this wave's batches wv + 4 i of the split (tile mt of batch i in lane
  // 2 i + mt) go out with the query words and positions, the split taken as full (indices
  // clamped into the table; tiles past the context are masked later): the batch loop takes its
  // tile offsets with readlane and never waits for a page-table load (such a wait, vmcnt(0),
  // also waits for every K/V load in flight). The rope words follow, then the wave's first
  // batches (all of them in the all-in-flight variant, R - 1 in the streaming one): s_waitcnt
  // counts loads in issue order, so the queries, built once the rope words are in, never wait
  // for a batch, and each batch is read whether or not the split has keys there (inside its
  // page) and used only if it does.
  // (split <= 3968 keys: at most 31 batches per wave, 62 lanes)
  const uint32_t nbw_full = p.split / 32 > (uint32_t)wv ? (p.split / 32 - wv + 3) / 4 : 0u;
  size_t tile_off = 0;
  const uint32_t ncols = T * p.G;
  bf16x8 qh[NCT][KST], ql[NCT][KST];
  KvBatchT<D> bt[NBW > 0 ? NBW : 1];
  {
    // Queries, positions and page-table words in one round trip; then the rope words, then
    // every batch of the wave (slots past the split's batches read nothing); the queries are
    // built once the rope words are in, while the batches stream.
    // 1. One round trip: query words and positions of the lane's columns (a column past the
    //    run's reads the last column's words and is zeroed), this wave's page-table words
    //    (lane 2 i + mt: tile mt of batch i, index clamped into the table) and p0.
    QRaw<D, NCT> qr;
#pragma unroll
    for (int ct = 0; ct < NCT; ct++) {
      const uint32_t c = min(16u * ct + c16, ncols - 1), i = c / p.G, h = g * p.G + c % p.G, t = t0 + i;
      qr.pos[ct] = p.meta[2 * t + 1];
      const size_t qo = (size_t)t * p.W + h * D + 8 * q;
#pragma unroll
      for (int ks = 0; ks < KST; ks++) {
        const f32x4 a = *(const f32x4*)(p.qkv + qo + 32 * ks), b = *(const f32x4*)(p.qkv + qo + 32 * ks + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          qr.v[ct][ks][e] = a[e];
          qr.v[ct][ks][4 + e] = b[e];
        }
      }
    }
    const uint32_t tpos = kbeg + 32 * (wv + 4 * (lane >> 1)) + 16 * (lane & 1);
    const uint32_t pword = p.page_table[(size_t)seq * p.max_pages + min(tpos >> p.page_shift, p.max_pages - 1)];
    if constexpr (!LOCAL) p0 = p.meta[2 * t0 + 1];  // (a window layer read it first: kbeg needs it)
    // Rope words through a descriptor whose range is empty without rope (zeros, no access), so
    // no branch splits the loads' accounting. Inline runs: the step's rows by token, in this
    // same round trip; else the table's rows at the positions, once those are in.
    float2 cs[NCT][KST][4];
    auto load_rope = [&](const float* base, bool by_token) {
      const __amdgpu_buffer_rsrc_t rrs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, p.rope_on ? 0x7fffffff : 0, 0x00020000);
#pragma unroll
      for (int ct = 0; ct < NCT; ct++)
#pragma unroll
        for (int ks = 0; ks < KST; ks++)
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const uint32_t j = 16 * ks + 4 * q + jj;
            const bool on = p.rope_on && 32 * ks + 8 * q < 64;
            const uint32_t c = min(16u * ct + c16, ncols - 1);
            const uint32_t row = by_token ? t0 + c / p.G : qr.pos[ct];
            const uint32_t off = (row * SV_ROPE_PAIRS + j) * 8 + (on ? 0u : 0x80000000u);
            cs[ct][ks][jj] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rrs, off, 0, 0));
          }
    };
    if constexpr (INL) load_rope(p.rope_rows, true);
    __builtin_amdgcn_sched_barrier(0);
    // 2. (Without inline runs, the rope words: they need the positions.) Then every batch of
    //    the wave (they need the page words; slots past the split's batches read nothing).
    if constexpr (!INL) load_rope(p.rope, false);
    // Streaming variant: a split past the run's context (the grid is sized for the longest
    // one), or a grid with too few splits for it, is known once p0 is in, in the round trip of
    // the page words: it leaves before requesting K/V or building queries. The all-in-flight
    // variant (about one workgroup per CU, few past the context) does not wait for p0 before
    // its K/V requests (measured 8 % slower at configs[1] when it did) and checks after.
    if constexpr (NBW == 0) {
      const uint32_t nsplit = attn_nsplit_t<LOCAL>(p, p0);
      if (nsplit > p.max_splits) {
        // Its output is NaN (never a partial sum) and the counter is left alone.
        if (s == 0)
          for (uint32_t idx = tid; idx < ncols * D; idx += 256) {
            const uint32_t col = idx / D, i = col / p.G, h = g * p.G + col % p.G;
            p.out[(size_t)(t0 + i) * p.NQ * D + h * D + idx % D] = __builtin_nanf("");
          }
        return;
      }
      if (s >= nsplit) return;
    }
    if ((uint32_t)lane < 2 * nbw_full) {
      const uint32_t page = min(pword, p.n_pages - 1);
      tile_off = ((((size_t)p.layer * p.n_pages + page) * p.NKV + g) << p.page_shift) * D +
                 (size_t)(tpos & ((1u << p.page_shift) - 1u)) * D;
    }
    if constexpr (NBW > 0) {
#pragma unroll
      for (int i = 0; i < NBW; i++) {
        const size_t toffs[2] = {readlane64(tile_off, 2 * i), readlane64(tile_off, 2 * i + 1)};
        load_batch_tiles_t<D>(p, toffs, bt[i], lane, (uint32_t)i < nbw_full ? 0u : 0x80000000u);
      }
    } else {
      // the ring's first R - 1 batches (the loop requests each next one R - 1 ahead)
#pragma unroll
      for (int i = 0; i < R - 1; i++) {
        const size_t toffs[2] = {readlane64(tile_off, 2 * i), readlane64(tile_off, 2 * i + 1)};
        load_batch_tiles_t<D>(p, toffs, ring[i], lane, (uint32_t)i < nbw_full ? 0u : 0x80000000u);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (tid < T) svis[tid] = visw;
    // 3. The queries, while the batches stream (columns past the run's are zero; no rope is
    //    the identity rotation).
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
    qfinish_cs<D, NCT>(p, ncols, qr, cs, qh, ql, lane);
  }

  const uint32_t nsplit = attn_nsplit_t<LOCAL>(p, p0);
  if constexpr (NBW > 0) {
    if (nsplit > p.max_splits) {
      // The grid has too few splits for this run's context: its output is NaN (never a
      // partial sum) and the counter is left alone.
      if (s == 0)
        for (uint32_t idx = tid; idx < ncols * D; idx += 256) {
          const uint32_t col = idx / D, i = col / p.G, h = g * p.G + col % p.G;
          p.out[(size_t)(t0 + i) * p.NQ * D + h * D + idx % D] = __builtin_nanf("");
        }
      return;
    }
    if (s >= nsplit) return;
  }
  // Each lane column's first visible cached key, and the highest of any column of the run (its
  // positions are at most p0 + T - 1): batches at or above it need no window mask.
  uint32_t clo[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    const uint32_t c = 16 * ct + c16;
    clo[ct] = LOCAL && c < ncols ? key_lo_t<LOCAL>(p, p.meta[2 * (t0 + c / p.G) + 1]) : 0u;
  }
  const uint32_t lo_hi = key_lo_t<LOCAL>(p, p0 + T - 1);
  // newest: a split of the new keys alone; takes_new: the last cached split also takes them
  // (attn_newest_own; the launch sets p.newest_own to match).
  const bool newest = attn_newest_own(NCT, NBW) && s == nsplit - 1, takes_new = !attn_newest_own(NCT, NBW) && s == nsplit - 1;

  const uint32_t kend = newest ? p0 : min(kbeg + p.split, p0);
  const uint32_t nb = newest ? 0u : (kend - kbeg + 31) / 32;

  if (newest) new_keys<D, false>(p, seq, g, t0, T, p0, nk, nv, tid, 256);
  __syncthreads();

  f32x4 O[VE][NCT];
  float lsum[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    lsum[ct] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < VE; dt++) O[dt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (newest) {
    if (wv == 0) {
      KvBatchT<D> nb0;
      load_batch_new_t<D>(nk, nv, p0, p0 + T, p0, nb0, lane);
      compute_batch_t<D, NCT, true>(p, nb0, p0, p0 + T, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo, svis);
    }
  } else if constexpr (NBW > 0) {
#pragma unroll
    for (int i = 0; i < NBW; i++) {
      const uint32_t b = wv + 4 * i, kb = kbeg + 32 * b;
      if (b < nb) {
        if (kb + 32 <= kend && kb >= lo_hi) compute_batch_t<D, NCT, false, true>(p, bt[i], kb, kend, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo);
        else compute_batch_t<D, NCT, false>(p, bt[i], kb, kend, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo);
      }
    }
  } else {
    // The wave's j-th batch (wv + 4 j of the split) lives in slot j % R; the batch R - 1 ahead
    // is requested (slots past the wave's last batch read nothing) before batch j is multiplied.
    const uint32_t nbw = nb > (uint32_t)wv ? (nb - wv + 3) / 4 : 0u;
    for (uint32_t j0 = 0; j0 < nbw; j0 += R) {
#pragma unroll
      for (int i = 0; i < R; i++) {
        const uint32_t j = j0 + i, jn = j + R - 1;
        const int li = (int)min(2 * jn, 62u);
        const size_t toffs[2] = {readlane64(tile_off, li), readlane64(tile_off, li + 1)};
        load_batch_tiles_t<D>(p, toffs, ring[(i + R - 1) % R], lane, jn < nbw ? 0u : 0x80000000u);
        __builtin_amdgcn_sched_barrier(0);  // the loads go out before this batch's work
        if (j < nbw) {
          const uint32_t kb = kbeg + 32 * (wv + 4 * j);
          if (kb + 32 <= kend && kb >= lo_hi) compute_batch_t<D, NCT, false, true>(p, ring[i], kb, kend, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo);
          else compute_batch_t<D, NCT, false>(p, ring[i], kb, kend, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo);
        }
      }
    }
    if (takes_new) {
      // The run's new keys after this split's cached ones: to the cache and LDS (no other
      // workgroup reads positions p0 on), then wave 0 multiplies them (the barrier orders every
      // wave's batches before it).
      new_keys<D, false>(p, seq, g, t0, T, p0, nk, nv, tid, 256);
      __syncthreads();
      if (wv == 0) {
        KvBatchT<D> nb0;
        load_batch_new_t<D>(nk, nv, p0, p0 + T, p0, nb0, lane);
        compute_batch_t<D, NCT, true>(p, nb0, p0, p0 + T, p0, ncols, t0, qh, ql, O, lsum, lane, stage, clo, svis);
      }
    }
  }

  __syncthreads();  // every wave's V stage read before the reduction buffer (over it) is written
  // This wave's (l, o) to LDS: lane holds column 16 ct + c16, dims 16 dt + 4 q + i.
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
  const size_t rec = ((size_t)r * p.NKV + g) * p.max_splits + s;
  const uint32_t n4 = ncols * D / 4;
  {
    const __amdgpu_buffer_rsrc_t po = coherent_rsrc(p.part_o + rec * p.maxcols * D);
    for (uint32_t i4 = tid; i4 < n4; i4 += 256) {
      const f32x4* o4 = (const f32x4*)ored;
      const uint32_t cs = COLS * D / 4;
      store_wt4(po, i4 * 16, ((o4[i4] + o4[cs + i4]) + o4[2 * cs + i4]) + o4[3 * cs + i4]);
    }
  }
  float* pl = p.part_l + rec * p.maxcols;
  for (uint32_t idx = tid; idx < ncols; idx += 256)
    store_wt(pl + idx, ((lred[idx] + lred[COLS + idx]) + lred[2 * COLS + idx]) + lred[3 * COLS + idx]);
  if (!p.counters) return;  // attn_merge_kernel merges

  // The last split of (run, kv head) to arrive merges (attn_dec_reduce, kernels.metal:1316-1362)
  // in attn_merge_kernel's order, so both give the same bits: P parts (p.merge_parts <= 4), part
  // j adding splits j, j + P, ... (at most eight) from zero, the parts then added in part order.
  // Thread (part, gi) takes items gi, gi + 256 / P, ... of four outputs (column, dims d .. d + 3),
  // three items' loads in flight at once; each part's sums meet in the reduction buffer.
  __shared__ uint32_t flag;
  if (!arrive_last(&p.counters[r * p.NKV + g], nsplit, &flag)) return;
  const uint32_t P = p.merge_parts, G4 = 256 / P, part = tid / G4, gi = tid % G4;
  const size_t rec0 = ((size_t)r * p.NKV + g) * p.max_splits;
  const uint32_t so = p.maxcols * D * 4;  // bytes per split partial
  const __amdgpu_buffer_rsrc_t po0 = coherent_rsrc(p.part_o + rec0 * p.maxcols * D);
  const float* pl0 = p.part_l + rec0 * p.maxcols;
  f32x4* red = (f32x4*)ored;  // [P][n4] (P n4 16 <= 4 COLS D 4 bytes)
  constexpr int IB = 3;
  for (uint32_t b0 = gi; b0 < n4; b0 += IB * G4) {
    f32x4 ov[IB][8];
#pragma unroll
    for (int b = 0; b < IB; b++)
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const uint32_t i4 = b0 + b * G4, x = part + u * P;
        ov[b][u] = i4 < n4 && x < nsplit ? load_wt4(po0, x * so + i4 * 16) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int b = 0; b < IB; b++) {
      f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (part + u * P < nsplit) o += ov[b][u];
      if (b0 + b * G4 < n4) red[part * n4 + b0 + b * G4] = o;
    }
  }
  // l per (part, column)
  if (tid < P * ncols) {
    const uint32_t lp = tid / ncols, col = tid % ncols;
    float lv[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const uint32_t x = lp + u * P;
      lv[u] = x < nsplit ? load_wt(pl0 + x * p.maxcols + col) : 0.0f;
    }
    float l = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (lp + u * P < nsplit) l += lv[u];
    lred[lp * COLS + col] = l;
  }
  __syncthreads();
  for (uint32_t i4 = tid; i4 < n4; i4 += 256) {
    const uint32_t col = (4 * i4) / D, d = (4 * i4) % D;
    f32x4 o = red[i4];
    float l = lred[col];
    for (uint32_t j = 1; j < P; j++) {
      o += red[j * n4 + i4];
      l += lred[j * COLS + col];
    }
    const uint32_t i = col / p.G, h = g * p.G + col % p.G;
    *(f32x4*)(p.out + (size_t)(t0 + i) * p.NQ * D + h * D + d) = o / l;
    if (p.cap_sdpa) *(f32x4*)(p.cap_sdpa + (size_t)(t0 + i) * p.NQ * D + h * D + d) = o / l;
  }
}

// attn_dec_reduce (kernels.metal:1316-1362) for the fused verify attention: plain sums over
// the splits (no running max) of four consecutive outputs (column, dims d .. d + 3) of one
// (run, kv head), then o / l. A workgroup of 256 threads is P parts x 256 / P output groups:
// part j adds splits j, j + P, ... (at most eight, all requested at once, before the context
// length in meta says how many count), then the parts are added in part order through LDS.
// P grows with the grid's splits (long contexts at one stream), so no thread waits for more
// than one round of loads. With the extras, XSA then the gate (kernels.metal:1355-1361): o -=
// xsa[h] (o . v) v, o *= 2 sigmoid(rms_norm(x)[:D] . attn_gate[h]); a column's D / 4 threads
// are consecutive lanes of part 0 (the launch keeps 256 / P >= D / 4) and add the dot products
// by lane exchange.
template <int D, bool INL>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p, uint32_t P) {
  __shared__ f32x4 so[256];
  __shared__ float sl[256];
  const uint32_t G4 = 256 / P, part = threadIdx.x / G4, gi = threadIdx.x % G4;
  const uint32_t r = blockIdx.x, g = blockIdx.y, i4 = blockIdx.z * G4 + gi;
  uint32_t t0, T, seq;
  run_header<INL>(p, r, t0, T, seq);
  const uint32_t ncols = T * p.G;
  const bool live = 4 * i4 < ncols * D;
  const uint32_t col = live ? (4 * i4) / D : 0u, d = (4 * i4) % D;
  const uint32_t p0 = p.meta[2 * t0 + 1];
  const size_t rec0 = ((size_t)r * p.NKV + g) * p.max_splits;
  const size_t so_stride = (size_t)p.maxcols * D;
  const float* po = p.part_o + rec0 * so_stride + (size_t)col * D + d;
  const float* pl = p.part_l + rec0 * p.maxcols + col;
  f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
  float l = 0.0f;
  for (uint32_t sp = part; sp < p.max_splits; sp += 8 * P) {
    f32x4 ov[8];
    float lv[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const uint32_t x = sp + u * P;
      const bool in = live && x < p.max_splits;
      ov[u] = in ? *(const f32x4*)(po + x * so_stride) : f32x4{0.f, 0.f, 0.f, 0.f};
      lv[u] = in ? pl[x * p.maxcols] : 0.0f;
    }
    const uint32_t nsplit = attn_nsplit(p, p0);  // after the loads are issued
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (sp + u * P < nsplit) {
        o += ov[u];
        l += lv[u];
      }
  }
  if (P > 1) {
    so[threadIdx.x] = o;
    sl[threadIdx.x] = l;
    __syncthreads();
    if (part != 0) return;
    for (uint32_t j = 1; j < P; j++) {
      o += so[j * G4 + gi];
      l += sl[j * G4 + gi];
    }
  }
  if (!live || attn_nsplit(p, p0) > p.max_splits) return;  // NaN written by the attention
  const uint32_t i = col / p.G, h = g * p.G + col % p.G, t = t0 + i;
  f32x4 res = o / l;
  if (p.cap_sdpa) *(f32x4*)(p.cap_sdpa + (size_t)t * p.NQ * D + h * D + d) = res;
  if (p.xsa) {
    const f32x4 vd = *(const f32x4*)(p.vdir + ((size_t)t * p.NKV + g) * D + d);
    float dp = ((res[0] * vd[0] + res[1] * vd[1]) + res[2] * vd[2]) + res[3] * vd[3];
#pragma unroll
    for (int m = 1; m < D / 4; m <<= 1) dp += __shfl_xor(dp, m, WAVE);
    const float c = p.xsa[h] * dp;
#pragma unroll
    for (int e = 0; e < 4; e++) res[e] = __builtin_fmaf(-c, vd[e], res[e]);
  }
  if (p.attn_gate) {
    const f32x4 xv = *(const f32x4*)(p.x + (size_t)t * p.H + d);
    const f32x4 gv = *(const f32x4*)(p.attn_gate + (size_t)h * D + d);
    const float iv = p.inv[t];
    float gs = (((xv[0] * iv) * gv[0] + (xv[1] * iv) * gv[1]) + (xv[2] * iv) * gv[2]) + (xv[3] * iv) * gv[3];
#pragma unroll
    for (int m = 1; m < D / 4; m <<= 1) gs += __shfl_xor(gs, m, WAVE);
    res *= 2.0f * sigmoid_f(gs);
  }
  *(f32x4*)(p.out + (size_t)t * p.NQ * D + h * D + d) = res;
}

// Prompt chunks (qkv_post, kernels.metal:749-801, for the chunk path of encode.rs:300-355):
// every attention run's new K/V rows (norm, RoPE, bf16) to the cache before any run reads
// them, so a chunk's later runs of 16 rows find its earlier rows as cached keys. The same
// new_keys code as the attention's own pass, so both write the same bits. Grid (runs, kv
// heads).
template <int D, bool INL>
__global__ __launch_bounds__(256) void kv_write_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t nk[SV_MAX_RUN * D], nv[SV_MAX_RUN * D];
  uint32_t t0, T, seq;
  run_header<INL>(p, blockIdx.x, t0, T, seq);
  new_keys<D, false>(p, seq, blockIdx.y, t0, T, p.meta[2 * t0 + 1], nk, nv, threadIdx.x, 256);
}

// Dynamic LDS of up to 4 x 64 x 128 floats (+ l): allow it once per instantiation, outside
// any graph capture (sv_engine_create calls this; attn_launch does on its first use).
void attn_init() {
  static bool done = false;
  if (done) return;
  done = true;
#define SV_ATTR3(DD, N, B, I, LC)                                                                   \
  (void)hipFuncSetAttribute((const void*)attn_verify_kernel<DD, N, B, I, LC>,                    \
                            hipFuncAttributeMaxDynamicSharedMemorySize,                           \
                            (int)((size_t)4 * 16 * N * DD * 4 + (size_t)4 * 16 * N * 4))
#define SV_ATTR2(DD, N, B, I) SV_ATTR3(DD, N, B, I, false)
#define SV_ATTR1(DD, N, B) \
  SV_ATTR2(DD, N, B, true); \
  SV_ATTR2(DD, N, B, false)
#define SV_ATTR(DD, N)                 \
  SV_ATTR1(DD, N, 0);                  \
  SV_ATTR3(DD, N, 0, true, true);      \
  SV_ATTR3(DD, N, 0, false, true)
  SV_ATTR1(64, 1, SV_ATTN_NBW);
  SV_ATTR1(64, 2, SV_ATTN_NBW);
  SV_ATTR(64, 1);
  SV_ATTR(64, 2);
  SV_ATTR(64, 3);
  SV_ATTR(64, 4);
  SV_ATTR(128, 1);
  SV_ATTR(128, 2);
  SV_ATTR(128, 3);
  SV_ATTR(128, 4);
#undef SV_ATTR
#undef SV_ATTR1
#undef SV_ATTR2
#undef SV_ATTR3
}

// Compute units of the current device (the all-batches-in-flight choice).
// sv_step_capture (engine.rs:318-355; kernels.metal:932,1035): each token's queries after the
// norm and RoPE, and its new keys after the norm and RoPE and values after the value embedding,
// computed by the verify kernel's own loads and device code (qfinish_cs, new_keys), so they are
// the bits the attention used; nothing else is written. Grid (kv heads, runs); launched only by
// the capture step, after the layer's attention.
template <int D, int NCT, bool INL>
__global__ __launch_bounds__(256) void attn_capture_kernel(AttnParams p) {
  constexpr int KST = D / 32;
  __shared__ __attribute__((aligned(16))) uint16_t nk[SV_MAX_RUN * D], nv[SV_MAX_RUN * D];
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, q = lane >> 4;
  const uint32_t g = blockIdx.x, r = blockIdx.y;
  uint32_t t0, T, seq;
  run_header<INL>(p, r, t0, T, seq);
  const uint32_t ncols = T * p.G;
  if (tid < 64) {
    QRaw<D, NCT> qr;
#pragma unroll
    for (int ct = 0; ct < NCT; ct++) {
      const uint32_t c = min(16u * ct + c16, ncols - 1), i = c / p.G, h = g * p.G + c % p.G, t = t0 + i;
      qr.pos[ct] = p.meta[2 * t + 1];
      const size_t qo = (size_t)t * p.W + h * D + 8 * q;
#pragma unroll
      for (int ks = 0; ks < KST; ks++) {
        const f32x4 a = *(const f32x4*)(p.qkv + qo + 32 * ks), b = *(const f32x4*)(p.qkv + qo + 32 * ks + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          qr.v[ct][ks][e] = a[e];
          qr.v[ct][ks][4 + e] = b[e];
        }
      }
    }
    float2 cs[NCT][KST][4];
    const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(INL ? p.rope_rows : p.rope), 0, p.rope_on ? 0x7fffffff : 0, 0x00020000);
#pragma unroll
    for (int ct = 0; ct < NCT; ct++)
#pragma unroll
      for (int ks = 0; ks < KST; ks++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const uint32_t j = 16 * ks + 4 * q + jj;
          const bool on = p.rope_on && 32 * ks + 8 * q < 64;
          const uint32_t c = min(16u * ct + c16, ncols - 1);
          const uint32_t row = INL ? t0 + c / p.G : qr.pos[ct];
          const uint32_t off = (row * SV_ROPE_PAIRS + j) * 8 + (on ? 0u : 0x80000000u);
          cs[ct][ks][jj] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rrs, off, 0, 0));
          if (!on) cs[ct][ks][jj] = float2{1.0f, 0.0f};
        }
#pragma unroll
    for (int ct = 0; ct < NCT; ct++)
      if (16u * ct + c16 >= ncols)
#pragma unroll
        for (int ks = 0; ks < KST; ks++)
#pragma unroll
          for (int e = 0; e < 8; e++) qr.v[ct][ks][e] = 0.0f;
    bf16x8 qh[NCT][KST], ql[NCT][KST];
    qfinish_cs<D, NCT, true>(p, ncols, qr, cs, qh, ql, lane, t0, g);
  }
  new_keys<D, false, true, false>(p, seq, g, t0, T, p.meta[2 * t0 + 1], nk, nv, tid, 256);
}

static uint32_t attn_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return (uint32_t)cus;
}
thread_local AttnCapture g_attn_capture;
bool g_attn_fused_merge = false;  // tests: the last split to arrive merges (bit-identical, measured slower)
int g_attn_allin = -1;  // -1: by shape; 0 / 1: force the one-batch-ahead / all-batches variant where built

static uint32_t cols_pad(const sv_shape* sh, uint32_t max_run) {
  const uint32_t cols = max_run * (sh->n_heads / sh->n_kv_heads);
  return (cols + 15) / 16 * 16;
}

size_t attn_ws_bytes(const sv_shape* sh, uint32_t n_runs, uint32_t max_splits, uint32_t max_run) {
  const size_t maxcols = cols_pad(sh, max_run);
  size_t b = ((size_t)n_runs * sh->n_kv_heads * 4 + 255) / 256 * 256;
  b += (size_t)n_runs * sh->n_kv_heads * max_splits * maxcols * sh->head_dim * 4;
  b = (b + 255) / 256 * 256;
  b += (size_t)n_runs * sh->n_kv_heads * max_splits * maxcols * 4;
  return b;
}

sv_status attn_launch(hipStream_t stream, const sv_shape* sh, const float* qkv, const uint32_t* meta,
                      uint16_t* k_cache, uint16_t* v_cache, const uint32_t* page_table, const float* rope,
                      const sv_kv_args* kv, const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs,
                      uint32_t max_run, const uint32_t* vis, float* out, void* ws, size_t ws_bytes,
                      uint32_t parts, const uint32_t* host_runs, bool may_fuse, const sv_attn_extras* ex,
                      const float* rope_rows) {
  if (!sh || !qkv || !meta || !k_cache || !v_cache || !page_table || !kv || !args || !runs || !vis || !out)
    return fail(SV_ERR_ARG, "attn_verify: null pointer");
  if (n_runs == 0) return SV_OK;
  const uint32_t D = sh->head_dim, NQ = sh->n_heads, NKV = sh->n_kv_heads;
  if (D != 64 && D != 128) return fail(SV_ERR_UNSUPPORTED, "attn_verify: head_dim %u (64 or 128 are built)", D);
  if (NKV == 0 || NQ % NKV) return fail(SV_ERR_ARG, "attn_verify: %u heads over %u kv heads", NQ, NKV);
  if (!kv->is_global && kv->window == 0) return fail(SV_ERR_ARG, "attn_verify: a sliding-window layer with window 0");
  if (ex) {
    if ((ex->d_ve_gate && (!ex->d_value_embed || !ex->d_tokens)) || ((ex->d_ve_gate || ex->d_attn_gate) && (!ex->d_x || !ex->d_inv)) ||
        (ex->d_xsa && !ex->d_vdir))
      return fail(SV_ERR_ARG, "attn_verify: an extra without its inputs (ve_gate needs x, inv, tokens, value_embed; "
                              "attn_gate x, inv; xsa vdir)");
    if ((ex->d_ve_gate || ex->d_attn_gate) && ex->hidden < D)
      return fail(SV_ERR_ARG, "attn_verify: hidden %u below head_dim %u", ex->hidden, D);
  }
  if (kv->page_shift < 4 || kv->page_shift > 16)
    return fail(SV_ERR_UNSUPPORTED, "attn_verify: pages of 2^%u tokens (16..65536 are built)", kv->page_shift);
  if (args->split == 0 || args->split % 32 || args->split > 3968)
    return fail(SV_ERR_ARG, "attn_verify: split %u (a multiple of 32, at most 3968)", args->split);
  if (max_run == 0 || max_run > SV_MAX_RUN) return fail(SV_ERR_ARG, "attn_verify: max_run %u", max_run);
  if (!rope && args->rope) return fail(SV_ERR_ARG, "attn_verify: rope table missing");
  const uint32_t maxcols = cols_pad(sh, max_run), nct = maxcols / 16;
  if (nct > SV_MAX_COLS / 16)
    return fail(SV_ERR_UNSUPPORTED, "attn_verify: %u columns per kv head (%u are built)", max_run * NQ / NKV, SV_MAX_COLS);
  // The merge runs as its own launch over (run, kv head, column) workgroups (measured
  // faster at 9-65 splits); with g_attn_fused_merge set the last split of each (run, kv head)
  // to arrive merges instead.
  const bool merge_extras = ex && (ex->d_xsa || ex->d_attn_gate);
  // merge parts: enough that a thread adds at most eight splits (a power of two, up to 64)
  // (with XSA or the gate, a column's D / 4 threads stay in part 0: P <= 1024 / D); the fused
  // merge holds its parts' sums in the reduction buffer: P <= 4
  const uint32_t P_max = merge_extras ? 1024u / D : 64u;
  uint32_t P = 1;
  while (P < P_max && 8 * P < args->max_splits) P *= 2;
  const bool fused_merge = may_fuse && g_attn_fused_merge && !merge_extras && P <= 4;
  const size_t need = attn_ws_bytes(sh, n_runs, args->max_splits, max_run);
  if (!ws || ws_bytes < need) return fail(SV_ERR_ARG, "attn_verify: workspace %zu < %zu bytes", ws_bytes, need);
  AttnParams p;
  p.qkv = qkv;
  p.meta = meta;
  p.kc = k_cache;
  p.vc = v_cache;
  p.page_table = page_table;
  p.rope = rope;
  p.runs = runs;
  p.vis = vis;
  p.out = out;
  // counters (zero at rest), then the partials
  p.counters = fused_merge ? (uint32_t*)ws : nullptr;
  p.merge_parts = P;
  size_t off = ((size_t)n_runs * NKV * 4 + 255) / 256 * 256;
  p.part_o = (float*)((char*)ws + off);
  off += (size_t)n_runs * NKV * args->max_splits * maxcols * D * 4;
  off = (off + 255) / 256 * 256;
  p.part_l = (float*)((char*)ws + off);
  p.NQ = NQ;
  p.NKV = NKV;
  p.G = NQ / NKV;
  p.W = (NQ + 2 * NKV) * D;
  p.KOFF = NQ * D;
  p.VOFF = (NQ + NKV) * D;
  p.split = args->split;
  p.max_splits = args->max_splits;
  p.scale_log2 = args->scale_log2;
  p.rope_on = args->rope;
  p.page_shift = kv->page_shift;
  p.n_pages = kv->n_pages;
  p.max_pages = kv->max_pages;
  p.layer = kv->kv_layer;
  p.maxcols = maxcols;
  p.n_inline = 0;
  p.newest_own = 1;
  p.local = kv->is_global ? 0u : 1u;
  p.window = kv->window;
  p.x = ex ? ex->d_x : nullptr;
  p.inv = ex ? ex->d_inv : nullptr;
  p.tokens = ex ? ex->d_tokens : nullptr;
  p.vemb = ex ? ex->d_value_embed : nullptr;
  p.ve_gate = ex ? ex->d_ve_gate : nullptr;
  p.attn_gate = ex ? ex->d_attn_gate : nullptr;
  p.xsa = ex ? ex->d_xsa : nullptr;
  p.vdir = ex && ex->d_xsa ? ex->d_vdir : nullptr;
  p.H = ex ? ex->hidden : 0u;
  p.cap_q = g_attn_capture.q;
  p.cap_k = g_attn_capture.k;
  p.cap_v = g_attn_capture.v;
  p.cap_sdpa = g_attn_capture.sdpa;
  p.rope_rows = rope_rows;
  // inline runs take the queries' rope words from the step's rows by token
  if (host_runs && rope_rows && n_runs <= SV_INLINE_RUNS) {
    p.n_inline = n_runs;
    for (uint32_t i = 0; i < 3 * n_runs; i++) p.inl[i] = host_runs[i];
  }
  attn_init();
  // All of a wave's batches in flight where the grid is about one workgroup per CU (latency,
  // not throughput, bounds it) and a wave has at most SV_ATTN_NBW batches. The new keys' split
  // follows attn_newest_own for the variant launched.
  const bool fits = D == 64 && nct <= 2 && args->split <= 128u * SV_ATTN_NBW && !p.local;
  const bool allin = fits && (g_attn_allin == 1 || (g_attn_allin < 0 && (size_t)args->max_splits * NKV * n_runs <= attn_cus()));
  p.newest_own = attn_newest_own((int)nct, allin ? SV_ATTN_NBW : 0) ? 1u : 0u;
  if (parts & 4) {
    const dim3 g4(n_runs, NKV);
    if (D == 64) {
      if (p.n_inline) launch(kv_write_kernel<64, true>, g4, dim3(256), 0, stream, p);
      else launch(kv_write_kernel<64, false>, g4, dim3(256), 0, stream, p);
    } else {
      if (p.n_inline) launch(kv_write_kernel<128, true>, g4, dim3(256), 0, stream, p);
      else launch(kv_write_kernel<128, false>, g4, dim3(256), 0, stream, p);
    }
    SV_TRY_LAUNCH("kv_write");
  }
  if (parts & 1) {
    dim3 grid(args->max_splits, NKV, n_runs);
    // the reduction buffer, at least the 4 waves' V stages (2 x 16 rows of 2 D + 32 bytes) it holds
    const size_t shm = std::max((size_t)4 * maxcols * D * 4 + (size_t)4 * maxcols * 4, (size_t)4 * 32 * (2 * D + 32));
    const bool inl = p.n_inline != 0;
#define SV_ATTN3(DD, N, B)                                                          \
  do {                                                                              \
    if (inl) launch((attn_verify_kernel<DD, N, B, true>), grid, dim3(256), shm, stream, p);  \
    else launch((attn_verify_kernel<DD, N, B, false>), grid, dim3(256), shm, stream, p);     \
  } while (0)
  // sliding-window layers: the streaming variant with the window compiled in
#define SV_ATTN(DD, N)                                                                                   \
  do {                                                                                                   \
    if (!p.local) SV_ATTN3(DD, N, 0);                                                                    \
    else if (inl) launch((attn_verify_kernel<DD, N, 0, true, true>), grid, dim3(256), shm, stream, p);   \
    else launch((attn_verify_kernel<DD, N, 0, false, true>), grid, dim3(256), shm, stream, p);           \
  } while (0)
    if (allin) {
      if (nct == 1) SV_ATTN3(64, 1, SV_ATTN_NBW);
      else SV_ATTN3(64, 2, SV_ATTN_NBW);
    } else if (D == 64) {
      switch (nct) {
        case 1: SV_ATTN(64, 1); break;
        case 2: SV_ATTN(64, 2); break;
        case 3: SV_ATTN(64, 3); break;
        default: SV_ATTN(64, 4); break;
      }
    } else {
      switch (nct) {
        case 1: SV_ATTN(128, 1); break;
        case 2: SV_ATTN(128, 2); break;
        case 3: SV_ATTN(128, 3); break;
        default: SV_ATTN(128, 4); break;
      }
    }
#undef SV_ATTN
#undef SV_ATTN3
    SV_TRY_LAUNCH("attn_verify");
  }
  if (parts & 8) {
    // the capture step's queries, keys and values (attn_capture_kernel)
    if (!p.cap_q || !p.cap_k || !p.cap_v) return fail(SV_ERR_ARG, "attn_verify: capture without its buffers");
    const dim3 gc(NKV, n_runs);
    const bool inl = p.n_inline != 0;
#define SV_ATTN_CAP(DD, N)                                                              \
  do {                                                                                  \
    if (inl) launch((attn_capture_kernel<DD, N, true>), gc, dim3(256), 0, stream, p);   \
    else launch((attn_capture_kernel<DD, N, false>), gc, dim3(256), 0, stream, p);      \
  } while (0)
    if (D == 64) {
      switch (nct) {
        case 1: SV_ATTN_CAP(64, 1); break;
        case 2: SV_ATTN_CAP(64, 2); break;
        case 3: SV_ATTN_CAP(64, 3); break;
        default: SV_ATTN_CAP(64, 4); break;
      }
    } else {
      switch (nct) {
        case 1: SV_ATTN_CAP(128, 1); break;
        case 2: SV_ATTN_CAP(128, 2); break;
        case 3: SV_ATTN_CAP(128, 3); break;
        default: SV_ATTN_CAP(128, 4); break;
      }
    }
#undef SV_ATTN_CAP
    SV_TRY_LAUNCH("attn_capture");
  }
  if (fused_merge || !(parts & 2)) return SV_OK;
  const uint32_t G4 = 256 / P, mz = (maxcols * D / 4 + G4 - 1) / G4;
  const dim3 mg(n_runs, NKV, mz);
  if (D == 64) {
    if (p.n_inline) launch(attn_merge_kernel<64, true>, mg, dim3(256), 0, stream, p, P);
    else launch(attn_merge_kernel<64, false>, mg, dim3(256), 0, stream, p, P);
  } else {
    if (p.n_inline) launch(attn_merge_kernel<128, true>, mg, dim3(256), 0, stream, p, P);
    else launch(attn_merge_kernel<128, false>, mg, dim3(256), 0, stream, p, P);
  }
  return check_launch("attn_merge");
}

// ------------------------------------------- the persistent layer kernel's attention
// Floats of one layer's split partials (o, then l at *l_off), 64-float aligned.
size_t attn_part_floats(const sv_shape* sh, uint32_t n_runs, uint32_t max_splits, uint32_t max_run, size_t* l_off) {
  const size_t maxcols = cols_pad(sh, max_run);
  const size_t o = ((size_t)n_runs * sh->n_kv_heads * max_splits * maxcols * sh->head_dim + 63) / 64 * 64;
  *l_off = o;
  return o + ((size_t)n_runs * sh->n_kv_heads * max_splits * maxcols + 63) / 64 * 64;
}

sv_status attn_params_fill(void* out, const sv_shape* sh, const float* qkv, const uint32_t* meta, uint16_t* k_cache,
                           uint16_t* v_cache, const uint32_t* page_table, const float* rope_rows,
                           const sv_kv_args* kv, const sv_attn_args* args, const uint32_t* host_runs,
                           uint32_t n_runs, uint32_t max_run, const uint32_t* vis, float* o, float* part_o,
                           float* part_l) {
  if (!out || !sh || !kv || !args || !host_runs) return fail(SV_ERR_ARG, "layers: attention arguments");
  if (n_runs == 0 || n_runs > SV_INLINE_RUNS) return fail(SV_ERR_UNSUPPORTED, "layers: %u attention runs", n_runs);
  if (sh->head_dim != 64 || !kv->is_global || args->split % 32 || args->split > 32u * 4 * 4)
    return fail(SV_ERR_UNSUPPORTED, "layers: head_dim %u, global %u, split %u", sh->head_dim, kv->is_global, args->split);
  if (args->rope && !rope_rows) return fail(SV_ERR_ARG, "layers: rope rows missing");
  AttnParams p{};
  p.qkv = qkv;
  p.meta = meta;
  p.kc = k_cache;
  p.vc = v_cache;
  p.page_table = page_table;
  p.rope = nullptr;
  p.rope_rows = rope_rows;
  p.runs = nullptr;
  p.vis = vis;
  p.out = o;
  p.part_o = part_o;
  p.part_l = part_l;
  p.counters = nullptr;
  p.merge_parts = 1;
  p.NQ = sh->n_heads;
  p.NKV = sh->n_kv_heads;
  p.G = sh->n_heads / sh->n_kv_heads;
  p.W = (sh->n_heads + 2 * sh->n_kv_heads) * sh->head_dim;
  p.KOFF = sh->n_heads * sh->head_dim;
  p.VOFF = (sh->n_heads + sh->n_kv_heads) * sh->head_dim;
  p.split = args->split;
  p.max_splits = args->max_splits;
  p.scale_log2 = args->scale_log2;
  p.rope_on = args->rope;
  p.page_shift = kv->page_shift;
  p.n_pages = kv->n_pages;
  p.max_pages = kv->max_pages;
  p.layer = kv->kv_layer;
  p.maxcols = cols_pad(sh, max_run);
  p.n_inline = n_runs;
  for (uint32_t i = 0; i < 3 * n_runs; i++) p.inl[i] = host_runs[i];
  p.newest_own = 1;
  p.local = 0;
  p.window = 0;
  memcpy(out, &p, sizeof p);
  return SV_OK;
}

// ------------------------------------------------- the entry point that allocates nothing
// Split partials of sv_attn_verify_noalloc live in this array: one copy per GPU, held until the
// process ends. Its name is a host-side stand-in; host code uses the device address that
// hipGetSymbolAddress returns for the current device. The partials need no clearing: every
// partial the merge reads is written by the same call (the counted merge, which needs counters
// at zero, is not used here).
constexpr size_t ATTN_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[ATTN_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static std::vector<void*> g_scratch_ptr;  // per device

static sv_status scratch_address(void** out) {
  int dev = 0;
  const hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) return check_hip(de, "attn_verify_noalloc: device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((size_t)dev >= g_scratch_ptr.size()) g_scratch_ptr.resize(dev + 1, nullptr);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(SV_ERR_HIP, "attn_verify_noalloc: scratch address: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SV_OK;
}

size_t attn_scratch_bytes() { return ATTN_SCRATCH_BYTES; }

sv_status attn_launch_noalloc(hipStream_t stream, const sv_shape* sh, const float* qkv, const uint32_t* meta,
                              uint16_t* k_cache, uint16_t* v_cache, const uint32_t* page_table, const float* rope,
                              const sv_kv_args* kv, const sv_attn_args* args, const uint32_t* runs, uint32_t n_runs,
                              uint32_t max_run, const uint32_t* vis, float* out) {
  if (!sh || !args) return fail(SV_ERR_ARG, "attn_verify_noalloc: null pointer");
  if (max_run == 0 || max_run > SV_MAX_RUN) return fail(SV_ERR_ARG, "attn_verify_noalloc: max_run %u", max_run);
  const size_t need = attn_ws_bytes(sh, n_runs, args->max_splits, max_run);
  if (need > ATTN_SCRATCH_BYTES)
    return fail(SV_ERR_CAPACITY, "attn_verify_noalloc: %zu bytes of split partials exceed the %zu-byte scratch", need,
                ATTN_SCRATCH_BYTES);
  void* ws = nullptr;
  const sv_status st = scratch_address(&ws);
  if (st != SV_OK) return st;
  return attn_launch(stream, sh, qkv, meta, k_cache, v_cache, page_table, rope, kv, args, runs, n_runs, max_run, vis,
                     out, ws, ATTN_SCRATCH_BYTES, 3, nullptr, false, nullptr);
}

}  // namespace sv
