// attn_device.h — device pieces of the verify attention (attn_verify_kernel, kv_write_kernel):
// paged K/V addressing, the 32-key batch (load + MFMA products), the query build and the
// new-key pass (the reference's attn_verify, engine/src/kernels.metal:891-1148).
#pragma once
#include "sv_device.h"

namespace sv {

constexpr uint32_t SV_INLINE_RUNS = 32;

struct AttnParams {
  const float* qkv;
  const uint32_t* meta;
  uint16_t* kc;
  uint16_t* vc;
  const uint32_t* page_table;
  const float* rope;
  // The step's rope words by token (the table's row at each token's position, written by the
  // embed kernel): with inline runs the queries' rope words need no position first.
  const float* rope_rows;
  const uint32_t* runs;
  const uint32_t* vis;
  float* out;
  float* part_o;
  float* part_l;
  uint32_t* counters;  // per (run, kv head): fused merge; null: attn_merge_kernel merges
  uint32_t merge_parts;  // the merge's parts P (both merges: splits j, j + P, ... per part)
  uint32_t NQ, NKV, G, W, KOFF, VOFF;
  uint32_t split, max_splits;
  float scale_log2;
  uint32_t rope_on;
  uint32_t page_shift, n_pages, max_pages, layer, maxcols;
  // Runs known to the host when the launch is encoded (the engine's plan): (first token,
  // rows, sequence slot) per run, so the kernels start without reading runs and meta; 0: read
  // them from `runs` / `meta`.
  uint32_t n_inline;
  uint32_t inl[3 * SV_INLINE_RUNS];
  // 1: a run's new keys have a split of their own (after its cached splits); 0: its last cached
  // split (or the only split, without cached keys) takes them too.
  uint32_t newest_own;
  // Sliding-window layer (kernels.metal:808-811): a query at pos sees cached keys from
  // pos - window on; 0: every cached key.
  uint32_t local, window;
  // The layer extras (null: off): value embeddings in the new V rows, the XSA directions they
  // leave in vdir, and the merge's XSA and gate.
  const float* x;
  const float* inv;
  const uint32_t* tokens;
  const uint16_t* vemb;
  const float* ve_gate;
  const float* attn_gate;
  const float* xsa;
  float* vdir;
  uint32_t H;
  // Per-layer capture (sv_step_capture; null: off): each token's queries after the norm and
  // RoPE [n][NQ D], its keys after the norm and RoPE and values after the value embedding
  // [n][NKV D] (written by attn_capture_kernel only), and the attention output before XSA and
  // the gate [n][NQ D] (by the merge), all fp32.
  float* cap_q;
  float* cap_k;
  float* cap_v;
  float* cap_sdpa;
};

// The first cached key the query at pos sees (kernels.metal:808-811 key_lo); LOCAL: the layer
// is a sliding-window one (a compile-time choice in the attention kernel, so global layers
// carry none of it).
template <bool LOCAL>
__device__ __forceinline__ uint32_t key_lo_t(const AttnParams& p, uint32_t pos) {
  return LOCAL && pos > p.window ? pos - p.window : 0u;
}
// A run's cached keys start at its first query's key_lo rounded down to a batch (32 keys):
// batches stay aligned to the tiles of 16 keys; keys below a column's key_lo are masked.
template <bool LOCAL>
__device__ __forceinline__ uint32_t key_base_t(const AttnParams& p, uint32_t p0) { return key_lo_t<LOCAL>(p, p0) & ~31u; }

// Splits of a run whose first position is p0.
template <bool LOCAL>
__device__ __forceinline__ uint32_t attn_nsplit_t(const AttnParams& p, uint32_t p0) {
  const uint32_t c = (p0 - key_base_t<LOCAL>(p, p0) + p.split - 1) / p.split;
  return p.newest_own ? c + 1 : (c ? c : 1u);
}
__device__ __forceinline__ uint32_t attn_nsplit(const AttnParams& p, uint32_t p0) {
  return p.local ? attn_nsplit_t<true>(p, p0) : attn_nsplit_t<false>(p, p0);
}

__device__ __forceinline__ float sigmoid_f(float x) {
  return 1.0f / (1.0f + __builtin_amdgcn_exp2f(-x * 1.44269504088896340736f));
}

// Run r's first token, rows and sequence slot: from the kernel arguments (INL: the launch
// carries the runs, read by scalar loads issued with the other arguments, so no round trip is
// spent on the header alone) or from runs / meta.
template <bool INL>
__device__ __forceinline__ void run_header(const AttnParams& p, uint32_t r, uint32_t& t0, uint32_t& T, uint32_t& seq) {
  if constexpr (INL) {
    t0 = p.inl[3 * r];
    T = p.inl[3 * r + 1];
    seq = p.inl[3 * r + 2];
  } else {
    t0 = p.runs[2 * r];
    T = p.runs[2 * r + 1];
    seq = p.meta[2 * t0];
  }
}

// Element offset of kv head g's row at cache position pos (kernels.metal:704-711, global).
template <int D>
__device__ __forceinline__ size_t kv_off(const AttnParams& p, uint32_t seq, uint32_t g, uint32_t pos) {
  // Clamped to the table and the pool: keys read ahead of knowing the context length (and
  // masked later) stay in bounds; valid positions are unchanged.
  const uint32_t pi = min(pos >> p.page_shift, p.max_pages - 1);
  const uint32_t page = min(p.page_table[(size_t)seq * p.max_pages + pi], p.n_pages - 1);
  return ((((size_t)p.layer * p.n_pages + page) * p.NKV + g) << p.page_shift) * D +
         (size_t)(pos & ((1u << p.page_shift) - 1u)) * D;
}

// Lane `l`'s 64-bit value, for a wave-uniform l.
__device__ __forceinline__ size_t readlane64(size_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l), hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
  return ((size_t)hi << 32) | lo;
}

template <int VE>
struct VWord;
template <>
struct VWord<4> {
  typedef u32x2 type;
};
template <>
struct VWord<8> {
  typedef u32x4 type;
};

// One batch of 32 keys [kb, kb + 32) below kend, for one wave: its K and V words (loaded
// ahead of use) and the products. NEW: the keys are the run's new ones, in LDS (index
// key - p0), masked by each column's vis.
template <int D>
struct KvBatch {
  static constexpr int KST = D / 32, VE = D / 16;
  typedef typename VWord<VE>::type vword;
  u32x4 kw[2][KST];  // lane (c16, q): key kb + 16 mt + c16, dims 32 ks + 8 q .. + 7
  vword vw[8];       // slot j: key kb + 16 (j / 4) + 4 q + j % 4, dims VE c16 .. + VE - 1
};

// toff: the element offsets of the batch's two 16-key tiles when the caller has them (no
// page-table load then).
template <int D, bool NEW>
__device__ __forceinline__ void load_batch(const AttnParams& p, uint32_t seq, uint32_t g, uint32_t kb, uint32_t kend,
                                           uint32_t p0, const uint16_t* nk, const uint16_t* nv, KvBatch<D>& b,
                                           int lane, const size_t* toff = nullptr) {
  constexpr int KST = D / 32, VE = D / 16;
  typedef typename KvBatch<D>::vword vword;
  const int c16 = lane & 15, q = lane >> 4;
  // A tile of 16 keys never straddles a page (pages hold >= 16 keys, kb is a multiple of 32).
#pragma unroll
  for (int mt = 0; mt < 2; mt++) {
    const uint32_t first = min(kb + 16 * mt, kend - 1);
    const uint16_t* kt;
    const uint16_t* vt;
    if (NEW) {
      kt = nk + (size_t)(first - p0) * D;
      vt = nv + (size_t)(first - p0) * D;
    } else {
      const size_t off = toff ? toff[mt] : kv_off<D>(p, seq, g, first);
      kt = p.kc + off;
      vt = p.vc + off;
    }
    const uint32_t key = min(kb + 16 * mt + c16, kend - 1);
    const uint16_t* kr = kt + (size_t)(key - first) * D;
#pragma unroll
    for (int ks = 0; ks < KST; ks++) b.kw[mt][ks] = *(const u32x4*)(kr + 32 * ks + 8 * q);
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      const uint32_t vk = min(kb + 16 * mt + 4 * q + jj, kend - 1);
      b.vw[4 * mt + jj] = *(const vword*)(vt + (size_t)(vk - first) * D + VE * c16);
    }
  }
}

// A cached batch through per-tile buffer descriptors: its two 16-key tiles start at the
// page-aligned positions kb and kb + 16 (toff: their element offsets, the page table applied,
// clamped into the pool), so a tile's 16 keys lie in its page and each lane's byte offset
// within a tile is the same for every batch: no per-key address arithmetic. Keys at or past
// the context end are read (inside the page) and masked by compute_batch.
template <int D>
__device__ __forceinline__ void load_batch_tiles(const AttnParams& p, const size_t* toff, KvBatch<D>& b, int lane) {
  constexpr int KST = D / 32, VE = D / 16;
  typedef typename KvBatch<D>::vword vword;
  const int c16 = lane & 15, q = lane >> 4;
  const uint32_t ko = (uint32_t)(c16 * D + 8 * q) * 2;      // key c16, dims 8 q .. (+ 32 ks)
  const uint32_t vo = (uint32_t)(4 * q * D + VE * c16) * 2;  // key 4 q (+ jj), dims VE c16 ..
#pragma unroll
  for (int mt = 0; mt < 2; mt++) {
    const __amdgpu_buffer_rsrc_t krs = coherent_rsrc(p.kc + toff[mt]), vrs = coherent_rsrc(p.vc + toff[mt]);
#pragma unroll
    for (int ks = 0; ks < KST; ks++) b.kw[mt][ks] = buf_ld16(krs, ko + 64 * ks, 0);
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      if constexpr (VE == 4)
        b.vw[4 * mt + jj] = __builtin_bit_cast(vword, __builtin_amdgcn_raw_buffer_load_b64(vrs, vo + jj * D * 2, 0, 0));
      else
        b.vw[4 * mt + jj] = __builtin_bit_cast(vword, buf_ld16(vrs, vo + jj * D * 2, 0));
    }
  }
}

// FULL: every key of the batch is below kend (no key mask). Columns past ncols need no mask
// either: their queries are zero, so they only fill partial sums that are never stored.
// p = 2^s by the hardware exp (v_exp_f32): q and k are rms-normed, so |s| <= D x scale x
// log2 e (11.6 at D = 64, scale 1/8) and no result is subnormal.
template <int D, int NCT, bool NEW, bool FULL = false>
__device__ __forceinline__ void compute_batch(const AttnParams& p, const KvBatch<D>& b, uint32_t kb, uint32_t kend,
                                              uint32_t p0, uint32_t ncols, uint32_t t0,
                                              const bf16x8 (&qh)[NCT][D / 32], const bf16x8 (&ql)[NCT][D / 32],
                                              f32x4 (&O)[D / 16][NCT], float (&lsum)[NCT], int lane,
                                              const uint32_t* vis_cached = nullptr) {
  constexpr int KST = D / 32, VE = D / 16;
  const int c16 = lane & 15, q = lane >> 4;
  // S^T tiles: lane holds keys kb + 16 mt + 4 q + i, column 16 ct + c16.
  f32x4 S[2][NCT];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int ct = 0; ct < NCT; ct++) {
      f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KST; ks++) {
        const bf16x8 kk = __builtin_bit_cast(bf16x8, b.kw[mt][ks]);
        a = mfma16(kk, qh[ct][ks], a);
        a = mfma16(kk, ql[ct][ks], a);
      }
      S[mt][ct] = a;
    }
  bf16x8 ph[NCT], pl[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    const uint32_t c = 16 * ct + c16;
    const bool col_ok = c < ncols;
    uint32_t vbits = 0;
    if (NEW && col_ok) vbits = vis_cached ? vis_cached[c / p.G] : p.vis[t0 + c / p.G];
    float pv[8];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t key = kb + 16 * mt + 4 * q + i;
        float e = __builtin_amdgcn_exp2f(S[mt][ct][i]);
        if (!FULL) {
          bool ok = col_ok && key < kend;
          if (NEW) ok = ok && ((vbits >> (key - p0)) & 1u);
          e = ok ? e : 0.0f;
        }
        pv[4 * mt + i] = e;
        lsum[ct] += e;
      }
    split8(pv, ph[ct], pl[ct]);
  }
  // O^T[dt] (rows: dims VE (4 q + i) + dt) += V^T[dt] P^T.
#pragma unroll
  for (int dt = 0; dt < VE; dt++) {
    u32x4 a;
    const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int jj = 0; jj < 4; jj++) a[jj] = __builtin_amdgcn_perm(b.vw[2 * jj + 1][dt >> 1], b.vw[2 * jj][dt >> 1], sel);
    const bf16x8 av = __builtin_bit_cast(bf16x8, a);
#pragma unroll
    for (int ct = 0; ct < NCT; ct++) {
      O[dt][ct] = mfma16(av, ph[ct], O[dt][ct]);
      O[dt][ct] = mfma16(av, pl[ct], O[dt][ct]);
    }
  }
}


// ----------------------------------------------------------------------------------------
// The attention kernel's batches carry V as the tile's own bytes (coalesced 16-byte loads) and
// transpose it on the way into the matrix cores through a wave-private LDS stage with gfx950's
// transposing LDS read (ds_read_b64_tr_b16: within each group of 16 lanes, lane j receives
// element j % 4 of the 8-byte rows addressed by lanes j / 4, 4 + j / 4, 8 + j / 4, 12 + j / 4).
// Output tile dt of O^T then holds dims 16 dt + row.
template <int D>
struct KvBatchT {
  static constexpr int KST = D / 32, NV = D / 32;
  u32x4 kw[2][KST];  // lane (c16, q): key kb + 16 mt + c16, dims 32 ks + 8 q .. + 7
  u32x4 vr[2][NV];   // tile mt (keys kb + 16 mt ..): its bytes 16 lane + 1024 v (rows of 2 D bytes)
};

// Cached batch through per-tile buffer descriptors (load_batch_tiles' contract).
// oob = 2^31 turns every load into a range-checked miss: zeros, no memory access (a batch
// slot past the split's last batch).
template <int D>
__device__ __forceinline__ void load_batch_tiles_t(const AttnParams& p, const size_t* toff, KvBatchT<D>& b, int lane,
                                                   uint32_t oob = 0) {
  constexpr int KST = D / 32, NV = D / 32;
  const int c16 = lane & 15, q = lane >> 4;
  const uint32_t ko = (uint32_t)(c16 * D + 8 * q) * 2 + oob, vo = 16u * lane + oob;
#pragma unroll
  for (int mt = 0; mt < 2; mt++) {
    const __amdgpu_buffer_rsrc_t krs = coherent_rsrc(p.kc + toff[mt]), vrs = coherent_rsrc(p.vc + toff[mt]);
#pragma unroll
    for (int ks = 0; ks < KST; ks++) b.kw[mt][ks] = buf_ld16(krs, ko + 64 * ks, 0);
#pragma unroll
    for (int v = 0; v < NV; v++) b.vr[mt][v] = buf_ld16(vrs, vo + 1024 * v, 0);
  }
}

// The run's new keys from LDS (nk / nv: [T][D], key p0 + row), keys clamped to kend - 1.
template <int D>
__device__ __forceinline__ void load_batch_new_t(const uint16_t* nk, const uint16_t* nv, uint32_t kb, uint32_t kend,
                                                 uint32_t p0, KvBatchT<D>& b, int lane) {
  constexpr int KST = D / 32, NV = D / 32;
  const int c16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < 2; mt++) {
    const uint32_t key = min(kb + 16 * mt + c16, kend - 1);
#pragma unroll
    for (int ks = 0; ks < KST; ks++) b.kw[mt][ks] = *(const u32x4*)(nk + (size_t)(key - p0) * D + 32 * ks + 8 * q);
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const uint32_t byte = 16 * lane + 1024 * v, row = byte / (2 * D), col = (byte % (2 * D)) / 2;
      const uint32_t vk = min(kb + 16 * mt + row, kend - 1);
      b.vr[mt][v] = *(const u32x4*)(nv + (size_t)(vk - p0) * D + col);
    }
  }
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Bytes per key row of the V stage: 2 D plus 32, an odd multiple of 32 bytes, so the 32-byte
// slabs that a transposing read takes from 8 consecutive rows fall on 8 different bank groups
// (at 2 D = 128 bytes, rows alternated between two: a 4-way conflict on gfx950's 256-byte
// banks); the stage's 16-byte writes stay 8 consecutive lanes to one row.
template <int D>
constexpr uint32_t stage_row() { return 2 * D + 32; }
template <int D>
constexpr uint32_t stage_bytes() { return 32 * stage_row<D>(); }  // 2 tiles x 16 keys

// compute_batch's semantics with V through the wave's LDS stage (2 tiles x 16 keys, rows of
// stage_row bytes).
// Keys at or past kend that a partial batch read from their page get V rows of zero, so
// whatever the cache holds there cannot reach the sums (p is 0 for them).
// clo: each lane column's first visible cached key (key_lo; 0 on global layers); a FULL batch
// lies at or above every column's.
template <int D, int NCT, bool NEW, bool FULL = false>
__device__ __forceinline__ void compute_batch_t(const AttnParams& p, const KvBatchT<D>& b, uint32_t kb, uint32_t kend,
                                                uint32_t p0, uint32_t ncols, uint32_t t0,
                                                const bf16x8 (&qh)[NCT][D / 32], const bf16x8 (&ql)[NCT][D / 32],
                                                f32x4 (&O)[D / 16][NCT], float (&lsum)[NCT], int lane, uint16_t* stage,
                                                const uint32_t (&clo)[NCT], const uint32_t* vis_cached = nullptr) {
  constexpr int KST = D / 32, VE = D / 16, NV = D / 32;
  const int c16 = lane & 15, q = lane >> 4;
  // V into the stage first (its LDS writes overlap the score products).
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < NV; v++) {
      u32x4 w = b.vr[mt][v];
      if (!FULL && !NEW) {
        const uint32_t row = (16 * lane + 1024 * v) / (2 * D);
        if (kb + 16 * mt + row >= kend) w = u32x4{0u, 0u, 0u, 0u};
      }
      const uint32_t byte = 16 * lane + 1024 * v;
      *(u32x4*)((char*)stage + (16 * mt + byte / (2 * D)) * stage_row<D>() + byte % (2 * D)) = w;
    }
  // S^T tiles: lane holds keys kb + 16 mt + 4 q + i, column 16 ct + c16.
  f32x4 S[2][NCT];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int ct = 0; ct < NCT; ct++) {
      f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KST; ks++) {
        const bf16x8 kk = __builtin_bit_cast(bf16x8, b.kw[mt][ks]);
        a = mfma16(kk, qh[ct][ks], a);
        a = mfma16(kk, ql[ct][ks], a);
      }
      S[mt][ct] = a;
    }
  bf16x8 ph[NCT], pl[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    const uint32_t c = 16 * ct + c16;
    const bool col_ok = c < ncols;
    uint32_t vbits = 0;
    if (NEW && col_ok) vbits = vis_cached ? vis_cached[c / p.G] : p.vis[t0 + c / p.G];
    float pv[8];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t key = kb + 16 * mt + 4 * q + i;
        float e = __builtin_amdgcn_exp2f(S[mt][ct][i]);
        if (!FULL) {
          bool ok = col_ok && key < kend;
          if (NEW) ok = ok && ((vbits >> (key - p0)) & 1u);
          else ok = ok && key >= clo[ct];
          e = ok ? e : 0.0f;
        }
        pv[4 * mt + i] = e;
        lsum[ct] += e;
      }
    split8(pv, ph[ct], pl[ct]);
  }
  // O^T[dt] (rows: dims 16 dt + 4 q + i) += V^T[dt] P^T; the A operand's k slots 4 mt + t are
  // keys kb + 16 mt + 4 q + t (P's layout), read transposed: lane (i, q) addresses key
  // 4 q + i / 4 of tile mt, dims 16 dt + 4 (i % 4) .. + 3.
  const uint32_t rd = (uint32_t)(4 * q + c16 / 4) * stage_row<D>() + (uint32_t)(4 * (c16 % 4)) * 2;
#pragma unroll
  for (int dt = 0; dt < VE; dt++) {
    const i16x4 h0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)((char*)stage + rd + 32 * dt));
    const i16x4 h1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)((char*)stage + 16 * stage_row<D>() + rd + 32 * dt));
    const u32x4 a = u32x4{__builtin_bit_cast(u32x2, h0)[0], __builtin_bit_cast(u32x2, h0)[1],
                          __builtin_bit_cast(u32x2, h1)[0], __builtin_bit_cast(u32x2, h1)[1]};
    const bf16x8 av = __builtin_bit_cast(bf16x8, a);
#pragma unroll
    for (int ct = 0; ct < NCT; ct++) {
      O[dt][ct] = mfma16(av, ph[ct], O[dt][ct]);
      O[dt][ct] = mfma16(av, pl[ct], O[dt][ct]);
    }
  }
}

// fp32 activation words at element offset `off` (a multiple of 4): plain, or coherent (sc1)
// when they were written earlier in the same launch by another workgroup.
template <bool COH>
__device__ __forceinline__ f32x4 ld_act(const float* base, size_t off) {
  if (COH) return load_wt4(coherent_rsrc(base), (uint32_t)(off * 4));
  return *(const f32x4*)(base + off);
}

// Raw query words of a lane's columns (loaded) before the norm, RoPE and split.
template <int D, int NCT>
struct QRaw {
  float v[NCT][D / 32][8];
  uint32_t pos[NCT];
};

template <int D, int NCT, bool COH>
__device__ __forceinline__ void qload(const AttnParams& p, uint32_t t0, uint32_t g, uint32_t ncols, QRaw<D, NCT>& r,
                                      int lane) {
  constexpr int KST = D / 32;
  const int c16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    const uint32_t c = 16 * ct + c16;
    r.pos[ct] = 0;
    if (c < ncols) {
      const uint32_t i = c / p.G, h = g * p.G + c % p.G, t = t0 + i;
      r.pos[ct] = p.meta[2 * t + 1];
      const size_t qo = (size_t)t * p.W + h * D + 8 * q;
#pragma unroll
      for (int ks = 0; ks < KST; ks++) {
        const f32x4 a = ld_act<COH>(p.qkv, qo + 32 * ks), b = ld_act<COH>(p.qkv, qo + 32 * ks + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          r.v[ct][ks][e] = a[e];
          r.v[ct][ks][4 + e] = b[e];
        }
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < KST; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) r.v[ct][ks][e] = 0.0f;
    }
  }
}

// The rope words of a lane's columns (all columns requested together).
template <int D, int NCT>
__device__ __forceinline__ void qrope_load(const AttnParams& p, uint32_t ncols, const QRaw<D, NCT>& r,
                                           float2 (&cs)[NCT][D / 32][4], int lane) {
  constexpr int KST = D / 32;
  const int c16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NCT; ct++)
#pragma unroll
    for (int ks = 0; ks < KST; ks++)
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        const uint32_t j = 16 * ks + 4 * q + jj;
        const bool on = p.rope_on && 16 * ct + c16 < ncols && 32 * ks + 8 * q < 64;
        cs[ct][ks][jj] = !on ? float2{1.0f, 0.0f} : *(const float2*)(p.rope + ((size_t)r.pos[ct] * SV_ROPE_PAIRS + j) * 2);
      }
}

// Norm, RoPE (words from qrope_load), scale and hi/lo split of the raw queries.
// CAP (the capture kernel only): the queries after the norm and RoPE also go to p.cap_q.
template <int D, int NCT, bool CAP = false>
__device__ __forceinline__ void qfinish_cs(const AttnParams& p, uint32_t ncols, QRaw<D, NCT>& r,
                                           const float2 (&cs)[NCT][D / 32][4], bf16x8 (&qh)[NCT][D / 32],
                                           bf16x8 (&ql)[NCT][D / 32], int lane, uint32_t t0 = 0, uint32_t g = 0) {
  constexpr int KST = D / 32;
  const int c16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NCT; ct++) {
    const bool ok = 16 * ct + c16 < ncols;
    float ss = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KST; ks++)
#pragma unroll
      for (int e = 0; e < 8; e++) ss = __builtin_fmaf(r.v[ct][ks][e], r.v[ct][ks][e], ss);
    ss += __shfl_xor(ss, 16, WAVE);
    ss += __shfl_xor(ss, 32, WAVE);
    const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + SV_RMS_EPS);
#pragma unroll
    for (int ks = 0; ks < KST; ks++) {
      float* v = r.v[ct][ks];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] *= inv;
      if (p.rope_on && ok && 32 * ks + 8 * q < 64) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const float a0 = v[2 * jj], a1 = v[2 * jj + 1];
          v[2 * jj] = cs[ct][ks][jj].x * a0 + cs[ct][ks][jj].y * a1;
          v[2 * jj + 1] = cs[ct][ks][jj].x * a1 - cs[ct][ks][jj].y * a0;
        }
      }
      if (CAP && ok) {
        // the query after the norm and RoPE (column 16 ct + c16: token c / G, head g G + c % G)
        const uint32_t c = 16 * ct + c16;
        float* dst = p.cap_q + (size_t)(t0 + c / p.G) * p.NQ * D + (g * p.G + c % p.G) * D + 32 * ks + 8 * q;
        *(f32x4*)dst = f32x4{v[0], v[1], v[2], v[3]};
        *(f32x4*)(dst + 4) = f32x4{v[4], v[5], v[6], v[7]};
      }
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] *= p.scale_log2;
      split8(v, qh[ct][ks], ql[ct][ks]);
    }
  }
}

template <int D, int NCT>
__device__ __forceinline__ void qfinish(const AttnParams& p, uint32_t ncols, QRaw<D, NCT>& r, bf16x8 (&qh)[NCT][D / 32],
                                        bf16x8 (&ql)[NCT][D / 32], int lane) {
  float2 cs[NCT][D / 32][4];
  qrope_load<D, NCT>(p, ncols, r, cs, lane);
  qfinish_cs<D, NCT>(p, ncols, r, cs, qh, ql, lane);
}

// Queries of columns 16 ct + c16 (kernels.metal:1022-1039 with norm_rope :727-736): rms-norm
// over the head, RoPE on pairs, times softmax scale x log2 e, split into bf16 hi + lo MFMA
// operands; k slot j of step ks is dim 32 ks + 8 q + j. COH: qkv is read with coherent
// loads (written earlier in the same launch by other workgroups).
template <int D, int NCT, bool COH>
__device__ __forceinline__ void build_queries(const AttnParams& p, uint32_t t0, uint32_t g, uint32_t ncols,
                                              bf16x8 (&qh)[NCT][D / 32], bf16x8 (&ql)[NCT][D / 32], int lane) {
  QRaw<D, NCT> r;
  qload<D, NCT, COH>(p, t0, g, ncols, r, lane);
  qfinish<D, NCT>(p, ncols, r, qh, ql, lane);
}

// The run's new keys (kernels.metal:910-942 new_key): norm, RoPE, bf16, to the cache at
// p0 + row and to LDS (nk / nv: [T][D]). 16 threads per key (D / 16 dims each, rope pairs
// within a thread); threads tid < nthreads of the caller take keys tid / 16, + nthreads / 16...
// With the extras: the value embedding added to V first (add_ve, kernels.metal:738-747) and
// V's direction V / max(|V|, 1e-4) to vdir for XSA (fp32, before rounding).
// CAP (the capture kernel only): the keys after the norm and RoPE and the values after the value
// embedding also go to p.cap_k / p.cap_v; with CACHE false nothing is written to the cache, LDS
// or vdir (the step's attention already wrote the same bits).
template <int D, bool COH, bool CAP = false, bool CACHE = true>
__device__ __forceinline__ void new_keys(const AttnParams& p, uint32_t seq, uint32_t g, uint32_t t0, uint32_t T,
                                         uint32_t p0, uint16_t* nk, uint16_t* nv, uint32_t tid, uint32_t nthreads) {
  constexpr int DL = D / 16;
  const uint32_t l16 = tid & 15;
  for (uint32_t i = tid >> 4; i < T; i += nthreads >> 4) {
    {
      const uint32_t t = t0 + i, pos = p.meta[2 * t + 1];
      const size_t ko = (size_t)t * p.W + p.KOFF + g * D + DL * l16;
      const size_t vo = (size_t)t * p.W + p.VOFF + g * D + DL * l16;
      float kv[DL], vv[DL];
#pragma unroll
      for (int e = 0; e < DL; e += 4) {
        const f32x4 a = ld_act<COH>(p.qkv, ko + e), b = ld_act<COH>(p.qkv, vo + e);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          kv[e + j] = a[j];
          vv[e + j] = b[j];
        }
      }
      if (p.ve_gate) {
        // 2 sigmoid(rms_norm(x)[:12] . ve_gate[g]) * value_embed[token][g D ..]
        float s = 0.0f;
        if (l16 < SV_VE_GATE_W / 4) {
          const f32x4 xv = *(const f32x4*)(p.x + (size_t)t * p.H + 4 * l16);
          const f32x4 gv = *(const f32x4*)(p.ve_gate + g * SV_VE_GATE_W + 4 * l16);
          const float iv = p.inv[t];
#pragma unroll
          for (int j = 0; j < 4; j++) s = __builtin_fmaf(xv[j] * iv, gv[j], s);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o, WAVE);
        const float gate = 2.0f * sigmoid_f(s);
        const uint16_t* ve = p.vemb + ((size_t)p.tokens[t] * p.NKV + g) * D + DL * l16;
#pragma unroll
        for (int e = 0; e < DL; e++) vv[e] = __builtin_fmaf(gate, bf(ve[e]), vv[e]);
      }
      if (CACHE && p.vdir) {
        float vs = 0.0f;
#pragma unroll
        for (int e = 0; e < DL; e++) vs = __builtin_fmaf(vv[e], vv[e], vs);
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) vs += __shfl_xor(vs, o, WAVE);
        const float den = __builtin_fmaxf(__builtin_sqrtf(vs), 1e-4f);
        float* vd = p.vdir + ((size_t)t * p.NKV + g) * D + DL * l16;
#pragma unroll
        for (int e = 0; e < DL; e += 4) *(f32x4*)(vd + e) = f32x4{vv[e] / den, vv[e + 1] / den, vv[e + 2] / den, vv[e + 3] / den};
      }
      const size_t row = kv_off<D>(p, seq, g, p0 + i);
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < DL; e++) ss = __builtin_fmaf(kv[e], kv[e], ss);
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o, WAVE);
      const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + SV_RMS_EPS);
      uint32_t kb[DL / 2], vb[DL / 2];
#pragma unroll
      for (int e = 0; e < DL; e += 2) {
        const uint32_t d = DL * l16 + e;
        float k0 = kv[e] * inv, k1 = kv[e + 1] * inv;
        if (p.rope_on && d < 64) {
          const float2 cs = p.rope_rows ? *(const float2*)(p.rope_rows + ((size_t)t * SV_ROPE_PAIRS + d / 2) * 2)
                                        : *(const float2*)(p.rope + ((size_t)pos * SV_ROPE_PAIRS + d / 2) * 2);
          const float r0 = cs.x * k0 + cs.y * k1, r1 = cs.x * k1 - cs.y * k0;
          k0 = r0;
          k1 = r1;
        }
        if constexpr (CAP) {
          const size_t co = (size_t)t * p.NKV * D + g * D + d;
          p.cap_k[co] = k0;
          p.cap_k[co + 1] = k1;
          p.cap_v[co] = vv[e];
          p.cap_v[co + 1] = vv[e + 1];
        }
        kb[e / 2] = (uint32_t)to_bf(k0) | ((uint32_t)to_bf(k1) << 16);
        vb[e / 2] = (uint32_t)to_bf(vv[e]) | ((uint32_t)to_bf(vv[e + 1]) << 16);
      }
#pragma unroll
      for (int e = 0; e < DL / 2 && CACHE; e += 2) {
        const u32x2 kw = u32x2{kb[e], kb[e + 1]}, vw = u32x2{vb[e], vb[e + 1]};
        *(u32x2*)(p.kc + row + DL * l16 + 2 * e) = kw;
        *(u32x2*)(p.vc + row + DL * l16 + 2 * e) = vw;
        *(u32x2*)(nk + i * D + DL * l16 + 2 * e) = kw;
        *(u32x2*)(nv + i * D + DL * l16 + 2 * e) = vw;
      }
    }
  }
}

}  // namespace sv
