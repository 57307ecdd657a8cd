// layers.h — the persistent layer kernel's parameters (layers.hip), shared with the engine.
#pragma once

#include "attn_device.h"
#include "sv_internal.h"

namespace sv {

constexpr uint32_t PL_MAX_LAYERS = 16;

// One layer's tiled int8 matrices (qkv, o, gate_up, down), their per-row scales and scalars.
struct LayerW {
  const uint8_t* w[4];
  const uint16_t* s[4];
  float qkv_scale, o_scale, ra_attn, rb_attn, ra_mlp, rb_mlp;
};

// Everything the kernel reads per layer is in its arguments (the kernel-argument segment,
// read through the scalar cache), not in device buffers whose first read would be a scalar
// cache miss on the critical path of a phase.
struct LayersParams {
  LayerW layers[PL_MAX_LAYERS];
  AttnParams ap;              // the attention of every layer: qkv, out, part_o/l, layer and rope
                              // are replaced per layer (slices below, bit l of rope_mask)
  uint32_t rope_mask;
  uint32_t n_layers, n, H, F, qkv_m, G;
  // activation slices, one per layer (h: n_layers + 1, slice 0 the embedding's rows)
  float *h, *qkv, *attn_out, *mixed, *act, *part;
  uint32_t h_stride, qkv_stride, attn_stride, mixed_stride, act_stride;
  uint32_t part_stride, part_l_off;  // floats: a layer's split partials, l after o
  uint32_t attn_items, merge_items, merge_P, merge_z;
  uint32_t cnt[6];            // workgroups that arrive at each of a layer's six phases
  uint32_t* sync;             // [n_layers * 6][16] counters, 256 bytes apart (never reset)
  const uint32_t* epoch;      // incremented by embed before every launch
  uint32_t* abort;            // set by a workgroup whose wait ran out
  uint32_t spin;              // polls before a wait gives up
  // Tests and probes: per (set, workgroup, layer, phase) the 100 MHz clock at points of the
  // phase ([2][256][n_layers][6][8]); null: none.
  uint64_t* stamps;
};

// Workgroups per set the device holds (0: the kernel does not fit two per compute unit).
int layers_grid_per_set();
sv_status layers_launch(hipStream_t stream, const LayersParams& p, uint32_t max_run);
// Tests: a smaller poll limit, and producers added to the attention phase's count (a barrier
// that cannot complete, so the abort path runs and every workgroup still exits); 0: off.
extern uint32_t g_layers_spin, g_layers_extra;
extern uint64_t g_layers_stamps;  // device address of a stamp buffer (0: none)

}  // namespace sv
