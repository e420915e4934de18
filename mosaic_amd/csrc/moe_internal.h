// Internal interface between the routing/layout kernels and the MoE launchers.
#pragma once
#include "common.h"

namespace mosaic {

// Device arrays written by the routing + stable-sort + tile-list kernel.
struct LayoutOut {
  int32_t* counts;       // [E_ext]
  int32_t* offsets;      // [E_ext + 1]
  int32_t* perm;         // [A_ext] flat assignment index at sorted position p
  int32_t* perm_token;   // [A_ext] token of sorted position p
  float* perm_weight;    // [A_ext] route weight of sorted position p (1 for shared)
  int32_t* sorted_ids;   // [A_ext] expert id of sorted position p (E for shared)
  int32_t* inv_pos;      // [A_ext] sorted position of flat assignment a (-1 if dropped)
  int32_t* combine_pos;  // [M, K(+1)] token's sorted positions, ascending expert id (shared last)
  int32_t* tile_expert;  // [tile_cap]
  int32_t* tile_start;   // [tile_cap]
  int32_t* tile_rows;    // [tile_cap]
  int32_t* tile_p0;      // [tile_cap] first sorted position of the tile
  int32_t* n_tiles;      // [1]
  int32_t* counters;     // [n_counters] zeroed by the layout kernel (arrival counters of later kernels)
  int n_counters;
  int small_ok;          // the caller does not read counts/offsets: A_ext <= 64 may take the
                         // single-wave path, which leaves them unwritten
};

// Enqueue routing (when logits != nullptr) + stable layout + tile list.
int launch_route_layout(const float* logits, const float* bias, const int32_t* ids_in, const float* weights_in,
                        int32_t* ids_out, float* weights_out, int64_t M, int64_t E, int64_t K, int func, int renorm,
                        float route_scale, int has_shared, int block_m, int64_t tile_cap, const LayoutOut& out,
                        hipStream_t st);

}  // namespace mosaic
