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
  int small_ok;          // the caller does not read counts/offsets: small batches may take the
                         // small-batch path, which leaves them unwritten
  int32_t* chunk_counts; // [layout_chunks(A_ext)][E_ext] scratch of the multi-workgroup path
  int32_t* chunk_base;   // [layout_chunks(A_ext)][E_ext]
};

// combine_pos row width bound: top_k (<= kRouteMaxTopK = 16) + the shared expert
constexpr int kCombineMaxW = 17;

constexpr int kLayoutChunk = 1024;  // assignments per workgroup of the multi-workgroup layout
inline int64_t layout_chunks(int64_t a_ext) { return (a_ext + kLayoutChunk - 1) / kLayoutChunk; }
// scratch bytes of the multi-workgroup layout (0 when the single-workgroup path applies)
inline size_t layout_scratch_bytes(int64_t a_ext, int64_t e_ext) {
  return a_ext > 4096 ? (size_t)layout_chunks(a_ext) * (size_t)e_ext * 4 * 2 : 0;
}

// Enqueue routing (when logits != nullptr) + stable layout + tile list.
int launch_route_layout(const float* logits, const float* bias, const int32_t* ids_in, const float* weights_in,
                        int32_t* ids_out, float* weights_out, int64_t M, int64_t E, int64_t K, int func, int renorm,
                        float route_scale, int has_shared, int block_m, int64_t tile_cap, const LayoutOut& out,
                        hipStream_t st);

constexpr int kMoeBlockM = 16;  // token rows per MoE tile (one 16-row MFMA tile)

// y[t][h] = bf16(sum over j of yp[combine_pos[t][j]][h]) (defined in mx_a16.hip)
__global__ void moe_combine_kernel(const float* __restrict__ yp, const int32_t* __restrict__ combine_pos,
                                   uint16_t* __restrict__ y, int M, int W, int H);

// Device workspace of one MoE forward (caller-allocated, carved here).
struct MoeWorkspace {
  int32_t *counts, *offsets, *perm, *perm_token, *sorted_ids, *inv_pos, *combine_pos;
  float* perm_weight;
  int32_t *tile_expert, *tile_start, *tile_rows, *tile_p0, *n_tiles;
  uint16_t* z;     // [A, I] bf16 SwiGLU output (route weight applied)
  float* yp;       // [A, H] fp32 expert partials
  uint8_t* xq;     // A8 only: [M, H] e4m3 tokens
  float* xs;       // A8 only: [M, H/128] scales
  uint8_t* zq;     // A8 only: [A, I] e4m3 z
  float* zs;       // A8 only: [A, I/128] scales
  int32_t *chunk_counts, *chunk_base;
  int64_t tile_cap;
  size_t bytes;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// base == nullptr only sizes the workspace
inline MoeWorkspace carve_moe_workspace(char* base, int64_t M, int64_t H, int64_t I, int64_t E, int64_t K,
                                        int has_shared, int block_m, bool a8) {
  MoeWorkspace w{};
  const int64_t A = M * K + (has_shared ? M : 0);
  const int64_t Ee = E + (has_shared ? 1 : 0);
  const int64_t u = A < Ee ? A : Ee;
  w.tile_cap = (A + u * (block_m - 1)) / block_m;
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  w.counts = (int32_t*)take(4 * (Ee + 1));
  w.offsets = (int32_t*)take(4 * (Ee + 2));
  w.perm = (int32_t*)take(4 * A);
  w.perm_token = (int32_t*)take(4 * A);
  w.perm_weight = (float*)take(4 * A);
  w.sorted_ids = (int32_t*)take(4 * A);
  w.inv_pos = (int32_t*)take(4 * A);
  w.combine_pos = (int32_t*)take(4 * A);
  w.tile_expert = (int32_t*)take(4 * w.tile_cap);
  w.tile_start = (int32_t*)take(4 * w.tile_cap);
  w.tile_rows = (int32_t*)take(4 * w.tile_cap);
  w.tile_p0 = (int32_t*)take(4 * w.tile_cap);
  w.n_tiles = (int32_t*)take(4);
  const size_t lsb = layout_scratch_bytes(A, Ee);
  w.chunk_counts = lsb ? (int32_t*)take(lsb / 2) : nullptr;
  w.chunk_base = lsb ? (int32_t*)take(lsb / 2) : nullptr;
  w.z = (uint16_t*)take(2 * A * I);
  w.yp = (float*)take(4 * A * H);
  if (a8) {
    w.xq = (uint8_t*)take(M * H);
    w.xs = (float*)take(4 * M * (H / 128));
    w.zq = (uint8_t*)take(A * I);
    w.zs = (float*)take(4 * A * (I / 128));
  }
  w.bytes = off;
  return w;
}

// Batch-1 decode layer in two launches (moe_decode.hip): routing + gate/up +
// SwiGLU, then down + combine.  `supported` says whether the shapes fit it.
bool moe_decode1_supported(int64_t m, int64_t hidden, int64_t inter, int64_t top_k, int has_shared);
int launch_moe_decode1(const uint16_t* x, const float* logits, const float* bias, const int32_t* ids_in,
                       const float* w_in, int32_t* ids_out, float* w_out, const uint8_t* gu_p, const uint8_t* gu_s,
                       const uint8_t* d_p, const uint8_t* d_s, const uint8_t* sh_gu_p, const uint8_t* sh_gu_s,
                       const uint8_t* sh_d_p, const uint8_t* sh_d_s, uint16_t* y, int64_t H, int64_t I, int64_t E,
                       int64_t K, int has_shared, int func, int renorm, float route_scale, float limit, uint16_t* z,
                       int32_t* tile_expert, int32_t* n_tiles, void* const* marks, hipStream_t st);

// Down + combine for 2..4 tokens after the layout and grouped gate/up kernels
// (moe_decode.hip): every workgroup walks the whole tile list and writes y.
bool moe_small_down_supported(int64_t m, int64_t hidden, int64_t inter, int64_t tile_cap);
void launch_moe_small_down(const uint16_t* z, const int32_t* tile_expert, const int32_t* tile_rows,
                           const int32_t* tile_p0, const int32_t* n_tiles, const int32_t* perm_token,
                           const uint8_t* d_p, const uint8_t* d_s, const uint8_t* sh_d_p, const uint8_t* sh_d_s,
                           uint16_t* y, int64_t M, int64_t H, int64_t I, int64_t E, int has_shared, hipStream_t st);

// Single MXT16 A16 linear at one token (moe_decode.hip).
bool linear_decode1_supported(int64_t m, int64_t n, int64_t k);
void launch_linear_decode1(const uint16_t* x, const uint8_t* pt, const uint8_t* st, uint16_t* y, int64_t n, int64_t k,
                           hipStream_t s);

}  // namespace mosaic
