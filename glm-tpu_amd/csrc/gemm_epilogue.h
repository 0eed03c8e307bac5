// Epilogues of the grouped FP8 projections: one MFMA output fragment (four
// consecutive weight rows n..n+3 of one route column) per call.
#pragma once

#include "moe_common.h"
#include "moe_kernels.h"

namespace glm_moe {

// Output row of route (sorted position) r, or -1 when it is outside the output.
__device__ __forceinline__ int64_t fragment_row(const GroupedGemmArgs& a, int r) {
  const int64_t orow = a.out_row_ids ? a.out_row_ids[r] : r;
  return orow < 0 || orow >= a.out_rows ? -1 : orow;
}

// The bf16 route weight the weighted epilogue multiplies output row orow by
// (1 for the other epilogues and rows outside the output).
template <int EPI>
__device__ __forceinline__ float fragment_weight(const GroupedGemmArgs& a, int64_t orow) {
  if constexpr (EPI == kEpiWeighted) return orow < 0 ? 1.0f : round_to_bf16(a.route_w[orow]);
  return 1.0f;
}

// Stores the four values of output row orow (fragment_row; < 0: nothing) at
// rows n..n+3, with the route weight wgt (fragment_weight) already loaded.
// g/u: table 0 / table 1 accumulators (u unused for one table).
template <int TABLES, int EPI>
__device__ __forceinline__ void store_fragment_at(const GroupedGemmArgs& a, int64_t orow, float wgt, int n,
                                                  const f32x4& g, const f32x4& u) {
  if (orow < 0) return;
  if constexpr (EPI == kEpiSwiglu) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = swiglu_bf16(round_to_bf16(g[j]), round_to_bf16(u[j]));
    const u32x2 pk{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + orow * a.ldo + n) = pk;
  } else if constexpr (EPI == kEpiWeighted) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = round_to_bf16(g[j]) * wgt;
    const u32x2 pk{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + orow * a.ldo + n) = pk;
  } else if constexpr (EPI == kEpiStoreF32) {
    float* o = static_cast<float*>(a.out) + orow * a.ldo + n;
    *reinterpret_cast<f32x4*>(o) = g;
    if constexpr (TABLES == 2) *reinterpret_cast<f32x4*>(o + a.table_stride) = u;
  } else {
    uint16_t* o = static_cast<uint16_t*>(a.out) + orow * a.ldo + n;
    *reinterpret_cast<u32x2*>(o) = u32x2{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3])};
    if constexpr (TABLES == 2)
      *reinterpret_cast<u32x2*>(o + a.table_stride) = u32x2{pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3])};
  }
}

// Stores the four values of route (sorted position) r at rows n..n+3.
template <int TABLES, int EPI>
__device__ __forceinline__ void store_fragment(const GroupedGemmArgs& a, int r, int n, const f32x4& g,
                                               const f32x4& u) {
  const int64_t orow = fragment_row(a, r);
  store_fragment_at<TABLES, EPI>(a, orow, fragment_weight<EPI>(a, orow), n, g, u);
}

}  // namespace glm_moe
