// Route-grouped FP8 expert projection on gfx950 bf16 MFMA: the skinny
// (decode) kernel, for work tiles of at most 4, 16 or 32 routes.
//
// Computes, for every work tile (expert e, sorted routes [r0, r0 + live)) and
// every BN-row stripe of the expert's weight table,
//     acc[n][r] = sum_k bf16(f32(e4m3(W[e][n][k])) * S[e][n/128][k/128]) * X[r][k]
// with FP32 accumulation over ascending 128-wide K blocks -- the projection of
// glm-tpu's fp8_routed_projection (reference
// glm_tpu/kernels/fp8_grouped_matmul/kernel.py:209-235) and
// prefill_panel_fp8_matmul (panel_kernel.py:83-101).
//
// Mapping onto v_mfma_f32_16x16x32_bf16 (D = A x B + C, A 16x32, B 32x16):
//   A = 16 weight rows x 32 K: lane l holds row l%16, eight K values of group l/16.
//   B = 32 K x 16 routes:      lane l holds route l%16, the same eight K values.
//   D = 16 weight rows x 16 routes: lane l holds rows 4*(l/16)+j, route l%16.
// The K index inside a 128-wide block is permuted identically for A and B
// (lane group g holds K = g*16+0..7 for the first MFMA, g*16+8..15 for the
// second, 64+g*16+... for the third and fourth), which only reorders the FP32
// sum inside one block.
//
// Weights are the streamed operand.  Each wave owns RG 16-row groups of every
// table and a K range (WK waves split K); it streams 256-byte row segments
// through its own swizzled LDS region (weight_stage.h), decodes each e4m3 byte
// once with its block scale into the bf16 A operand.  The tile's activation
// rows (B, at most XROWS routes) are staged the same way, and both operands of
// two steps are kept in flight in one register ring, so that waiting for a
// step never waits for a later one.  Split-K partial sums meet in LDS and are added in wave
// order, so results are deterministic.  Epilogues fuse the bf16 SwiGLU of
// gate/up (routed_experts.py:102) and the bf16 route weighting of down
// (routed_experts.py:104-105).
#include "gemm_epilogue.h"
#include "moe_common.h"
#include "moe_kernels.h"
#include "weight_stage.h"

namespace glm_moe {

namespace {

// Streaming needs many resident waves: the decode shapes ask for four per SIMD
// (at most 128 VGPRs), the wider ones for what fits.
template <int TABLES, int RG, int XROWS, int WN, int WK, int DEPTH, int EPI>
__global__ __launch_bounds__(64 * WN * WK) void grouped_fp8_gemm_kernel(const GroupedGemmArgs a) {
  constexpr int BN = WN * RG * 16;
  constexpr int WAVES = WN * WK;
  constexpr int REGIONS = TABLES * RG;       // 4 KB weight regions per wave
  constexpr int CG = (XROWS + 15) / 16;      // 16-route column groups
  constexpr int XI = XROWS / 4;              // activation loads per K block
  constexpr int XBYTES = XROWS * 256;        // staged activations per K block
  static_assert(XROWS % 4 == 0 && XROWS <= 32, "staged activation rows");
  __shared__ __attribute__((aligned(16))) uint8_t wlds[WAVES][REGIONS][kStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t xlds[WAVES][2][XBYTES];

  const int tile = blockIdx.x;
  if (tile >= a.tile_count[0]) return;
  if (a.valid != nullptr && a.valid[0] == 0) return;
  const int e = a.tile_expert[tile];
  const int r0 = a.tile_row[tile];
  const int live = a.tile_live[tile];
  // A consistent plan always passes; a corrupt one computes nothing instead of
  // reading out of bounds.
  if (e < 0 || e >= a.experts || r0 < 0 || live <= 0 || live > XROWS || r0 + live > a.rows) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wn = wave % WN;
  const int wk = wave / WN;
  const int lrow = lane & 15;
  const int lgrp = lane >> 4;
  const int N = a.n;
  const int K = a.k;
  const int KB = K / kScaleBlock;
  const int NS = (KB + 1) / 2;  // steps of two K blocks
  const int s0 = (NS * wk) / WK;
  const int s1 = (NS * (wk + 1)) / WK;
  const int n0 = blockIdx.y * BN + wn * RG * 16;

  WeightRows wrows[TABLES][RG];
  const float* sptr[TABLES][RG];
#pragma unroll
  for (int t = 0; t < TABLES; ++t) {
    const uint8_t* wb = t == 0 ? a.w0 : a.w1;
    const float* sb = t == 0 ? a.s0 : a.s1;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      wrows[t][rg] = weight_rows(wb, (int64_t)e * N + n0 + rg * 16, K, lane);
      sptr[t][rg] = sb + ((size_t)e * (N / kScaleBlock) + (n0 + rg * 16) / kScaleBlock) * KB;
    }
  }
  // activation rows this lane loads: row 4q + lane/16 of the tile, chunk lane%16
  const uint16_t* xsrc[XI];
  bool xok[XI];
#pragma unroll
  for (int q = 0; q < XI; ++q) {
    const int i = 4 * q + lgrp;
    xok[q] = i < live;
    const int r = r0 + (xok[q] ? i : 0);
    int64_t phys = a.x_row_ids ? a.x_row_ids[r] / a.x_row_div : r;
    phys = phys < 0 ? 0 : (phys >= a.x_rows ? a.x_rows - 1 : phys);
    xsrc[q] = a.x + (size_t)phys * K + lrow * 8;
  }

  f32x4 acc[TABLES][RG][CG];
#pragma unroll
  for (int t = 0; t < TABLES; ++t)
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) acc[t][rg][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint8_t(*region)[kStageBytes] = wlds[wave];
  uint8_t(*xregion)[XBYTES] = xlds[wave];
  // DEPTH steps of weights and activations are in flight (in registers) while
  // the previous one is multiplied out of LDS; both operands of a step are
  // issued together, so waiting for a step never waits for a later one.
  u32x4 wring[DEPTH][TABLES][RG][4];
  u32x4 xring[DEPTH][2][XI];

  auto load_step = [&](int slot, int s) {
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) load_weight_step(wrows[t][rg], s, lane, wring[slot][t][rg]);
#pragma unroll
    for (int kbl = 0; kbl < 2; ++kbl) {
      const int kb = 2 * s + kbl;
#pragma unroll
      for (int q = 0; q < XI; ++q)
        xring[slot][kbl][q] = (xok[q] && kb < KB)
                                  ? *reinterpret_cast<const u32x4*>(xsrc[q] + (size_t)kb * kScaleBlock)
                                  : u32x4{0u, 0u, 0u, 0u};
    }
  };

  // stage step s (already in the ring) into LDS, then refill its slot with s + DEPTH
  auto compute_step = [&](int slot, int s) {
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) store_weight_step(region[t * RG + rg], lane, wring[slot][t][rg]);
#pragma unroll
    for (int kbl = 0; kbl < 2; ++kbl)
#pragma unroll
      for (int q = 0; q < XI; ++q) store_act_rows(xregion[kbl], q, lane, xring[slot][kbl][q]);
    __builtin_amdgcn_wave_barrier();
    if (s + DEPTH < s1) load_step(slot, s + DEPTH);
#pragma unroll
    for (int kbl = 0; kbl < 2; ++kbl) {
      const int kb = 2 * s + kbl;
      if (kb >= KB) break;
      bf16x8 B[CG][4];
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        const int i = cg * 16 + lrow;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          B[cg][j] = i < XROWS ? as_bf16x8(read_act_chunk(xregion[kbl], i, lane, j))
                               : as_bf16x8(u32x4{0u, 0u, 0u, 0u});
      }
#pragma unroll
      for (int t = 0; t < TABLES; ++t)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
          bf16x8 A[4];
          decode_weight_block(region[t * RG + rg], lane, kbl, sptr[t][rg][kb], A);
#pragma unroll
          for (int cg = 0; cg < CG; ++cg) {
            f32x4 c = acc[t][rg][cg];
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[0], B[cg][0], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[1], B[cg][1], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2], B[cg][2], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[3], B[cg][3], c, 0, 0, 0);
            acc[t][rg][cg] = c;
          }
        }
    }
    __builtin_amdgcn_wave_barrier();
  };

#pragma unroll
  for (int d = 0; d < DEPTH; ++d)
    if (s0 + d < s1) load_step(d, s0 + d);
  for (int s = s0; s < s1; s += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (s + d < s1) compute_step(d, s + d);
  }

  // Split-K: waves wk > 0 hand their partial sums to wave wk == 0 through LDS,
  // which adds them in wave order (deterministic).
  if constexpr (WK > 1) {
    constexpr int NV = TABLES * RG * CG;
    __shared__ f32x4 red[WK - 1][WN][NV][64];
    if (wk > 0) {
#pragma unroll
      for (int t = 0; t < TABLES; ++t)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
          for (int cg = 0; cg < CG; ++cg)
            red[wk - 1][wn][(t * RG + rg) * CG + cg][lane] = acc[t][rg][cg];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int w = 0; w < WK - 1; ++w)
#pragma unroll
      for (int t = 0; t < TABLES; ++t)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
          for (int cg = 0; cg < CG; ++cg)
            acc[t][rg][cg] += red[w][wn][(t * RG + rg) * CG + cg][lane];
  }

  // Epilogue: lane holds rows n .. n+3 of route column cg*16 + lrow.
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int col = cg * 16 + lrow;
    if (col >= live) continue;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
      store_fragment<TABLES, EPI>(a, r0 + col, n0 + rg * 16 + lgrp * 4, acc[0][rg][cg],
                                  acc[TABLES - 1][rg][cg]);
  }
}

template <int TABLES, int RG, int XROWS, int WN, int WK, int DEPTH>
hipError_t launch_shape(const GroupedGemmArgs& a, int epilogue, hipStream_t stream) {
  constexpr int BN = WN * RG * 16;
  const dim3 grid(a.max_tiles, a.n / BN);
  const dim3 block(64 * WN * WK);
  label_grouped_gemm(a, TABLES, XROWS, BN, "");
  switch (epilogue) {
    case kEpiStoreF32:
      return launch_kernel(grouped_fp8_gemm_kernel<TABLES, RG, XROWS, WN, WK, DEPTH, kEpiStoreF32>, grid, block, 0, stream, a);
    case kEpiStoreBf16:
      return launch_kernel(grouped_fp8_gemm_kernel<TABLES, RG, XROWS, WN, WK, DEPTH, kEpiStoreBf16>, grid, block, 0, stream, a);
    case kEpiSwiglu:
      if constexpr (TABLES == 2) {
        return launch_kernel(grouped_fp8_gemm_kernel<TABLES, RG, XROWS, WN, WK, DEPTH, kEpiSwiglu>, grid, block, 0, stream, a);
      }
      return hipErrorInvalidValue;
    case kEpiWeighted:
      if constexpr (TABLES == 1) {
        return launch_kernel(grouped_fp8_gemm_kernel<TABLES, RG, XROWS, WN, WK, DEPTH, kEpiWeighted>, grid, block, 0, stream, a);
      }
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

// Routes per tile of each shape family.
int gemm_shape_rows(int shape) {
  switch (shape) {
    case kShapeDecode: return 4;
    case kShapeSkinny: return 16;
    case kShapePanel32: return 32;
    case kShapeWide: return 128;
    default: return 0;
  }
}

// Weight rows per workgroup (the N stripe) of each shape family.
int gemm_shape_bn(int shape, int tables) {
  switch (shape) {
    case kShapeDecode: return tables == 2 ? 16 : 32;
    case kShapeSkinny: return tables == 2 ? 16 : 32;
    case kShapePanel32: return tables == 2 ? 64 : 128;
    case kShapeWide: return tables == 2 ? 128 : 256;
    default: return 0;
  }
}

hipError_t launch_grouped_gemm(const GroupedGemmArgs& a, int shape, int tables, int epilogue,
                               hipStream_t stream) {
  if (a.max_tiles <= 0) return hipSuccess;
  if (tables == 2) {
    switch (shape) {
      case kShapeDecode: return launch_shape<2, 1, 4, 1, 4, 1>(a, epilogue, stream);
      case kShapeSkinny: return launch_shape<2, 1, 16, 1, 4, 1>(a, epilogue, stream);
      case kShapePanel32: return launch_shape<2, 1, 32, 4, 1, 1>(a, epilogue, stream);
      case kShapeWide:
        return prefill_fits(a.n, a.k, 2) && prefill_rows_fit(a.x_rows, a.k)
                   ? launch_grouped_gemm_prefill(a, 2, epilogue, stream)
                                         : launch_grouped_gemm_wide(a, 2, epilogue, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (tables == 1) {
    switch (shape) {
      case kShapeDecode: return launch_shape<1, 1, 4, 2, 2, 1>(a, epilogue, stream);
      case kShapeSkinny: return launch_shape<1, 1, 16, 2, 2, 1>(a, epilogue, stream);
      case kShapePanel32: return launch_shape<1, 2, 32, 4, 1, 1>(a, epilogue, stream);
      case kShapeWide:
        return prefill_fits(a.n, a.k, 1) && prefill_rows_fit(a.x_rows, a.k)
                   ? launch_grouped_gemm_prefill(a, 1, epilogue, stream)
                                         : launch_grouped_gemm_wide(a, 1, epilogue, stream);
      default: return hipErrorInvalidValue;
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace glm_moe
