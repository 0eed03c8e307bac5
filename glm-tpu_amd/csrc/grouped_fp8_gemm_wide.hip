// Wide (prefill) route-grouped FP8 projection: up to 128 routes per work tile.
//
// Same arithmetic as the skinny kernel (bf16(f32(e4m3) * block scale) weights,
// bf16 activations, FP32 accumulation over ascending 128-wide K blocks on
// v_mfma_f32_16x16x32_bf16), organised for operand reuse:
//   * a workgroup of WAVES waves owns a stripe of BN = WAVES * RG * 16 weight
//     rows of one expert and one tile of up to BM = CGMAX * 16 sorted routes;
//   * every wave streams and decodes only its own RG*16 rows of every table
//     (each weight byte is loaded from HBM and decoded once per tile), and
//     feeds the decoded bf16 straight to the MFMA A operand;
//   * the tile's activation rows (gathered token rows for gate/up, sorted
//     activation rows for down) are staged once per 128-wide K block into LDS
//     (double buffered, 16-byte row padding keeps the 128-bit reads
//     conflict-free) and shared by all waves as the B operand;
//   * only the 16-route column groups that hold live routes are multiplied.
// One barrier per K block; the next block's weights and activations are in
// flight while the current one is decoded and multiplied.
#include "gemm_epilogue.h"
#include "moe_common.h"
#include "moe_kernels.h"

namespace glm_moe {

namespace {

template <int TABLES, int RG, int CGMAX, int WAVES, int EPI>
__global__ __launch_bounds__(WAVES * 64) void grouped_fp8_gemm_wide_kernel(const GroupedGemmArgs a) {
  constexpr int BN = WAVES * RG * 16;
  constexpr int BM = CGMAX * 16;
  constexpr int THREADS = WAVES * 64;
  constexpr int LDS_ROW = kScaleBlock + 8;           // bf16 per staged row (16-byte pad)
  constexpr int ROWS_PER_PASS = THREADS / 16;         // 16 threads x 16 B per 256-byte row
  constexpr int PASSES = (BM + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][BM * LDS_ROW];

  const int tile = blockIdx.x;
  if (tile >= a.tile_count[0]) return;
  if (a.valid != nullptr && a.valid[0] == 0) return;
  const int e = a.tile_expert[tile];
  const int r0 = a.tile_row[tile];
  const int live = a.tile_live[tile];
  if (e < 0 || e >= a.experts || r0 < 0 || live <= 0 || live > BM || r0 + live > a.rows) return;
  const int ncg = (live + 15) >> 4;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lrow = lane & 15;
  const int lgrp = lane >> 4;
  const int N = a.n;
  const int K = a.k;
  const int KB = K / kScaleBlock;
  const int n0 = blockIdx.y * BN + wave * RG * 16;

  // ---- activation staging: thread -> (row, 16-byte chunk) of the 128-wide block
  const int schunk = tid & 15;
  const uint16_t* src[PASSES];
  bool sok[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = (tid >> 4) + p * ROWS_PER_PASS;
    sok[p] = row < live;
    const int r = r0 + (sok[p] ? row : 0);
    int64_t phys = a.x_row_ids ? a.x_row_ids[r] / a.x_row_div : r;
    phys = phys < 0 ? 0 : (phys >= a.x_rows ? a.x_rows - 1 : phys);
    src[p] = a.x + (size_t)phys * K + schunk * 8;
  }

  // ---- weight rows of this wave
  const uint8_t* wptr[TABLES][RG];
  const float* sptr[TABLES][RG];
#pragma unroll
  for (int t = 0; t < TABLES; ++t) {
    const uint8_t* wb = t == 0 ? a.w0 : a.w1;
    const float* sb = t == 0 ? a.s0 : a.s1;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      const int row = n0 + rg * 16 + lrow;
      wptr[t][rg] = wb + ((size_t)e * N + row) * (size_t)K + lgrp * 16;
      sptr[t][rg] = sb + ((size_t)e * (N / kScaleBlock) + (n0 + rg * 16) / kScaleBlock) * KB;
    }
  }

  f32x4 acc[TABLES][RG][CGMAX];
#pragma unroll
  for (int t = 0; t < TABLES; ++t)
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
      for (int cg = 0; cg < CGMAX; ++cg) acc[t][rg][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 xr[PASSES];
  u32x4 wreg[2][TABLES][RG][2];
  float sreg[2][TABLES][RG];

  auto load_x = [&](int kb) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      if (sok[p]) xr[p] = *reinterpret_cast<const u32x4*>(src[p] + (size_t)kb * kScaleBlock);
      else xr[p] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = (tid >> 4) + p * ROWS_PER_PASS;
      if (row < BM) *reinterpret_cast<u32x4*>(&xs[buf][row * LDS_ROW + schunk * 8]) = xr[p];
    }
  };
  auto load_w = [&](int slot, int kb) {
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const uint8_t* p = wptr[t][rg] + (size_t)kb * kScaleBlock;
        wreg[slot][t][rg][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        wreg[slot][t][rg][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 64));
        sreg[slot][t][rg] = sptr[t][rg][kb];
      }
  };
  auto compute = [&](int slot, int buf) {
    bf16x8 A[TABLES][RG][4];
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const float s = sreg[slot][t][rg];
        const u32x4 w0 = wreg[slot][t][rg][0];
        const u32x4 w1 = wreg[slot][t][rg][1];
        A[t][rg][0] = decode_fp8x8(w0.x, w0.y, s);
        A[t][rg][1] = decode_fp8x8(w0.z, w0.w, s);
        A[t][rg][2] = decode_fp8x8(w1.x, w1.y, s);
        A[t][rg][3] = decode_fp8x8(w1.z, w1.w, s);
      }
#pragma unroll
    for (int cg = 0; cg < CGMAX; ++cg) {
      if (cg < ncg) {
        const uint16_t* bp = &xs[buf][(cg * 16 + lrow) * LDS_ROW + lgrp * 16];
        const bf16x8 b0 = as_bf16x8(*reinterpret_cast<const u32x4*>(bp));
        const bf16x8 b1 = as_bf16x8(*reinterpret_cast<const u32x4*>(bp + 8));
        const bf16x8 b2 = as_bf16x8(*reinterpret_cast<const u32x4*>(bp + 64));
        const bf16x8 b3 = as_bf16x8(*reinterpret_cast<const u32x4*>(bp + 72));
#pragma unroll
        for (int t = 0; t < TABLES; ++t)
#pragma unroll
          for (int rg = 0; rg < RG; ++rg) {
            f32x4 c = acc[t][rg][cg];
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t][rg][0], b0, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t][rg][1], b1, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t][rg][2], b2, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t][rg][3], b3, c, 0, 0, 0);
            acc[t][rg][cg] = c;
          }
      }
    }
  };

  // prologue: block 0 staged, its weights in flight
  load_x(0);
  load_w(0, 0);
  store_x(0);
  __syncthreads();
  // two K blocks per trip so that register buffers are addressed statically
  for (int kb = 0; kb < KB; kb += 2) {
    if (kb + 1 < KB) {
      load_x(kb + 1);
      load_w(1, kb + 1);
    }
    compute(0, 0);
    if (kb + 1 < KB) store_x(1);
    __syncthreads();
    if (kb + 1 < KB) {
      if (kb + 2 < KB) {
        load_x(kb + 2);
        load_w(0, kb + 2);
      }
      compute(1, 1);
      if (kb + 2 < KB) store_x(0);
      __syncthreads();
    }
  }

#pragma unroll
  for (int cg = 0; cg < CGMAX; ++cg) {
    const int col = cg * 16 + lrow;
    if (cg >= ncg || col >= live) continue;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
      store_fragment<TABLES, EPI>(a, r0 + col, n0 + rg * 16 + lgrp * 4, acc[0][rg][cg],
                                  acc[TABLES - 1][rg][cg]);
  }
}

template <int TABLES, int RG, int CGMAX, int WAVES>
hipError_t launch_wide_shape(const GroupedGemmArgs& a, int epilogue, hipStream_t stream) {
  constexpr int BN = WAVES * RG * 16;
  const dim3 grid(a.max_tiles, a.n / BN);
  const dim3 block(64 * WAVES);
  label_grouped_gemm(a, TABLES, 128, BN, "");
  switch (epilogue) {
    case kEpiStoreF32:
      return launch_kernel(grouped_fp8_gemm_wide_kernel<TABLES, RG, CGMAX, WAVES, kEpiStoreF32>, grid, block, 0, stream, a);
    case kEpiStoreBf16:
      return launch_kernel(grouped_fp8_gemm_wide_kernel<TABLES, RG, CGMAX, WAVES, kEpiStoreBf16>, grid, block, 0, stream, a);
    case kEpiSwiglu:
      if constexpr (TABLES == 2) {
        return launch_kernel(grouped_fp8_gemm_wide_kernel<TABLES, RG, CGMAX, WAVES, kEpiSwiglu>, grid, block, 0, stream, a);
      }
      return hipErrorInvalidValue;
    case kEpiWeighted:
      if constexpr (TABLES == 1) {
        return launch_kernel(grouped_fp8_gemm_wide_kernel<TABLES, RG, CGMAX, WAVES, kEpiWeighted>, grid, block, 0, stream, a);
      }
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_grouped_gemm_wide(const GroupedGemmArgs& a, int tables, int epilogue, hipStream_t stream) {
  if (a.max_tiles <= 0) return hipSuccess;
  if (tables == 2) return launch_wide_shape<2, 1, 8, 8>(a, epilogue, stream);
  if (tables == 1) return launch_wide_shape<1, 2, 8, 8>(a, epilogue, stream);
  return hipErrorInvalidValue;
}

}  // namespace glm_moe
