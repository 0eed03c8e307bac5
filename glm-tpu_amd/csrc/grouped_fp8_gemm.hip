// Route-grouped FP8 expert projection on gfx950 bf16 MFMA.
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
// Weights are the streamed operand: every lane loads 16 contiguous e4m3 bytes
// of its row with one 128-bit load (two loads cover a 128-wide K block, a
// whole 128-byte line per row), decodes them in registers with the block
// scale to bf16 and feeds them straight to the MFMA A operand; each weight
// byte is read from HBM once per tile and decoded once.  The K index inside a
// block is permuted identically for A and B (lane group g holds K = g*16+0..7
// for the first MFMA and g*16+8..15 for the second), which only reorders the
// FP32 sum inside one K block.
// Activations (B) are gathered rows (the route's token row for gate/up, the
// sorted activation row for down), read with 128-bit loads.
// Epilogues fuse the bf16 SwiGLU of gate/up (routed_experts.py:102) and the
// bf16 route weighting of down (routed_experts.py:104-105).
#include "moe_common.h"
#include "moe_kernels.h"

namespace glm_moe {

namespace {

template <int TABLES, int RG, int CG>
struct Frag {
  f32x4 v[TABLES][RG][CG];
};

template <int TABLES, int RG, int CG, int WN, int WK, int EPI>
__global__ __launch_bounds__(64 * WN * WK) void grouped_fp8_gemm_kernel(const GroupedGemmArgs a) {
  constexpr int BN = WN * RG * 16;
  const int tile = blockIdx.x;
  if (tile >= a.tile_count[0]) return;
  if (a.valid != nullptr && a.valid[0] == 0) return;
  const int e = a.tile_expert[tile];
  const int r0 = a.tile_row[tile];
  const int live = a.tile_live[tile];
  // A consistent plan always passes; a corrupt one computes nothing instead of
  // reading out of bounds.
  if (e < 0 || e >= a.experts || r0 < 0 || live <= 0 || live > CG * 16 || r0 + live > a.rows) return;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % WN;
  const int wk = wave / WN;
  const int lrow = lane & 15;
  const int lgrp = lane >> 4;
  const int N = a.n;
  const int K = a.k;
  const int KB = K / kScaleBlock;
  const int n0 = blockIdx.y * BN + wn * RG * 16;
  const int kb0 = (KB * wk) / WK;
  const int kb1 = (KB * (wk + 1)) / WK;

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
  const uint16_t* xptr[CG];
  bool xok[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int col = cg * 16 + lrow;
    xok[cg] = col < live;
    const int r = r0 + (xok[cg] ? col : 0);
    int64_t phys = a.x_row_ids ? a.x_row_ids[r] / a.x_row_div : r;
    phys = phys < 0 ? 0 : (phys >= a.x_rows ? a.x_rows - 1 : phys);
    xptr[cg] = a.x + (size_t)phys * K + lgrp * 16;
  }

  Frag<TABLES, RG, CG> acc;
#pragma unroll
  for (int t = 0; t < TABLES; ++t)
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) acc.v[t][rg][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Register double buffer: the next K block's weights and activations are in
  // flight while the current block is decoded and multiplied.
  u32x4 wbuf[2][TABLES][RG][2];
  u32x4 xbuf[2][CG][4];
  float sbuf[2][TABLES][RG];

  auto load = [&](int buf, int kb) {
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const uint8_t* p = wptr[t][rg] + (size_t)kb * kScaleBlock;
        wbuf[buf][t][rg][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        wbuf[buf][t][rg][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 64));
        sbuf[buf][t][rg] = sptr[t][rg][kb];
      }
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      if (xok[cg]) {
        const uint16_t* p = xptr[cg] + (size_t)kb * kScaleBlock;
        xbuf[buf][cg][0] = *reinterpret_cast<const u32x4*>(p);
        xbuf[buf][cg][1] = *reinterpret_cast<const u32x4*>(p + 8);
        xbuf[buf][cg][2] = *reinterpret_cast<const u32x4*>(p + 64);
        xbuf[buf][cg][3] = *reinterpret_cast<const u32x4*>(p + 72);
      } else {
        xbuf[buf][cg][0] = xbuf[buf][cg][1] = xbuf[buf][cg][2] = xbuf[buf][cg][3] =
            u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  auto compute = [&](int buf) {
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const float s = sbuf[buf][t][rg];
        const u32x4 w0 = wbuf[buf][t][rg][0];
        const u32x4 w1 = wbuf[buf][t][rg][1];
        const bf16x8 a0 = decode_fp8x8(w0.x, w0.y, s);
        const bf16x8 a1 = decode_fp8x8(w0.z, w0.w, s);
        const bf16x8 a2 = decode_fp8x8(w1.x, w1.y, s);
        const bf16x8 a3 = decode_fp8x8(w1.z, w1.w, s);
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
          f32x4 c = acc.v[t][rg][cg];
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, as_bf16x8(xbuf[buf][cg][0]), c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, as_bf16x8(xbuf[buf][cg][1]), c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, as_bf16x8(xbuf[buf][cg][2]), c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, as_bf16x8(xbuf[buf][cg][3]), c, 0, 0, 0);
          acc.v[t][rg][cg] = c;
        }
      }
  };

  if (kb0 < kb1) {
    load(0, kb0);
    for (int kb = kb0; kb < kb1; kb += 2) {
      if (kb + 1 < kb1) load(1, kb + 1);
      compute(0);
      if (kb + 1 < kb1) {
        if (kb + 2 < kb1) load(0, kb + 2);
        compute(1);
      }
    }
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
            red[wk - 1][wn][(t * RG + rg) * CG + cg][lane] = acc.v[t][rg][cg];
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
            acc.v[t][rg][cg] += red[w][wn][(t * RG + rg) * CG + cg][lane];
  }

  // Epilogue: lane holds rows n .. n+3 of route column cg*16 + lrow.
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int col = cg * 16 + lrow;
    if (col >= live) continue;
    const int r = r0 + col;
    const int64_t orow = a.out_row_ids ? a.out_row_ids[r] : r;
    if (orow < 0 || orow >= a.out_rows) continue;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      const int n = n0 + rg * 16 + lgrp * 4;
      if constexpr (EPI == kEpiSwiglu) {
        const f32x4 g = acc.v[0][rg][cg];
        const f32x4 u = acc.v[TABLES - 1][rg][cg];
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = swiglu_bf16(round_to_bf16(g[j]), round_to_bf16(u[j]));
        u32x2 pk{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + orow * a.ldo + n) = pk;
      } else if constexpr (EPI == kEpiWeighted) {
        const float wgt = round_to_bf16(a.route_w[orow]);
        const f32x4 d = acc.v[0][rg][cg];
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = round_to_bf16(d[j]) * wgt;
        u32x2 pk{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + orow * a.ldo + n) = pk;
      } else if constexpr (EPI == kEpiStoreF32) {
#pragma unroll
        for (int t = 0; t < TABLES; ++t) {
          const f32x4 d = acc.v[t][rg][cg];
          *reinterpret_cast<float4*>(static_cast<float*>(a.out) + orow * a.ldo + t * a.table_stride + n) =
              float4{d[0], d[1], d[2], d[3]};
        }
      } else {
#pragma unroll
        for (int t = 0; t < TABLES; ++t) {
          const f32x4 d = acc.v[t][rg][cg];
          u32x2 pk{pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3])};
          *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + orow * a.ldo + t * a.table_stride + n) = pk;
        }
      }
    }
  }
}

template <int TABLES, int RG, int CG, int WN, int WK>
hipError_t launch_shape(const GroupedGemmArgs& a, int epilogue, hipStream_t stream) {
  constexpr int BN = WN * RG * 16;
  const dim3 grid(a.max_tiles, a.n / BN);
  const dim3 block(64 * WN * WK);
  switch (epilogue) {
    case kEpiStoreF32:
      hipLaunchKernelGGL((grouped_fp8_gemm_kernel<TABLES, RG, CG, WN, WK, kEpiStoreF32>), grid, block, 0, stream, a);
      break;
    case kEpiStoreBf16:
      hipLaunchKernelGGL((grouped_fp8_gemm_kernel<TABLES, RG, CG, WN, WK, kEpiStoreBf16>), grid, block, 0, stream, a);
      break;
    case kEpiSwiglu:
      if constexpr (TABLES == 2) {
        hipLaunchKernelGGL((grouped_fp8_gemm_kernel<TABLES, RG, CG, WN, WK, kEpiSwiglu>), grid, block, 0, stream, a);
        break;
      }
      return hipErrorInvalidValue;
    case kEpiWeighted:
      if constexpr (TABLES == 1) {
        hipLaunchKernelGGL((grouped_fp8_gemm_kernel<TABLES, RG, CG, WN, WK, kEpiWeighted>), grid, block, 0, stream, a);
        break;
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
    case kShapeSkinny: return 16;
    case kShapePanel32: return 32;
    case kShapeWide: return 64;
    default: return 0;
  }
}

// Weight rows per workgroup (the N stripe) of each shape family.
int gemm_shape_bn(int shape, int tables) {
  switch (shape) {
    case kShapeSkinny: return tables == 2 ? 16 : 32;
    case kShapePanel32: return tables == 2 ? 64 : 128;
    case kShapeWide: return tables == 2 ? 64 : 128;
    default: return 0;
  }
}

hipError_t launch_grouped_gemm(const GroupedGemmArgs& a, int shape, int tables, int epilogue,
                               hipStream_t stream) {
  if (a.max_tiles <= 0) return hipSuccess;
  if (tables == 2) {
    switch (shape) {
      case kShapeSkinny: return launch_shape<2, 1, 1, 1, 4>(a, epilogue, stream);
      case kShapePanel32: return launch_shape<2, 1, 2, 4, 1>(a, epilogue, stream);
      case kShapeWide: return launch_shape<2, 1, 4, 4, 1>(a, epilogue, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (tables == 1) {
    switch (shape) {
      case kShapeSkinny: return launch_shape<1, 2, 1, 1, 4>(a, epilogue, stream);
      case kShapePanel32: return launch_shape<1, 2, 2, 4, 1>(a, epilogue, stream);
      case kShapeWide: return launch_shape<1, 2, 4, 4, 1>(a, epilogue, stream);
      default: return hipErrorInvalidValue;
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace glm_moe
