// Per-wave staging of e4m3 weight rows: HBM -> registers -> LDS -> MFMA layout.
//
// The MFMA A operand wants lane l to hold row l%16, so loading it directly
// makes every 128-bit load instruction touch 16 rows x 64 bytes, which caps
// HBM streaming near 5 TB/s on MI355X.  Instead each wave loads a "step" of
// 16 rows x 256 contiguous bytes (two 128-wide K blocks) with instructions
// that each cover 4 rows x 256 B (16 lanes per row), writes the step into its
// own 4 KB LDS region with an XOR swizzle (16-byte chunk c of row i lives in
// slot c ^ i), and reads it back in MFMA layout, where the 16 lanes of a group
// hit 16 distinct bank groups.  A wave only reads LDS it wrote itself, in
// order, so no workgroup barrier is involved.
#pragma once

#include "moe_common.h"

namespace glm_moe {

constexpr int kStepBytes = 256;        // K bytes of one row per step (two scale blocks)
constexpr int kStageBytes = 16 * 256;  // one 16-row group of one table per step

struct WeightRows {
  const uint8_t* base;  // this lane's load address at step 0: row (lane >> 4), byte (lane & 15) * 16
  int64_t row_stride;   // bytes between rows (K)
  int k_bytes;          // K
};

// Rows [row0, row0 + 16) of an [rows, K] e4m3 table, as loaded by this lane.
__device__ __forceinline__ WeightRows weight_rows(const uint8_t* table, int64_t row0, int64_t k, int lane) {
  WeightRows w;
  w.base = table + (row0 + (lane >> 4)) * k + (lane & 15) * 16;
  w.row_stride = k;
  w.k_bytes = (int)k;
  return w;
}

// Four 128-bit loads: rows 4q + lane/16, bytes step*256 + (lane%16)*16.  A
// half step at the end of an odd number of K blocks loads only its first 128 B.
__device__ __forceinline__ void load_weight_step(const WeightRows& w, int step, int lane, u32x4 (&r)[4]) {
  const int off = step * kStepBytes;
  const bool ok = off + (lane & 15) * 16 < w.k_bytes;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u32x4* p = reinterpret_cast<const u32x4*>(w.base + (int64_t)(4 * q) * w.row_stride + off);
    r[q] = ok ? *p : u32x4{0u, 0u, 0u, 0u};
  }
}

// Swizzled store of one step into a 4 KB LDS region.
__device__ __forceinline__ void store_weight_step(uint8_t* region, int lane, const u32x4 (&r)[4]) {
  const int c = lane & 15;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * q + (lane >> 4);
    *reinterpret_cast<u32x4*>(region + i * 256 + ((c ^ i) << 4)) = r[q];
  }
}

// 16 bytes of logical chunk c of row lane%16 (MFMA layout).
__device__ __forceinline__ u32x4 read_weight_chunk(const uint8_t* region, int lane, int c) {
  const int i = lane & 15;
  return *reinterpret_cast<const u32x4*>(region + i * 256 + ((c ^ i) << 4));
}

// The four bf16 A operands of K block kbl (0 or 1) of a staged step: lane
// group g holds K = g*16 + 0..15 and 64 + g*16 + 0..15 of the block, decoded
// with the block's scale.
__device__ __forceinline__ void decode_weight_block(const uint8_t* region, int lane, int kbl, float scale,
                                                    bf16x8 (&a)[4]) {
  const int g = lane >> 4;
  const u32x4 w0 = read_weight_chunk(region, lane, kbl * 8 + g);
  const u32x4 w1 = read_weight_chunk(region, lane, kbl * 8 + 4 + g);
  a[0] = decode_fp8x8(w0.x, w0.y, scale);
  a[1] = decode_fp8x8(w0.z, w0.w, scale);
  a[2] = decode_fp8x8(w1.x, w1.y, scale);
  a[3] = decode_fp8x8(w1.z, w1.w, scale);
}

// Activation rows of a skinny tile staged the same way: per 128-wide K block,
// XROWS rows x 256 B, loaded by XROWS/4 instructions of 4 rows x 256 B (lane l:
// row 4q + l/16, 16-byte chunk l%16), stored with chunk c of row i in slot
// c ^ (i & 15), and read back in MFMA B layout.
__device__ __forceinline__ void store_act_rows(uint8_t* region, int q, int lane, const u32x4& v) {
  const int i = 4 * q + (lane >> 4);
  const int c = lane & 15;
  *reinterpret_cast<u32x4*>(region + i * 256 + ((c ^ (i & 15)) << 4)) = v;
}

// B operand j (0..3) of a staged K block for route row i (lane group g = lane/16):
// K = g*16 + 0..7, g*16 + 8..15, 64 + g*16 + 0..7, 64 + g*16 + 8..15.
__device__ __forceinline__ u32x4 read_act_chunk(const uint8_t* region, int i, int lane, int j) {
  const int g = lane >> 4;
  const int c = (j >> 1) * 8 + 2 * g + (j & 1);
  return *reinterpret_cast<const u32x4*>(region + i * 256 + ((c ^ (i & 15)) << 4));
}

}  // namespace glm_moe
