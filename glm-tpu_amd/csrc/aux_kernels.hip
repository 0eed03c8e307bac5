// Row movement, FP8 table decode and the route combine of the MoE path.
#include "moe_common.h"
#include "moe_kernels.h"
#include "router_wave.h"

namespace glm_moe {

namespace {

// decode_fp8_table (reference glm_tpu/layers/fp8.py:113-126):
// out[n][k] = bf16(f32(e4m3(bits[n][k])) * scale[n / bn][k / bk]).
__global__ void decode_fp8_table_kernel(const uint8_t* bits, const float* scale, int64_t n, int64_t k,
                                        int32_t bn, int32_t bk, uint16_t* out) {
  const int64_t kblocks = (k + bk - 1) / bk;
  const int64_t total = n * k;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / k;
    const int64_t col = i - row * k;
    const float s = scale[(row / bn) * kblocks + col / bk];
    const float v = __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)bits[i], false)[0];
    out[i] = f32_to_bf16_bits(v * s);
  }
}

// The expert activation (reference glm_tpu/layers/moe/routed_experts.py:102):
// out[i] = swiglu_bf16(g[i], u[i]) on bf16 values, the epilogues' device function.
__global__ void swiglu_bf16_kernel(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = f32_to_bf16_bits(swiglu_bf16(bf16_bits_to_f32(g[i]), bf16_bits_to_f32(u[i])));
}

// The same on 16-byte-aligned tensors of n8 x 8 values: one 128-bit load of
// each operand and one store per 8 values.
__global__ void swiglu_bf16_x8_kernel(const u32x4* g, const u32x4* u, int64_t n8, u32x4* out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const u32x4 gv = g[i], uv = u[i];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = swiglu_bf16(bf16_bits_to_f32(gv[j] & 0xFFFFu), bf16_bits_to_f32(uv[j] & 0xFFFFu));
      const float hi = swiglu_bf16(bf16_bits_to_f32(gv[j] >> 16), bf16_bits_to_f32(uv[j] >> 16));
      o[j] = pack_bf16x2(lo, hi);
    }
    out[i] = o;
  }
}

// dst[i] = mask[i] ? src[clamp(index[i] / div, 0, src_rows - 1)] : 0, row-wise (dwords).
__global__ void gather_rows_kernel(const uint32_t* src, int64_t src_rows, int64_t row_words,
                                   const int32_t* index, int32_t div, const uint8_t* mask, int64_t n,
                                   uint32_t* dst) {
  const int64_t total = n * row_words;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / row_words;
    const int64_t w = i - row * row_words;
    const bool keep = mask == nullptr || mask[row] != 0;
    uint32_t v = 0;
    if (keep) {
      int64_t s = index[row] / div;
      s = s < 0 ? 0 : (s >= src_rows ? src_rows - 1 : s);
      v = src[s * row_words + w];
    }
    dst[i] = v;
  }
}

// pack_expert_panel_rows (panels.py:86-95): [capacity, panel_rows, row] with
// rows beyond a panel's live count zero.
__global__ void pack_panel_rows_kernel(const uint32_t* src, int64_t src_rows, int64_t row_words,
                                       const int32_t* row_starts, const int32_t* live_counts,
                                       int32_t capacity, int32_t panel_rows, uint32_t* dst) {
  const int64_t total = (int64_t)capacity * panel_rows * row_words;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / row_words;
    const int64_t w = i - row * row_words;
    const int p = (int)(row / panel_rows);
    const int lane = (int)(row - (int64_t)p * panel_rows);
    uint32_t v = 0;
    if (lane < live_counts[p]) {
      int64_t s = (int64_t)row_starts[p] + lane;
      s = s < 0 ? 0 : (s >= src_rows ? src_rows - 1 : s);
      v = src[s * row_words + w];
    }
    dst[i] = v;
  }
}

// Zero every row whose keep flag is 0, or every row when *valid == 0.
__global__ void zero_rows_kernel(uint32_t* out, int64_t rows, int64_t row_words, const uint8_t* keep,
                                 const uint8_t* valid) {
  const bool all = valid != nullptr && valid[0] == 0;
  const int64_t total = rows * row_words;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / row_words;
    if (all || (keep != nullptr && keep[row] == 0)) out[i] = 0u;
  }
}

// FP32 sum of a token's top-k weighted route rows in slot order, one bf16
// rounding (routed_experts.py:106-117; also the decode body's per-owner bf16
// sum, :293, which JAX computes in FP32 and rounds once).  With ids given, a slot whose raw expert id lies outside [0, experts) is not
// owned and contributes nothing (the decode ownership rule, :250-253).
// y is [tokens * top_k, h] in flat (token, slot) order.  Eight columns per thread.
// With shared given, the layer epilogue follows (routed_experts.py:125, :303):
// out = bf16(bf16(routed * routed_scale) + shared), and any non-finite output
// clears the health byte (:126); every other health writer ran before.
__global__ void combine_routes_kernel(const uint16_t* y, int64_t tokens, int32_t top_k, int64_t h,
                                      const int32_t* ids, const RouteOwnership own, const float* route_w,
                                      const uint16_t* shared, float routed_scale, uint8_t* valid,
                                      uint16_t* out, float* out_f32, int32_t round_partial) {
  const int64_t groups = h / 8;
  const int64_t total = tokens * groups;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / groups;
    const int64_t c = (i - t * groups) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // the token's slots eight at a time: the slots computed here (another
    // share's routes are skipped) are listed first, then their rows are all
    // loaded before any is summed, so the loads overlap instead of each
    // waiting behind its slot's ownership test
    for (int s0 = 0; s0 < top_k; s0 += 8) {
      int id[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) id[u] = ids != nullptr ? ids[t * top_k + min(s0 + u, top_k - 1)] : 0;
      int slot[8];
      int n = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < top_k && (ids == nullptr || owned_expert(id[u], own) >= 0)) slot[n++] = s0 + u;
      u32x4 v[8];
      float w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (u < n) {
          v[u] = *reinterpret_cast<const u32x4*>(y + ((t * top_k + slot[u]) * h + c));
          w[u] = route_w != nullptr ? route_w[t * top_k + slot[u]] : 1.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (u >= n) break;
        // bf16 route weight (routed_experts.py:104-105): bf16(bf16(down) * bf16(w))
        w[u] = round_to_bf16(w[u]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float lo = bf16_bits_to_f32(v[u][j] & 0xFFFFu), hi = bf16_bits_to_f32(v[u][j] >> 16);
          if (route_w != nullptr) {
            lo = round_to_bf16(lo * w[u]);
            hi = round_to_bf16(hi * w[u]);
          }
          acc[2 * j] += lo;
          acc[2 * j + 1] += hi;
        }
      }
    }
    if (shared != nullptr) {
      const u32x4 sv = *reinterpret_cast<const u32x4*>(shared + t * h + c);
      bool finite = true;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = round_to_bf16(round_to_bf16(round_to_bf16(acc[2 * j]) * routed_scale) +
                                   bf16_bits_to_f32(sv[j] & 0xFFFFu));
        acc[2 * j + 1] = round_to_bf16(round_to_bf16(round_to_bf16(acc[2 * j + 1]) * routed_scale) +
                                       bf16_bits_to_f32(sv[j] >> 16));
        finite &= isfinite(acc[2 * j]) && isfinite(acc[2 * j + 1]);
      }
      if (!finite) valid[0] = 0;
    }
    if (out_f32 != nullptr) {
      // a share's partial for the caller's sum over the expert axis
      f32x4 lo4, hi4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo4[j] = round_partial ? round_to_bf16(acc[j]) : acc[j];
        hi4[j] = round_partial ? round_to_bf16(acc[4 + j]) : acc[4 + j];
      }
      *reinterpret_cast<f32x4*>(out_f32 + t * h + c) = lo4;
      *reinterpret_cast<f32x4*>(out_f32 + t * h + c + 4) = hi4;
      continue;
    }
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(acc[2 * j], acc[2 * j + 1]);
    *reinterpret_cast<u32x4*>(out + t * h + c) = o;
  }
}

// The layer epilogue after the sum over the expert axis (routed_experts.py:
// 113-127 / :295-304): the FP32 routed sum rounded to bf16, then
// bf16(bf16(routed * routed_scale) + shared); a non-finite output clears the
// health byte.  Eight columns per thread.
__global__ void layer_epilogue_kernel(const float* routed, int64_t tokens, int64_t h, const uint16_t* shared,
                                      float routed_scale, uint8_t* valid, uint16_t* out) {
  const int64_t total = tokens * (h / 8);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = i * 8;
    const f32x4 r0 = *reinterpret_cast<const f32x4*>(routed + e);
    const f32x4 r1 = *reinterpret_cast<const f32x4*>(routed + e + 4);
    const u32x4 sv = *reinterpret_cast<const u32x4*>(shared + e);
    bool finite = true;
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a0 = j < 2 ? r0[2 * j] : r1[2 * j - 4];
      const float a1 = j < 2 ? r0[2 * j + 1] : r1[2 * j - 3];
      const float v0 = round_to_bf16(round_to_bf16(round_to_bf16(a0) * routed_scale) +
                                     bf16_bits_to_f32(sv[j] & 0xFFFFu));
      const float v1 = round_to_bf16(round_to_bf16(round_to_bf16(a1) * routed_scale) +
                                     bf16_bits_to_f32(sv[j] >> 16));
      finite &= isfinite(v0) && isfinite(v1);
      o[j] = pack_bf16x2(v0, v1);
    }
    *reinterpret_cast<u32x4*>(out + e) = o;
    if (!finite) valid[0] = 0;
  }
}

// GLM noaux_tc routing (glm_tpu/layers/moe/router.py:20-55), one wave per
// token: FP32 sigmoid scores, selection by score + correction bias, k rounds of
// a wave-wide arg-max (each lane holds experts lane + 64 j, j < KPER), and the
// selected *unbiased* scores renormalised in FP32 in selection order.
template <int KPER>
__global__ __launch_bounds__(256) void route_noaux_tc_kernel(const float* logits, int64_t tokens, int32_t experts,
                                                             const float* bias, int32_t top_k, int32_t* ids,
                                                             float* weights) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (t >= tokens) return;
  int my_id;
  float my_weight;
  route_token_noaux<KPER>(logits + t * experts, experts, bias, top_k, lane, my_id, my_weight);
  if (lane < top_k) {
    ids[t * top_k + lane] = my_id;
    weights[t * top_k + lane] = my_weight;
  }
}

// Wave-wide maximum (every lane active), wave-uniform: the 16-lane row maxima
// by DPP moves (row16_max_f32), then the four of them through v_readlane -- no
// LDS round trip.
__device__ __forceinline__ float wave_max_f32(float v) {
  v = row16_max_f32(v);
  const auto lane_value = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
  return fmaxf(fmaxf(lane_value(0), lane_value(16)), fmaxf(lane_value(32), lane_value(48)));
}

// Activation quantisation of the native FP8 mode: one wave per (row, 128-wide
// K block), two values a lane.  scale = amax / 448 (1 for an all-zero block);
// q = e4m3fn(clamp(x / scale, +-448)) with round-to-nearest-even
// (v_cvt_pk_fp8_f32); NaN stays NaN.  The scales go out block-major by sorted
// position, scales[kb * n_pos + pos], for each of the row's per_row positions
// positions[row * per_row + j] (the row itself when positions is null), so
// that the FP8 prefill GEMM reads a tile's scales of one block as one
// contiguous run instead of one line per row.
__global__ __launch_bounds__(256) void quantize_rows_fp8_kernel(const uint16_t* x, int64_t rows, int64_t k,
                                                                uint8_t* q, float* scales, const int32_t* positions,
                                                                int per_row, int64_t n_pos) {
  const int lane = threadIdx.x & 63;
  const int64_t kb = k / 128;
  const int64_t blocks = rows * kb;
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t blk = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); blk < blocks; blk += waves) {
    const int64_t row = blk / kb, col = (blk - row * kb) * 128 + 2 * lane;
    const uint32_t pair = *reinterpret_cast<const uint32_t*>(x + row * k + col);
    const float v0 = bf16_bits_to_f32(pair & 0xFFFFu), v1 = bf16_bits_to_f32(pair >> 16);
    const float m = wave_max_f32(fmaxf(fabsf(v0), fabsf(v1)));
    const float scale = m > 0.0f ? m / 448.0f : 1.0f;
    auto clamp448 = [](float v) { return v != v ? v : fminf(fmaxf(v, -448.0f), 448.0f); };
    const float a0 = clamp448(v0 / scale), a1 = clamp448(v1 / scale);
    const uint32_t packed = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, 0, false);
    *reinterpret_cast<uint16_t*>(q + row * k + col) = (uint16_t)(packed & 0xFFFFu);
    if (lane < per_row) {
      const int64_t pos = positions != nullptr ? positions[row * per_row + lane] : row;
      if (pos >= 0 && pos < n_pos) scales[(blk - row * kb) * n_pos + pos] = scale;
    }
  }
}

// The same with 16 lanes per (row, 128-wide K block): four blocks a wave, 8
// values a lane (one 16-byte load, one 8-byte store), the block maximum over
// the lane's 16-lane row by DPP moves (quantize_block16_fp8, which the FP8
// prefill kernel's gate/up epilogue shares).  Same values, scales and NaN
// handling as quantize_rows_fp8_kernel.
__global__ __launch_bounds__(256) void quantize_rows_fp8_x8_kernel(const uint16_t* x, int64_t rows, int64_t k,
                                                                   uint8_t* q, float* scales,
                                                                   const int32_t* positions, int per_row,
                                                                   int64_t n_pos) {
  const int lane = threadIdx.x & 63, l16 = lane & 15;
  const int64_t kb = k / 128;
  const int64_t blocks = rows * kb;
  const int64_t step = (int64_t)gridDim.x * (blockDim.x / 16);
  for (int64_t blk = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / 16; blk < blocks; blk += step) {
    const int64_t row = blk / kb, b = blk - row * kb, col = b * 128 + 8 * l16;
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + row * k + col);
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = bf16_bits_to_f32(v[j] & 0xFFFFu);
      f[2 * j + 1] = bf16_bits_to_f32(v[j] >> 16);
    }
    uint32_t w0, w1;
    const float scale = quantize_block16_fp8(f, w0, w1);
    *reinterpret_cast<uint2*>(q + row * k + col) = make_uint2(w0, w1);
    for (int j = l16; j < per_row; j += 16) {
      const int64_t pos = positions != nullptr ? positions[row * per_row + j] : row;
      if (pos >= 0 && pos < n_pos) scales[b * n_pos + pos] = scale;
    }
  }
}

__global__ void fill_u32_kernel(uint32_t* dst, int64_t words, uint32_t value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = value;
}


// Synthetic FP8 expert weights for tests and benchmarks, the recipe of the
// reference's fixture generator (tools/equivalence/fixture.py:158-172) with
// per-block scales: w ~ N(0, sigma) from a counter-based hash (splitmix64
// finaliser) and Box-Muller; per 128x128 block scale = amax / 448; bits =
// e4m3fn(clamp(w / scale, +-448)) rounded to nearest even.  One workgroup per
// block, 256 threads x 64 values (two threads per 128-byte row).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void synth_fp8_kernel(uint64_t seed, int64_t n, int64_t k, float sigma,
                                                        uint8_t* bits, float* scales) {
  __shared__ float s_max[4];
  const int64_t nb = n / 128, kb = k / 128;
  const int64_t blk = blockIdx.x;
  const int64_t e = blk / (nb * kb);
  const int64_t rem = blk - e * nb * kb;
  const int64_t bn = rem / kb, bk = rem - bn * kb;
  const int tid = threadIdx.x;
  const int64_t row = bn * 128 + (tid >> 1);
  const int64_t col0 = bk * 128 + (tid & 1) * 64;
  const int64_t elem0 = (e * n + row) * k + col0;
  float v[64];
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 64; j += 2) {
    const uint64_t h = splitmix64(seed ^ splitmix64((uint64_t)(elem0 + j)));
    const float u1 = ((uint32_t)(h >> 40) + 1.0f) * (1.0f / 16777217.0f);  // (0, 1]
    const float u2 = (uint32_t)(h & 0xFFFFFFu) * (1.0f / 16777216.0f);     // [0, 1)
    const float r = sigma * sqrtf(-2.0f * __logf(u1));
    float sn, cs;
    __sincosf(6.283185307179586f * u2, &sn, &cs);
    v[j] = r * cs;
    v[j + 1] = r * sn;
    m = fmaxf(m, fmaxf(fabsf(v[j]), fabsf(v[j + 1])));
  }
  for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  if ((tid & 63) == 0) s_max[tid >> 6] = m;
  __syncthreads();
  const float amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  if (tid == 0) scales[(e * nb + bn) * kb + bk] = scale;
  u32x4 out[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int j = q * 16 + w * 4;
      float a0 = fminf(fmaxf(v[j] / scale, -448.0f), 448.0f);
      float a1 = fminf(fmaxf(v[j + 1] / scale, -448.0f), 448.0f);
      float a2 = fminf(fmaxf(v[j + 2] / scale, -448.0f), 448.0f);
      float a3 = fminf(fmaxf(v[j + 3] / scale, -448.0f), 448.0f);
      int packed = __builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, 0, false);
      packed = __builtin_amdgcn_cvt_pk_fp8_f32(a2, a3, packed, true);
      out[q][w] = (uint32_t)packed;
    }
  }
  u32x4* dst = reinterpret_cast<u32x4*>(bits + elem0);
#pragma unroll
  for (int q = 0; q < 4; ++q) dst[q] = out[q];
}

dim3 grid_for(int64_t work, int threads) {
  int64_t blocks = (work + threads - 1) / threads;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  return dim3((unsigned)blocks);
}

// Count of e4m3fn NaN encodings (0x7F, 0xFF) in n bytes, added to *count:
// the checkpoint's finite-bit gate (glm_tpu/model_loader/sharded_state/
// format.py:307-315).  Four bytes a lane per 32-bit word: a byte b is NaN iff
// (b & 0x7F) == 0x7F, found for all four at once with the zero-byte trick on
// (w & 0x7F7F7F7F) ^ 0x7F7F7F7F.  Per-wave sums, one global atomic per wave.
__global__ void count_nonfinite_fp8_kernel(const uint8_t* bits, int64_t n, unsigned long long* count) {
  const int64_t words = n >> 2;
  const uint32_t* w32 = reinterpret_cast<const uint32_t*>(bits);
  unsigned long long local = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t x = (w32[i] & 0x7F7F7F7Fu) ^ 0x7F7F7F7Fu;
    // exact per-byte zero test: bit 7 of each byte of ~(((x & 0x7F..) + 0x7F..) | x) is set iff that byte is 0
    const uint32_t z = ~(((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x | 0x7F7F7F7Fu);
    local += (unsigned long long)__popc(z);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
    const uint8_t b = bits[(words << 2) + threadIdx.x];
    local += (b & 0x7F) == 0x7F ? 1ull : 0ull;
  }
  for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off, 64);
  if ((threadIdx.x & 63) == 0 && local != 0) atomicAdd(count, local);
}

}  // namespace

hipError_t launch_synth_fp8(uint64_t seed, int32_t experts, int64_t n, int64_t k, float sigma,
                            uint8_t* bits, float* scales, hipStream_t stream) {
  const int64_t blocks = (int64_t)experts * (n / 128) * (k / 128);
  if (blocks == 0) return hipSuccess;
  label_next_launch("synthesize_fp8_weights_e%d_n%lld_k%lld", experts, (long long)n, (long long)k);
  return launch_kernel(synth_fp8_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, seed, n, k, sigma,
                     bits, scales);
}

hipError_t launch_decode_fp8_table(const uint8_t* bits, const float* scale, int64_t n, int64_t k,
                                   int32_t block_n, int32_t block_k, uint16_t* out,
                                   hipStream_t stream) {
  if (n * k == 0) return hipSuccess;
  label_next_launch("decode_fp8_table_n%lld_k%lld", (long long)n, (long long)k);
  return launch_kernel(decode_fp8_table_kernel, grid_for(n * k, 256), dim3(256), 0, stream, bits, scale,
                     n, k, block_n, block_k, out);
}

hipError_t launch_swiglu_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* out, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const bool aligned = ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u) |
                         reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  label_next_launch("swiglu_bf16_n%lld", (long long)n);
  if (aligned && n % 8 == 0)
    return launch_kernel(swiglu_bf16_x8_kernel, grid_for(n / 8, 256), dim3(256), 0, stream,
                         reinterpret_cast<const u32x4*>(g), reinterpret_cast<const u32x4*>(u), n / 8,
                         reinterpret_cast<u32x4*>(out));
  return launch_kernel(swiglu_bf16_kernel, grid_for(n, 256), dim3(256), 0, stream, g, u, n, out);
}

hipError_t launch_gather_rows(const void* src, int64_t src_rows, int64_t row_bytes,
                              const int32_t* index, int32_t div, const uint8_t* mask, int64_t n,
                              void* dst, hipStream_t stream) {
  const int64_t words = row_bytes / 4;
  if (n * words == 0) return hipSuccess;
  label_next_launch("gather_prefill_route_rows_r%lld_b%lld", (long long)n, (long long)row_bytes);
  return launch_kernel(gather_rows_kernel, grid_for(n * words, 256), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(src), src_rows, words, index, div, mask, n,
                     static_cast<uint32_t*>(dst));
}

hipError_t launch_pack_panel_rows(const void* src, int64_t src_rows, int64_t row_bytes,
                                  const int32_t* row_starts, const int32_t* live_counts,
                                  int32_t capacity, int32_t panel_rows, void* dst,
                                  hipStream_t stream) {
  const int64_t words = row_bytes / 4;
  const int64_t total = (int64_t)capacity * panel_rows * words;
  if (total == 0) return hipSuccess;
  label_next_launch("pack_expert_panel_rows_p%d_b%lld", capacity, (long long)row_bytes);
  return launch_kernel(pack_panel_rows_kernel, grid_for(total, 256), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(src), src_rows, words, row_starts, live_counts,
                     capacity, panel_rows, static_cast<uint32_t*>(dst));
}

hipError_t launch_zero_rows(void* out, int64_t rows, int64_t row_bytes, const uint8_t* keep,
                            const uint8_t* valid, hipStream_t stream) {
  const int64_t words = row_bytes / 4;
  if (rows * words == 0) return hipSuccess;
  label_next_launch("unpack_expert_panel_rows_r%lld_b%lld", (long long)rows, (long long)row_bytes);
  return launch_kernel(zero_rows_kernel, grid_for(rows * words, 256), dim3(256), 0, stream,
                     static_cast<uint32_t*>(out), rows, words, keep, valid);
}

hipError_t launch_combine_routes(const uint16_t* y, int64_t tokens, int32_t top_k, int64_t h,
                                 const int32_t* ids, const RouteOwnership& own, const float* route_w,
                                 const uint16_t* shared, float routed_scale, uint8_t* valid, uint16_t* out,
                                 float* out_f32, int32_t round_partial, hipStream_t stream) {
  const int64_t total = tokens * (h / 8);
  if (total == 0) return hipSuccess;
  if (h % 8 != 0 || (shared != nullptr && valid == nullptr) || (out_f32 != nullptr && shared != nullptr))
    return hipErrorInvalidValue;
  label_next_launch("restore_prefill_route_rows_t%lld_k%d_h%lld%s", (long long)tokens, top_k, (long long)h,
                    shared != nullptr ? "_epilogue" : "");
  return launch_kernel(combine_routes_kernel, grid_for(total, 256), dim3(256), 0, stream, y, tokens,
                     top_k, h, ids, own, route_w, shared, routed_scale, valid, out, out_f32, round_partial);
}

hipError_t launch_layer_epilogue(const float* routed, int64_t tokens, int64_t h, const uint16_t* shared,
                                 float routed_scale, uint16_t* out, uint8_t* valid, hipStream_t stream) {
  const int64_t total = tokens * (h / 8);
  if (total == 0) return hipSuccess;
  if (h % 8 != 0 || valid == nullptr) return hipErrorInvalidValue;
  label_next_launch("moe_layer_epilogue_t%lld_h%lld", (long long)tokens, (long long)h);
  return launch_kernel(layer_epilogue_kernel, grid_for(total, 256), dim3(256), 0, stream, routed, tokens, h,
                       shared, routed_scale, valid, out);
}

hipError_t launch_count_nonfinite_fp8(const uint8_t* bits, int64_t n, unsigned long long* count,
                                      hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t words = (n >> 2) > 0 ? (n >> 2) : 1;
  const int64_t blocks = words / 256 + 1 < 4096 ? words / 256 + 1 : 4096;
  label_next_launch("count_nonfinite_fp8_n%lld", (long long)n);
  return launch_kernel(count_nonfinite_fp8_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, bits, n, count);
}

hipError_t launch_route_noaux_tc(const float* logits, int64_t tokens, int32_t experts, const float* bias,
                                 int32_t top_k, int32_t* ids, float* weights, hipStream_t stream) {
  if (tokens <= 0) return hipSuccess;
  if (experts <= 0 || experts > kMaxExperts || top_k <= 0 || top_k > kWave || top_k > experts)
    return hipErrorInvalidValue;
  const int64_t blocks = (tokens + 3) / 4;
  label_next_launch("route_glm_noaux_tc_t%lld_e%d_k%d", (long long)tokens, experts, top_k);
  if (experts <= 256)
    return launch_kernel(route_noaux_tc_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, logits, tokens,
                         experts, bias, top_k, ids, weights);
  return launch_kernel(route_noaux_tc_kernel<kMaxExperts / 64>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       logits, tokens, experts, bias, top_k, ids, weights);
}

hipError_t launch_quantize_rows_fp8(const uint16_t* x, int64_t rows, int64_t k, uint8_t* q, float* scales,
                                    const int32_t* positions, int32_t per_row, int64_t n_pos, hipStream_t stream) {
  if (rows <= 0 || k <= 0) return hipSuccess;
  if (k % 128 != 0 || per_row < 1 || per_row > 64 || (positions == nullptr && per_row != 1)) return hipErrorInvalidValue;
  const int64_t blocks = rows * (k / 128);
  label_next_launch("quantize_rows_fp8_r%lld_k%lld", (long long)rows, (long long)k);
  if (((reinterpret_cast<uintptr_t>(x) & 15) | (reinterpret_cast<uintptr_t>(q) & 7)) == 0) {
    const int64_t wgs = (blocks + 15) / 16;  // 16 blocks a workgroup
    return launch_kernel(quantize_rows_fp8_x8_kernel, dim3((unsigned)(wgs < 65536 ? wgs : 65536)), dim3(256), 0,
                         stream, x, rows, k, q, scales, positions, (int)per_row, n_pos);
  }
  const int64_t wgs = (blocks + 3) / 4;
  return launch_kernel(quantize_rows_fp8_kernel, dim3((unsigned)(wgs < 65536 ? wgs : 65536)), dim3(256), 0,
                       stream, x, rows, k, q, scales, positions, (int)per_row, n_pos);
}

hipError_t launch_fill_u32(void* dst, int64_t words, uint32_t value, hipStream_t stream) {
  if (words == 0) return hipSuccess;
  return launch_kernel(fill_u32_kernel, grid_for(words, 256), dim3(256), 0, stream,
                     static_cast<uint32_t*>(dst), words, value);
}

}  // namespace glm_moe
