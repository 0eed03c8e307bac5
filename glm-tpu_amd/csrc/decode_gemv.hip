// Decode path of the routed experts (at most 64 routes, e.g. T <= 8 tokens x
// top-8): two kernels, no separate route plan and no separate combine.
//
// 1. gate/up: workgroup = (tile j, 16 intermediate rows); WK waves split K.
// 2. down:    workgroup = 16 hidden rows x every tile; its waves take tiles in
//    turn, write each route's weighted bf16 result to LDS, and the workgroup
//    then sums every token's slots in slot order (the route combine of
//    glm_tpu/layers/moe/routed_experts.py:104-117 / :291-293).
//
// Route grouping happens inside every wave (decode_tile): the <= 64 route ids
// are matched with one ballot per key bit; each distinct expert (in order of
// its first route) forms tiles of up to R of its routes.  Every route is
// computed by exactly one tile, so the order of tiles changes no result.
//
// Projections are GEMVs on the vector ALU.  A wave owns 16 weight rows; each
// 128-bit load instruction covers 4 rows x 256 contiguous bytes (lane l: row
// 4q + l/16, bytes (l%16)*16), the access pattern that streams HBM at full
// rate.  Every e4m3 byte is decoded once, bf16(f32(e4m3) * block scale)
// (glm_tpu/layers/fp8.py:113-126), and multiplied with the bf16 activations
// by v_dot2c_f32_bf16 (exact bf16 products, FP32 accumulation).  The 16 lanes
// that share a row add their partial sums at the end.  Two steps of weights
// and activations are kept in flight per wave; every load of a step is issued
// unconditionally, so waiting for a step never drains later ones.
#include "moe_common.h"
#include "moe_kernels.h"

namespace glm_moe {

namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kGemvRows = 16;  // weight rows per wave

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Two packed bf16 of a 32-bit word.  The word is taken by value: hipcc 7.2
// lowers __builtin_bit_cast applied directly to a vector element (v[h]) to a
// read of element 0 whatever h is.
__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2, v); }

template <int R>
struct DecodeTile {
  int expert;
  int count;        // routes in the tile (1..R)
  int route[R];     // flat route ids t * top_k + slot (route[0] repeated past count)
};

// The j-th tile of the route set, wave-uniform.  Routes with an id outside
// [0, experts) are skipped (drop_unowned) or take expert 0 (the reference's
// safe id).  Returns false when j >= tile count.
template <int R>
__device__ bool decode_tile(const int32_t* ids, int n, int experts, int key_bits, bool drop_unowned, int j,
                            DecodeTile<R>& t) {
  const int lane = threadIdx.x & 63;
  const int raw = lane < n ? ids[lane] : -1;
  const bool owned = raw >= 0 && raw < experts;
  const int key = lane < n ? (owned ? raw : (drop_unowned ? -1 : 0)) : -1;
  const bool act = key >= 0;
  uint64_t peers = __ballot(act);
  for (int b = 0; b < key_bits; ++b) {
    const bool bit = act && ((key >> b) & 1);
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  if (!act) peers = 0;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const bool leader = act && (peers & lt) == 0;
  const int cnt = __popcll(peers);
  const int ntiles = leader ? (cnt + R - 1) / R : 0;
  int incl = ntiles;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int v = __shfl_up(incl, d, 64);
    if (lane >= d) incl += v;
  }
  const int excl = incl - ntiles;
  const int total = uniform(__shfl(incl, 63, 64));
  if (j >= total) return false;
  const uint64_t hit = __ballot(leader && j >= excl && j < incl);
  const int src = uniform(__ffsll((unsigned long long)hit) - 1);
  const int chunk = j - uniform(__shfl(excl, src, 64));
  t.expert = uniform(__shfl(key, src, 64));
  const uint32_t lo = uniform(__shfl((int)(uint32_t)peers, src, 64));
  const uint32_t hi = uniform(__shfl((int)(uint32_t)(peers >> 32), src, 64));
  uint64_t members = ((uint64_t)hi << 32) | lo;
  for (int skip = 0; skip < chunk * R; ++skip) members &= members - 1;
  t.count = 0;
  int first = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (members != 0) {
      t.route[r] = __ffsll((unsigned long long)members) - 1;
      members &= members - 1;
      t.count = r + 1;
      if (r == 0) first = t.route[0];
    } else {
      t.route[r] = first;
    }
  }
  return true;
}

// One step of one wave: 16 rows x 256 K of TABLES tables, and R routes' activations.
template <int TABLES, int R>
struct GemvSlot {
  u32x4 w[TABLES][4];   // rows 4q + lane/16, 16 bytes at lane%16
  u32x4 x[R][2];        // 16 bf16 activations per route at the same K
  float s_lo[TABLES];   // scales of the step's two K blocks (wave-uniform)
  float s_hi[TABLES];
  bool keep;            // false for the masked lanes of a half step
};

template <int TABLES, int R>
struct GemvStream {
  const uint8_t* wrow[TABLES];  // start of the lane's first row (row0 + lane/16)
  const float* srow[TABLES];    // scale row of the 16 rows (K/128 entries)
  const uint16_t* xrow[R];
  int64_t row_stride;
  int k;
};

template <int TABLES, int R>
__device__ __forceinline__ void gemv_load(const GemvStream<TABLES, R>& g, int step, int lane,
                                          GemvSlot<TABLES, R>& sl) {
  const int kofs = step * 256 + (lane & 15) * 16;
  // a half step (the last one of an odd K/128) masks its upper eight lanes;
  // their loads read in-bounds bytes that are then multiplied by zero
  sl.keep = kofs < g.k;
  const int kk = sl.keep ? kofs : g.k - 16;
  const int kb_hi = min(2 * step + 1, (g.k >> 7) - 1);
#pragma unroll
  for (int t = 0; t < TABLES; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      sl.w[t][q] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(g.wrow[t] + (int64_t)(4 * q) * g.row_stride + kk));
    sl.s_lo[t] = g.srow[t][2 * step];
    sl.s_hi[t] = g.srow[t][kb_hi];
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const u32x4* p = reinterpret_cast<const u32x4*>(g.xrow[r] + kk);
    sl.x[r][0] = p[0];
    sl.x[r][1] = p[1];
  }
}

// acc[t][q][r] += sum over the lane's 16 K of bf16(e4m3 * scale) * x
template <int TABLES, int R>
__device__ __forceinline__ void gemv_fma(const GemvSlot<TABLES, R>& sl, int nr, int lane,
                                         float (&acc)[TABLES][4][R]) {
#pragma unroll
  for (int t = 0; t < TABLES; ++t) {
    const float scale = sl.keep ? ((lane & 15) < 8 ? sl.s_lo[t] : sl.s_hi[t]) : 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 w = sl.w[t][q];
      const u32x4 lo = __builtin_bit_cast(u32x4, decode_fp8x8(w[0], w[1], scale));
      const u32x4 hi = __builtin_bit_cast(u32x4, decode_fp8x8(w[2], w[3], scale));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r < nr) {
          float a = acc[t][q][r];
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const uint32_t wv = lo[h], xv = sl.x[r][0][h];
            a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv), as_bf16x2(xv), a, false);
          }
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const uint32_t wv = hi[h], xv = sl.x[r][1][h];
            a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv), as_bf16x2(xv), a, false);
          }
          acc[t][q][r] = a;
        }
      }
    }
  }
}

// Straight-line stream of exactly NSTEPS steps from s0, two steps in flight:
// with no loop back-edge the compiler counts outstanding loads exactly and
// waits only for the step it is about to multiply.
template <int NSTEPS, int TABLES, int R>
__device__ __forceinline__ void gemv_run_fixed(const GemvStream<TABLES, R>& g, int s0, int nr, int lane,
                                               float (&acc)[TABLES][4][R]) {
  GemvSlot<TABLES, R> ring[2];
  gemv_load(g, s0, lane, ring[0]);
  if constexpr (NSTEPS > 1) gemv_load(g, s0 + 1, lane, ring[1]);
#pragma unroll
  for (int s = 0; s < NSTEPS; ++s) {
    gemv_fma(ring[s & 1], nr, lane, acc);
    if (s + 2 < NSTEPS) {
      __builtin_amdgcn_sched_barrier(0);
      gemv_load(g, s0 + s + 2, lane, ring[s & 1]);
    }
  }
}

// Stream steps [s0, s1) of the 16 rows, two steps in flight.  The usual step
// counts run straight-line; others use a loop whose refills are issued
// unconditionally (a refill past the end reloads the last step, an L2 hit).
template <int TABLES, int R>
__device__ __forceinline__ void gemv_run(const GemvStream<TABLES, R>& g, int s0, int s1, int nr, int lane,
                                         float (&acc)[TABLES][4][R]) {
  if (s0 >= s1) return;
  switch (s1 - s0) {
    case 1: gemv_run_fixed<1>(g, s0, nr, lane, acc); return;
    case 2: gemv_run_fixed<2>(g, s0, nr, lane, acc); return;
    case 3: gemv_run_fixed<3>(g, s0, nr, lane, acc); return;
    case 4: gemv_run_fixed<4>(g, s0, nr, lane, acc); return;
    case 6: gemv_run_fixed<6>(g, s0, nr, lane, acc); return;
    case 8: gemv_run_fixed<8>(g, s0, nr, lane, acc); return;
    case 12: gemv_run_fixed<12>(g, s0, nr, lane, acc); return;
    default: break;
  }
  const int last = s1 - 1;
  GemvSlot<TABLES, R> ring[2];
  gemv_load(g, s0, lane, ring[0]);
  gemv_load(g, min(s0 + 1, last), lane, ring[1]);
  // The scheduling barriers keep each refill after the multiplications that
  // consume its slot, so a slot's registers are reused in place (no copies of
  // in-flight registers at the loop back-edge, which would force full waits).
  for (int s = s0; s < s1; s += 2) {
    gemv_fma(ring[0], nr, lane, acc);
    __builtin_amdgcn_sched_barrier(0);
    gemv_load(g, min(s + 2, last), lane, ring[0]);
    if (s + 1 < s1) gemv_fma(ring[1], nr, lane, acc);
    __builtin_amdgcn_sched_barrier(0);
    gemv_load(g, min(s + 3, last), lane, ring[1]);
  }
}

// Sum over the 16 lanes that share rows; every lane of the group gets the sum.
__device__ __forceinline__ float sum16(float v) {
  v += __shfl_xor(v, 8, 16);
  v += __shfl_xor(v, 4, 16);
  v += __shfl_xor(v, 2, 16);
  v += __shfl_xor(v, 1, 16);
  return v;
}

// ------------------------------------------------------------------ gate/up + SwiGLU
template <int R, int WK>
__global__ __launch_bounds__(64 * WK) void decode_gate_up_kernel(const DecodeArgs a) {
  __shared__ float red[WK][2][kGemvRows][R];
  const int lane = threadIdx.x & 63;
  const int wk = uniform(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  DecodeTile<R> tile;
  if (!decode_tile<R>(a.ids, a.routes, a.experts, a.key_bits, a.drop_unowned, blockIdx.x, tile)) return;
  const int I = a.intermediate, H = a.hidden;
  const int row0 = blockIdx.y * kGemvRows;
  GemvStream<2, R> g;
  const uint8_t* tables[2] = {a.gate_bits, a.up_bits};
  const float* scales[2] = {a.gate_scale, a.up_scale};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    g.wrow[t] = tables[t] + ((int64_t)tile.expert * I + row0 + (lane >> 4)) * H;
    g.srow[t] = scales[t] + ((int64_t)tile.expert * (I / kScaleBlock) + row0 / kScaleBlock) * (H / kScaleBlock);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) g.xrow[r] = a.hidden_in + (int64_t)(tile.route[r] / a.top_k) * H;
  g.row_stride = H;
  g.k = H;
  const int steps = (H / kScaleBlock + 1) / 2;
  float acc[2][4][R] = {};
  gemv_run(g, (steps * wk) / WK, (steps * (wk + 1)) / WK, tile.count, lane, acc);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float v = sum16(acc[t][q][r]);
        if ((lane & 15) == 0) red[wk][t][4 * q + (lane >> 4)][r] = v;
      }
  __syncthreads();
  // one thread per (row, route): wave-order split-K sum, then the bf16 SwiGLU
  const int tid = threadIdx.x;
  if (tid < kGemvRows * R) {
    const int row = tid / R, r = tid % R;
    if (r < tile.count) {
      float gsum = 0.f, usum = 0.f;
      for (int w = 0; w < WK; ++w) {
        gsum += red[w][0][row][r];
        usum += red[w][1][row][r];
      }
      const float v = swiglu_bf16(round_to_bf16(gsum), round_to_bf16(usum));
      a.act[(int64_t)tile.route[r] * I + row0 + row] = f32_to_bf16_bits(v);
    }
  }
}

// ------------------------------------------------------------------ down + weighting + combine
template <int R, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void decode_down_kernel(const DecodeArgs a) {
  __shared__ float res[kMaxDecodeRoutes][kGemvRows];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  const int tid = threadIdx.x;
  const int I = a.intermediate, H = a.hidden;
  const int row0 = blockIdx.x * kGemvRows;
  for (int i = tid; i < a.routes * kGemvRows; i += 64 * WAVES) res[i / kGemvRows][i % kGemvRows] = 0.f;
  __syncthreads();
  const int steps = (I / kScaleBlock + 1) / 2;
  for (int j = wave;; j += WAVES) {
    DecodeTile<R> tile;
    if (!decode_tile<R>(a.ids, a.routes, a.experts, a.key_bits, a.drop_unowned, j, tile)) break;
    GemvStream<1, R> g;
    g.wrow[0] = a.down_bits + ((int64_t)tile.expert * H + row0 + (lane >> 4)) * I;
    g.srow[0] = a.down_scale + ((int64_t)tile.expert * (H / kScaleBlock) + row0 / kScaleBlock) * (I / kScaleBlock);
#pragma unroll
    for (int r = 0; r < R; ++r) g.xrow[r] = a.act + (int64_t)tile.route[r] * I;
    g.row_stride = I;
    g.k = I;
    float acc[1][4][R] = {};
    gemv_run(g, 0, steps, tile.count, lane, acc);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float v = sum16(acc[0][q][r]);
        if ((lane & 15) == 0 && r < tile.count) {
          const int route = tile.route[r];
          // bf16 down output times the bf16 route weight, rounded (routed_experts.py:104-105)
          res[route][4 * q + (lane >> 4)] = round_to_bf16(round_to_bf16(v) * round_to_bf16(a.weights[route]));
        }
      }
  }
  __syncthreads();
  // route combine: every token's slots in slot order, FP32 (or bf16 running) sum
  const int tokens = a.routes / a.top_k;
  for (int i = tid; i < tokens * kGemvRows; i += 64 * WAVES) {
    const int t = i / kGemvRows, row = i % kGemvRows;
    float sum = 0.f;
    for (int s = 0; s < a.top_k; ++s) {
      sum += res[t * a.top_k + s][row];
      if (a.bf16_sum) sum = round_to_bf16(sum);
    }
    a.out[(int64_t)t * H + row0 + row] = f32_to_bf16_bits(sum);
  }
  // health: ids in range, no duplicate id in a row, weights finite and >= 0 if asked
  if (blockIdx.x == 0 && wave == 0) {
    bool bad = false;
    if (lane < a.routes) {
      const int id = a.ids[lane];
      bad = id < 0 || id >= a.experts;
      const int t0 = (lane / a.top_k) * a.top_k;
      for (int s = t0; s < lane; ++s) bad |= a.ids[s] == id;
      if (a.check_weights) {
        const float w = a.weights[lane];
        bad |= !(w >= 0.0f) || isinf(w);
      }
    }
    const uint64_t any = __ballot(bad);
    if (lane == 0) a.valid[0] = any ? 0 : 1;
  }
}

template <int R>
hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const dim3 g1(a.routes, a.intermediate / kGemvRows);
  hipLaunchKernelGGL((decode_gate_up_kernel<R, 4>), g1, dim3(256), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (a.between_event) {
    err = hipEventRecord(static_cast<hipEvent_t>(a.between_event), stream);
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL((decode_down_kernel<R, 8>), dim3(a.hidden / kGemvRows), dim3(512), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

// One token: every expert carries one route (duplicates split into one-route
// tiles); more tokens: tiles of up to four routes share each weight byte.
hipError_t launch_decode_routed(const DecodeArgs& a, hipStream_t stream) {
  return a.routes <= a.top_k ? launch_decode<1>(a, stream) : launch_decode<4>(a, stream);
}

}  // namespace glm_moe
