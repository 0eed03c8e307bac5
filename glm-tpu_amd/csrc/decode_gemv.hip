// Decode path of the routed experts (at most 64 routes, e.g. T <= 8 tokens x
// top-8): two kernels, no separate route plan and no separate combine.
//
// 1. gate/up: workgroup = (route j, 16 intermediate rows); WK waves split K.
// 2. down:    workgroup = 8 hidden rows x every route; its waves take routes
//    in turn, write each route's weighted bf16 result to LDS, and the
//    workgroup then sums every token's slots in slot order (the route combine
//    of glm_tpu/layers/moe/routed_experts.py:104-117 / :291-293).
//
// With two or more tokens (and no routing inside the kernel) the multi kernels
// below run instead: routes selecting the same expert are grouped into units
// of up to two, so each unit streams its expert's rows once, and the resident
// shared expert streams its rows once per group of up to four tokens
// (gate/up) or once for all tokens (down, K split over the waves).
//
// Every active route is computed by exactly one wave; the j-th active route
// (flat order t * top_k + slot) is found with one ballot.  A route is active
// when the call owns its expert (RouteOwnership: an expert-parallel share owns
// a range of global ids; an invalid id is dropped or stands for the
// reference's safe id 0).
//
// Projections are GEMVs on the vector ALU.  A wave owns 16 (gate/up) or 8 (down) weight rows and a
// range of K "steps" of 256.  Each 128-bit load instruction covers 4 rows x
// 256 contiguous bytes (lane l: row 4q + l/16, bytes (l%16)*16), the access
// pattern that streams HBM at full rate; weight loads are the only vector
// memory traffic of the stream:
//   * the 128x128 block scales of the wave's K range are loaded once, one per
//     lane, and picked per step with v_readlane (the step is wave-uniform);
//   * the route's activations for the wave's K range are staged once into the
//     wave's own LDS region (their loads are issued before the first weight
//     loads, so waiting for them never waits for weights), followed by 16 zero
//     bf16 that the masked lanes of a half step read.
// Every e4m3 byte is decoded once, bf16(f32(e4m3) * block scale)
// (glm_tpu/layers/fp8.py:113-126), and multiplied with the bf16 activations
// by v_dot2c_f32_bf16 (exact bf16 products, FP32 accumulation).  The 16 lanes
// that share a row add their partial sums at the end.  DEPTH steps of weights
// are kept in flight per wave.
#include "moe_common.h"
#include "moe_kernels.h"
#include "router_wave.h"

namespace glm_moe {

namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kGemvRows = 16;      // weight rows per wave
constexpr int kStepK = 256;        // K per step: 16 lanes x 16 e4m3 bytes
constexpr int kMaxWaveSteps = 8;   // K range of one wave: 2048 (LDS staging, lane-held scales)
constexpr int kGateUpWaves = 4;
constexpr int kDownWaves = 8;
constexpr int kDownWavesFew = 4;   // <= 8 routes, no shared expert: 3 four-wave workgroups per CU, one pass
constexpr int kDownMultiWaves = 4; // the multi kernel (2+ tokens): 768 workgroups fit the GPU at once
constexpr int kGateUpDepth = 2;    // two tables: 2 x 32 VGPRs in flight
constexpr int kDownRows = 8;       // down: weight rows per workgroup (H / 8 = 768 workgroups: 3 per CU)
constexpr int kDownQuads = kDownRows / 4;
constexpr int kDownDepth = 6;      // one table, 8 rows: 6 x 8 VGPRs in flight
constexpr int kDownMultiDepth = 4; // the multi kernel's units of two routes: 4 x 8 VGPRs in flight
constexpr int kSharedGateUpRows = 8;   // resident shared expert: bf16 gate/up rows per workgroup
constexpr int kSharedGateUpDepth = 4;  // 2 tables x 8 bf16 rows: 4 steps (4 x 16 VGPRs) in flight

constexpr int kNonTemporal = 2;            // buffer load cache policy: streamed once (nt)
constexpr int kBufferFormat = 0x00020000;  // raw buffer descriptor word 3: 32-bit data format

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Buffer descriptor over `bytes` bytes from base (out-of-range loads return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_buffer(const uint8_t* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, (int)bytes, kBufferFormat);
}

// 16 bytes a lane from rsrc + voffset + soffset straight into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds).  The builtin exists only for the device target.
__device__ __forceinline__ void load_lds_16(__amdgpu_buffer_rsrc_t rsrc, uint16_t* lds, int voffset, int soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0,
                                           0);
#endif
}

// Wait until at most N of this wave's vector memory loads are outstanding
// (loads complete in issue order, direct-to-LDS loads included): the loads
// issued before the newest N are done.  The memory clobber keeps the compiler
// from moving memory accesses across it.
template <int N>
__device__ __forceinline__ void wait_loads_but() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Two packed bf16 of a 32-bit word.  The word is taken by value: hipcc 7.2
// lowers __builtin_bit_cast applied directly to a vector element (v[h]) to a
// read of element 0 whatever h is.
__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2, v); }

// v's value in lane `src` (wave-uniform index), as a scalar
__device__ __forceinline__ float lane_value(float v, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

struct DecodeRoute {
  int expert;
  int route;   // flat route id t * top_k + slot
};

// The j-th active (owned) route, wave-uniform; false when there are at most j.
__device__ __forceinline__ bool decode_route(const int32_t* ids, int n, const RouteOwnership& own, int j,
                                             DecodeRoute& r) {
  const int lane = threadIdx.x & 63;
  const int key = lane < n ? owned_expert(ids[lane], own) : -1;
  uint64_t active = __ballot(key >= 0);
  if (__popcll(active) <= j) return false;
  for (int skip = 0; skip < j; ++skip) active &= active - 1;
  r.route = uniform(__ffsll((unsigned long long)active) - 1);
  r.expert = __builtin_amdgcn_readlane(key, r.route);  // r.route is wave-uniform
  return true;
}

// The number of active routes (those decode_route enumerates), wave-uniform.
__device__ __forceinline__ int decode_active_routes(const int32_t* ids, int n, const RouteOwnership& own) {
  const int lane = threadIdx.x & 63;
  const bool active = lane < n && owned_expert(ids[lane], own) >= 0;
  return __popcll(__ballot(active));
}

// The K range [step_begin, step_end) of one wave over TABLES tables of the
// same 16 rows, against NR activation rows (NR routes of one expert: its
// weights are streamed and decoded once for all of them).
template <int TABLES, int NR = 1>
struct GemvStream {
  __amdgpu_buffer_rsrc_t w[TABLES];  // the 16 rows of each table (descriptor in SGPRs)
  uint32_t lane_off;            // (lane/16) * row_stride + (lane%16) * 16
  float sreg[TABLES];           // lane l: block scale 2 * step_begin + l of the rows
  int64_t row_stride;           // bytes between weight rows (= k)
  int k;
  int kblocks;                  // k / 128
  int step_begin, step_end;
  const uint16_t* x[NR];        // global activation rows (bf16, k entries)
  uint16_t* xs;                 // the wave's LDS region: per row, the K range then 16 zero bf16
  int xs_stride;                // elements between the rows' regions
  int pad;                      // element offset of the zeros in a row's region
};

// Activations of the wave's K range into registers (at most 4 x 16 bytes a lane a row).
template <int TABLES, int NR>
__device__ __forceinline__ void stage_x_load(const GemvStream<TABLES, NR>& g, int lane, u32x4 (&xv)[NR][4]) {
  const int kbeg = g.step_begin * kStepK;
  const int chunks = (min(g.step_end * kStepK, g.k) - kbeg) >> 3;
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane + 64 * i;
      if (c < chunks) xv[r][i] = *reinterpret_cast<const u32x4*>(g.x[r] + kbeg + 8 * c);
    }
}

template <int TABLES, int NR>
__device__ __forceinline__ void stage_x_store(const GemvStream<TABLES, NR>& g, int lane, const u32x4 (&xv)[NR][4]) {
  const int kbeg = g.step_begin * kStepK;
  const int chunks = (min(g.step_end * kStepK, g.k) - kbeg) >> 3;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    uint16_t* xs = g.xs + r * g.xs_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane + 64 * i;
      if (c < chunks) *reinterpret_cast<u32x4*>(xs + 8 * c) = xv[r][i];
    }
    if (lane < 2) *reinterpret_cast<u32x4*>(xs + g.pad + 8 * lane) = u32x4{0u, 0u, 0u, 0u};
  }
}

// The same staging by direct-to-LDS loads (1 KB an instruction, lanes past the
// range masked): no registers hold the rows, the caller waits for them with
// vmcnt (wait_loads_but) after issuing the weight loads that follow.
template <int TABLES, int NR>
__device__ __forceinline__ void stage_x_dma(const GemvStream<TABLES, NR>& g, int lane) {
  const int kbeg = g.step_begin * kStepK;
  const int len = min(g.step_end * kStepK, g.k) - kbeg;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    uint16_t* xs = g.xs + r * g.xs_stride;
    const __amdgpu_buffer_rsrc_t src = rows_buffer(reinterpret_cast<const uint8_t*>(g.x[r]), (int64_t)g.k * 2);
    for (int i = 0; i * 512 < len; ++i)
      if (i * 512 + 8 * lane < len) load_lds_16(src, xs + 512 * i, 16 * lane, 2 * (kbeg + 512 * i));
    if (lane < 2) *reinterpret_cast<u32x4*>(xs + g.pad + 8 * lane) = u32x4{0u, 0u, 0u, 0u};
  }
}

// Weights of step s0 + s: rows 4q + lane/16, 16 bytes at K = (s0 + s) * 256 + (lane%16) * 16.
// FULL: every step of the range is whole.  Otherwise the masked lanes of a
// half step (the last step of an odd k/128) load the row's last 16 bytes, in
// bounds; their products are zero.
template <bool FULL, int TABLES, int NR, int QN>
__device__ __forceinline__ void gemv_load(const GemvStream<TABLES, NR>& g, int s, int lane, u32x4 (&w)[TABLES][QN]) {
  // buffer loads: lane offset (VGPR) + step (immediate) + row group and range start (SGPR)
  uint32_t off = g.lane_off + s * kStepK;
  if constexpr (!FULL) {
    const int kofs = (g.step_begin + s) * kStepK + (lane & 15) * 16;
    if (kofs >= g.k) off -= (uint32_t)(kofs - (g.k - 16));
  }
#pragma unroll
  for (int t = 0; t < TABLES; ++t)
#pragma unroll
    for (int q = 0; q < QN; ++q)
      w[t][q] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(g.w[t], off, 4 * q * (int)g.row_stride + g.step_begin * kStepK,
                                                       kNonTemporal));
}

// acc[t][q][r] += sum over the lane's 16 K of bf16(e4m3 * scale) * x_r, for step s0 + s
template <bool FULL, int TABLES, int NR, int QN>
__device__ __forceinline__ void gemv_fma(const GemvStream<TABLES, NR>& g, const u32x4 (&w)[TABLES][QN], int s,
                                         int lane, float (&acc)[TABLES][QN][NR]) {
  int xoff = s * kStepK + (lane & 15) * 16;
  int b_hi = 2 * s + 1;
  bool keep = true;
  if constexpr (!FULL) {
    keep = (g.step_begin + s) * kStepK + (lane & 15) * 16 < g.k;
    xoff = keep ? xoff : g.pad;
    b_hi = min(2 * (g.step_begin + s) + 1, g.kblocks - 1) - 2 * g.step_begin;
  }
  u32x4 x0[NR], x1[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    x0[r] = *reinterpret_cast<const u32x4*>(g.xs + r * g.xs_stride + xoff);
    x1[r] = *reinterpret_cast<const u32x4*>(g.xs + r * g.xs_stride + xoff + 8);
  }
#pragma unroll
  for (int t = 0; t < TABLES; ++t) {
    const float s_lo = lane_value(g.sreg[t], 2 * s);
    const float s_hi = lane_value(g.sreg[t], b_hi);
    float scale = (lane & 15) < 8 ? s_lo : s_hi;
    if constexpr (!FULL) scale = keep ? scale : 0.0f;
#pragma unroll
    for (int q = 0; q < QN; ++q) {
      const u32x4 lo = __builtin_bit_cast(u32x4, decode_fp8x8(w[t][q][0], w[t][q][1], scale));
      const u32x4 hi = __builtin_bit_cast(u32x4, decode_fp8x8(w[t][q][2], w[t][q][3], scale));
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float a = acc[t][q][r];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t wv = lo[h], xv = x0[r][h];
          a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv), as_bf16x2(xv), a, false);
        }
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t wv = hi[h], xv = x1[r][h];
          a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv), as_bf16x2(xv), a, false);
        }
        acc[t][q][r] = a;
      }
    }
  }
}

// Straight-line stream of exactly NSTEPS steps, DEPTH in flight: with no loop
// back-edge the compiler counts outstanding loads exactly and waits only for
// the step it is about to multiply.  Order of issue: activation staging
// loads, the first DEPTH weight steps, then the staging stores (which wait
// for the activations only).
template <int NSTEPS, int DEPTH, bool DMA, int TABLES, int NR, int QN>
__device__ __forceinline__ void gemv_run_fixed(const GemvStream<TABLES, NR>& g, int lane,
                                               float (&acc)[TABLES][QN][NR]) {
  constexpr int D = DEPTH < NSTEPS ? DEPTH : NSTEPS;
  u32x4 xv[DMA ? 1 : NR][4];
  if constexpr (DMA) {
    stage_x_dma(g, lane);
  } else {
    stage_x_load(g, lane, xv);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 ring[D][TABLES][QN];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    gemv_load<true>(g, d, lane, ring[d]);
    __builtin_amdgcn_sched_barrier(0);  // issue step by step: waiting for one never waits for the next
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (DMA) {
    wait_loads_but<D * TABLES * QN>();
  } else {
    stage_x_store(g, lane, xv);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < NSTEPS; ++s) {
    gemv_fma<true>(g, ring[s % D], s, lane, acc);
    if (s + D < NSTEPS) {
      __builtin_amdgcn_sched_barrier(0);
      gemv_load<true>(g, s + D, lane, ring[s % D]);
    }
  }
}

// Any range, half step included: a loop over groups of DEPTH steps whose
// refills are issued unconditionally (a refill past the end reloads the last step).
template <int DEPTH, bool DMA, int TABLES, int NR, int QN>
__device__ __forceinline__ void gemv_run_loop(const GemvStream<TABLES, NR>& g, int lane,
                                              float (&acc)[TABLES][QN][NR]) {
  const int n = g.step_end - g.step_begin, last = n - 1;
  u32x4 xv[DMA ? 1 : NR][4];
  if constexpr (DMA) {
    stage_x_dma(g, lane);
  } else {
    stage_x_load(g, lane, xv);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 ring[DEPTH][TABLES][QN];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    gemv_load<false>(g, min(d, last), lane, ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (DMA) {
    wait_loads_but<DEPTH * TABLES * QN>();
  } else {
    stage_x_store(g, lane, xv);
  }
  __builtin_amdgcn_sched_barrier(0);
  for (int s = 0; s < n; s += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      if (s + d < n) gemv_fma<false>(g, ring[d], s + d, lane, acc);
      __builtin_amdgcn_sched_barrier(0);
      gemv_load<false>(g, min(s + d + DEPTH, last), lane, ring[d]);
    }
  }
}

// DMA: stage the activation rows by direct-to-LDS loads instead of through registers.
template <int DEPTH, bool DMA = false, int TABLES, int NR, int QN>
__device__ __forceinline__ void gemv_run(const GemvStream<TABLES, NR>& g, int lane, float (&acc)[TABLES][QN][NR]) {
  const int n = g.step_end - g.step_begin;
  if (n <= 0) return;
  // a half step exists when k / 128 is odd; it is the last step of the last range
  const bool half = (g.kblocks & 1) && g.step_end * kStepK > g.k;
  if (!half) {
    switch (n) {
      case 2: gemv_run_fixed<2, DEPTH, DMA>(g, lane, acc); return;
      case 4: gemv_run_fixed<4, DEPTH, DMA>(g, lane, acc); return;
      case 6: gemv_run_fixed<6, DEPTH, DMA>(g, lane, acc); return;
      case 8:
        // two tables: eight straight-line steps exceed the register budget
        if constexpr (TABLES == 1) {
          gemv_run_fixed<8, DEPTH, DMA>(g, lane, acc);
          return;
        }
        break;
      default: break;
    }
  }
  gemv_run_loop<DEPTH, DMA>(g, lane, acc);
}

// Block scales 2 * step_begin + lane of the 16 rows (rows share one 128-row block).
__device__ __forceinline__ float lane_scale(const float* srow, int kblocks, int step_begin, int lane) {
  const int b = 2 * step_begin + lane;
  return b < kblocks ? srow[b] : 0.0f;
}

// v plus the same value DPP-moved from another lane of its 16-lane row (dpp_ctrl).
template <int CTRL>
__device__ __forceinline__ float add_dpp(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                   false));
}

// Sum over the 16 lanes that share rows (one 16-lane row of the wave); every
// lane of the group gets the sum.  A butterfly of DPP moves -- quad lanes xor 1
// and xor 2, then the half-row and row mirrors, each pairing lanes whose
// partial sums cover disjoint halves -- so no step waits on an LDS round trip.
__device__ __forceinline__ float sum16(float v) {
  v = add_dpp<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = add_dpp<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = add_dpp<0x141>(v);  // row_half_mirror
  v = add_dpp<0x140>(v);  // row_mirror
  return v;
}

__host__ __device__ constexpr int xs_elems(int wave_steps) { return wave_steps * kStepK + 16; }

// ------------------------------------------------------------------ bf16 weights (resident shared expert)
// The same 16-row streams over bf16 tables: a step is still 256 bytes of a row
// (4 rows x 256 B per load instruction), now 128 K; products are exact bf16 x
// bf16 in v_dot2c_f32_bf16 with FP32 sums, as the reference's resident_matmul
// (glm_tpu/layers/linear.py:26-33).  K is a multiple of 128 (whole steps).
constexpr int kBf16StepK = kStepK / 2;

template <int TABLES>
struct Bf16Stream {
  __amdgpu_buffer_rsrc_t w[TABLES];
  uint32_t lane_off;   // (lane/16) * row_bytes + (lane%16) * 16
  int row_bytes;       // 2 k
  int k;
  int step_begin, step_end;  // steps of 128 elements
  const uint16_t* x;   // activation row (bf16, k entries)
  uint16_t* xs;        // the wave's LDS region (the K range)
};

template <int TABLES, int QN>
__device__ __forceinline__ void bf16_load(const Bf16Stream<TABLES>& g, int s, u32x4 (&w)[TABLES][QN]) {
  const uint32_t off = g.lane_off + s * kStepK;
#pragma unroll
  for (int t = 0; t < TABLES; ++t)
#pragma unroll
    for (int q = 0; q < QN; ++q)
      w[t][q] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(g.w[t], off, 4 * q * g.row_bytes + g.step_begin * kStepK,
                                                       kNonTemporal));
}

template <int TABLES, int QN>
__device__ __forceinline__ void bf16_fma(const Bf16Stream<TABLES>& g, const u32x4 (&w)[TABLES][QN], int s, int lane,
                                         float (&acc)[TABLES][QN]) {
  const u32x4 x = *reinterpret_cast<const u32x4*>(g.xs + s * kBf16StepK + (lane & 15) * 8);
#pragma unroll
  for (int t = 0; t < TABLES; ++t)
#pragma unroll
    for (int q = 0; q < QN; ++q) {
      float a = acc[t][q];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t wv = w[t][q][h], xv = x[h];
        a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv), as_bf16x2(xv), a, false);
      }
      acc[t][q] = a;
    }
}

// The wave's K range with DEPTH steps of weights in flight; the activations
// are staged once into the wave's LDS region (loads issued before the weights).
template <int DEPTH, int TABLES, int QN>
__device__ __forceinline__ void bf16_run(const Bf16Stream<TABLES>& g, int lane, float (&acc)[TABLES][QN]) {
  const int n = g.step_end - g.step_begin;
  if (n <= 0) return;
  const int last = n - 1;
  const int kbeg = g.step_begin * kBf16StepK;
  const int chunks = (n * kBf16StepK) >> 3;  // 8 bf16 a chunk, at most 256
  u32x4 xv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) xv[i] = *reinterpret_cast<const u32x4*>(g.x + kbeg + 8 * c);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 ring[DEPTH][TABLES][QN];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    bf16_load(g, min(d, last), ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) *reinterpret_cast<u32x4*>(g.xs + 8 * c) = xv[i];
  }
  __builtin_amdgcn_sched_barrier(0);
  for (int s = 0; s < n; s += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      if (s + d < n) bf16_fma(g, ring[d], s + d, lane, acc);
      __builtin_amdgcn_sched_barrier(0);
      bf16_load(g, min(s + d + DEPTH, last), ring[d]);
    }
  }
}

// LDS elements a wave's staging region needs for K range `wave_steps` steps of
// e4m3 (256 K each) or the same range in bf16 steps.
__host__ __device__ constexpr int bf16_wave_steps(int k, int waves) {
  return ((k / kBf16StepK) + waves - 1) / waves;
}

// ------------------------------------------------------------------ gate/up + SwiGLU
template <int WK>
__global__ __launch_bounds__(64 * WK) __attribute__((amdgpu_waves_per_eu(4)))
void decode_gate_up_kernel(const DecodeArgs a, int wave_steps) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float(*red)[2][kGemvRows] = reinterpret_cast<float(*)[2][kGemvRows]>(smem);
  const int lane = threadIdx.x & 63;
  const int wk = uniform(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  // health starts true; the down kernel (next on the stream) only clears it
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) a.valid[0] = 1;
  const int I = a.intermediate, H = a.hidden;
  const int row0 = blockIdx.y * kGemvRows;
  if ((int)blockIdx.x >= a.routes) {
    // the resident shared expert of token (blockIdx.x - routes) / 2: bf16 gate/up +
    // SwiGLU of 8 of the row block's 16 rows, so that a shared workgroup streams
    // as many bytes as a routed one (8 bf16 rows = 16 e4m3 rows)
    const int t = (blockIdx.x - a.routes) >> 1;
    const int srow0 = row0 + kSharedGateUpRows * ((blockIdx.x - a.routes) & 1);
    const int ws = bf16_wave_steps(H, WK);
    Bf16Stream<2> g;
    g.k = H;
    g.row_bytes = 2 * H;
    g.lane_off = (uint32_t)((lane >> 4) * 2 * H + (lane & 15) * 16);
    g.step_begin = min(wk * ws, H / kBf16StepK);
    g.step_end = min(g.step_begin + ws, H / kBf16StepK);
    g.w[0] = rows_buffer(reinterpret_cast<const uint8_t*>(a.shared_gate + (int64_t)srow0 * H),
                         (int64_t)kSharedGateUpRows * 2 * H);
    g.w[1] = rows_buffer(reinterpret_cast<const uint8_t*>(a.shared_up + (int64_t)srow0 * H),
                         (int64_t)kSharedGateUpRows * 2 * H);
    g.x = a.hidden_in + (int64_t)t * H;
    g.xs = reinterpret_cast<uint16_t*>(smem + sizeof(float) * WK * 2 * kGemvRows) + wk * xs_elems(wave_steps);
    constexpr int QN = kSharedGateUpRows / 4;
    float acc[2][QN] = {};
    bf16_run<kSharedGateUpDepth>(g, lane, acc);
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int q = 0; q < QN; ++q) {
        const float v = sum16(acc[tb][q]);
        if ((lane & 15) == 0) red[wk][tb][4 * q + (lane >> 4)] = v;
      }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < kSharedGateUpRows) {
      float gsum = 0.f, usum = 0.f;
      for (int w = 0; w < WK; ++w) {
        gsum += red[w][0][tid];
        usum += red[w][1][tid];
      }
      const float v = swiglu_bf16(round_to_bf16(gsum), round_to_bf16(usum));
      a.act_shared[(int64_t)t * I + srow0 + tid] = f32_to_bf16_bits(v);
    }
    return;
  }
  DecodeRoute rt;
  if (a.router_logits != nullptr) {
    // route j = t * top_k + s of token t: every wave routes the token itself
    // (top-k ids are distinct and in range, so every route is active); the
    // token's first-slot workgroup of row block 0 publishes ids and weights
    const int j = blockIdx.x, t = j / a.top_k, s = j % a.top_k;
    int my_id;
    float my_weight;
    route_token_noaux<kDecodeRouterExperts / 64>(a.router_logits + (int64_t)t * a.own.experts, a.own.experts,
                                                 a.router_bias, a.top_k, lane, my_id, my_weight);
    rt.route = j;
    rt.expert = __builtin_amdgcn_readlane(my_id, s);  // s is wave-uniform
    if (s == 0 && blockIdx.y == 0 && wk == 0 && lane < a.top_k) {
      a.ids_out[j + lane] = my_id;
      a.weights_out[j + lane] = my_weight;
    }
  } else if (!decode_route(a.ids, a.routes, a.own, blockIdx.x, rt)) {
    return;
  }
  const int steps = (H + kStepK - 1) / kStepK;
  GemvStream<2> g;
  g.k = H;
  g.kblocks = H / kScaleBlock;
  g.row_stride = H;
  g.lane_off = (uint32_t)((lane >> 4) * H + (lane & 15) * 16);
  g.step_begin = min(wk * wave_steps, steps);
  g.step_end = min(g.step_begin + wave_steps, steps);
  const uint8_t* tables[2] = {a.gate_bits, a.up_bits};
  const float* scales[2] = {a.gate_scale, a.up_scale};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    g.w[t] = rows_buffer(tables[t] + ((int64_t)rt.expert * I + row0) * H, (int64_t)kGemvRows * H);
    const float* srow = scales[t] + ((int64_t)rt.expert * (I / kScaleBlock) + row0 / kScaleBlock) * g.kblocks;
    g.sreg[t] = lane_scale(srow, g.kblocks, g.step_begin, lane);
  }
  g.x[0] = a.hidden_in + (int64_t)(rt.route / a.top_k) * H;
  g.xs = reinterpret_cast<uint16_t*>(smem + sizeof(float) * WK * 2 * kGemvRows) + wk * xs_elems(wave_steps);
  g.xs_stride = xs_elems(wave_steps);
  g.pad = wave_steps * kStepK;
  float acc[2][4][1] = {};
  gemv_run<kGateUpDepth>(g, lane, acc);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float v = sum16(acc[t][q][0]);
      if ((lane & 15) == 0) red[wk][t][4 * q + (lane >> 4)] = v;
    }
  __syncthreads();
  // one thread per row: wave-order split-K sum, then the bf16 SwiGLU
  const int tid = threadIdx.x;
  if (tid < kGemvRows) {
    float gsum = 0.f, usum = 0.f;
    for (int w = 0; w < WK; ++w) {
      gsum += red[w][0][tid];
      usum += red[w][1][tid];
    }
    const float v = swiglu_bf16(round_to_bf16(gsum), round_to_bf16(usum));
    a.act[(int64_t)rt.route * I + row0 + tid] = f32_to_bf16_bits(v);
  }
}

// ------------------------------------------------------------------ down + weighting + combine
// RESIDENT: the resident shared expert's down rows are computed here too (a
// separate instantiation, so the routed-only kernel keeps its registers).
template <int WAVES, bool RESIDENT>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(4)))
void decode_down_kernel(const DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float(*res)[kGemvRows] = reinterpret_cast<float(*)[kGemvRows]>(smem);  // [kMaxDecodeRoutes][16]
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  const int tid = threadIdx.x;
  const int I = a.intermediate, H = a.hidden;
  const int row0 = blockIdx.x * kDownRows;
  const int steps = (I + kStepK - 1) / kStepK;
  for (int i = tid; i < a.routes * kGemvRows; i += 64 * WAVES) res[i / kGemvRows][i % kGemvRows] = 0.f;
  __syncthreads();
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem + sizeof(float) * kMaxDecodeRoutes * kGemvRows) +
                 wave * xs_elems(steps);
  // [tokens][16] bf16 shared-expert down rows, after every wave's staging region
  float(*res_sh)[kGemvRows] = reinterpret_cast<float(*)[kGemvRows]>(
      smem + sizeof(float) * kMaxDecodeRoutes * kGemvRows + sizeof(uint16_t) * WAVES * xs_elems(steps));
  const int tokens = a.routes / a.top_k;
  const int active = RESIDENT ? decode_active_routes(a.ids, a.routes, a.own) : kMaxDecodeRoutes;
  const int jobs = RESIDENT ? active + tokens : kMaxDecodeRoutes;
  for (int j = wave; j < jobs; j += WAVES) {
    if (RESIDENT && j >= active) {
      // the resident shared expert's down projection of token j - active (bf16, unweighted)
      const int t = j - active;
      Bf16Stream<1> g;
      g.k = I;
      g.row_bytes = 2 * I;
      g.lane_off = (uint32_t)((lane >> 4) * 2 * I + (lane & 15) * 16);
      g.step_begin = 0;
      g.step_end = I / kBf16StepK;
      g.w[0] = rows_buffer(reinterpret_cast<const uint8_t*>(a.shared_down + (int64_t)row0 * I),
                           (int64_t)kDownRows * 2 * I);
      g.x = a.act_shared + (int64_t)t * I;
      g.xs = xs;
      float acc[1][kDownQuads] = {};
      bf16_run<kDownDepth>(g, lane, acc);
#pragma unroll
      for (int q = 0; q < kDownQuads; ++q) {
        const float v = sum16(acc[0][q]);
        if ((lane & 15) == 0) res_sh[t][4 * q + (lane >> 4)] = round_to_bf16(v);
      }
      continue;
    }
    DecodeRoute rt;
    if (!decode_route(a.ids, a.routes, a.own, j, rt)) break;
    GemvStream<1> g;
    g.k = I;
    g.kblocks = I / kScaleBlock;
    g.row_stride = I;
    g.step_begin = 0;
    g.step_end = steps;
    g.w[0] = rows_buffer(a.down_bits + ((int64_t)rt.expert * H + row0) * I, (int64_t)kDownRows * I);
    g.lane_off = (uint32_t)((lane >> 4) * I + (lane & 15) * 16);
    const float* srow = a.down_scale + ((int64_t)rt.expert * (H / kScaleBlock) + row0 / kScaleBlock) * g.kblocks;
    g.sreg[0] = lane_scale(srow, g.kblocks, 0, lane);
    g.x[0] = a.act + (int64_t)rt.route * I;
    g.xs = xs;
    g.xs_stride = xs_elems(steps);
    g.pad = steps * kStepK;
    const float wr = round_to_bf16(a.weights[rt.route]);  // loaded before the weight stream
    float acc[1][kDownQuads][1] = {};
    gemv_run<kDownDepth>(g, lane, acc);
#pragma unroll
    for (int q = 0; q < kDownQuads; ++q) {
      const float v = sum16(acc[0][q][0]);
      // bf16 down output times the bf16 route weight, rounded (routed_experts.py:104-105)
      if ((lane & 15) == 0) res[rt.route][4 * q + (lane >> 4)] = round_to_bf16(round_to_bf16(v) * wr);
    }
  }
  __syncthreads();
  // route combine: every token's slots in slot order, FP32 sum rounded once to
  // bf16 (the prefill body's route sum, and the decode body's per-owner bf16 sum,
  // which JAX computes in FP32: routed_experts.py:110-115, :293)
  for (int i = tid; i < tokens * kDownRows; i += 64 * WAVES) {
    const int t = i / kDownRows, row = i % kDownRows;
    float sum = 0.f;
    for (int s = 0; s < a.top_k; ++s) sum += res[t * a.top_k + s][row];
    const int64_t o = (int64_t)t * H + row0 + row;
    if (a.out_f32 != nullptr) {
      // a share's partial for the caller's sum over the expert axis
      a.out_f32[o] = a.round_partial ? round_to_bf16(sum) : sum;
      continue;
    }
    if (RESIDENT) {
      // layer epilogue with the resident shared expert computed above
      sum = round_to_bf16(round_to_bf16(round_to_bf16(sum) * a.routed_scale) + res_sh[t][row]);
      if (!isfinite(sum)) a.valid[0] = 0;
    } else if (a.shared != nullptr) {
      // layer epilogue (routed_experts.py:125, :303): bf16(bf16(routed * scale) + shared)
      sum = round_to_bf16(round_to_bf16(round_to_bf16(sum) * a.routed_scale) + bf16_bits_to_f32(a.shared[o]));
      if (!isfinite(sum)) a.valid[0] = 0;
    }
    a.out[o] = f32_to_bf16_bits(sum);
  }
  // health: ids in range, no duplicate id in a row, weights finite and >= 0 if asked
  if (blockIdx.x == 0 && wave == 0) {
    bool bad = false;
    if (lane < a.routes) {
      const int id = a.ids[lane];
      bad = id < 0 || id >= a.own.global_experts;
      const int t0 = (lane / a.top_k) * a.top_k;
      for (int s = t0; s < lane; ++s) bad |= a.ids[s] == id;
      if (a.check_weights) {
        const float w = a.weights[lane];
        bad |= !(w >= 0.0f) || isinf(w);
      }
    }
    const uint64_t any = __ballot(bad);
    if (lane == 0 && any) a.valid[0] = 0;
  }
}


// ------------------------------------------------------------------ bf16 shared expert over a few rows
// For tokens > 1 the resident path above streams the shared tables once per
// token; these two kernels stream them once for all NT rows.  Workgroup = 8
// weight rows (two quads) x every row; its 4 waves split K; a wave stages its
// K range of all NT activation rows in its LDS region and, per step of 128 K,
// multiplies the 8 weight rows' bf16 chunks (4 rows x 256 B per load, as the
// resident path) with each row's chunk in v_dot2c_f32_bf16 (exact products,
// FP32 sums).  Rounding points as the resident path: bf16 gate and up sums,
// bf16 SwiGLU, bf16 down sums.
constexpr int kSharedWgRows = 8;
constexpr int kSharedWaves = 4;
constexpr int kSharedQuads = kSharedWgRows / 4;

template <int TABLES, int NT>
__device__ __forceinline__ void bf16_rows_fma(const u32x4 (&w)[TABLES][kSharedQuads], const uint16_t* xs, int range,
                                              int s, int lane, float (&acc)[TABLES][kSharedQuads][NT]) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(xs + t * range + s * kBf16StepK + (lane & 15) * 8);
#pragma unroll
    for (int tb = 0; tb < TABLES; ++tb)
#pragma unroll
      for (int q = 0; q < kSharedQuads; ++q) {
        float a = acc[tb][q][t];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t wv = w[tb][q][h], xv = x[h];
          a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv), as_bf16x2(xv), a, false);
        }
        acc[tb][q][t] = a;
      }
  }
}

// One wave: K range [step_begin, step_end) of the 8 rows of every table against
// NT rows x[t * k + ...], staged at xs (NT x range elements).
template <int TABLES, int NT>
__device__ __forceinline__ void bf16_rows_run(Bf16Stream<TABLES>& g, const uint16_t* x, int range, int lane,
                                              float (&acc)[TABLES][kSharedQuads][NT]) {
  const int n = g.step_end - g.step_begin;
  if (n <= 0) return;
  const int last = n - 1;
  const int kbeg = g.step_begin * kBf16StepK;
  const int per_row = (n * kBf16StepK) >> 3;  // 16-byte chunks of one row's range
  for (int c = lane; c < NT * per_row; c += 64) {
    const int t = c / per_row, i = c % per_row;
    *reinterpret_cast<u32x4*>(g.xs + t * range + 8 * i) =
        *reinterpret_cast<const u32x4*>(x + (int64_t)t * g.k + kbeg + 8 * i);
  }
  constexpr int D = 2;
  u32x4 ring[D][TABLES][kSharedQuads];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    bf16_load(g, min(d, last), ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int s = 0; s < n; s += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (s + d < n) bf16_rows_fma<TABLES, NT>(ring[d], g.xs, range, s + d, lane, acc);
      __builtin_amdgcn_sched_barrier(0);
      bf16_load(g, min(s + d + D, last), ring[d]);
    }
  }
}

__host__ __device__ constexpr int shared_wave_steps(int k) { return ((k / kBf16StepK) + kSharedWaves - 1) / kSharedWaves; }

// TABLES == 2: gate/up rows of `intermediate`, SwiGLU into act [NT, I].
// TABLES == 1: down rows of `hidden` from act, into out [NT, H].
template <int TABLES, int NT>
__global__ __launch_bounds__(64 * kSharedWaves) void shared_rows_kernel(const uint16_t* x, int k,
                                                                         const uint16_t* w0, const uint16_t* w1,
                                                                         int n, uint16_t* out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float(*red)[TABLES][kSharedWgRows][NT] = reinterpret_cast<float(*)[TABLES][kSharedWgRows][NT]>(smem);
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int row0 = blockIdx.x * kSharedWgRows;
  const int ws = shared_wave_steps(k);
  const int range = ws * kBf16StepK;
  Bf16Stream<TABLES> g;
  g.k = k;
  g.row_bytes = 2 * k;
  g.lane_off = (uint32_t)((lane >> 4) * 2 * k + (lane & 15) * 16);
  g.step_begin = min(wave * ws, k / kBf16StepK);
  g.step_end = min(g.step_begin + ws, k / kBf16StepK);
  const uint16_t* tables[2] = {w0, w1};
#pragma unroll
  for (int tb = 0; tb < TABLES; ++tb)
    g.w[tb] = rows_buffer(reinterpret_cast<const uint8_t*>(tables[tb] + (int64_t)row0 * k),
                          (int64_t)kSharedWgRows * 2 * k);
  g.x = nullptr;
  g.xs = reinterpret_cast<uint16_t*>(smem + sizeof(float) * kSharedWaves * TABLES * kSharedWgRows * NT) +
         wave * NT * range;
  float acc[TABLES][kSharedQuads][NT] = {};
  bf16_rows_run<TABLES, NT>(g, x, range, lane, acc);
#pragma unroll
  for (int tb = 0; tb < TABLES; ++tb)
#pragma unroll
    for (int q = 0; q < kSharedQuads; ++q)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float v = sum16(acc[tb][q][t]);
        if ((lane & 15) == 0) red[wave][tb][4 * q + (lane >> 4)][t] = v;
      }
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < kSharedWgRows * NT) {
    const int row = tid % kSharedWgRows, t = tid / kSharedWgRows;
    float s0 = 0.f, s1 = 0.f;
    for (int w = 0; w < kSharedWaves; ++w) {  // wave order: deterministic
      s0 += red[w][0][row][t];
      s1 += red[w][TABLES - 1][row][t];
    }
    const float v = TABLES == 2 ? swiglu_bf16(round_to_bf16(s0), round_to_bf16(s1)) : s0;
    out[(int64_t)t * n + row0 + row] = f32_to_bf16_bits(v);
  }
}

template <int TABLES, int NT>
hipError_t launch_shared_rows(const uint16_t* x, int k, const uint16_t* w0, const uint16_t* w1, int n, uint16_t* out,
                              hipStream_t stream) {
  static std::atomic<uint64_t> lds_set{0};
  const hipError_t err = allow_full_lds(reinterpret_cast<const void*>(shared_rows_kernel<TABLES, NT>), lds_set);
  if (err != hipSuccess) return err;
  const size_t lds = sizeof(float) * kSharedWaves * TABLES * kSharedWgRows * NT +
                     sizeof(uint16_t) * kSharedWaves * NT * shared_wave_steps(k) * kBf16StepK;
  label_next_launch("shared_expert_rows_s%d_t%d_k%d_n%d", NT, TABLES, k, n);
  return launch_kernel(shared_rows_kernel<TABLES, NT>, dim3(n / kSharedWgRows), dim3(64 * kSharedWaves), lds, stream,
                       x, k, w0, w1, n, out);
}

template <int NT>
hipError_t launch_shared_expert_nt(const uint16_t* x, int hidden, int intermediate, const uint16_t* gate,
                                   const uint16_t* up, const uint16_t* down, uint16_t* act, uint16_t* out,
                                   hipStream_t stream) {
  hipError_t err = launch_shared_rows<2, NT>(x, hidden, gate, up, intermediate, act, stream);
  if (err != hipSuccess) return err;
  return launch_shared_rows<1, NT>(act, intermediate, down, nullptr, hidden, out, stream);
}

int gate_up_wave_steps(int hidden) {
  const int steps = (hidden + kStepK - 1) / kStepK;
  return (steps + kGateUpWaves - 1) / kGateUpWaves;
}


// ------------------------------------------------------------------ batched decode (2 .. 64 routes of 2+ tokens)
// With more than one token, routes of different tokens often select the same
// expert (T=4, top-8: 32 routes over ~30.5 distinct experts).  The multi
// kernels group the active routes by expert and stream each expert's rows once
// for a "unit" of up to kUnitRoutes of its routes (flat order within the
// expert), decoding every e4m3 byte once for all of them.  The resident bf16
// shared expert runs for every token in the same two launches: gate/up streams
// its rows once per group of up to kSharedGroupTokens tokens, down streams
// them once, its K split over the workgroup's waves.  Arithmetic and rounding
// points are those of the one-token kernels above.
constexpr int kUnitRoutes = 2;       // at most, a unit's routes (down kernel)
constexpr int kGateUpUnitRoutes = 2;  // a gate/up unit's routes
constexpr int kSharedGroupTokens = 4;
constexpr int kMultiStageRows = 4;    // activation rows a gate/up wave stages (max of the two above)
constexpr int kMultiSharedTokens = 8;  // tokens of the resident shared expert in the multi kernels

// LDS elements of one down wave's staging region: a unit's act rows, or with
// the resident shared expert every token's K slice if that is larger.
__host__ __device__ constexpr int down_multi_region(int intermediate, int waves, bool resident) {
  const int unit = kUnitRoutes * xs_elems((intermediate + kStepK - 1) / kStepK);
  const int slice = kMultiSharedTokens * ((intermediate / kBf16StepK + waves - 1) / waves) * kBf16StepK;
  return resident && slice > unit ? slice : unit;
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int src) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, src);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ int key_bits_of(int keys) {
  int b = 0;
  while ((1 << b) < keys) ++b;
  return b;
}

struct DecodeUnit {
  int expert;
  int count;                // 1 .. kUnitRoutes
  int route[kUnitRoutes];   // flat route ids, ascending
};

// Lanes (routes) with this lane's owned expert: one ballot per key bit
// (ballots of the active routes with the bit set, intersected or excluded).
__device__ __forceinline__ uint64_t same_expert_routes(int key, uint64_t active, int key_bits) {
  uint64_t same = active;
  for (int b = 0; b < key_bits; ++b) {
    const uint64_t ones = __ballot(key >= 0 && ((key >> b) & 1));
    same &= ((key >> b) & 1) ? ones : ~ones;
  }
  return same;
}

// The j-th unit (wave-uniform): each owned expert's active routes in flat
// order, cut into runs of U <= kUnitRoutes; units ordered by their first
// route.  false when there are at most j units.
template <int U>
__device__ __forceinline__ bool decode_unit(const int32_t* ids, int n, const RouteOwnership& own, int key_bits, int j,
                                            DecodeUnit& u) {
  static_assert(U >= 1 && U <= kUnitRoutes, "unit size");
  const int lane = threadIdx.x & 63;
  const int key = lane < n ? owned_expert(ids[lane], own) : -1;
  const uint64_t active = __ballot(key >= 0);
  const uint64_t same = same_expert_routes(key, active, key_bits);
  const int rank = __popcll(same & ((1ull << lane) - 1));
  uint64_t starts = __ballot(key >= 0 && rank % U == 0);
  if (__popcll(starts) <= j) return false;
  for (int skip = 0; skip < j; ++skip) starts &= starts - 1;
  const int r0 = uniform(__ffsll((unsigned long long)starts) - 1);
  u.expert = __builtin_amdgcn_readlane(key, r0);
  uint64_t rest = readlane64(same, r0) & ~((2ull << r0) - 1);  // the expert's routes after r0 (r0 = 63: none)
  u.route[0] = r0;
  u.count = 1;
#pragma unroll
  for (int i = 1; i < kUnitRoutes; ++i) {
    const bool more = i < U && rest != 0;
    u.route[i] = more ? uniform(__ffsll((unsigned long long)rest) - 1) : r0;
    u.count += more ? 1 : 0;
    rest &= rest - 1;
  }
  return true;
}

// The number of units of U routes (wave-uniform).
template <int U>
__device__ __forceinline__ int decode_units(const int32_t* ids, int n, const RouteOwnership& own, int key_bits) {
  const int lane = threadIdx.x & 63;
  const int key = lane < n ? owned_expert(ids[lane], own) : -1;
  const uint64_t active = __ballot(key >= 0);
  const uint64_t same = same_expert_routes(key, active, key_bits);
  const int rank = __popcll(same & ((1ull << lane) - 1));
  return __popcll(__ballot(key >= 0 && rank % U == 0));
}

// Activation rows r < NS (element offsets row_elem[r] into src) of the K range
// [kbeg, kbeg + len) into xs + r * stride, by direct-to-LDS loads of 1 KB an
// instruction (lanes past the range masked, so nothing beyond it is written).
// No registers hold them; the wave waits for them with vmcnt before it reads.
template <int NS>
__device__ __forceinline__ void stage_rows_lds(__amdgpu_buffer_rsrc_t src, const int (&row_elem)[NS], int kbeg, int len,
                                               uint16_t* xs, int stride, int lane) {
#pragma unroll
  for (int r = 0; r < NS; ++r)
    for (int i = 0; i * 512 < len; ++i)
      if (i * 512 + 8 * lane < len) load_lds_16(src, xs + r * stride + 512 * i, 16 * lane, 2 * (row_elem[r] + kbeg + 512 * i));
}

// bf16 rows (QN quads) of TABLES tables against NS staged activation rows.
template <int TABLES, int QN, int NS>
__device__ __forceinline__ void bf16_group_fma(const u32x4 (&w)[TABLES][QN], const uint16_t* xs, int stride, int s,
                                               int lane, float (&acc)[TABLES][QN][NS]) {
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(xs + t * stride + s * kBf16StepK + (lane & 15) * 8);
#pragma unroll
    for (int tb = 0; tb < TABLES; ++tb)
#pragma unroll
      for (int q = 0; q < QN; ++q) {
        float a = acc[tb][q][t];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t wv = w[tb][q][h], xv = x[h];
          a = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wv), as_bf16x2(xv), a, false);
        }
        acc[tb][q][t] = a;
      }
  }
}

// One wave's K range of 4 * QN bf16 rows of TABLES tables against NS
// activation rows (src + row_elem[t]), staged direct to LDS at xs (stride
// elements a row); DEPTH steps of weights in flight.
template <int DEPTH, int TABLES, int QN, int NS>
__device__ __forceinline__ void bf16_group_run(const Bf16Stream<TABLES>& g, __amdgpu_buffer_rsrc_t src,
                                               const int (&row_elem)[NS], uint16_t* xs, int stride, int lane,
                                               float (&acc)[TABLES][QN][NS]) {
  const int n = g.step_end - g.step_begin;
  if (n <= 0) return;
  const int last = n - 1;
  stage_rows_lds<NS>(src, row_elem, g.step_begin * kBf16StepK, n * kBf16StepK, xs, stride, lane);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 ring[DEPTH][TABLES][QN];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    bf16_load(g, min(d, last), ring[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_loads_but<DEPTH * TABLES * QN>();  // the staged rows are in LDS; the weight steps stay in flight
  for (int s = 0; s < n; s += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      if (s + d < n) bf16_group_fma<TABLES, QN, NS>(ring[d], xs, stride, s + d, lane, acc);
      __builtin_amdgcn_sched_barrier(0);
      bf16_load(g, min(s + d + DEPTH, last), ring[d]);
    }
  }
}

// gate/up of one unit: NR routes of one expert, 16 intermediate rows.
template <int WK, int NR>
__device__ __forceinline__ void gate_up_unit(const DecodeArgs& a, const DecodeUnit& u, int wave_steps, int stage_rows,
                                             int wk, int lane, uint8_t* smem) {
  float(*red)[kMultiStageRows][2][kGemvRows] = reinterpret_cast<float(*)[kMultiStageRows][2][kGemvRows]>(smem);
  const int I = a.intermediate, H = a.hidden;
  const int row0 = blockIdx.y * kGemvRows;
  const int steps = (H + kStepK - 1) / kStepK;
  GemvStream<2, NR> g;
  g.k = H;
  g.kblocks = H / kScaleBlock;
  g.row_stride = H;
  g.lane_off = (uint32_t)((lane >> 4) * H + (lane & 15) * 16);
  g.step_begin = min(wk * wave_steps, steps);
  g.step_end = min(g.step_begin + wave_steps, steps);
  const uint8_t* tables[2] = {a.gate_bits, a.up_bits};
  const float* scales[2] = {a.gate_scale, a.up_scale};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    g.w[t] = rows_buffer(tables[t] + ((int64_t)u.expert * I + row0) * H, (int64_t)kGemvRows * H);
    const float* srow = scales[t] + ((int64_t)u.expert * (I / kScaleBlock) + row0 / kScaleBlock) * g.kblocks;
    g.sreg[t] = lane_scale(srow, g.kblocks, g.step_begin, lane);
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) g.x[r] = a.hidden_in + (int64_t)(u.route[r] / a.top_k) * H;
  g.xs_stride = xs_elems(wave_steps);
  g.xs = reinterpret_cast<uint16_t*>(smem + sizeof(float) * WK * kMultiStageRows * 2 * kGemvRows) +
         wk * stage_rows * g.xs_stride;
  g.pad = wave_steps * kStepK;
  float acc[2][4][NR] = {};
  gemv_run<kGateUpDepth, true>(g, lane, acc);
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v = sum16(acc[t][q][r]);
        if ((lane & 15) == 0) red[wk][r][t][4 * q + (lane >> 4)] = v;
      }
  __syncthreads();
  // one thread per (route, row): wave-order split-K sum, then the bf16 SwiGLU
  const int tid = threadIdx.x;
  if (tid < kGemvRows * NR) {
    const int row = tid % kGemvRows, r = tid / kGemvRows;
    float gsum = 0.f, usum = 0.f;
    for (int w = 0; w < WK; ++w) {
      gsum += red[w][r][0][row];
      usum += red[w][r][1][row];
    }
    const float v = swiglu_bf16(round_to_bf16(gsum), round_to_bf16(usum));
    const int route = r == 0 ? u.route[0] : u.route[kUnitRoutes - 1];  // no runtime index into u (registers)
    a.act[(int64_t)route * I + row0 + row] = f32_to_bf16_bits(v);
  }
}

// Resident shared expert gate/up: 8 bf16 rows x NS tokens [t0, t0 + NS).
template <int WK, int NS>
__device__ __forceinline__ void gate_up_shared_group(const DecodeArgs& a, int t0, int srow0, int wave_steps,
                                                     int stage_rows, int wk, int lane, uint8_t* smem) {
  constexpr int QN = kSharedGateUpRows / 4;
  float(*red)[kMultiStageRows][2][kGemvRows] = reinterpret_cast<float(*)[kMultiStageRows][2][kGemvRows]>(smem);
  const int I = a.intermediate, H = a.hidden;
  const int ws = bf16_wave_steps(H, WK);
  Bf16Stream<2> g;
  g.k = H;
  g.row_bytes = 2 * H;
  g.lane_off = (uint32_t)((lane >> 4) * 2 * H + (lane & 15) * 16);
  g.step_begin = min(wk * ws, H / kBf16StepK);
  g.step_end = min(g.step_begin + ws, H / kBf16StepK);
  g.w[0] = rows_buffer(reinterpret_cast<const uint8_t*>(a.shared_gate + (int64_t)srow0 * H),
                       (int64_t)kSharedGateUpRows * 2 * H);
  g.w[1] = rows_buffer(reinterpret_cast<const uint8_t*>(a.shared_up + (int64_t)srow0 * H),
                       (int64_t)kSharedGateUpRows * 2 * H);
  const int stride = xs_elems(wave_steps);
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem + sizeof(float) * WK * kMultiStageRows * 2 * kGemvRows) +
                 wk * stage_rows * stride;
  const int tokens = a.routes / a.top_k;
  const __amdgpu_buffer_rsrc_t src =
      rows_buffer(reinterpret_cast<const uint8_t*>(a.hidden_in), (int64_t)tokens * H * 2);
  int row_elem[NS];
#pragma unroll
  for (int t = 0; t < NS; ++t) row_elem[t] = (t0 + t) * H;
  float acc[2][QN][NS] = {};
  bf16_group_run<kSharedGateUpDepth / 2>(g, src, row_elem, xs, stride, lane, acc);
#pragma unroll
  for (int t = 0; t < NS; ++t)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int q = 0; q < QN; ++q) {
        const float v = sum16(acc[tb][q][t]);
        if ((lane & 15) == 0) red[wk][t][tb][4 * q + (lane >> 4)] = v;
      }
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < kSharedGateUpRows * NS) {
    const int row = tid % kSharedGateUpRows, t = tid / kSharedGateUpRows;
    float gsum = 0.f, usum = 0.f;
    for (int w = 0; w < WK; ++w) {
      gsum += red[w][t][0][row];
      usum += red[w][t][1][row];
    }
    const float v = swiglu_bf16(round_to_bf16(gsum), round_to_bf16(usum));
    a.act_shared[(int64_t)(t0 + t) * I + srow0 + row] = f32_to_bf16_bits(v);
  }
}

// Grid: (units upper bound = routes, plus 2 columns per shared token group, I / 16).
// A wave stages stage_rows activation rows: kUnitRoutes, or the shared token
// group's size if larger.
template <int WK>
__global__ __launch_bounds__(64 * WK) __attribute__((amdgpu_waves_per_eu(4)))
void decode_gate_up_multi_kernel(const DecodeArgs a, int wave_steps, int group_tokens, int stage_rows) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wk = uniform(threadIdx.x >> 6);
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) a.valid[0] = 1;  // the down kernel only clears it
  if ((int)blockIdx.x >= a.routes) {
    const int c = blockIdx.x - a.routes;
    const int tokens = a.routes / a.top_k;
    const int t0 = (c >> 1) * group_tokens;
    const int srow0 = blockIdx.y * kGemvRows + kSharedGateUpRows * (c & 1);
    switch (min(group_tokens, tokens - t0)) {
      case 1: gate_up_shared_group<WK, 1>(a, t0, srow0, wave_steps, stage_rows, wk, lane, smem); return;
      case 2: gate_up_shared_group<WK, 2>(a, t0, srow0, wave_steps, stage_rows, wk, lane, smem); return;
      case 3: gate_up_shared_group<WK, 3>(a, t0, srow0, wave_steps, stage_rows, wk, lane, smem); return;
      default: gate_up_shared_group<WK, 4>(a, t0, srow0, wave_steps, stage_rows, wk, lane, smem); return;
    }
  }
  DecodeUnit u;
  if (!decode_unit<kGateUpUnitRoutes>(a.ids, a.routes, a.own, key_bits_of(a.own.experts), blockIdx.x, u)) return;
  if (u.count == 2)
    gate_up_unit<WK, 2>(a, u, wave_steps, stage_rows, wk, lane, smem);
  else
    gate_up_unit<WK, 1>(a, u, wave_steps, stage_rows, wk, lane, smem);
}

// down of one unit: NR routes of one expert, this workgroup's 8 hidden rows.
template <int NR>
__device__ __forceinline__ void down_unit(const DecodeArgs& a, const DecodeUnit& u, int steps, uint16_t* xs, int lane,
                                          float (*res)[kGemvRows]) {
  const int I = a.intermediate, H = a.hidden;
  const int row0 = blockIdx.x * kDownRows;
  GemvStream<1, NR> g;
  g.k = I;
  g.kblocks = I / kScaleBlock;
  g.row_stride = I;
  g.step_begin = 0;
  g.step_end = steps;
  g.w[0] = rows_buffer(a.down_bits + ((int64_t)u.expert * H + row0) * I, (int64_t)kDownRows * I);
  g.lane_off = (uint32_t)((lane >> 4) * I + (lane & 15) * 16);
  const float* srow = a.down_scale + ((int64_t)u.expert * (H / kScaleBlock) + row0 / kScaleBlock) * g.kblocks;
  g.sreg[0] = lane_scale(srow, g.kblocks, 0, lane);
  float wr[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    g.x[r] = a.act + (int64_t)u.route[r] * I;
    wr[r] = round_to_bf16(a.weights[u.route[r]]);  // loaded before the weight stream
  }
  g.xs = xs;
  g.xs_stride = xs_elems(steps);
  g.pad = steps * kStepK;
  float acc[1][kDownQuads][NR] = {};
  gemv_run<kDownMultiDepth, true>(g, lane, acc);
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int q = 0; q < kDownQuads; ++q) {
      const float v = sum16(acc[0][q][r]);
      // bf16 down output times the bf16 route weight, rounded (routed_experts.py:104-105)
      if ((lane & 15) == 0) res[u.route[r]][4 * q + (lane >> 4)] = round_to_bf16(round_to_bf16(v) * wr[r]);
    }
}

// Workgroup = 8 hidden rows x every unit (waves take units in turn) and, with
// the resident shared expert, the shared down rows of every token (K split
// over the waves, partials summed in wave order).
template <int WAVES, bool RESIDENT>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(4)))
void decode_down_multi_kernel(const DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float(*res)[kGemvRows] = reinterpret_cast<float(*)[kGemvRows]>(smem);  // [kMaxDecodeRoutes][16]
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int tid = threadIdx.x;
  const int I = a.intermediate, H = a.hidden;
  const int row0 = blockIdx.x * kDownRows;
  const int steps = (I + kStepK - 1) / kStepK;
  const int tokens = a.routes / a.top_k;
  for (int i = tid; i < a.routes * kGemvRows; i += 64 * WAVES) res[i / kGemvRows][i % kGemvRows] = 0.f;
  const int region = down_multi_region(I, WAVES, RESIDENT);
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem + sizeof(float) * kMaxDecodeRoutes * kGemvRows) + wave * region;
  // [WAVES][tokens][8] FP32 partial sums of the shared down rows, after the staging regions
  float(*red_sh)[kMultiSharedTokens][kDownRows] = reinterpret_cast<float(*)[kMultiSharedTokens][kDownRows]>(
      smem + sizeof(float) * kMaxDecodeRoutes * kGemvRows + sizeof(uint16_t) * WAVES * region);
  __syncthreads();
  if constexpr (RESIDENT) {
    // this wave's K slice of the shared down rows for every token (bf16, unweighted)
    const int ws = (I / kBf16StepK + WAVES - 1) / WAVES;
    Bf16Stream<1> g;
    g.k = I;
    g.row_bytes = 2 * I;
    g.lane_off = (uint32_t)((lane >> 4) * 2 * I + (lane & 15) * 16);
    g.step_begin = min(wave * ws, I / kBf16StepK);
    g.step_end = min(g.step_begin + ws, I / kBf16StepK);
    g.w[0] = rows_buffer(reinterpret_cast<const uint8_t*>(a.shared_down + (int64_t)row0 * I),
                         (int64_t)kDownRows * 2 * I);
    const __amdgpu_buffer_rsrc_t src =
        rows_buffer(reinterpret_cast<const uint8_t*>(a.act_shared), (int64_t)tokens * I * 2);
    int row_elem[kMultiSharedTokens];
#pragma unroll
    for (int t = 0; t < kMultiSharedTokens; ++t) row_elem[t] = min(t, tokens - 1) * I;  // rows past T: row T-1 again
    float acc[1][kDownQuads][kMultiSharedTokens] = {};
    bf16_group_run<2>(g, src, row_elem, xs, ws * kBf16StepK, lane, acc);
#pragma unroll
    for (int t = 0; t < kMultiSharedTokens; ++t)
#pragma unroll
      for (int q = 0; q < kDownQuads; ++q) {
        const float v = sum16(acc[0][q][t]);
        if ((lane & 15) == 0) red_sh[wave][t][4 * q + (lane >> 4)] = v;
      }
  }
  const int key_bits = key_bits_of(a.own.experts);
  const int units = decode_units<kUnitRoutes>(a.ids, a.routes, a.own, key_bits);
  for (int j = wave; j < units; j += WAVES) {
    DecodeUnit u;
    decode_unit<kUnitRoutes>(a.ids, a.routes, a.own, key_bits, j, u);
    if (u.count == 2)
      down_unit<2>(a, u, steps, xs, lane, res);
    else
      down_unit<1>(a, u, steps, xs, lane, res);
  }
  __syncthreads();
  // route combine: every token's slots in slot order, FP32 sum rounded once
  for (int i = tid; i < tokens * kDownRows; i += 64 * WAVES) {
    const int t = i / kDownRows, row = i % kDownRows;
    float sum = 0.f;
    for (int s = 0; s < a.top_k; ++s) sum += res[t * a.top_k + s][row];
    const int64_t o = (int64_t)t * H + row0 + row;
    if (a.out_f32 != nullptr) {
      a.out_f32[o] = a.round_partial ? round_to_bf16(sum) : sum;
      continue;
    }
    if constexpr (RESIDENT) {
      float sh = 0.f;
      for (int w = 0; w < WAVES; ++w) sh += red_sh[w][t][row];  // wave order: deterministic
      sum = round_to_bf16(round_to_bf16(round_to_bf16(sum) * a.routed_scale) + round_to_bf16(sh));
      if (!isfinite(sum)) a.valid[0] = 0;
    } else if (a.shared != nullptr) {
      sum = round_to_bf16(round_to_bf16(round_to_bf16(sum) * a.routed_scale) + bf16_bits_to_f32(a.shared[o]));
      if (!isfinite(sum)) a.valid[0] = 0;
    }
    a.out[o] = f32_to_bf16_bits(sum);
  }
  // health: ids in range, no duplicate id in a row, weights finite and >= 0 if asked
  if (blockIdx.x == 0 && wave == 0) {
    bool bad = false;
    if (lane < a.routes) {
      const int id = a.ids[lane];
      bad = id < 0 || id >= a.own.global_experts;
      const int t0 = (lane / a.top_k) * a.top_k;
      for (int s = t0; s < lane; ++s) bad |= a.ids[s] == id;
      if (a.check_weights) {
        const float w = a.weights[lane];
        bad |= !(w >= 0.0f) || isinf(w);
      }
    }
    const uint64_t any = __ballot(bad);
    if (lane == 0 && any) a.valid[0] = 0;
  }
}
}  // namespace

bool decode_path_fits(int64_t hidden, int64_t intermediate) {
  return hidden % kGemvRows == 0 && hidden <= (int64_t)kGateUpWaves * kMaxWaveSteps * kStepK &&
         intermediate <= (int64_t)kMaxWaveSteps * kStepK;
}

// The staged rows of a wave (NT x its K range, bf16) must fit in LDS next to
// the sums; weight rows come in workgroups of 8 and K in steps of 128.
bool shared_rows_fit(int64_t tokens, int64_t hidden, int64_t intermediate) {
  if (tokens < 1 || tokens > kSharedRowsMax || hidden <= 0 || intermediate <= 0) return false;
  if (hidden % kScaleBlock != 0 || intermediate % kScaleBlock != 0) return false;
  if (hidden > (1 << 20) || intermediate > (1 << 20)) return false;
  const int64_t kmax = hidden > intermediate ? hidden : intermediate;
  const int64_t lds = (int64_t)sizeof(float) * kSharedWaves * 2 * kSharedWgRows * tokens +
                      2 * kSharedWaves * tokens * (int64_t)shared_wave_steps((int)kmax) * kBf16StepK;
  return lds <= 160 * 1024;
}

hipError_t launch_shared_expert_rows(const uint16_t* x, int tokens, int hidden, int intermediate,
                                     const uint16_t* gate, const uint16_t* up, const uint16_t* down,
                                     uint16_t* act, uint16_t* out, hipStream_t stream) {
  if (!shared_rows_fit(tokens, hidden, intermediate)) return hipErrorInvalidValue;
  switch (tokens) {
    case 1: return launch_shared_expert_nt<1>(x, hidden, intermediate, gate, up, down, act, out, stream);
    case 2: return launch_shared_expert_nt<2>(x, hidden, intermediate, gate, up, down, act, out, stream);
    case 3: return launch_shared_expert_nt<3>(x, hidden, intermediate, gate, up, down, act, out, stream);
    case 4: return launch_shared_expert_nt<4>(x, hidden, intermediate, gate, up, down, act, out, stream);
    case 5: return launch_shared_expert_nt<5>(x, hidden, intermediate, gate, up, down, act, out, stream);
    case 6: return launch_shared_expert_nt<6>(x, hidden, intermediate, gate, up, down, act, out, stream);
    case 7: return launch_shared_expert_nt<7>(x, hidden, intermediate, gate, up, down, act, out, stream);
    default: return launch_shared_expert_nt<8>(x, hidden, intermediate, gate, up, down, act, out, stream);
  }
}

// Two or more tokens without routing inside the kernel: the multi kernels
// (routes grouped by expert; the resident shared expert's rows streamed once
// per token group).
hipError_t launch_decode_multi(const DecodeArgs& a, hipStream_t stream, const LaunchEvents* stage_events) {
  const int tokens = a.routes / a.top_k;
  const bool resident = a.shared_gate != nullptr;
  const int gu_steps = gate_up_wave_steps(a.hidden);
  const int group = min(tokens, kSharedGroupTokens);
  const int stage_rows = resident ? max(kUnitRoutes, group) : kUnitRoutes;
  const size_t gu_lds = sizeof(float) * kGateUpWaves * kMultiStageRows * 2 * kGemvRows +
                        sizeof(uint16_t) * kGateUpWaves * stage_rows * xs_elems(gu_steps);
  const int shared_cols = resident ? 2 * ((tokens + group - 1) / group) : 0;
  const dim3 g1(a.routes + shared_cols, a.intermediate / kGemvRows);
  if (stage_events) next_launch_events() = stage_events[0];
  label_next_launch("fp8_routed_projection_s%d_t2_k%d_n%d_tn%d_tk%d_units%s", a.routes, a.hidden, a.intermediate,
                    kGemvRows, kStepK, resident ? "_shared" : "");
  hipError_t err = launch_kernel(decode_gate_up_multi_kernel<kGateUpWaves>, g1, dim3(64 * kGateUpWaves), gu_lds,
                                 stream, a, gu_steps, group, stage_rows);
  if (err != hipSuccess) return err;
  const size_t d_lds = sizeof(float) * kMaxDecodeRoutes * kGemvRows +
                       sizeof(uint16_t) * kDownMultiWaves * down_multi_region(a.intermediate, kDownMultiWaves, resident) +
                       (resident ? sizeof(float) * kDownMultiWaves * kMultiSharedTokens * kDownRows : 0);
  if (stage_events) next_launch_events() = stage_events[1];
  label_next_launch("fp8_routed_projection_s%d_t1_k%d_n%d_tn%d_tk%d_units%s", a.routes, a.intermediate, a.hidden,
                    kDownRows, kStepK, resident ? "_shared" : "");
  if (resident)
    return launch_kernel(decode_down_multi_kernel<kDownMultiWaves, true>, dim3(a.hidden / kDownRows),
                         dim3(64 * kDownMultiWaves), d_lds, stream, a);
  return launch_kernel(decode_down_multi_kernel<kDownMultiWaves, false>, dim3(a.hidden / kDownRows),
                       dim3(64 * kDownMultiWaves), d_lds, stream, a);
}

hipError_t launch_decode_routed(const DecodeArgs& a, hipStream_t stream, const LaunchEvents* stage_events) {
  if (a.routes <= 0 || a.routes > kMaxDecodeRoutes || a.top_k <= 0 || a.routes % a.top_k != 0 ||
      !decode_path_fits(a.hidden, a.intermediate) || a.hidden % kScaleBlock != 0 ||
      a.intermediate % kScaleBlock != 0)
    return hipErrorInvalidValue;
  const int gu_steps = gate_up_wave_steps(a.hidden);
  const size_t gu_lds = sizeof(float) * kGateUpWaves * 2 * kGemvRows +
                        sizeof(uint16_t) * kGateUpWaves * xs_elems(gu_steps);
  if (a.router_logits != nullptr &&
      (a.own.experts > kDecodeRouterExperts || a.top_k > 64 || a.ids_out == nullptr || a.weights_out == nullptr ||
       a.ids != a.ids_out || a.weights != a.weights_out ||
       a.own.expert_offset != 0 || a.own.global_experts != a.own.experts))  // routes every expert: no share
    return hipErrorInvalidValue;
  if (a.out_f32 != nullptr && (a.shared != nullptr || a.shared_gate != nullptr)) return hipErrorInvalidValue;
  const bool resident = a.shared_gate != nullptr;
  if (resident && (a.shared_up == nullptr || a.shared_down == nullptr || a.act_shared == nullptr ||
                   bf16_wave_steps(a.hidden, kGateUpWaves) * kBf16StepK > xs_elems(gu_steps) ||
                   a.intermediate > xs_elems((a.intermediate + kStepK - 1) / kStepK)))
    return hipErrorInvalidValue;
  const int tokens = a.routes / a.top_k;
  if (tokens > 1 && a.router_logits == nullptr && (!resident || tokens <= kMultiSharedTokens))
    return launch_decode_multi(a, stream, stage_events);
  const dim3 g1(a.routes + (resident ? 2 * tokens : 0), a.intermediate / kGemvRows);
  if (stage_events) next_launch_events() = stage_events[0];
  // the reference's decode kernel name: routes (slots), tables, K, N, the
  // intermediate rows of a workgroup and the K of one load step
  label_next_launch("fp8_routed_projection_s%d_t2_k%d_n%d_tn%d_tk%d%s%s", a.routes, a.hidden, a.intermediate,
                    kGemvRows, kStepK, resident ? "_shared" : "", a.router_logits != nullptr ? "_router" : "");
  hipError_t err = launch_kernel(decode_gate_up_kernel<kGateUpWaves>, g1, dim3(64 * kGateUpWaves), gu_lds, stream,
                                 a, gu_steps);
  if (err != hipSuccess) return err;
  const int d_steps = (a.intermediate + kStepK - 1) / kStepK;
  // Eight-wave workgroups (one route per wave) for many routes or the resident
  // shared expert; for a single token's routes four-wave workgroups of two
  // routes a wave, which all fit on the GPU at once (768 x 4 waves).
  const bool few = !resident && a.routes <= 2 * kDownWavesFew;
  const int d_waves = few ? kDownWavesFew : kDownWaves;
  const size_t d_lds = sizeof(float) * kMaxDecodeRoutes * kGemvRows +
                       sizeof(uint16_t) * d_waves * xs_elems(d_steps) +
                       (resident ? sizeof(float) * kMaxDecodeRoutes * kGemvRows : 0);
  if (stage_events) next_launch_events() = stage_events[1];
  label_next_launch("fp8_routed_projection_s%d_t1_k%d_n%d_tn%d_tk%d%s", a.routes, a.intermediate, a.hidden, kDownRows,
                    kStepK, resident ? "_shared" : "");
  if (resident)
    return launch_kernel(decode_down_kernel<kDownWaves, true>, dim3(a.hidden / kDownRows), dim3(64 * kDownWaves),
                         d_lds, stream, a);
  if (few)
    return launch_kernel(decode_down_kernel<kDownWavesFew, false>, dim3(a.hidden / kDownRows),
                         dim3(64 * kDownWavesFew), d_lds, stream, a);
  return launch_kernel(decode_down_kernel<kDownWaves, false>, dim3(a.hidden / kDownRows), dim3(64 * kDownWaves),
                       d_lds, stream, a);
}

}  // namespace glm_moe
