// Internal launch interface between the C-ABI layer (capi.hip) and the kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <rocprofiler-sdk-roctx/roctx.h>
#include <stdint.h>

#include <atomic>
#include <utility>

namespace glm_moe {

// Lets `kernel` use the whole 160 KB of LDS of a CU on the current device.
// `done` is the caller's per-kernel mask of devices already set (the attribute
// is per device; setting it twice is harmless, so racing threads are fine).
inline hipError_t allow_full_lds(const void* kernel, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (err == hipSuccess) done.fetch_or(bit, std::memory_order_release);
  return err;
}

// ------------------------------------------------------------------ launches
// Stage timing: a caller may arm a (start, stop) pair of HIP events for the
// next kernel launched on this thread; the launch then records them at the
// kernel's own start and end (hipExtLaunchKernelGGL), so the elapsed time is
// the kernel's duration without event packets between kernels.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
LaunchEvents& next_launch_events();  // thread-local; defined in capi.hip

// Profiler name of the next launch on this thread: the reference's kernel
// names with their shape suffix (glm_tpu/kernels/names.py:1-31, e.g.
// fp8_routed_projection_s{slots}_t{tables}_k{K}_n{N}_tn{tn}_tk{tk},
// fp8_grouped_matmul/kernel.py:283).  launch_kernel wraps the launch in a
// roctx range of that name, which `rocprofv3 --kernel-trace --kernel-rename`
// reports as the kernel's name, so one profile splits by configuration.
// The next launch consumes it; an empty label opens no range.  A refused C-ABI
// call clears it (capi.hip), so no stale name reaches a later launch.
constexpr int kLabelBytes = 128;
char* next_launch_label();  // thread-local, kLabelBytes; defined in capi.hip
void label_next_launch(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

template <typename... KArgs, typename... Args>
hipError_t launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                         Args&&... args) {
  char* label = next_launch_label();
  const bool labelled = label[0] != '\0';
  if (labelled) roctxRangePushA(label);
  LaunchEvents& ev = next_launch_events();
  if (ev.start != nullptr || ev.stop != nullptr) {
    const LaunchEvents armed = ev;
    ev = LaunchEvents{};
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, armed.start, armed.stop, 0u,
                          std::forward<Args>(args)...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, std::forward<Args>(args)...);
  }
  const hipError_t err = hipGetLastError();
  if (labelled) {
    roctxRangePop();
    label[0] = '\0';
  }
  return err;
}

// ------------------------------------------------------------------ route plan
constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kMaxExperts = 1024;

// Which routes a call owns.  A call holds the tables of `experts` consecutive
// experts starting at global id `expert_offset` (an expert-parallel share; the
// whole layer when expert_offset = 0 and global_experts = experts).  Ids in
// [0, global_experts) are valid.  An invalid id is unowned when drop_invalid is
// set (the decode body's ownership mask, routed_experts.py:250-253), else it
// stands for the safe id 0 (group_prefill_routes, routed_experts.py:159-161).
struct RouteOwnership {
  int32_t experts;
  int32_t global_experts;
  int32_t expert_offset;
  int32_t drop_invalid;
};

// The local expert (0 .. experts - 1) of a raw route id, or -1 when unowned.
__host__ __device__ inline int owned_expert(int raw, const RouteOwnership& o) {
  const int g = (raw >= 0 && raw < o.global_experts) ? raw : (o.drop_invalid ? -1 : 0);
  const int l = g - o.expert_offset;
  return (g >= 0 && l >= 0 && l < o.experts) ? l : -1;
}

// Whether some route can be unowned (a share, or invalid ids dropped).
__host__ __device__ inline bool may_leave_routes_unowned(const RouteOwnership& o) {
  return o.drop_invalid || o.expert_offset != 0 || o.global_experts != o.experts;
}

inline RouteOwnership whole_layer(int32_t experts) { return RouteOwnership{experts, experts, 0, 0}; }

struct RoutePlanArgs {
  const int32_t* ids;        // [tokens * top_k] route expert ids (flat t * k + slot)
  int32_t n;                 // tokens * top_k
  int32_t top_k;
  int32_t experts;           // owned (local) experts: the groups counted, offset and tiled
  RouteOwnership own;        // which ids are valid and owned (own.experts == experts)
  int32_t keys;              // sort keys: the owned experts, plus one key past them for the
                             // unowned routes (sorted last, never tiled) when there can be any
  int32_t key_bits;          // bits needed to hold keys - 1 (wave match keys)
  const float* route_w;      // nullable: also require finite, non-negative weights
  int32_t* sorted;           // [n] sorted_flat_ids (unowned routes last)
  int32_t* inverse;          // [n] inverse permutation (nullable)
  int32_t* counts;           // [experts] group sizes
  int32_t* offsets;          // [experts + 1] exclusive prefix of counts; [experts] = owned routes (nullable)
  uint8_t* valid;            // [1]
  // optional GEMM work list: one tile per tile_rows sorted routes of an expert
  int32_t tile_rows;         // 0: no tiles
  int32_t wide_twice;        // nonzero: a tile of more than tile_rows / 2 routes is listed twice,
                             // the second time with kTileSecondHalf set in its tile_live
  int32_t max_tiles;
  int32_t* tile_expert;
  int32_t* tile_row;
  int32_t* tile_live;
  int32_t* tile_count;       // [1]
  int32_t* tile_desc;          // nullable [max_tiles][4], 16-byte aligned: per listing, its expert's
                               // id, first listing, first sorted position and route count
  // optional scratch for the multi-workgroup plan (route_plan_chunks() chunks):
  int32_t* chunk_hist;         // [chunks, keys] key counts of each chunk
  int32_t* chunk_bad;          // [chunks] health of each chunk
  int32_t chunk;               // routes per chunk (set by launch_route_plan)
};
// Flag of a tile_live entry: the second listing of a wide tile (wide_twice),
// whose work items take the second half of each tall weight stripe; the
// route count is tile_live & kTileLiveMask.
constexpr int32_t kTileSecondHalf = 1 << 16;
constexpr int32_t kTileLiveMask = kTileSecondHalf - 1;
// Listings of an expert of c routes: ceil(c / rows) tiles, plus (wide_twice)
// a second listing of every tile of more than rows / 2 routes -- then listing
// i of the expert is tile i / 2, the second listing when i is odd.
__host__ __device__ inline int tiles_of_count(int c, int rows, int wide_twice) {
  const int full = c / rows, rem = c - full * rows;
  const int nt = full + (rem > 0 ? 1 : 0);
  return wide_twice ? nt + full + (rem > rows / 2 ? 1 : 0) : nt;
}
// Route chunks of the multi-workgroup plan (whole token rows, about 2048 routes each).
constexpr int kPlanChunkRoutes = 2048;
int route_plan_chunks(int32_t n, int32_t top_k);
hipError_t launch_route_plan(const RoutePlanArgs& a, hipStream_t stream);

// The same plan for routes the noaux_tc router computes from logits on the way:
// the router writes ids and weights (a.ids must be r.ids) and, on the
// multi-workgroup path, the histogram rows of its workgroups (kRouterHistTokens
// tokens each) in its own launch, so the plan is two launches: router with
// counting, then the scatter.  chunk_hist / chunk_bad then need
// route_plan_hist_rows() rows.
constexpr int kRouterHistTokens = 16;
struct RouterPass {
  const float* logits;   // [tokens, experts] FP32
  const float* bias;     // nullable [experts] correction bias (selects, does not weight)
  int32_t experts;       // global experts routed over (<= 1024)
  int64_t tokens;
  int32_t* ids;          // [tokens, top_k] out
  float* weights;        // [tokens, top_k] out
};
int64_t route_plan_hist_rows(int64_t tokens, int32_t top_k);
hipError_t launch_route_plan_from_logits(const RoutePlanArgs& a, const RouterPass& r, hipStream_t stream);

struct PanelPlanArgs {
  const int32_t* group_sizes;  // [groups]
  int32_t groups;
  const int32_t* group_offset; // device scalar
  int32_t rows;
  int32_t local_groups;
  int32_t panel_rows;
  int32_t capacity;
  int32_t* expert_ids;       // [capacity]
  int32_t* row_starts;       // [capacity]
  int32_t* live_counts;      // [capacity]
  int32_t* active_panels;    // [1]
  int32_t* restore_indices;  // [rows]
  uint8_t* owned_rows;       // [rows]
  uint8_t* valid;            // [1]
};
hipError_t launch_panel_plan(const PanelPlanArgs& a, hipStream_t stream);

// Owned decode slots as one-row tiles (kernel.py:185-191 slot compaction).
hipError_t launch_slot_tiles(const int32_t* local_ids, const uint8_t* owned, int32_t slots,
                             int32_t experts, int32_t* tile_expert, int32_t* tile_row,
                             int32_t* tile_live, int32_t* tile_count, hipStream_t stream);

// ------------------------------------------------------------------ grouped FP8 GEMM
enum Epilogue : int {
  kEpiStoreF32 = 0,   // out[row][t*table_stride + n] = acc (f32)
  kEpiStoreBf16 = 1,  // same, rounded to bf16
  kEpiSwiglu = 2,     // out[row][n] = bf16 SwiGLU(bf16(gate), bf16(up))
  kEpiWeighted = 3,   // out[row][n] = bf16(bf16(acc) * bf16(route_w[row]))
};

struct GroupedGemmArgs {
  int32_t experts;             // tiles naming another expert are skipped
  int32_t rows;                // sorted positions; tiles must lie in [0, rows)
  int64_t x_rows;              // activation rows (gathered row ids are clamped to it)
  int64_t out_rows;            // output rows (larger output row ids are skipped)
  const uint16_t* x;           // bf16 activation rows of length k
  const int32_t* x_row_ids;    // nullable: activation row of sorted position r = x_row_ids[r] / x_row_div
  int32_t x_row_div;
  const uint8_t* w0;           // [experts, n, k] e4m3fn bits
  const float* s0;             // [experts, n/128, k/128]
  const uint8_t* w1;           // second table (fused gate/up) or null
  const float* s1;
  int32_t n;
  int32_t k;
  const int32_t* tile_expert;  // work list
  const int32_t* tile_row;
  const int32_t* tile_live;
  const int32_t* tile_count;
  int32_t max_tiles;
  const int32_t* tile_desc;    // prefill kernels: the plan's per-listing expert descriptors
                               // (RoutePlanArgs::tile_desc), with tile_rows and wide_twice
  const uint8_t* xq;           // nullable: e4m3 activations [x_rows, k] for the native FP8 mode
  const float* xscale;         // their FP32 block scales by sorted position [k / 128, rows]
  const uint8_t* valid;        // nullable: no work at all when *valid == 0
  void* out;
  int64_t ldo;                 // elements between output rows
  int64_t table_stride;        // elements between the tables of one output row
  const int32_t* out_row_ids;  // nullable: output row of sorted position r
  const float* route_w;        // kEpiWeighted: weight of output row
  int32_t stripe_run;          // FP8 prefill kernel: weight stripes of one work item (0 or 1: one)
  int32_t tile_rows;           // routes per tile of the work list (0: unknown, up to 256)
  int32_t wide_twice;          // the work list names tiles of more than 128 routes twice (RoutePlanArgs)
  int32_t tall;                // prefill kernels: tall stripes (512 weight rows) where N allows them
  const char* name;            // profiler base name (null: fp8_expert_panel_matmul)
  // FP8 prefill kernel, SwiGLU epilogue on tall stripes (prefill_quantizes_output): nullable; the
  // output rows quantised for the next projection instead of stored bf16 -- e4m3 codes
  // [out_rows, ldo] and FP32 scales block-major by output row [n / 128][out_rows], the values of
  // launch_quantize_rows_fp8 over the bf16 output
  uint8_t* outq;
  float* outq_scale;
};

// Profiler name of a grouped-GEMM launch: fp8_routed_projection_s{slots}_t{tables}
// _k{K}_n{N}_tn{weight rows a workgroup}_tk128 for the routed-projection entry
// point (the reference's suffix), fp8_expert_panel_matmul{variant}_m{routes}
// _t{tables}_k{K}_n{N}_tm{routes a tile}_tn{weight rows a work item} otherwise.
inline void label_grouped_gemm(const GroupedGemmArgs& a, int tables, int tile_rows, int bn, const char* variant) {
  if (a.name != nullptr)
    label_next_launch("%s_s%d_t%d_k%d_n%d_tn%d_tk128", a.name, a.rows, tables, a.k, a.n, bn);
  else
    label_next_launch("fp8_expert_panel_matmul%s_m%d_t%d_k%d_n%d_tm%d_tn%d", variant, a.rows, tables, a.k, a.n,
                      tile_rows, bn);
}

// Kernel shape families chosen by the host from the number of routes per tile.
enum GemmShape : int {
  kShapeSkinny = 0,  // <= 16 routes per tile, split-K waves
  kShapePanel32 = 1, // <= 32 routes per tile (reference M32 panels)
  kShapeWide = 2,    // <= 128 routes per tile (256 on the bf16 prefill kernel), LDS-staged activations
  kShapeDecode = 3,  // <= 4 routes per tile, split-K waves (decode)
};
int gemm_shape_rows(int shape);
int gemm_shape_bn(int shape, int tables);
hipError_t launch_grouped_gemm_wide(const GroupedGemmArgs& a, int tables, int epilogue, hipStream_t stream);
// The pipelined prefill kernel (expert-major XCD-aware work order); needs the
// plan's tile_desc.  Its bf16 kernel takes tiles of up
// to prefill_wide_tile_rows() routes, the FP8 kernel up to 128.  N must be a
// multiple of prefill_bn(tables); both kernels run tall stripes of
// prefill_tall_bn(tables) rows where GroupedGemmArgs::tall asks for them and
// N is a multiple of that.
int prefill_bn(int tables);
int prefill_tall_bn(int tables);
int prefill_wide_tile_rows();
// Weight stripes one FP8 prefill work item runs for a projection of `tables` tables.
int prefill_stripe_run(int tables);
// Whether launch_grouped_gemm_prefill on these args runs the FP8 kernel's tall
// stripes with the SwiGLU epilogue, the launches that take GroupedGemmArgs::outq.
bool prefill_quantizes_output(const GroupedGemmArgs& a, int tables, int epilogue);
bool prefill_fits(int64_t n, int64_t k, int tables);
// The prefill kernels' 32-bit activation offsets: x_rows x k x 2 bytes below 2 GiB.
bool prefill_rows_fit(int64_t x_rows, int64_t k);
hipError_t launch_grouped_gemm_prefill(const GroupedGemmArgs& a, int tables, int epilogue, hipStream_t stream);
hipError_t launch_grouped_gemm(const GroupedGemmArgs& a, int shape, int tables, int epilogue,
                               hipStream_t stream);

// ------------------------------------------------------------------ decode path (<= 64 routes)
constexpr int kMaxDecodeRoutes = 64;

struct DecodeArgs {
  const int32_t* ids;          // [routes] flat route expert ids
  const float* weights;        // [routes] route weights
  int32_t routes;              // tokens * top_k, <= kMaxDecodeRoutes
  int32_t top_k;
  RouteOwnership own;          // the owned experts (the tables) and the valid ids
  int32_t check_weights;       // health also requires finite, non-negative weights
  const uint16_t* hidden_in;   // [tokens, hidden] bf16
  int32_t hidden;
  int32_t intermediate;
  const uint8_t* gate_bits;
  const float* gate_scale;
  const uint8_t* up_bits;
  const float* up_scale;
  const uint8_t* down_bits;
  const float* down_scale;
  uint16_t* act;               // workspace [routes, intermediate] bf16, flat route order
  uint16_t* out;               // [tokens, hidden] bf16 (or out_f32)
  float* out_f32;              // nullable: the FP32 route sum [tokens, hidden] instead of out (a share's
                               // partial for the caller's sum over the expert axis)
  int32_t round_partial;       // out_f32 holds the route sum rounded to bf16 (the decode body's per-owner sum)
  uint8_t* valid;
  // layer epilogue (null shared: out is the routed sum): out = bf16(bf16(routed
  // * routed_scale) + shared), and health also requires a finite output
  const uint16_t* shared;      // [tokens, hidden] bf16 shared-expert output
  float routed_scale;          // already a bf16 value
  // the resident bf16 shared expert computed in the same two kernels (null:
  // none); its intermediate size equals `intermediate`
  const uint16_t* shared_gate; // [intermediate, hidden] bf16
  const uint16_t* shared_up;   // [intermediate, hidden] bf16
  const uint16_t* shared_down; // [hidden, intermediate] bf16
  uint16_t* act_shared;        // workspace [tokens, intermediate] bf16
  // routing inside the gate/up kernel (null: ids / weights are inputs): each
  // workgroup routes its token from the router logits [tokens, experts] f32
  // (+ correction bias [experts], nullable); the first slot's workgroups write
  // the token's ids and weights to ids_out / weights_out, which ids / weights
  // then point to for the down kernel.  experts <= kDecodeRouterExperts.
  const float* router_logits;
  const float* router_bias;
  int32_t* ids_out;
  float* weights_out;
};
constexpr int kDecodeRouterExperts = 256;
// The decode kernels stage one wave's K range (<= 2048) in LDS: hidden <= 8192
// (four waves split it), intermediate <= 2048.
bool decode_path_fits(int64_t hidden, int64_t intermediate);
// stage_events: null, or the armed events of the gate/up [0] and down [1] kernels.
hipError_t launch_decode_routed(const DecodeArgs& a, hipStream_t stream, const LaunchEvents* stage_events);

// The bf16 shared expert over a few rows (tokens <= kSharedRowsMax): gate/up
// [I, H], SwiGLU and down [H, I] with the resident path's rounding points,
// every weight byte read once for all rows.  act: workspace [tokens, I] bf16.
constexpr int kSharedRowsMax = 8;
bool shared_rows_fit(int64_t tokens, int64_t hidden, int64_t intermediate);
hipError_t launch_shared_expert_rows(const uint16_t* x, int tokens, int hidden, int intermediate,
                                     const uint16_t* gate, const uint16_t* up, const uint16_t* down,
                                     uint16_t* act, uint16_t* out, hipStream_t stream);

// ------------------------------------------------------------------ auxiliary
hipError_t launch_decode_fp8_table(const uint8_t* bits, const float* scale, int64_t n, int64_t k,
                                   int32_t block_n, int32_t block_k, uint16_t* out,
                                   hipStream_t stream);
hipError_t launch_swiglu_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* out, hipStream_t stream);
hipError_t launch_gather_rows(const void* src, int64_t src_rows, int64_t row_bytes,
                              const int32_t* index, int32_t div, const uint8_t* mask, int64_t n,
                              void* dst, hipStream_t stream);
hipError_t launch_pack_panel_rows(const void* src, int64_t src_rows, int64_t row_bytes,
                                  const int32_t* row_starts, const int32_t* live_counts,
                                  int32_t capacity, int32_t panel_rows, void* dst,
                                  hipStream_t stream);
hipError_t launch_zero_rows(void* out, int64_t rows, int64_t row_bytes, const uint8_t* keep,
                            const uint8_t* valid, hipStream_t stream);
// out[t] = bf16(sum over slots of y[t * top_k + s]); with ids != nullptr a slot
// whose raw id the call does not own (owned_expert < 0) contributes nothing;
// with route_w != nullptr slot s contributes bf16(y * bf16(route_w[t * top_k + s])).
// shared: null, or the layer epilogue's bf16 shared-expert rows (out =
// bf16(bf16(routed * routed_scale) + shared), and a non-finite output clears valid).
// out_f32: null, or the FP32 sum [tokens, h] instead of out (rounded to bf16
// values when round_partial), for a share's partial; shared must then be null.
hipError_t launch_combine_routes(const uint16_t* y, int64_t tokens, int32_t top_k, int64_t h,
                                 const int32_t* ids, const RouteOwnership& own, const float* route_w,
                                 const uint16_t* shared, float routed_scale, uint8_t* valid, uint16_t* out,
                                 float* out_f32, int32_t round_partial, hipStream_t stream);
// The layer epilogue on an FP32 routed sum (after the sum over the expert
// axis): out = bf16(bf16(bf16(routed) * routed_scale) + shared); a non-finite
// output clears valid.
hipError_t launch_layer_epilogue(const float* routed, int64_t tokens, int64_t h, const uint16_t* shared,
                                 float routed_scale, uint16_t* out, uint8_t* valid, hipStream_t stream);
// GLM noaux_tc routing of [tokens, experts] FP32 logits (experts <= 1024, top_k <= 64).
// Adds the count of e4m3fn NaN bytes (0x7F / 0xFF) among n bytes to *count.
hipError_t launch_count_nonfinite_fp8(const uint8_t* bits, int64_t n, unsigned long long* count,
                                      hipStream_t stream);
hipError_t launch_route_noaux_tc(const float* logits, int64_t tokens, int32_t experts, const float* bias,
                                 int32_t top_k, int32_t* ids, float* weights, hipStream_t stream);
// Per (row, 128-wide block): scale = amax / 448 (1 for an all-zero block),
// q = e4m3fn(clamp(x / scale, +-448)) rounded to nearest even.  The scales go
// to scales[kb * n_pos + pos] for each pos = positions[row * per_row + j]
// (j < per_row; pos = row when positions is null and per_row is 1).
hipError_t launch_quantize_rows_fp8(const uint16_t* x, int64_t rows, int64_t k, uint8_t* q, float* scales,
                                    const int32_t* positions, int32_t per_row, int64_t n_pos, hipStream_t stream);
hipError_t launch_fill_u32(void* dst, int64_t words, uint32_t value, hipStream_t stream);
hipError_t launch_synth_fp8(uint64_t seed, int32_t experts, int64_t n, int64_t k, float sigma,
                            uint8_t* bits, float* scales, hipStream_t stream);

}  // namespace glm_moe
