// extern "C" entry points of libglm_moe.so (declared in include/glm_moe.h).
//
// Static geometry checks mirror the reference's trace-time ValueErrors; the
// kernels never see a shape they were not built for.  Nothing here allocates.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/glm_moe.h"
#include "moe_common.h"
#include "moe_kernels.h"

using namespace glm_moe;

namespace glm_moe {

LaunchEvents& next_launch_events() {
  thread_local LaunchEvents armed;
  return armed;
}

char* next_launch_label() {
  thread_local char label[kLabelBytes] = {};
  return label;
}

void label_next_launch(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(next_launch_label(), kLabelBytes, fmt, ap);
  va_end(ap);
}

}  // namespace glm_moe

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  next_launch_label()[0] = '\0';  // a refused call's label must not name a later launch
  return status;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return GLM_MOE_OK;
  return fail(GLM_MOE_ERR_DEVICE, "%s: %s", what, hipGetErrorString(err));
}

#define GLM_REQUIRE(cond, ...) \
  do {                         \
    if (!(cond)) return fail(GLM_MOE_ERR_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define GLM_HIP(call, what)                        \
  do {                                             \
    const int _st = check_hip((call), (what));     \
    if (_st != GLM_MOE_OK) return _st;             \
  } while (0)

constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

int key_bits_for(int experts) {
  int bits = 0;
  while ((1 << bits) < experts) ++bits;
  return bits;
}

// Shape family of the grouped GEMM for a route set: the pipelined prefill
// kernel wherever its geometry fits -- measured faster than the split-K
// shapes at every route count above the decode kernels' 64 (GLM-5 shape,
// T = 9 / 16 / 32 / 64 / 128 / 256: -5 / -9 / -11 / -18 / -20 / -26 %);
// otherwise split-K kernels while experts see few routes each (<= 4 routes
// per tile up to one route per expert on average, <= 16 up to eight) and the
// 64-bit-offset LDS-tiled kernel beyond.
int routed_shape(int64_t tokens, int64_t routes, int32_t experts, int64_t hidden, int64_t intermediate) {
  if (prefill_fits(intermediate, hidden, 2) && prefill_fits(hidden, intermediate, 1) &&
      prefill_rows_fit(tokens, hidden) && prefill_rows_fit(routes, intermediate))
    return kShapeWide;
  if (routes <= (int64_t)experts) return kShapeDecode;
  return routes <= 8 * (int64_t)experts ? kShapeSkinny : kShapeWide;
}

int64_t max_tiles_for(int64_t routes, int32_t experts, int rows) {
  return (routes + rows - 1) / rows + (routes < experts ? routes : experts);
}

// Routed-expert calls of at most 64 routes take the two-kernel decode path.
bool uses_decode_path(int64_t routes, int64_t hidden, int64_t intermediate) {
  return routes <= kMaxDecodeRoutes && decode_path_fits(hidden, intermediate);
}

// Whether the bf16 down projection keeps tall stripes (512 weight rows a work
// item) for about `listings` route tiles: unless its work items would leave
// most CUs of the last round idle where 256-row stripes (twice the items)
// fill the rounds -- an expert-parallel share's few experts (32 tiles x 12
// tall stripes = 384 items on 256 CUs: 1.5 rounds).
bool down_tall_fills(int64_t listings, int64_t hidden) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess || cus <= 0)
    return true;
  auto fill = [&](int64_t items) { return (double)items / (double)(((items + cus - 1) / cus) * cus); };
  const int64_t tall_items = listings * (hidden / prefill_tall_bn(1));
  const int64_t short_items = listings * (hidden / prefill_bn(1));
  return !(fill(tall_items) < 0.85 && fill(short_items) > fill(tall_items) + 0.1);
}

// Byte layout of the glm_moe_routed_experts workspace.
struct RoutedLayout {
  size_t sorted, inverse, counts, offsets, tiles, tile_desc, chunk_hist, chunk_bad, act, y, xq, xscale, actq,
      actscale, act_shared, total;
  int64_t max_tiles;
};

RoutedLayout routed_layout(int64_t tokens, int32_t top_k, int32_t experts, int64_t hidden,
                           int64_t intermediate) {
  RoutedLayout L{};
  const int64_t n = tokens * top_k;
  const int shape = routed_shape(tokens, n, experts, hidden, intermediate);
  L.max_tiles = max_tiles_for(n, experts, gemm_shape_rows(shape));
  size_t off = 0;
  L.sorted = off;  off = align_up(off + sizeof(int32_t) * n);
  L.inverse = off; off = align_up(off + sizeof(int32_t) * n);
  L.counts = off;  off = align_up(off + sizeof(int32_t) * experts);
  L.offsets = off; off = align_up(off + sizeof(int32_t) * (experts + 1));
  L.tiles = off;   off = align_up(off + sizeof(int32_t) * (3 * L.max_tiles + 1));
  L.tile_desc = off; off = align_up(off + sizeof(int32_t) * 4 * L.max_tiles);
  // histogram rows of the plan (per chunk, or per router workgroup when the
  // router counts on the way): one sort key per expert, plus the key of unowned routes
  const int64_t hist_rows = route_plan_hist_rows(tokens, top_k);
  L.chunk_hist = off; off = align_up(off + sizeof(int32_t) * (size_t)hist_rows * (experts + 1));
  L.chunk_bad = off;  off = align_up(off + sizeof(int32_t) * (size_t)hist_rows);
  L.act = off;     off = align_up(off + sizeof(uint16_t) * n * intermediate);
  L.y = off;       off = align_up(off + sizeof(uint16_t) * n * hidden);
  // native FP8 mode: quantised activations and their block scales
  L.xq = off;       off = align_up(off + (size_t)tokens * hidden);
  L.xscale = off;   off = align_up(off + sizeof(float) * n * (hidden / 128));  // by sorted position
  L.actq = off;     off = align_up(off + (size_t)n * intermediate);
  L.actscale = off; off = align_up(off + sizeof(float) * n * (intermediate / 128));
  // resident shared expert (decode shapes): its bf16 SwiGLU activations
  L.act_shared = off; off = align_up(off + sizeof(uint16_t) * tokens * intermediate);
  L.total = off;
  return L;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Scratch of the decode path alone (the compact layout of the allocation-free
// entry point): the routes' bf16 SwiGLU rows [routes, I], then the resident
// shared expert's [tokens, I].
size_t decode_act_bytes(int64_t tokens, int32_t top_k, int64_t intermediate) {
  return align_up(sizeof(uint16_t) * (size_t)(tokens * top_k) * (size_t)intermediate);
}
size_t decode_scratch_bytes(int64_t tokens, int32_t top_k, int64_t intermediate) {
  return decode_act_bytes(tokens, top_k, intermediate) +
         align_up(sizeof(uint16_t) * (size_t)tokens * (size_t)intermediate);
}

// Stage timing of glm_moe_routed_experts_timed: stage i's kernel records
// events[2i] at its start and events[2i + 1] at its end.
enum Stage { kStagePlan = 0, kStageGateUp = 1, kStageDown = 2, kStageCombine = 3, kStages = 4 };

struct StageTimer {
  void* const* events;  // null: untimed call
  uint32_t* timed;      // bit i set when stage i ran a kernel

  LaunchEvents at(int stage) const {
    LaunchEvents e;
    if (events != nullptr) {
      e.start = static_cast<hipEvent_t>(events[2 * stage]);
      e.stop = static_cast<hipEvent_t>(events[2 * stage + 1]);
    }
    return e;
  }
  // arm the next launch with stage i's events
  void arm(int stage) const {
    if (events == nullptr) return;
    next_launch_events() = at(stage);
    *timed |= 1u << stage;
  }
  // after stage i: if no kernel took its events (nothing to launch), disarm
  void done(int stage) const {
    if (events == nullptr) return;
    LaunchEvents& armed = next_launch_events();
    if (armed.start != nullptr || armed.stop != nullptr) {
      armed = LaunchEvents{};
      *timed &= ~(1u << stage);
    }
  }
};

// RNE float -> bf16 value (finite input): the reference casts the routed scale
// to bf16 before the epilogue multiply (routed_experts.py:125, :303).
float bf16_round_host(float f) {
  uint32_t u;
  std::memcpy(&u, &f, sizeof(u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  u &= 0xFFFF0000u;
  std::memcpy(&f, &u, sizeof(f));
  return f;
}

// Routing computed inside the decode gate/up kernel: the router logits
// [tokens, experts] f32 and the correction bias [experts] (nullable); the
// route_indices / route_weights of routed_experts_impl are then its outputs.
struct RouterIn {
  const float* logits;
  const float* bias;
};

int routed_experts_impl(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                        const int32_t* route_indices, const float* route_weights, int32_t top_k,
                        int32_t num_experts, int64_t intermediate, const uint8_t* gate_bits,
                        const float* gate_scale, const uint8_t* up_bits, const float* up_scale,
                        const uint8_t* down_bits, const float* down_scale, uint32_t flags,
                        const uint16_t* shared, const uint16_t* const* resident, float routed_scale,
                        uint16_t* out, uint8_t* valid, void* workspace, size_t workspace_bytes,
                        const StageTimer& timer, void* stream_ptr, const RouterIn* router = nullptr,
                        bool compact_decode_scratch = false, int32_t global_experts = 0,
                        int32_t expert_offset = 0, float* out_f32 = nullptr) {
  // a whole layer unless the caller names a share: tables of num_experts experts
  // from global id expert_offset on, of global_experts in all
  if (global_experts == 0) global_experts = num_experts;
  GLM_REQUIRE(tokens > 0 && top_k > 0 && num_experts > 0, "routed experts need tokens, top_k, experts > 0");
  GLM_REQUIRE(top_k <= global_experts, "top_k exceeds expert count");
  GLM_REQUIRE(global_experts <= kMaxExperts, "at most %d experts", kMaxExperts);
  GLM_REQUIRE(num_experts <= global_experts && expert_offset >= 0 && expert_offset <= global_experts - num_experts,
              "a share's experts [%d, %d) must lie in [0, %d)", (int)expert_offset,
              (int)(expert_offset + num_experts), (int)global_experts);
  const RouteOwnership own{num_experts, global_experts, expert_offset,
                           (flags & GLM_MOE_DROP_UNOWNED) ? 1 : 0};
  const bool unowned = may_leave_routes_unowned(own);
  GLM_REQUIRE(!unowned || num_experts < kMaxExperts, "a share or dropped routes: at most %d local experts",
              kMaxExperts - 1);
  GLM_REQUIRE(tokens * top_k <= INT32_MAX / 2, "too many routes");
  GLM_REQUIRE(hidden_size > 0 && hidden_size % 128 == 0, "hidden size must be a positive multiple of 128");
  GLM_REQUIRE(intermediate > 0 && intermediate % 128 == 0, "intermediate size must be a positive multiple of 128");
  GLM_REQUIRE(hidden_size <= INT32_MAX / 2 && intermediate <= INT32_MAX / 2, "dimension too large");
  GLM_REQUIRE(hidden && route_indices && route_weights && gate_bits && gate_scale && up_bits &&
                  up_scale && down_bits && down_scale && (out || out_f32) && valid,
              "null tensor pointer");
  GLM_REQUIRE(out_f32 == nullptr || (shared == nullptr && resident == nullptr && router == nullptr),
              "a share's FP32 partial takes no layer epilogue (it follows the sum over the expert axis)");
  const int64_t n = tokens * top_k;
  const int shape = routed_shape(tokens, n, num_experts, hidden_size, intermediate);
  const bool fp8 = (flags & GLM_MOE_FP8_ACTIVATIONS) != 0;
  GLM_REQUIRE(!fp8 || (!uses_decode_path(n, hidden_size, intermediate) && shape == kShapeWide &&
                       prefill_fits(intermediate, hidden_size, 2) && prefill_fits(hidden_size, intermediate, 1)),
              "FP8 activations need a prefill shape: more than %d routes, H a multiple of 256 and I of 128, "
              "both at most 8192",
              kMaxDecodeRoutes);
  GLM_REQUIRE(!fp8 || (prefill_rows_fit(tokens, hidden_size) && prefill_rows_fit(n, intermediate)),
              "FP8 activations: tokens x hidden and routes x intermediate bf16 must stay below 2 GiB");
  const int bn13 = gemm_shape_bn(shape, 2);
  const int bn2 = gemm_shape_bn(shape, 1);
  GLM_REQUIRE(intermediate % bn13 == 0, "intermediate size must be a multiple of %d", bn13);
  GLM_REQUIRE(hidden_size % bn2 == 0, "hidden size must be a multiple of %d", bn2);
  const RoutedLayout L = routed_layout(tokens, top_k, num_experts, hidden_size, intermediate);
  const bool decode = uses_decode_path(n, hidden_size, intermediate);
  GLM_REQUIRE(decode || !compact_decode_scratch, "the decode-path scratch layout takes decode shapes only");
  const size_t need = compact_decode_scratch ? decode_scratch_bytes(tokens, top_k, intermediate) : L.total;
  if (workspace_bytes < need || workspace == nullptr)
    return fail(GLM_MOE_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  hipStream_t stream = as_stream(stream_ptr);
  char* ws = static_cast<char*>(workspace);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
  int32_t* inverse = reinterpret_cast<int32_t*>(ws + L.inverse);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* tile_expert = reinterpret_cast<int32_t*>(ws + L.tiles);
  int32_t* tile_row = tile_expert + L.max_tiles;
  int32_t* tile_live = tile_row + L.max_tiles;
  int32_t* tile_count = tile_live + L.max_tiles;
  int32_t* tile_desc = reinterpret_cast<int32_t*>(ws + L.tile_desc);
  uint16_t* act = reinterpret_cast<uint16_t*>(ws + (compact_decode_scratch ? 0 : L.act));
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + L.y);
  uint8_t* xq = reinterpret_cast<uint8_t*>(ws + L.xq);
  float* xscale = reinterpret_cast<float*>(ws + L.xscale);
  uint8_t* actq = reinterpret_cast<uint8_t*>(ws + L.actq);
  float* actscale = reinterpret_cast<float*>(ws + L.actscale);

  if (timer.events) *timer.timed = 0;
  if (decode) {
    // decode: two kernels that find their routes themselves and fuse the combine
    DecodeArgs d{};
    d.ids = route_indices;
    d.weights = route_weights;
    d.routes = (int32_t)n;
    d.top_k = top_k;
    d.own = own;
    d.check_weights = (flags & GLM_MOE_CHECK_WEIGHTS) ? 1 : 0;
    d.hidden_in = hidden;
    d.hidden = (int32_t)hidden_size;
    d.intermediate = (int32_t)intermediate;
    d.gate_bits = gate_bits;
    d.gate_scale = gate_scale;
    d.up_bits = up_bits;
    d.up_scale = up_scale;
    d.down_bits = down_bits;
    d.down_scale = down_scale;
    d.act = act;
    d.out = out;
    d.out_f32 = out_f32;
    d.round_partial = (flags & GLM_MOE_ROUTE_SUM_BF16) ? 1 : 0;
    d.valid = valid;
    d.shared = shared;
    d.routed_scale = routed_scale;
    if (router != nullptr && num_experts > kDecodeRouterExperts) {
      // the decode gate/up kernel routes at most kDecodeRouterExperts experts:
      // the router kernel runs ahead of it (after every check above, so a
      // refused call has launched nothing and left the route outputs alone)
      GLM_HIP(launch_route_noaux_tc(router->logits, tokens, num_experts, router->bias, top_k,
                                    const_cast<int32_t*>(route_indices), const_cast<float*>(route_weights), stream),
              "router launch");
    } else if (router != nullptr) {
      d.router_logits = router->logits;
      d.router_bias = router->bias;
      d.ids_out = const_cast<int32_t*>(route_indices);
      d.weights_out = const_cast<float*>(route_weights);
    }
    if (resident != nullptr) {
      d.shared_gate = resident[0];
      d.shared_up = resident[1];
      d.shared_down = resident[2];
      d.act_shared = reinterpret_cast<uint16_t*>(
          ws + (compact_decode_scratch ? decode_act_bytes(tokens, top_k, intermediate) : L.act_shared));
    }
    const LaunchEvents stage_events[2] = {timer.at(kStageGateUp), timer.at(kStageDown)};
    if (timer.events) *timer.timed = (1u << kStageGateUp) | (1u << kStageDown);
    GLM_HIP(launch_decode_routed(d, stream, timer.events ? stage_events : nullptr), "decode launch");
    return GLM_MOE_OK;
  }

  GLM_REQUIRE(resident == nullptr,
              "the resident shared expert runs on decode shapes (at most %d routes); pass the shared "
              "expert's output to glm_moe_moe_layer instead",
              kMaxDecodeRoutes);
  RoutePlanArgs p{};
  p.ids = route_indices;
  p.n = (int32_t)n;
  p.top_k = top_k;
  p.experts = num_experts;
  p.own = own;
  p.keys = num_experts + (unowned ? 1 : 0);  // unowned routes: one key past the owned experts, never tiled
  p.key_bits = key_bits_for(p.keys);
  p.route_w = (flags & GLM_MOE_CHECK_WEIGHTS) ? route_weights : nullptr;
  p.sorted = sorted;
  p.inverse = inverse;
  p.counts = counts;
  p.offsets = offsets;
  p.valid = valid;
  // bf16 prefill: tiles of up to 256 routes when both projections run on the
  // prefill kernel (its wide variants decode each weight block once for twice
  // the routes); the FP8 kernel and the other shapes take the shape's tiles.
  const bool wide_tiles = !fp8 && shape == kShapeWide && prefill_fits(intermediate, hidden_size, 2) &&
                          prefill_fits(hidden_size, intermediate, 1) && prefill_rows_fit(tokens, hidden_size) &&
                          prefill_rows_fit(n, intermediate);
  const int tile_rows = wide_tiles ? prefill_wide_tile_rows() : gemm_shape_rows(shape);
  // Tall stripes (512 weight rows a work item) pay where experts see enough
  // routes to fill a few column groups: GLM-5 shape, T=1024 / 2048 layer
  // -3 / -5 %, T=512 even, but T=9 / 16 / 64 / 256 +7 / +7 / +3.5 / +1 %, so
  // they run from 16 routes per expert on average.  Where a projection runs
  // on them, its wide tiles run as two work items per stripe, one per 256-row
  // half: the plan lists each tile of more than half the tile rows twice.  At
  // most ceil(c / 128) listings per expert of c routes: within L.max_tiles.
  const bool tall = n >= 16 * (int64_t)global_experts;  // routes per expert of the whole layer
  const bool wide_twice = tall && wide_tiles &&
                          (intermediate % prefill_tall_bn(2) == 0 || hidden_size % prefill_tall_bn(1) == 0);
  const int32_t max_tiles =
      (int32_t)max_tiles_for(n, num_experts, wide_twice ? tile_rows / 2 : tile_rows);  // <= L.max_tiles
  p.tile_rows = tile_rows;
  p.wide_twice = wide_twice ? 1 : 0;
  p.max_tiles = max_tiles;
  p.tile_expert = tile_expert;
  p.tile_row = tile_row;
  p.tile_live = tile_live;
  p.tile_count = tile_count;
  p.tile_desc = tile_desc;
  p.chunk_hist = reinterpret_cast<int32_t*>(ws + L.chunk_hist);
  p.chunk_bad = reinterpret_cast<int32_t*>(ws + L.chunk_bad);
  timer.arm(kStagePlan);
  if (router != nullptr) {
    // routing from the logits on grouped shapes: the router (one wave per token
    // over the whole GPU) counts the plan's histogram rows on the way, so the
    // plan is the router and the scatter (one-workgroup plans: the router
    // kernel ahead of the plan).  Routing inside the plan's own workgroups was
    // built and measured slower at every prefill size: the plan runs one
    // workgroup per 2048 routes, and a token's routing costs a wave ~600 VALU
    // instructions.
    const RouterPass rp{router->logits, router->bias, global_experts, tokens,
                        const_cast<int32_t*>(route_indices), const_cast<float*>(route_weights)};
    GLM_HIP(launch_route_plan_from_logits(p, rp, stream), "router and route plan launch");
  } else {
    GLM_HIP(launch_route_plan(p, stream), "route plan launch");
  }
  timer.done(kStagePlan);

  // Every owned route is covered by exactly one tile, so every row of act and y
  // the combine reads is written before it is read (the combine skips unowned routes).
  GroupedGemmArgs g{};
  g.experts = num_experts;
  g.rows = (int32_t)n;
  g.x_rows = tokens;
  g.out_rows = n;
  g.x = hidden;
  g.x_row_ids = sorted;
  g.x_row_div = top_k;
  g.w0 = gate_bits;
  g.s0 = gate_scale;
  g.w1 = up_bits;
  g.s1 = up_scale;
  g.n = (int32_t)intermediate;
  g.k = (int32_t)hidden_size;
  g.tile_expert = tile_expert;
  g.tile_row = tile_row;
  g.tile_live = tile_live;
  g.tile_count = tile_count;
  g.max_tiles = max_tiles;
  g.tile_desc = tile_desc;
  if (fp8) {
    GLM_HIP(launch_quantize_rows_fp8(hidden, tokens, hidden_size, xq, xscale, inverse, top_k, n, stream),
            "quantize launch");
    g.xq = xq;
    g.xscale = xscale;
  }
  g.valid = nullptr;
  g.out = act;
  g.ldo = intermediate;
  g.table_stride = 0;
  g.out_row_ids = nullptr;
  g.route_w = nullptr;
  g.stripe_run = prefill_stripe_run(2);
  g.tile_rows = tile_rows;
  g.wide_twice = p.wide_twice;
  g.tall = tall ? 1 : 0;
  // FP8 mode on tall stripes: the gate/up epilogue quantises its SwiGLU rows
  // for the down projection itself (the values the quantize launch below
  // would write from the bf16 rows, which are then not written at all)
  const bool fused_quant = fp8 && shape == kShapeWide && prefill_quantizes_output(g, 2, kEpiSwiglu);
  if (fused_quant) {
    g.outq = actq;
    g.outq_scale = actscale;
  }
  timer.arm(kStageGateUp);
  GLM_HIP(launch_grouped_gemm(g, shape, 2, kEpiSwiglu, stream), "gate/up launch");
  timer.done(kStageGateUp);

  GroupedGemmArgs d{};
  d.experts = num_experts;
  d.rows = (int32_t)n;
  d.x_rows = n;
  d.out_rows = n;
  d.x = act;
  d.x_row_ids = nullptr;
  d.x_row_div = 1;
  d.w0 = down_bits;
  d.s0 = down_scale;
  d.n = (int32_t)hidden_size;
  d.k = (int32_t)intermediate;
  d.tile_expert = tile_expert;
  d.tile_row = tile_row;
  d.tile_live = tile_live;
  d.tile_count = tile_count;
  d.max_tiles = max_tiles;
  d.tile_desc = tile_desc;
  if (fp8) {
    if (!fused_quant)
      GLM_HIP(launch_quantize_rows_fp8(act, n, intermediate, actq, actscale, nullptr, 1, n, stream),
              "quantize launch");
    d.xq = actq;
    d.xscale = actscale;
  }
  d.valid = nullptr;
  d.out = y;
  d.ldo = hidden_size;
  d.table_stride = 0;
  d.out_row_ids = sorted;
  d.route_w = nullptr;  // the combine applies the route weights (same rounding, no dependent loads here)
  d.stripe_run = prefill_stripe_run(1);
  d.tile_rows = tile_rows;
  d.wide_twice = p.wide_twice;
  // about one tile per expert of the call, or its share of the routes in whole tiles
  // (wide tiles counted as their two listings)
  const int64_t listing_rows = p.wide_twice ? tile_rows / 2 : tile_rows;
  const int64_t listings_est =
      std::max<int64_t>(num_experts, (n * num_experts / global_experts + listing_rows - 1) / listing_rows);
  d.tall = tall && (fp8 || down_tall_fills(listings_est, hidden_size)) ? 1 : 0;
  timer.arm(kStageDown);
  GLM_HIP(launch_grouped_gemm(d, shape, 1, kEpiStoreBf16, stream), "down launch");
  timer.done(kStageDown);

  timer.arm(kStageCombine);
  GLM_HIP(launch_combine_routes(y, tokens, top_k, hidden_size, unowned ? route_indices : nullptr, own,
                                route_weights, shared, routed_scale, valid, out, out_f32,
                                (flags & GLM_MOE_ROUTE_SUM_BF16) ? 1 : 0, stream),
          "combine launch");
  timer.done(kStageCombine);
  return GLM_MOE_OK;
}

}  // namespace

// ------------------------------------------------------------------ allocation-free decode layer
// Scratch of glm_moe_moe_layer_resident_noalloc: a static device array, one
// copy per GPU, held until the process ends.  Host code never uses the array's
// name as an address (on the host it is only a stand-in for the symbol): the
// device address of each GPU's copy comes from hipGetSymbolAddress, taken once
// per device with that device current, and is what the kernels receive.
constexpr size_t kStaticScratchBytes = 512 * 1024;  // decode path: <= 64 routes x I <= 2048, bf16, twice
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices] = {};

// The copy of `scratch` on the device the call's kernels run on (looked up on
// the first call on the device).  Kernels run on the stream's device, but the
// symbol's address is taken for the current device, so a stream of another
// device than the current one is refused (the null stream runs on the current
// device).
int static_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  GLM_HIP(hipGetDevice(&dev), "hipGetDevice");
  if (stream != nullptr) {
    hipDevice_t stream_dev = 0;
    GLM_HIP(hipStreamGetDevice(stream, &stream_dev), "hipStreamGetDevice");
    GLM_REQUIRE(stream_dev == dev,
                "the stream runs on device %d but device %d is current: make the stream's device current "
                "(the static scratch is looked up per device)",
                (int)stream_dev, dev);
  }
  GLM_REQUIRE(dev >= 0 && dev < kScratchDevices, "device %d beyond the %d the static scratch tracks", dev,
              kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    GLM_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    GLM_REQUIRE(ptr != nullptr, "no device address for the static scratch");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GLM_MOE_OK;
}

}  // namespace

extern "C" {

int glm_moe_abi_version(void) { return GLM_MOE_ABI_VERSION; }

const char* glm_moe_last_error(void) { return g_last_error.c_str(); }

int glm_moe_decode_fp8_table(const uint8_t* bits, const float* scale, int64_t n, int64_t k,
                             int32_t block_n, int32_t block_k, uint16_t* out_bf16, void* stream) {
  GLM_REQUIRE(n >= 0 && k >= 0, "negative table shape");
  GLM_REQUIRE(block_n > 0 && block_k > 0, "block_shape must contain two positive integers");
  GLM_REQUIRE((n == 0 || k == 0) || (bits && scale && out_bf16), "null tensor pointer");
  GLM_HIP(launch_decode_fp8_table(bits, scale, n, k, block_n, block_k, out_bf16, as_stream(stream)),
          "decode launch");
  return GLM_MOE_OK;
}

int glm_moe_swiglu_bf16(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* out, void* stream) {
  GLM_REQUIRE(n >= 0, "negative element count");
  GLM_REQUIRE(n == 0 || (gate && up && out), "null tensor pointer");
  GLM_HIP(launch_swiglu_bf16(gate, up, n, out, as_stream(stream)), "swiglu launch");
  return GLM_MOE_OK;
}

int glm_moe_route_noaux_tc(const float* router_logits, int64_t tokens, int32_t num_experts,
                           const float* correction_bias, int32_t top_k, int32_t* route_indices,
                           float* route_weights, void* stream) {
  GLM_REQUIRE(tokens >= 0, "router_logits must have shape [tokens, experts]");
  GLM_REQUIRE(num_experts > 0 && num_experts <= kMaxExperts, "at most %d experts", kMaxExperts);
  GLM_REQUIRE(top_k > 0 && top_k <= num_experts, "top_k must be in [1, num_experts]");
  GLM_REQUIRE(top_k <= kWave, "the GPU router selects at most %d experts per token (one wave lane each)", kWave);
  if (tokens == 0) return GLM_MOE_OK;
  GLM_REQUIRE(router_logits && route_indices && route_weights, "null tensor pointer");
  GLM_HIP(launch_route_noaux_tc(router_logits, tokens, num_experts, correction_bias, top_k, route_indices,
                                route_weights, as_stream(stream)),
          "router launch");
  return GLM_MOE_OK;
}

int glm_moe_count_nonfinite_fp8(const uint8_t* bits, int64_t n, uint64_t* count, void* stream) {
  GLM_REQUIRE(n >= 0, "byte count must be >= 0");
  if (n == 0) return GLM_MOE_OK;
  GLM_REQUIRE(bits && count, "null tensor pointer");
  GLM_REQUIRE(reinterpret_cast<uintptr_t>(bits) % 4 == 0 && reinterpret_cast<uintptr_t>(count) % 8 == 0,
              "FP8 bytes must be 4-byte aligned and the count 8-byte aligned");
  GLM_HIP(launch_count_nonfinite_fp8(bits, n, reinterpret_cast<unsigned long long*>(count), as_stream(stream)),
          "finite-bit scan launch");
  return GLM_MOE_OK;
}

int glm_moe_group_routes(const int32_t* route_indices, int64_t tokens, int32_t top_k,
                         int32_t num_experts, int32_t* sorted_flat_ids,
                         int32_t* inverse_permutation, int32_t* group_sizes, uint8_t* valid,
                         void* workspace, size_t workspace_bytes, void* stream) {
  GLM_REQUIRE(tokens > 0 && top_k > 0, "routes must be nonempty [tokens,top_k]");
  GLM_REQUIRE(num_experts > 0, "num_experts must be a positive integer");
  GLM_REQUIRE(top_k <= num_experts, "top_k exceeds expert count");
  GLM_REQUIRE(num_experts <= kMaxExperts, "at most %d experts", kMaxExperts);
  GLM_REQUIRE(tokens * top_k <= INT32_MAX / 2, "too many routes");
  GLM_REQUIRE(route_indices && sorted_flat_ids && inverse_permutation && group_sizes && valid,
              "null tensor pointer");
  RoutePlanArgs p{};
  p.ids = route_indices;
  p.n = (int32_t)(tokens * top_k);
  p.top_k = top_k;
  p.experts = num_experts;
  p.own = whole_layer(num_experts);
  p.keys = num_experts;
  p.key_bits = key_bits_for(num_experts);
  p.sorted = sorted_flat_ids;
  p.inverse = inverse_permutation;
  p.counts = group_sizes;
  p.valid = valid;
  if (workspace != nullptr &&
      workspace_bytes >= glm_moe_group_routes_workspace_bytes(tokens, top_k, num_experts)) {
    const int chunks = route_plan_chunks(p.n, top_k);
    p.chunk_hist = static_cast<int32_t*>(workspace);
    p.chunk_bad = p.chunk_hist + (size_t)chunks * num_experts;
  }
  GLM_HIP(launch_route_plan(p, as_stream(stream)), "route plan launch");
  return GLM_MOE_OK;
}

size_t glm_moe_group_routes_workspace_bytes(int64_t tokens, int32_t top_k, int32_t num_experts) {
  if (tokens <= 0 || top_k <= 0 || num_experts <= 0 || tokens * top_k > INT32_MAX / 2) return 0;
  const size_t chunks = (size_t)route_plan_chunks((int32_t)(tokens * top_k), top_k);
  return sizeof(int32_t) * chunks * ((size_t)num_experts + 1);
}

int glm_moe_gather_rows(const void* src, int64_t src_rows, int64_t row_bytes,
                        const int32_t* index, int32_t div, const uint8_t* mask, int64_t rows,
                        void* dst, void* stream) {
  GLM_REQUIRE(rows >= 0 && row_bytes >= 0 && src_rows >= 0, "negative geometry");
  GLM_REQUIRE(row_bytes % 4 == 0, "row bytes must be a multiple of 4");
  GLM_REQUIRE(div > 0, "divisor must be positive");
  if (rows == 0 || row_bytes == 0) return GLM_MOE_OK;
  GLM_REQUIRE(src_rows > 0, "gather from an empty source");
  GLM_REQUIRE(src && index && dst, "null tensor pointer");
  GLM_HIP(launch_gather_rows(src, src_rows, row_bytes, index, div, mask, rows, dst, as_stream(stream)),
          "gather launch");
  return GLM_MOE_OK;
}

int glm_moe_build_expert_panels(const int32_t* group_sizes, int32_t num_groups,
                                const int32_t* group_offset, int32_t rows, int32_t local_groups,
                                int32_t* expert_ids, int32_t* row_starts, int32_t* live_counts,
                                int32_t* active_panels, int32_t* restore_indices,
                                uint8_t* owned_rows, uint8_t* valid, void* stream) {
  GLM_REQUIRE(rows > 0 && local_groups > 0, "expert panels require bounded rows and int32 group counts");
  GLM_REQUIRE(num_groups >= local_groups, "expert panels require bounded rows and int32 group counts");
  GLM_REQUIRE((int64_t)(rows + 31) * num_groups <= INT32_MAX, "expert panels require bounded rows and int32 group counts");
  GLM_REQUIRE(num_groups <= kMaxExperts, "at most %d groups", kMaxExperts);
  GLM_REQUIRE(group_sizes && group_offset && expert_ids && row_starts && live_counts && active_panels &&
                  restore_indices && owned_rows && valid,
              "null tensor pointer");
  PanelPlanArgs p{};
  p.group_sizes = group_sizes;
  p.groups = num_groups;
  p.group_offset = group_offset;
  p.rows = rows;
  p.local_groups = local_groups;
  p.panel_rows = 32;
  p.capacity = (rows + 31) / 32 + local_groups - 1;
  p.expert_ids = expert_ids;
  p.row_starts = row_starts;
  p.live_counts = live_counts;
  p.active_panels = active_panels;
  p.restore_indices = restore_indices;
  p.owned_rows = owned_rows;
  p.valid = valid;
  GLM_HIP(launch_panel_plan(p, as_stream(stream)), "panel plan launch");
  return GLM_MOE_OK;
}

int glm_moe_pack_expert_panel_rows(const void* values, int64_t rows, int64_t row_bytes,
                                   const int32_t* row_starts, const int32_t* live_counts,
                                   int32_t capacity, void* out, void* stream) {
  GLM_REQUIRE(rows > 0 && capacity >= 0 && row_bytes >= 0, "panel packing row geometry disagrees");
  GLM_REQUIRE(row_bytes % 4 == 0, "row bytes must be a multiple of 4");
  if (capacity == 0 || row_bytes == 0) return GLM_MOE_OK;
  GLM_REQUIRE(values && row_starts && live_counts && out, "null tensor pointer");
  GLM_HIP(launch_pack_panel_rows(values, rows, row_bytes, row_starts, live_counts, capacity, 32, out,
                                 as_stream(stream)),
          "pack launch");
  return GLM_MOE_OK;
}

int glm_moe_panel_fp8_matmul(const uint16_t* lhs, int64_t m, int64_t k, const uint8_t* weight_bits,
                             const float* scale, int32_t groups, int64_t n,
                             const int32_t* panel_expert_ids, const int32_t* panel_row_starts,
                             const int32_t* panel_live_counts, const int32_t* active_panels,
                             int32_t capacity, const uint8_t* owned_rows, const uint8_t* valid,
                             int32_t result_dtype, void* out, void* stream) {
  GLM_REQUIRE(m > 0 && k > 0 && groups > 0 && n > 0, "panel FP8 geometry/dtypes disagree with M32/N256/K128");
  GLM_REQUIRE(k % 128 == 0 && n % 256 == 0 && n / 128 <= 128, "panel FP8 geometry/dtypes disagree with M32/N256/K128");
  GLM_REQUIRE(capacity == (m + 31) / 32 + groups - 1, "panel FP8 geometry/dtypes disagree with M32/N256/K128");
  GLM_REQUIRE(result_dtype == GLM_MOE_F32 || result_dtype == GLM_MOE_BF16, "result must be FP32 or BF16");
  GLM_REQUIRE(k <= INT32_MAX / 2 && n <= INT32_MAX / 2 && m <= INT32_MAX / 2, "dimension too large");
  GLM_REQUIRE(lhs && weight_bits && scale && panel_expert_ids && panel_row_starts && panel_live_counts &&
                  active_panels && owned_rows && valid && out,
              "null tensor pointer");
  hipStream_t s = as_stream(stream);
  const int64_t elem = result_dtype == GLM_MOE_F32 ? 4 : 2;
  GLM_HIP(launch_zero_rows(out, m, n * elem, owned_rows, valid, s), "zero launch");
  GroupedGemmArgs g{};
  g.experts = groups;
  g.rows = (int32_t)m;
  g.x_rows = m;
  g.out_rows = m;
  g.x = lhs;
  g.x_row_div = 1;
  g.w0 = weight_bits;
  g.s0 = scale;
  g.n = (int32_t)n;
  g.k = (int32_t)k;
  g.tile_expert = panel_expert_ids;
  g.tile_row = panel_row_starts;
  g.tile_live = panel_live_counts;
  g.tile_count = active_panels;
  g.max_tiles = capacity;
  g.valid = valid;
  g.out = out;
  g.ldo = n;
  g.table_stride = 0;
  GLM_HIP(launch_grouped_gemm(g, kShapePanel32, 1, result_dtype == GLM_MOE_F32 ? kEpiStoreF32 : kEpiStoreBf16, s),
          "panel matmul launch");
  return GLM_MOE_OK;
}

size_t glm_moe_routed_projection_workspace_bytes(int32_t slots) {
  return align_up(sizeof(int32_t) * (3 * (size_t)(slots > 0 ? slots : 0) + 1));
}

int glm_moe_routed_projection(const uint16_t* lhs, int32_t slots, int64_t k, int32_t tables,
                              const uint8_t* bits0, const float* scale0, const uint8_t* bits1,
                              const float* scale1, int32_t experts, int64_t n,
                              const int32_t* local_expert_ids, const uint8_t* owned,
                              int32_t result_dtype, void* out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  GLM_REQUIRE(tables == 1 || tables == 2, "routed FP8 projection takes one or two weight table pairs");
  GLM_REQUIRE(slots > 0 && k > 0, "routed FP8 lhs dimensions must be positive");
  GLM_REQUIRE(experts > 0 && n > 0, "routed FP8 weight/input geometry disagrees");
  GLM_REQUIRE(k % 128 == 0 && n % 128 == 0, "routed FP8 requires N/K divisible by the scale block");
  GLM_REQUIRE(result_dtype == GLM_MOE_F32 || result_dtype == GLM_MOE_BF16, "routed FP8 result must be FP32 or BF16");
  GLM_REQUIRE(k <= INT32_MAX / 2 && n <= INT32_MAX / 2, "dimension too large");
  GLM_REQUIRE(lhs && bits0 && scale0 && local_expert_ids && owned && out, "null tensor pointer");
  GLM_REQUIRE(tables == 1 || (bits1 && scale1), "null tensor pointer");
  if (workspace_bytes < glm_moe_routed_projection_workspace_bytes(slots) || workspace == nullptr)
    return fail(GLM_MOE_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given",
                glm_moe_routed_projection_workspace_bytes(slots), workspace_bytes);
  hipStream_t s = as_stream(stream);
  int32_t* tile_expert = static_cast<int32_t*>(workspace);
  int32_t* tile_row = tile_expert + slots;
  int32_t* tile_live = tile_row + slots;
  int32_t* tile_count = tile_live + slots;
  const int64_t elem = result_dtype == GLM_MOE_F32 ? 4 : 2;
  GLM_HIP(launch_fill_u32(out, (int64_t)slots * tables * n * elem / 4, 0u, s), "zero launch");
  GLM_HIP(launch_slot_tiles(local_expert_ids, owned, slots, experts, tile_expert, tile_row, tile_live,
                            tile_count, s),
          "slot plan launch");
  GroupedGemmArgs g{};
  g.name = "fp8_routed_projection";
  g.experts = experts;
  g.rows = slots;
  g.x_rows = slots;
  g.out_rows = slots;
  g.x = lhs;
  g.x_row_div = 1;
  g.w0 = bits0;
  g.s0 = scale0;
  g.w1 = tables == 2 ? bits1 : nullptr;
  g.s1 = tables == 2 ? scale1 : nullptr;
  g.n = (int32_t)n;
  g.k = (int32_t)k;
  g.tile_expert = tile_expert;
  g.tile_row = tile_row;
  g.tile_live = tile_live;
  g.tile_count = tile_count;
  g.max_tiles = slots;
  g.out = out;
  g.ldo = (int64_t)tables * n;
  g.table_stride = n;
  GLM_HIP(launch_grouped_gemm(g, kShapeDecode, tables, result_dtype == GLM_MOE_F32 ? kEpiStoreF32 : kEpiStoreBf16, s),
          "routed projection launch");
  return GLM_MOE_OK;
}

size_t glm_moe_routed_experts_workspace_bytes(int64_t tokens, int32_t top_k, int32_t num_experts,
                                              int64_t hidden, int64_t intermediate) {
  if (tokens <= 0 || top_k <= 0 || num_experts <= 0 || hidden <= 0 || intermediate <= 0) return 0;
  return routed_layout(tokens, top_k, num_experts, hidden, intermediate).total;
}

int glm_moe_routed_experts(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                           const int32_t* route_indices, const float* route_weights,
                           int32_t top_k, int32_t num_experts, int64_t intermediate,
                           const uint8_t* gate_bits, const float* gate_scale,
                           const uint8_t* up_bits, const float* up_scale,
                           const uint8_t* down_bits, const float* down_scale, uint32_t flags,
                           uint16_t* out, uint8_t* valid, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k,
                             num_experts, intermediate, gate_bits, gate_scale, up_bits, up_scale,
                             down_bits, down_scale, flags, nullptr, nullptr, 0.0f, out, valid, workspace, workspace_bytes,
                             StageTimer{nullptr, nullptr}, stream);
}

int glm_moe_routed_experts_timed(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                                 const int32_t* route_indices, const float* route_weights,
                                 int32_t top_k, int32_t num_experts, int64_t intermediate,
                                 const uint8_t* gate_bits, const float* gate_scale,
                                 const uint8_t* up_bits, const float* up_scale,
                                 const uint8_t* down_bits, const float* down_scale,
                                 uint32_t flags, uint16_t* out, uint8_t* valid, void* workspace,
                                 size_t workspace_bytes, void* const* events, uint32_t* timed_stages,
                                 void* stream) {
  GLM_REQUIRE(events != nullptr && timed_stages != nullptr, "eight events and a stage mask required");
  for (int i = 0; i < 2 * kStages; ++i) GLM_REQUIRE(events[i] != nullptr, "eight events required");
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k,
                             num_experts, intermediate, gate_bits, gate_scale, up_bits, up_scale,
                             down_bits, down_scale, flags, nullptr, nullptr, 0.0f, out, valid, workspace, workspace_bytes,
                             StageTimer{events, timed_stages}, stream);
}

int glm_moe_moe_layer(const uint16_t* hidden, int64_t tokens, int64_t hidden_size, const int32_t* route_indices,
                      const float* route_weights, int32_t top_k, int32_t num_experts, int64_t intermediate,
                      const uint8_t* gate_bits, const float* gate_scale, const uint8_t* up_bits,
                      const float* up_scale, const uint8_t* down_bits, const float* down_scale, uint32_t flags,
                      const uint16_t* shared, float routed_scale, uint16_t* out, uint8_t* valid, void* workspace,
                      size_t workspace_bytes, void* stream) {
  GLM_REQUIRE(shared != nullptr, "null shared-expert rows");
  GLM_REQUIRE(std::isfinite(routed_scale), "routed scale must be finite");
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k,
                             num_experts, intermediate, gate_bits, gate_scale, up_bits, up_scale,
                             down_bits, down_scale, flags, shared, nullptr, bf16_round_host(routed_scale), out,
                             valid, workspace, workspace_bytes, StageTimer{nullptr, nullptr}, stream);
}

int glm_moe_moe_layer_from_router_logits(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                                         const float* router_logits, const float* correction_bias, int32_t top_k,
                                         int32_t num_experts, int64_t intermediate, const uint8_t* gate_bits,
                                         const float* gate_scale, const uint8_t* up_bits, const float* up_scale,
                                         const uint8_t* down_bits, const float* down_scale, uint32_t flags,
                                         const uint16_t* shared, float routed_scale, int32_t* route_indices,
                                         float* route_weights, uint16_t* out, uint8_t* valid, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  GLM_REQUIRE(router_logits != nullptr && route_indices != nullptr && route_weights != nullptr,
              "null router logits or route outputs");
  GLM_REQUIRE(num_experts > 0 && num_experts <= kMaxExperts, "the router takes 1 to %d experts", kMaxExperts);
  GLM_REQUIRE(top_k > 0 && top_k <= num_experts && top_k <= 64, "top_k must be in [1, min(%d, 64)]",
              (int)num_experts);
  GLM_REQUIRE(shared == nullptr || std::isfinite(routed_scale), "routed scale must be finite");
  const RouterIn router{router_logits, correction_bias};
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k, num_experts,
                             intermediate, gate_bits, gate_scale, up_bits, up_scale, down_bits, down_scale, flags,
                             shared, nullptr, shared ? bf16_round_host(routed_scale) : 0.0f, out, valid, workspace,
                             workspace_bytes, StageTimer{nullptr, nullptr}, stream, &router);
}

int glm_moe_routed_experts_share(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                                 const int32_t* route_indices, const float* route_weights, int32_t top_k,
                                 int32_t num_experts, int32_t expert_offset, int32_t local_experts,
                                 int64_t intermediate, const uint8_t* gate_bits, const float* gate_scale,
                                 const uint8_t* up_bits, const float* up_scale, const uint8_t* down_bits,
                                 const float* down_scale, uint32_t flags, float* out, uint8_t* valid,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  GLM_REQUIRE(out != nullptr, "null tensor pointer");
  GLM_REQUIRE(num_experts > 0 && local_experts > 0, "a share needs num_experts and local_experts > 0");
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k, local_experts,
                             intermediate, gate_bits, gate_scale, up_bits, up_scale, down_bits, down_scale, flags,
                             nullptr, nullptr, 0.0f, nullptr, valid, workspace, workspace_bytes,
                             StageTimer{nullptr, nullptr}, stream, nullptr, false, num_experts, expert_offset, out);
}

int glm_moe_moe_layer_epilogue(const float* routed, int64_t tokens, int64_t hidden_size, const uint16_t* shared,
                               float routed_scale, uint16_t* out, uint8_t* valid, void* stream) {
  GLM_REQUIRE(tokens > 0 && hidden_size > 0 && hidden_size % 8 == 0,
              "the epilogue takes [tokens, hidden] rows, hidden a multiple of 8");
  GLM_REQUIRE(routed && shared && out && valid, "null tensor pointer");
  GLM_REQUIRE(std::isfinite(routed_scale), "routed scale must be finite");
  GLM_HIP(launch_layer_epilogue(routed, tokens, hidden_size, shared, bf16_round_host(routed_scale), out, valid,
                                as_stream(stream)),
          "epilogue launch");
  return GLM_MOE_OK;
}

int glm_moe_uses_decode_kernels(int64_t tokens, int32_t top_k, int64_t hidden_size, int64_t intermediate) {
  return tokens > 0 && top_k > 0 && hidden_size > 0 && intermediate > 0 &&
                 uses_decode_path(tokens * top_k, hidden_size, intermediate)
             ? 1
             : 0;
}

int glm_moe_moe_layer_resident(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                               const int32_t* route_indices, const float* route_weights, int32_t top_k,
                               int32_t num_experts, int64_t intermediate, const uint8_t* gate_bits,
                               const float* gate_scale, const uint8_t* up_bits, const float* up_scale,
                               const uint8_t* down_bits, const float* down_scale, uint32_t flags,
                               const uint16_t* shared_gate, const uint16_t* shared_up, const uint16_t* shared_down,
                               int64_t shared_intermediate, float routed_scale, uint16_t* out, uint8_t* valid,
                               void* workspace, size_t workspace_bytes, void* stream) {
  GLM_REQUIRE(shared_gate && shared_up && shared_down, "null shared-expert table");
  GLM_REQUIRE(shared_intermediate == intermediate,
              "the resident shared expert needs the routed experts' intermediate size (%lld), got %lld",
              (long long)intermediate, (long long)shared_intermediate);
  GLM_REQUIRE(std::isfinite(routed_scale), "routed scale must be finite");
  GLM_REQUIRE((flags & GLM_MOE_FP8_ACTIVATIONS) == 0, "the resident shared expert takes bf16 activations");
  GLM_REQUIRE(tokens > 0 && top_k > 0 && uses_decode_path(tokens * top_k, hidden_size, intermediate),
              "the resident shared expert runs on decode shapes (at most %d routes); pass the shared "
              "expert's output to glm_moe_moe_layer instead",
              kMaxDecodeRoutes);
  const uint16_t* resident[3] = {shared_gate, shared_up, shared_down};
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k,
                             num_experts, intermediate, gate_bits, gate_scale, up_bits, up_scale,
                             down_bits, down_scale, flags, nullptr, resident, bf16_round_host(routed_scale), out,
                             valid, workspace, workspace_bytes, StageTimer{nullptr, nullptr}, stream);
}

int glm_moe_moe_layer_resident_noalloc(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                                       const int32_t* route_indices, const float* route_weights, int32_t top_k,
                                       int32_t num_experts, int64_t intermediate, const uint8_t* gate_bits,
                                       const float* gate_scale, const uint8_t* up_bits, const float* up_scale,
                                       const uint8_t* down_bits, const float* down_scale, uint32_t flags,
                                       const uint16_t* shared_gate, const uint16_t* shared_up,
                                       const uint16_t* shared_down, int64_t shared_intermediate,
                                       float routed_scale, uint16_t* out, uint8_t* valid, void* stream) {
  GLM_REQUIRE(shared_gate && shared_up && shared_down, "null shared-expert table");
  GLM_REQUIRE(shared_intermediate == intermediate,
              "the resident shared expert needs the routed experts' intermediate size (%lld), got %lld",
              (long long)intermediate, (long long)shared_intermediate);
  GLM_REQUIRE(std::isfinite(routed_scale), "routed scale must be finite");
  GLM_REQUIRE((flags & GLM_MOE_FP8_ACTIVATIONS) == 0, "the resident shared expert takes bf16 activations");
  GLM_REQUIRE(tokens > 0 && top_k > 0 && uses_decode_path(tokens * top_k, hidden_size, intermediate),
              "the allocation-free layer runs on decode shapes (at most %d routes, intermediate <= 2048)",
              kMaxDecodeRoutes);
  const size_t need = decode_scratch_bytes(tokens, top_k, intermediate);
  GLM_REQUIRE(need <= kStaticScratchBytes,
              "the allocation-free layer has %zu bytes of static scratch per device; this call needs %zu",
              kStaticScratchBytes, need);
  void* ws = nullptr;
  const int st = static_scratch(as_stream(stream), &ws);
  if (st != GLM_MOE_OK) return st;
  const uint16_t* resident[3] = {shared_gate, shared_up, shared_down};
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k,
                             num_experts, intermediate, gate_bits, gate_scale, up_bits, up_scale,
                             down_bits, down_scale, flags, nullptr, resident, bf16_round_host(routed_scale), out,
                             valid, ws, kStaticScratchBytes, StageTimer{nullptr, nullptr}, stream, nullptr,
                             /*compact_decode_scratch=*/true);
}

int glm_moe_moe_layer_from_logits(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                                  const float* router_logits, const float* correction_bias, int32_t top_k,
                                  int32_t num_experts, int64_t intermediate, const uint8_t* gate_bits,
                                  const float* gate_scale, const uint8_t* up_bits, const float* up_scale,
                                  const uint8_t* down_bits, const float* down_scale, uint32_t flags,
                                  const uint16_t* shared_gate, const uint16_t* shared_up,
                                  const uint16_t* shared_down, int64_t shared_intermediate, float routed_scale,
                                  int32_t* route_indices, float* route_weights, uint16_t* out, uint8_t* valid,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  GLM_REQUIRE(router_logits != nullptr && route_indices != nullptr && route_weights != nullptr,
              "null router logits or route outputs");
  GLM_REQUIRE(num_experts > 0 && num_experts <= kDecodeRouterExperts,
              "routing inside the decode kernels takes at most %d experts; route with glm_moe_route_noaux_tc "
              "and call glm_moe_moe_layer_resident",
              kDecodeRouterExperts);
  GLM_REQUIRE(top_k > 0 && top_k <= num_experts, "top_k must be in [1, %d]", (int)num_experts);
  GLM_REQUIRE(shared_gate && shared_up && shared_down, "null shared-expert table");
  GLM_REQUIRE(shared_intermediate == intermediate,
              "the resident shared expert needs the routed experts' intermediate size (%lld), got %lld",
              (long long)intermediate, (long long)shared_intermediate);
  GLM_REQUIRE(std::isfinite(routed_scale), "routed scale must be finite");
  GLM_REQUIRE((flags & GLM_MOE_FP8_ACTIVATIONS) == 0, "the decode layer takes bf16 activations");
  GLM_REQUIRE(tokens > 0 && uses_decode_path(tokens * top_k, hidden_size, intermediate),
              "routing inside the layer runs on decode shapes (at most %d routes); route with "
              "glm_moe_route_noaux_tc and call glm_moe_moe_layer instead",
              kMaxDecodeRoutes);
  const uint16_t* resident[3] = {shared_gate, shared_up, shared_down};
  const RouterIn router{router_logits, correction_bias};
  return routed_experts_impl(hidden, tokens, hidden_size, route_indices, route_weights, top_k,
                             num_experts, intermediate, gate_bits, gate_scale, up_bits, up_scale,
                             down_bits, down_scale, flags, nullptr, resident, bf16_round_host(routed_scale), out,
                             valid, workspace, workspace_bytes, StageTimer{nullptr, nullptr}, stream, &router);
}

size_t glm_moe_shared_expert_rows_workspace_bytes(int64_t tokens, int64_t shared_intermediate) {
  if (tokens <= 0 || shared_intermediate <= 0) return 0;
  return (size_t)tokens * (size_t)shared_intermediate * sizeof(uint16_t);
}

int glm_moe_shared_expert_rows(const uint16_t* hidden, int64_t tokens, int64_t hidden_size,
                               const uint16_t* shared_gate, const uint16_t* shared_up, const uint16_t* shared_down,
                               int64_t shared_intermediate, uint16_t* out, void* workspace, size_t workspace_bytes,
                               void* stream) {
  GLM_REQUIRE(hidden && shared_gate && shared_up && shared_down && out, "null tensor pointer");
  GLM_REQUIRE(shared_rows_fit(tokens, hidden_size, shared_intermediate),
              "the few-row shared expert takes 1 to %d rows and hidden / intermediate sizes that are multiples "
              "of 128 (at most 8192 for 8 rows)",
              kSharedRowsMax);
  const size_t need = glm_moe_shared_expert_rows_workspace_bytes(tokens, shared_intermediate);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(GLM_MOE_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  GLM_HIP(launch_shared_expert_rows(hidden, (int)tokens, (int)hidden_size, (int)shared_intermediate, shared_gate,
                                    shared_up, shared_down, static_cast<uint16_t*>(workspace), out,
                                    as_stream(stream)),
          "shared expert launch");
  return GLM_MOE_OK;
}

int glm_moe_event_create(void** event) {
  GLM_REQUIRE(event != nullptr, "null event slot");
  hipEvent_t e = nullptr;
  GLM_HIP(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return GLM_MOE_OK;
}

int glm_moe_event_destroy(void* event) {
  if (event == nullptr) return GLM_MOE_OK;
  GLM_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
  return GLM_MOE_OK;
}

int glm_moe_event_elapsed_ms(void* start, void* stop, float* ms) {
  GLM_REQUIRE(start && stop && ms, "null event");
  GLM_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
          "hipEventElapsedTime");
  return GLM_MOE_OK;
}

int glm_moe_synthesize_fp8_weights(uint64_t seed, int32_t experts, int64_t n, int64_t k, float sigma,
                                   uint8_t* bits, float* scales, void* stream) {
  GLM_REQUIRE(experts > 0 && n > 0 && k > 0, "synthetic weights need positive geometry");
  GLM_REQUIRE(n % 128 == 0 && k % 128 == 0, "synthetic weights need N and K multiples of 128");
  GLM_REQUIRE(sigma > 0.0f, "sigma must be positive");
  GLM_REQUIRE(bits && scales, "null tensor pointer");
  GLM_HIP(launch_synth_fp8(seed, experts, n, k, sigma, bits, scales, as_stream(stream)), "synth launch");
  return GLM_MOE_OK;
}

}  // extern "C"
