// Route planning: the stable expert grouping of glm-tpu's
// group_prefill_routes (reference glm_tpu/layers/moe/routed_experts.py:139-164),
// its expert-panel planner build_expert_panels
// (glm_tpu/kernels/fp8_grouped_matmul/panels.py:26-83), and the GEMM work list.
//
// The grouping is a one-pass stable counting sort over the expert id:
//   histogram (LDS integer counters: order-independent, so deterministic)
//   -> exclusive scan over experts
//   -> stable scatter: the rank of a route among equal ids before it comes from
//      wave64 ballots (a 'match any' built from one ballot per key bit) plus a
//      per-chunk scan of per-wave counts across the 16 waves, in wave order.
// The result is bit-exact np.argsort(flat, kind="stable") / np.bincount.
#include "moe_common.h"
#include "moe_kernels.h"
#include "router_wave.h"

namespace glm_moe {

namespace {

// Exclusive scan of one int per thread over a 1024-thread block.
// scratch holds kPlanWaves + 1 ints.  Returns the prefix; *total gets the sum.
__device__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  if (wave == 0) {
    const int t = lane < kPlanWaves ? scratch[lane] : 0;
    int s = t;
#pragma unroll
    for (int d = 1; d < kPlanWaves; d <<= 1) {
      const int y = __shfl_up(s, d, 64);
      if (lane >= d) s += y;
    }
    if (lane < kPlanWaves) scratch[lane] = s - t;
    if (lane == kPlanWaves - 1) scratch[kPlanWaves] = s;
  }
  __syncthreads();
  const int r = x - v + scratch[wave];
  *total = scratch[kPlanWaves];
  __syncthreads();
  return r;
}

// First work-list index of this thread's expert when experts are listed
// heaviest first (route count descending, ties by expert id): the tile list
// then falls in cost, and the prefill kernels deal it to the XCDs in a snake
// order, so that every XCD gets an even share of it.  c, nt: the routes and
// tiles of expert threadIdx.x (0 past E); s_free: 3 * E ints of free LDS.
// An expert's rank (its place in that order) is counted by `parts` threads,
// each over every parts-th expert, and summed with LDS atomics.
__device__ __forceinline__ int heavy_first_tile(int c, int nt, int E, int* s_free, int* s_scan, int* total) {
  const int tid = threadIdx.x;
  int* const s_cnt = s_free;           // [E] route counts, then list prefixes
  int* const s_rank = s_free + E;      // [E] places in the heaviest-first order
  int* const s_pos = s_free + 2 * E;   // [E] tiles of the expert at each place
  __syncthreads();  // the caller's last reads of the LDS reused here
  if (tid < E) {
    s_cnt[tid] = c;
    s_rank[tid] = 0;
  }
  __syncthreads();
  const int parts = E <= kPlanThreads / 4 ? 4 : (E <= kPlanThreads / 2 ? 2 : 1);
  const int i = tid / parts, part = tid % parts;
  if (i < E) {
    const int ci = s_cnt[i];
    int r = 0;
#pragma unroll 8
    for (int j = part; j < E; j += parts) {
      const int cj = s_cnt[j];
      r += (cj > ci) | ((cj == ci) & (j < i));
    }
    atomicAdd(&s_rank[i], r);
  }
  __syncthreads();
  const int rank = tid < E ? s_rank[tid] : 0;
  if (tid < E) s_pos[rank] = nt;
  __syncthreads();
  const int v = tid < E ? s_pos[tid] : 0;
  const int pre = block_exclusive_scan(v, s_scan, total);
  if (tid < E) s_cnt[tid] = pre;  // the prefix of list place tid
  __syncthreads();
  return tid < E ? s_cnt[rank] : 0;
}

// The work-list entries of expert e (c routes from sorted position start) from
// list index t0 on, in route order; a second listing follows its tile.  With
// a.tile_desc, each listing also gets the expert's descriptor {e, t0, start,
// c}: a prefill work item places its tile from that one 16-byte read.
__device__ __forceinline__ void write_tiles(const RoutePlanArgs& a, int e, int start, int c, int t0) {
  int idx = t0;
  for (int j = 0; j * a.tile_rows < c; ++j) {
    const int live = min(a.tile_rows, c - j * a.tile_rows);
    const int copies = a.wide_twice && live > a.tile_rows / 2 ? 2 : 1;
    for (int h = 0; h < copies; ++h, ++idx) {
      if (idx < a.max_tiles) {
        a.tile_expert[idx] = e;
        a.tile_row[idx] = start + j * a.tile_rows;
        a.tile_live[idx] = live | (h ? kTileSecondHalf : 0);
        if (a.tile_desc) *reinterpret_cast<int4*>(a.tile_desc + 4 * (int64_t)idx) = make_int4(e, t0, start, c);
      }
    }
  }
}

// Sort key of a raw route id: its owned (local) expert, or a.experts -- the key
// of the unowned routes, sorted after every owned expert and never tiled.
// For a whole layer (no unowned routes) this is the reference's safe id:
// valid ids as they are, invalid ones 0 (routed_experts.py:159-161).
__device__ __forceinline__ int plan_key(int raw, const RoutePlanArgs& a) {
  const int l = owned_expert(raw, a.own);
  return l >= 0 ? l : a.experts;
}

__device__ __forceinline__ bool id_valid(int raw, const RoutePlanArgs& a) {
  return raw >= 0 && raw < a.own.global_experts;
}

__global__ __launch_bounds__(kPlanThreads) void route_plan_kernel(const RoutePlanArgs a) {
  extern __shared__ int smem[];
  const int E = a.experts;
  const int KEYS = a.keys;
  const int ep = (KEYS + 63) & ~63;
  int* s_run = smem;                          // [ep] routes of each expert already placed
  int* s_off = s_run + ep;                    // [ep] exclusive offsets
  int* s_base = s_off + ep;                   // [ep] first position of an expert in this chunk
  int* s_scan = s_base + ep;                  // [kPlanWaves + 1]
  int* s_bad = s_scan + kPlanWaves + 1;       // [1]
  uint16_t* s_pre = reinterpret_cast<uint16_t*>(s_bad + 1);            // [kPlanWaves][ep] wave prefix in chunk
  uint8_t* s_wc = reinterpret_cast<uint8_t*>(s_pre + kPlanWaves * ep); // [kPlanWaves][ep] wave counts (<= 64)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int i = tid; i < ep; i += kPlanThreads) s_run[i] = 0;
  for (int i = tid; i < kPlanWaves * ep; i += kPlanThreads) s_wc[i] = 0;
  for (int i = tid; i < kPlanWaves * ep; i += kPlanThreads) s_pre[i] = 0;
  if (tid == 0) *s_bad = 0;
  __syncthreads();

  // histogram + range / weight validation
  for (int i = tid; i < a.n; i += kPlanThreads) {
    const int raw = a.ids[i];
    if (!id_valid(raw, a)) atomicOr(s_bad, 1);
    if (a.route_w) {
      const float w = a.route_w[i];
      if (!(w >= 0.0f) || isinf(w)) atomicOr(s_bad, 1);
    }
    atomicAdd(&s_run[plan_key(raw, a)], 1);
  }
  // duplicate ids within one token's row (raw ids, as the reference compares them)
  const int k = a.top_k;
  const int tokens = a.n / k;
  for (int t = tid; t < tokens; t += kPlanThreads) {
    const int32_t* row = a.ids + (int64_t)t * k;
    bool dup = false;
    for (int i = 0; i < k && !dup; ++i) {
      const int vi = row[i];
      for (int j = i + 1; j < k; ++j) {
        if (row[j] == vi) { dup = true; break; }
      }
    }
    if (dup) atomicOr(s_bad, 1);
  }
  __syncthreads();

  // counts and exclusive offsets (one key per thread; keys <= 1024); the
  // unowned key's offset is the number of owned routes
  {
    const int c = tid < KEYS ? s_run[tid] : 0;
    int total = 0;
    const int ex = block_exclusive_scan(c, s_scan, &total);
    if (tid < KEYS) {
      s_off[tid] = ex;
      s_run[tid] = 0;
    }
    if (tid < E) {
      a.counts[tid] = c;
      if (a.offsets) a.offsets[tid] = ex;
    }
    if (a.offsets && ((KEYS > E && tid == E) || (KEYS == E && tid == 0)))
      a.offsets[E] = KEYS > E ? ex : total;
  }
  __syncthreads();

  // stable scatter, one 1024-route chunk at a time in route order
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = 0; base < a.n; base += kPlanThreads) {
    const int i = base + tid;
    const bool act = i < a.n;
    const int e = act ? plan_key(a.ids[i], a) : 0;
    uint64_t peers = __ballot(act);
    for (int b = 0; b < a.key_bits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint64_t before = peers & lt_mask;
    const int rank = __popcll(before);
    if (act && before == 0) s_wc[wave * ep + e] = (uint8_t)__popcll(peers);
    __syncthreads();
    // per key: prefix over waves (in wave order), then advance the running count
    for (int x = tid; x < KEYS; x += kPlanThreads) {
      int acc = 0;
      for (int w = 0; w < kPlanWaves; ++w) {
        const int c = s_wc[w * ep + x];
        s_pre[w * ep + x] = (uint16_t)acc;
        s_wc[w * ep + x] = 0;
        acc += c;
      }
      s_base[x] = s_off[x] + s_run[x];
      s_run[x] += acc;
    }
    __syncthreads();
    if (act) {
      const int pos = s_base[e] + s_pre[wave * ep + e] + rank;
      if (pos >= 0 && pos < a.n) a.sorted[pos] = i;  // always true for a consistent plan
      if (a.inverse) a.inverse[i] = pos;
    }
  }

  const bool bad = *s_bad != 0;
  if (tid == 0) a.valid[0] = bad ? 0 : 1;

  // GEMM work list: ceil(count / tile_rows) tiles per expert, expert-major,
  // heaviest expert first
  if (a.tile_rows > 0) {
    const int c = tid < E ? a.counts[tid] : 0;  // written above by this thread
    const int nt = tiles_of_count(c, a.tile_rows, a.wide_twice);
    int total = 0;
    int* s_free = reinterpret_cast<int*>(s_pre);  // [kPlanWaves][ep] u16, free once the scatter is done
    const int t0 = heavy_first_tile(c, nt, E, s_free, s_scan, &total);
    if (tid < E) {
      const int start = s_off[tid];
      write_tiles(a, tid, start, c, t0);
    }
    // An invalid route set is still planned with its safe ids (invalid -> 0),
    // as the reference computes it; only the health byte reports it.
    if (tid == 0) a.tile_count[0] = min(total, a.max_tiles);
  }
}

// ---------------------------------------------------------------------------
// The same grouping over many workgroups, for large route sets: the routes are
// cut into chunks of whole token rows; pass 1 counts every chunk's experts
// (order-independent LDS counters) and checks its rows; pass 2 gives every
// chunk its starting position per expert -- the expert's offset plus the
// counts of the earlier chunks -- and scatters the chunk exactly as the
// one-workgroup kernel does (ballot ranks, wave-order prefixes).  Chunk 0 also
// writes counts, offsets, health and the GEMM work list.  Bit-exact with the
// one-workgroup kernel: the position of a route depends only on the routes
// before it.
__global__ __launch_bounds__(kPlanThreads) void route_hist_kernel(const RoutePlanArgs a) {
  __shared__ int s_count[kMaxExperts];
  __shared__ int s_bad;
  const int KEYS = a.keys, tid = threadIdx.x, c = blockIdx.x;
  const int begin = c * a.chunk, end = min(a.n, begin + a.chunk);
  for (int i = tid; i < KEYS; i += kPlanThreads) s_count[i] = 0;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  for (int i = begin + tid; i < end; i += kPlanThreads) {
    const int raw = a.ids[i];
    bool bad = !id_valid(raw, a);
    if (a.route_w) {
      const float w = a.route_w[i];
      bad |= !(w >= 0.0f) || isinf(w);
    }
    if (bad) atomicOr(&s_bad, 1);
    atomicAdd(&s_count[plan_key(raw, a)], 1);
  }
  // duplicate ids within one token's row (a chunk holds whole rows)
  const int k = a.top_k;
  for (int t = begin / k + tid; t < end / k; t += kPlanThreads) {
    const int32_t* row = a.ids + (int64_t)t * k;
    bool dup = false;
    for (int i = 0; i < k && !dup; ++i)
      for (int j = i + 1; j < k; ++j)
        if (row[j] == row[i]) { dup = true; break; }
    if (dup) atomicOr(&s_bad, 1);
  }
  __syncthreads();
  for (int e = tid; e < KEYS; e += kPlanThreads) a.chunk_hist[(int64_t)c * KEYS + e] = s_count[e];
  if (tid == 0) a.chunk_bad[c] = s_bad;
}

// The first pass of the grouping for routes that come from router logits: the
// noaux_tc routing of route_noaux_tc_kernel (one wave per token, the same
// device code, so the same ids and weights) fused with route_hist_kernel's
// counting and row checks.  A workgroup routes kRouterHistTokens tokens,
// writes their ids and weights, and writes its histogram row and health
// (duplicate ids in a token's row, ids out of range, weights not finite and
// >= 0 when checked, as route_hist_kernel checks them) -- the ids and weights
// are not read back.  Routing stays spread over the whole GPU, one wave per
// token; counting a whole 2048-route chunk inside one workgroup's routing was
// measured slower than the separate router kernel at every size.
template <int KPER>
__global__ __launch_bounds__(64 * kRouterHistTokens) void route_hist_from_logits_kernel(const RoutePlanArgs a,
                                                                                       const RouterPass r) {
  __shared__ int s_count[kMaxExperts];
  __shared__ int s_bad;
  const int KEYS = a.keys, tid = threadIdx.x, lane = tid & 63, row = blockIdx.x;
  for (int i = tid; i < KEYS; i += 64 * kRouterHistTokens) s_count[i] = 0;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  const int64_t t = (int64_t)row * kRouterHistTokens + (tid >> 6);
  if (t < r.tokens) {
    int id;
    float w;
    route_token_noaux<KPER>(r.logits + t * r.experts, r.experts, r.bias, a.top_k, lane, id, w);
    if (lane < a.top_k) {
      r.ids[t * a.top_k + lane] = id;
      r.weights[t * a.top_k + lane] = w;
    }
    bool bad = false;
    for (int s = 0; s < a.top_k; ++s) {
      const int other = __shfl(id, s, 64);
      bad |= s < lane && other == id;  // a duplicate of an earlier slot of the row
    }
    if (lane < a.top_k) {
      bad |= !id_valid(id, a);
      if (a.route_w) bad |= !(w >= 0.0f) || isinf(w);
      atomicAdd(&s_count[plan_key(id, a)], 1);
    }
    if (__ballot(lane < a.top_k && bad) != 0 && lane == 0) atomicOr(&s_bad, 1);
  }
  __syncthreads();
  for (int e = tid; e < KEYS; e += 64 * kRouterHistTokens) a.chunk_hist[(int64_t)row * KEYS + e] = s_count[e];
  if (tid == 0) a.chunk_bad[row] = s_bad;
}

// Histogram rows: `rows` rows of keys counts, rows_per_chunk of them per chunk
// (one per chunk after route_hist_kernel; one per router workgroup of
// kRouterHistTokens tokens after route_hist_from_logits_kernel).
__global__ __launch_bounds__(kPlanThreads) void route_scatter_kernel(const RoutePlanArgs a, int chunks, int rows,
                                                                     int rows_per_chunk) {
  extern __shared__ int smem[];
  const int E = a.experts;
  const int KEYS = a.keys;
  const int ep = (KEYS + 63) & ~63;
  int* s_run = smem;                          // [ep] routes of each expert placed by this chunk so far
  int* s_off = s_run + ep;                    // [ep] first position of each expert for this chunk
  int* s_base = s_off + ep;                   // [ep] first position of an expert in this sub-chunk
  int* s_scan = s_base + ep;                  // [kPlanWaves + 1]
  int* s_bad = s_scan + kPlanWaves + 1;       // [1]
  uint16_t* s_pre = reinterpret_cast<uint16_t*>(s_bad + 1);
  uint8_t* s_wc = reinterpret_cast<uint8_t*>(s_pre + kPlanWaves * ep);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = blockIdx.x;
  const int begin = c * a.chunk, end = min(a.n, begin + a.chunk);

  for (int i = tid; i < kPlanWaves * ep; i += kPlanThreads) {
    s_wc[i] = 0;
    s_pre[i] = 0;
  }
  if (tid == 0) *s_bad = 0;
  // per key: the counts of the earlier chunks and the total (column sums)
  int before = 0, total_e = 0;
  if (tid < KEYS) {
    const int first = c * rows_per_chunk;
#pragma unroll 8
    for (int q = 0; q < rows; ++q) {
      const int v = a.chunk_hist[(int64_t)q * KEYS + tid];
      before += q < first ? v : 0;
      total_e += v;
    }
  }
  int total = 0;
  const int ex = block_exclusive_scan(tid < KEYS ? total_e : 0, s_scan, &total);
  if (tid < KEYS) {
    s_off[tid] = ex + before;
    s_run[tid] = 0;
  }
  if (c == 0) {
    if (tid < E) {
      a.counts[tid] = total_e;
      if (a.offsets) a.offsets[tid] = ex;
    }
    // the unowned key's offset is the number of owned routes
    if (a.offsets && ((KEYS > E && tid == E) || (KEYS == E && tid == 0)))
      a.offsets[E] = KEYS > E ? ex : total;
    for (int q = tid; q < rows; q += kPlanThreads)
      if (a.chunk_bad[q]) atomicOr(s_bad, 1);
  }
  __syncthreads();

  // stable scatter of this chunk, 1024 routes at a time in route order
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int sub = begin; sub < end; sub += kPlanThreads) {
    const int i = sub + tid;
    const bool act = i < end;
    const int e = act ? plan_key(a.ids[i], a) : 0;
    uint64_t peers = __ballot(act);
    for (int b = 0; b < a.key_bits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint64_t before_lane = peers & lt_mask;
    const int rank = __popcll(before_lane);
    if (act && before_lane == 0) s_wc[wave * ep + e] = (uint8_t)__popcll(peers);
    __syncthreads();
    for (int x = tid; x < KEYS; x += kPlanThreads) {
      int acc = 0;
      for (int w = 0; w < kPlanWaves; ++w) {
        const int cnt = s_wc[w * ep + x];
        s_pre[w * ep + x] = (uint16_t)acc;
        s_wc[w * ep + x] = 0;
        acc += cnt;
      }
      s_base[x] = s_off[x] + s_run[x];
      s_run[x] += acc;
    }
    __syncthreads();
    if (act) {
      const int pos = s_base[e] + s_pre[wave * ep + e] + rank;
      if (pos >= 0 && pos < a.n) a.sorted[pos] = i;  // always true for a consistent plan
      if (a.inverse) a.inverse[i] = pos;
    }
  }
  if (c != 0) return;
  __syncthreads();
  if (tid == 0) a.valid[0] = *s_bad ? 0 : 1;
  if (a.tile_rows > 0) {
    const int cnt = tid < E ? total_e : 0;
    const int nt = tiles_of_count(cnt, a.tile_rows, a.wide_twice);
    int tiles = 0;
    int* s_free = reinterpret_cast<int*>(s_pre);  // [kPlanWaves][ep] u16, free once the scatter is done
    const int t0 = heavy_first_tile(cnt, nt, E, s_free, s_scan, &tiles);
    if (tid < E) {
      const int start = ex;
      write_tiles(a, tid, start, cnt, t0);
    }
    if (tid == 0) a.tile_count[0] = min(tiles, a.max_tiles);
  }
}

// build_expert_panels (panels.py:26-83) for groups <= 1024 on one block.
__global__ __launch_bounds__(kPlanThreads) void panel_plan_kernel(const PanelPlanArgs a) {
  __shared__ int64_t s_ends[kMaxExperts];        // inclusive prefix of masked counts
  __shared__ int64_t s_panel_ends[kMaxExperts];  // inclusive prefix of local panel counts
  __shared__ int s_scan[kPlanWaves + 1];
  __shared__ int s_bad;
  __shared__ long long s_sum;
  const int tid = threadIdx.x;
  const int G = a.groups, L = a.local_groups, PR = a.panel_rows;
  if (tid == 0) { s_bad = 0; s_sum = 0; }
  __syncthreads();
  const int size = tid < G ? a.group_sizes[tid] : 0;
  if (tid < G && (size < 0 || size > a.rows)) atomicOr(&s_bad, 1);
  if (tid < G) atomicAdd((unsigned long long*)&s_sum, (unsigned long long)(long long)size);
  __syncthreads();
  const int offset_raw = a.group_offset[0];
  const bool valid = s_bad == 0 && s_sum == (long long)a.rows && offset_raw >= 0 &&
                     offset_raw <= G - L;
  const int offset = min(max(offset_raw, 0), G - L);
  // ends = cumsum(where(valid, sizes, 0)); counts are in [0, rows] when valid
  int total = 0;
  const int c = valid ? size : 0;
  const int ex = block_exclusive_scan(c, s_scan, &total);
  if (tid < G) s_ends[tid] = (int64_t)ex + c;
  __syncthreads();
  // local panel counts and their inclusive prefix
  const int lc = tid < L ? (int)(s_ends[offset + tid] - (offset + tid > 0 ? s_ends[offset + tid - 1] : 0)) : 0;
  const int pc = (lc + PR - 1) / PR;
  int ptotal = 0;
  const int pex = block_exclusive_scan(pc, s_scan, &ptotal);
  if (tid < L) s_panel_ends[tid] = (int64_t)pex + pc;
  __syncthreads();
  const int64_t last_panel_end = s_panel_ends[L - 1];
  auto start_of = [&](int g) -> int64_t { return g > 0 ? s_ends[g - 1] : 0; };
  auto panel_start_of = [&](int j) -> int64_t { return j > 0 ? s_panel_ends[j - 1] : 0; };
  for (int p = tid; p < a.capacity; p += kPlanThreads) {
    // searchsorted(panel_ends, p, side="right"): number of local groups with end <= p
    int lo = 0, hi = L;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_panel_ends[mid] <= p) lo = mid + 1; else hi = mid;
    }
    const int expert = min(lo, L - 1);
    const int64_t within = ((int64_t)p - panel_start_of(expert)) * PR;
    const bool active = p < last_panel_end;
    const int64_t lcount = s_ends[offset + expert] - start_of(offset + expert);
    a.expert_ids[p] = active ? expert : 0;
    a.row_starts[p] = active ? (int32_t)(start_of(offset + expert) + within) : 0;
    int64_t live = lcount - within;
    live = live < 0 ? 0 : (live > PR ? PR : live);
    a.live_counts[p] = active ? (int32_t)live : 0;
  }
  for (int r = tid; r < a.rows; r += kPlanThreads) {
    int lo = 0, hi = G;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_ends[mid] <= r) lo = mid + 1; else hi = mid;
    }
    const int re = min(lo, G - 1);
    const bool owned = valid && re >= offset && re < offset + L;
    const int lre = min(max(re - offset, 0), L - 1);
    const int64_t rel = (int64_t)r - start_of(re);
    const int64_t restore = panel_start_of(lre) * PR + rel;
    a.restore_indices[r] = owned ? (int32_t)restore : 0;
    a.owned_rows[r] = owned ? 1 : 0;
  }
  if (tid == 0) {
    a.active_panels[0] = (int32_t)last_panel_end;
    a.valid[0] = valid ? 1 : 0;
  }
}

// Owned slots first, in slot order, as one-row tiles; ids clipped to [0, E).
__global__ void slot_tiles_kernel(const int32_t* ids, const uint8_t* owned, int slots, int experts,
                                  int32_t* tile_expert, int32_t* tile_row, int32_t* tile_live,
                                  int32_t* tile_count) {
  if (threadIdx.x != 0) return;
  int n = 0;
  for (int s = 0; s < slots; ++s) {
    if (!owned[s]) continue;
    const int e = min(max(ids[s], 0), experts - 1);
    tile_expert[n] = e;
    tile_row[n] = s;
    tile_live[n] = 1;
    ++n;
  }
  tile_count[0] = n;
}

}  // namespace

int route_plan_chunks(int32_t n, int32_t top_k) {
  const int chunk = (kPlanChunkRoutes / top_k) * top_k;
  return (n + chunk - 1) / chunk;
}

hipError_t launch_route_plan(const RoutePlanArgs& a, hipStream_t stream) {
  if (a.own.experts != a.experts || a.keys < a.experts || a.keys > kMaxExperts ||
      (a.keys == a.experts && may_leave_routes_unowned(a.own)) || (1 << a.key_bits) < a.keys)
    return hipErrorInvalidValue;
  const int ep = (a.keys + 63) & ~63;
  // int32 run/off/base + scan + flag, uint16 wave prefixes, uint8 wave counts:
  // 60 KB at 1024 experts, 15 KB at 256.
  const size_t lds = sizeof(int) * (size_t)(3 * ep + kPlanWaves + 2) +
                     sizeof(uint16_t) * (size_t)kPlanWaves * ep + (size_t)kPlanWaves * ep;
  const int chunks = route_plan_chunks(a.n, a.top_k);
  if (a.chunk_hist == nullptr || a.chunk_bad == nullptr || chunks <= 1) {
    label_next_launch("group_prefill_routes_r%d_e%d_tm%d", a.n, a.experts, a.tile_rows);
    return launch_kernel(route_plan_kernel, dim3(1), dim3(kPlanThreads), lds, stream, a);
  }
  RoutePlanArgs b = a;
  b.chunk = (kPlanChunkRoutes / a.top_k) * a.top_k;
  // the stage timer (if armed) measures the scatter pass: the plan's last kernel
  const LaunchEvents armed = next_launch_events();
  next_launch_events() = LaunchEvents{};
  label_next_launch("group_prefill_routes_hist_r%d_e%d", a.n, a.experts);
  hipError_t err = launch_kernel(route_hist_kernel, dim3(chunks), dim3(kPlanThreads), 0, stream, b);
  if (err != hipSuccess) return err;
  next_launch_events() = armed;
  label_next_launch("group_prefill_routes_scatter_r%d_e%d_tm%d", a.n, a.experts, a.tile_rows);
  return launch_kernel(route_scatter_kernel, dim3(chunks), dim3(kPlanThreads), lds, stream, b, chunks, chunks, 1);
}

// Chunks of the fused path: whole router workgroups of tokens, about 2048 routes.
static int64_t fused_chunk_tokens(int32_t top_k) {
  return (int64_t)(kPlanChunkRoutes / top_k) / kRouterHistTokens * kRouterHistTokens;
}

int64_t route_plan_hist_rows(int64_t tokens, int32_t top_k) {
  const int64_t chunks = route_plan_chunks((int32_t)(tokens * top_k), top_k);
  const int64_t router_rows = (tokens + kRouterHistTokens - 1) / kRouterHistTokens;
  return chunks > router_rows ? chunks : router_rows;
}

hipError_t launch_route_plan_from_logits(const RoutePlanArgs& a, const RouterPass& r, hipStream_t stream) {
  if (a.top_k <= 0 || a.n % a.top_k != 0 || r.tokens != a.n / a.top_k || r.ids != a.ids ||
      r.experts <= 0 || r.experts > kMaxExperts || a.top_k > kWave || a.top_k > r.experts)
    return hipErrorInvalidValue;
  const int64_t ct = fused_chunk_tokens(a.top_k);
  if (a.chunk_hist == nullptr || a.chunk_bad == nullptr || route_plan_chunks(a.n, a.top_k) <= 1 || ct <= 0) {
    // one workgroup plans everything: the router kernel ahead of it
    const LaunchEvents armed = next_launch_events();
    next_launch_events() = LaunchEvents{};
    hipError_t err = launch_route_noaux_tc(r.logits, r.tokens, r.experts, r.bias, a.top_k, r.ids, r.weights, stream);
    if (err != hipSuccess) return err;
    next_launch_events() = armed;
    return launch_route_plan(a, stream);
  }
  if (a.own.experts != a.experts || a.keys < a.experts || a.keys > kMaxExperts ||
      (a.keys == a.experts && may_leave_routes_unowned(a.own)) || (1 << a.key_bits) < a.keys)
    return hipErrorInvalidValue;
  const int ep = (a.keys + 63) & ~63;
  const size_t lds = sizeof(int) * (size_t)(3 * ep + kPlanWaves + 2) +
                     sizeof(uint16_t) * (size_t)kPlanWaves * ep + (size_t)kPlanWaves * ep;
  RoutePlanArgs b = a;
  b.chunk = (int32_t)(ct * a.top_k);
  const int chunks = (int)((r.tokens + ct - 1) / ct);
  const int rows = (int)((r.tokens + kRouterHistTokens - 1) / kRouterHistTokens);
  const LaunchEvents armed = next_launch_events();
  next_launch_events() = LaunchEvents{};
  label_next_launch("route_glm_noaux_tc_hist_t%lld_e%d_k%d", (long long)r.tokens, r.experts, a.top_k);
  hipError_t err =
      r.experts <= 256
          ? launch_kernel(route_hist_from_logits_kernel<4>, dim3(rows), dim3(64 * kRouterHistTokens), 0, stream, b, r)
          : launch_kernel(route_hist_from_logits_kernel<kMaxExperts / 64>, dim3(rows), dim3(64 * kRouterHistTokens), 0,
                          stream, b, r);
  if (err != hipSuccess) return err;
  next_launch_events() = armed;
  label_next_launch("group_prefill_routes_scatter_r%d_e%d_tm%d", a.n, a.experts, a.tile_rows);
  return launch_kernel(route_scatter_kernel, dim3(chunks), dim3(kPlanThreads), lds, stream, b, chunks, rows,
                       (int)(ct / kRouterHistTokens));
}

hipError_t launch_panel_plan(const PanelPlanArgs& a, hipStream_t stream) {
  label_next_launch("build_expert_panels_r%d_g%d_p%d", a.rows, a.groups, a.panel_rows);
  return launch_kernel(panel_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, a);
}

hipError_t launch_slot_tiles(const int32_t* local_ids, const uint8_t* owned, int32_t slots,
                             int32_t experts, int32_t* tile_expert, int32_t* tile_row,
                             int32_t* tile_live, int32_t* tile_count, hipStream_t stream) {
  label_next_launch("fp8_routed_projection_plan_s%d", slots);
  return launch_kernel(slot_tiles_kernel, dim3(1), dim3(64), 0, stream, local_ids, owned, slots,
                     experts, tile_expert, tile_row, tile_live, tile_count);
}

}  // namespace glm_moe
