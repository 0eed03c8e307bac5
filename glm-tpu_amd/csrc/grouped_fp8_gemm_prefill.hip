// Prefill route-grouped FP8 projection: tiles of up to 256 sorted routes (bf16
// kernel) or 128 (native FP8 kernel).
//
// Same arithmetic as every projection of this library (weights decoded as
// bf16(f32(e4m3) * block scale), bf16 activations, FP32 accumulation over
// ascending 128-wide K blocks on v_mfma_f32_16x16x32_bf16) -- the projection
// of glm-tpu's prefill_panel_fp8_matmul (reference
// glm_tpu/kernels/fp8_grouped_matmul/panel_kernel.py:83-101).
//
// Work item = (expert, tile of <= 256 / 128 sorted routes, run of stripes of BN
// weight rows; the FP8 kernel runs up to kMaxStripeRun stripes per item).
//   * Each of the 8 waves owns RG x 16 rows of every table of the stripe
//     (32 KB of e4m3 bytes per K block for the work item; 64 KB on the bf16
//     kernel's tall stripes, 512 rows: 32 gate + 32 up or 64 down rows a
//     wave, so every activation fragment read from LDS feeds twice the MFMAs
//     -- T=2048 layer -5 %).  The rows go HBM -> LDS with direct-to-LDS
//     buffer loads (no registers), 8 rows x 128 bytes per instruction (whole
//     lines), into a ring of blocks private to the wave, so 64-128 KB per CU
//     stay in flight; chunk c of row r sits in slot c ^ (r % 8) so the
//     MFMA-layout reads hit distinct banks.  Every byte is decoded once per
//     work item, one 32-wide K step ahead of the MFMAs that use it.
//   * The tile's activation rows (gathered token rows for gate/up, sorted
//     activation rows for down) go HBM/L2 -> LDS the same way into a ring of
//     SX stages shared by all waves as the B operand; each 1 KB load covers 4
//     rows x 256 bytes, chunk c of row r in slot c ^ (r % 16).
//   * One workgroup barrier per K block: after it the block's rows are in LDS
//     and every wave is done with the previous block, whose slots are refilled.
//     Ring slots are runtime indices, so any K / 128 <= 64 works; blocks past
//     the last are loaded out of range (no traffic) to keep wait counts exact.
//   * One code variant per count of 16-route column groups (1..8), each with
//     its own accumulators, ring depths and epilogue; wide tiles (9..16
//     groups) and, on tall stripes, tiles of 5..8 groups stage the
//     activations in half K blocks.  On tall stripes a wide tile is listed
//     twice by the plan and each listing takes one 256-row half of the
//     stripe (the accumulators of all 512 rows would not fit in registers).
// Work items are ordered expert-major, heaviest expert first (the plan lists
// experts by route count, descending), then in blocks of route tiles x
// stripes (item_of_expert), and dealt to the XCDs in chunks of 32 consecutive
// items (one per CU of an XCD; workgroup b runs on XCD b % 8): chunk c goes to
// XCD c % 8 in even rounds of 8 chunks and 7 - c % 8 in odd ones (a snake), so
// the tiles that share an expert's weight stripe (hot experts) and the stripes
// that share a tile's activation rows run together on one XCD, and, the list
// falling in cost, every XCD gets an even share of it (whole eighths of the
// list left the XCD holding the cold tail idle for a third of a T=8192 Zipf
// launch).
#include <atomic>
#include <type_traits>

#include "gemm_epilogue.h"
#include "moe_common.h"
#include "moe_kernels.h"

namespace glm_moe {

namespace {

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

constexpr int kNonTemporal = 2;             // buffer load cache policy: streamed once (nt)
constexpr int kBufferFormat = 0x00020000;   // raw buffer descriptor word 3: 32-bit data format

constexpr int kBM = 128;           // routes per tile of the FP8 kernel (and of the bf16 kernel's narrow variants)
constexpr int kXcds = 8;           // MI355X: 8 XCDs, workgroups dealt round-robin
constexpr int kChunk = 32;         // work items dealt to an XCD together: one per CU

// Work item of workgroup b (-1: none) when `total` items are dealt in chunks:
// the q-th workgroup of XCD x = b % 8 runs item (j * 8 + x') * 32 + q % 32 with
// j = q / 32 and x' = x for even j, 7 - x for odd j.  Each XCD runs `per`
// workgroups, a whole number of chunks.
__device__ __forceinline__ int xcd_item(int b, int total) {
  const int chunks = (total + kChunk - 1) / kChunk;
  const int per = (chunks + kXcds - 1) / kXcds * kChunk;
  const int q = b / kXcds;
  if (q >= per) return -1;
  const int j = q / kChunk, x = b % kXcds;
  return (j * kXcds + ((j & 1) ? kXcds - 1 - x : x)) * kChunk + q % kChunk;
}
// Stripes one work item runs: a.stripe_run, clamped to 1 .. kMaxStripeRun,
// and 1 when K has fewer than kMinRunBlocks blocks (the rings look up to 3
// blocks ahead; from 4 blocks on that reaches no further than the next
// stripe's first blocks).  The host sizes the grid with the same function.
// A run's stripes share the tile's activation rows and one continuous ring:
// the next stripe's first blocks are loaded during the current stripe's last
// blocks and its epilogue, in place of a workgroup's start and end.  Measured
// (FP8 layer): down with 4 stripes -8.5 % at T=8192 Zipf, -2.5 % at T=2048;
// gate/up with 2 no better (its K loops slow down as the idle time between
// items goes: the stream is near the HBM limit).  The bf16 kernel runs one
// stripe per item: the same rewrite of it measured 1.3 % slower at T=2048
// (longer item start) for 1.1 % at T=8192 Zipf.  On tall stripes (512 rows)
// both kernels run one stripe per item.
constexpr int kMaxStripeRun = 4;
constexpr int kMinRunBlocks = 4;
constexpr int kRunGateUp = 1;
constexpr int kRunDown = 4;
__host__ __device__ __forceinline__ int stripe_run_of(const GroupedGemmArgs& a) {
  if (a.k / kScaleBlock < kMinRunBlocks) return 1;
  return a.stripe_run < 1 ? 1 : (a.stripe_run > kMaxStripeRun ? kMaxStripeRun : a.stripe_run);
}

// p with both halves marked workgroup-uniform: a buffer descriptor built from
// it stays in scalar registers (one the compiler takes for divergent costs
// every load a loop over the lanes).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return reinterpret_cast<T*>((hi << 32) | lo);
}

// Workgroups of a launch over at most `items` work items: every XCD's whole
// chunks of the largest work list.
inline int64_t prefill_grid(int64_t items) {
  return (items + kXcds * kChunk - 1) / (kXcds * kChunk) * (kXcds * kChunk);
}
constexpr int kRowBytes = kScaleBlock * 2;   // one staged activation row of a K block (bf16)

// Work items of one expert (runs of stripes x nt route tiles; a run is one
// stripe unless the kernel runs several per item), in the order an XCD walks
// them: tile blocks of kTileBlock tiles, each over every run, each run over
// the block's tiles.  Consecutive items -- the ones an XCD's CUs run together
// -- then share kTileBlock activation tiles and ~32 / kTileBlock weight
// stripes.  An expert with one tile (uniform prefill) walks its runs over the
// same activation rows.  On tall stripes a wide tile's two listings share
// its rows, so a block holds 8 listings: again 4 tiles and ~32 / 4 half
// stripes per 32 items.
constexpr int kTileBlock = 4;
// The FP8 kernel's tile blocks: 16 tiles of 128 routes, so a block of a hot
// expert spans several chunks (XCDs), each running the 16 tiles over two runs
// (GLM-5 shape on tall stripes: gate/up 8 runs, 4 chunks; down 12 runs, 6).
// Its K loop takes half the bf16 kernel's time per weight byte, so the
// re-reads of a hot expert's stripes by every tile block cost more: blocks of
// 16 tiles read each stripe a quarter as often as blocks of 4, for more
// activation reads (T=8192 Zipf FP8 layer -2..3 %; blocks of 8: -1.5 %; the
// bf16 kernel gains nothing from larger blocks).
constexpr int kTileBlockFp8 = 16;

template <int TB = kTileBlock>
__device__ __forceinline__ void item_of_expert(int rel, int runs, int nt, int& run, int& tile) {
  const int tb = rel / (runs * TB);
  const int first = tb * TB;
  const int bs = min(TB, nt - first);
  const int r = rel - tb * runs * TB;
  run = r / bs;
  tile = first + r % bs;
}

__device__ __forceinline__ void wait_all_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The listings of the launch's work list, 0 when the plan reported bad routes
// (the health byte read through its aligned dword, a scalar load; the count
// stands in when there is no health byte).
__device__ __forceinline__ int healthy_listings(const GroupedGemmArgs& a) {
  const int mis = (int)(reinterpret_cast<uintptr_t>(a.valid) & 3);
  const uint32_t* word = a.valid != nullptr ? reinterpret_cast<const uint32_t*>(a.valid - mis)
                                            : reinterpret_cast<const uint32_t*>(a.tile_count);
  const uint32_t health = *word;
  const int listings = *a.tile_count;
  return a.valid == nullptr || ((health >> (8 * mis)) & 0xFFu) != 0 ? listings : 0;
}

// A work item's expert from its listing's descriptor (expert e, first listing
// t0, first sorted position, routes; RoutePlanArgs::tile_desc) -- one 16-byte
// load -- and then its tile: listing rel of the expert's nt is tile rel
// (rel / 2 when wide tiles are listed twice, the second listing when rel is
// odd), the sorted rows r0 .. r0 + live - 1, exactly as the plan lists them.
// False for a descriptor that cannot come from a consistent plan.
struct ItemTile {
  int e, t0, nt, start, count;  // the expert's
  int half, live;               // the item's tile
  int64_t r0;
};
__device__ __forceinline__ bool item_expert(const GroupedGemmArgs& a, int listing, ItemTile& t) {
  listing = uniform(listing);
  const int4 d = *reinterpret_cast<const int4*>(a.tile_desc + 4 * (int64_t)listing);
  t.e = uniform(d.x);
  t.t0 = uniform(d.y);
  t.start = uniform(d.z);
  t.count = uniform(d.w);
  if (t.e < 0 || t.e >= a.experts || t.t0 < 0 || t.t0 > listing || t.start < 0 || t.count <= 0) return false;
  t.nt = tiles_of_count(t.count, a.tile_rows, a.wide_twice);
  return listing < t.t0 + t.nt;
}
__device__ __forceinline__ void item_place(const GroupedGemmArgs& a, int rel, ItemTile& t) {
  const int j = a.wide_twice ? rel >> 1 : rel;
  t.half = a.wide_twice ? rel & 1 : 0;
  t.r0 = (int64_t)t.start + (int64_t)j * a.tile_rows;
  t.live = min(a.tile_rows, t.count - j * a.tile_rows);
}

// This wave's loads but the newest N have completed (direct-to-LDS loads
// included: their data is in LDS).  Unlike __syncthreads() the waits below
// leave later loads in flight, so the weight and activation prefetches of
// later K blocks stay in flight across the barrier.  Inline asm with a memory
// clobber: the compiler moves no memory access across it.
template <int N>
__device__ __forceinline__ void wait_loads() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The workgroup barrier alone: no wait for outstanding loads or LDS reads.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// Output rows of the lane's route columns r0 + cg * 16 + lrow, as stored (the
// epilogue checks them: out_row()).  The loads are unconditional (padding
// columns read column 0's entry) and issued together; nothing uses them
// before the epilogue, so nothing waits for them before it.
template <int NCG>
__device__ __forceinline__ void load_out_rows(const GroupedGemmArgs& a, int r0, int live, int lrow, int (&orow)[NCG]) {
  int r[NCG];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) r[cg] = r0 + (cg * 16 + lrow < live ? cg * 16 + lrow : 0);
  if (a.out_row_ids != nullptr) {
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) orow[cg] = a.out_row_ids[r[cg]];
  } else {
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) orow[cg] = r[cg];
  }
}

// The output row of column `col` given load_out_rows' entry, or -1 (padding
// column, or a row outside the output).
__device__ __forceinline__ int64_t out_row(const GroupedGemmArgs& a, int col, int live, int stored) {
  return col < live && stored >= 0 && stored < a.out_rows ? stored : -1;
}



// 16 bytes a lane from rsrc + voffset + soffset straight into LDS at
// lds + 16 * lane (buffer_load_dwordx4 ... lds).  The builtin only exists for
// the device target; the host pass of the kernel template must not see it.
// AUX is the cache policy (kNonTemporal for bytes that are read only once).
template <int AUX = 0>
__device__ __forceinline__ void load_lds_16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, int voffset, int soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset,
                                           0, AUX);
#endif
}

constexpr int kStripeBlockBytes = 32768;  // e4m3 bytes of 256 weight rows per K block
constexpr int kTallBlockBytes = 65536;    // e4m3 bytes of 512 weight rows per K block
constexpr int kPrefillLds = 160 * 1024;  // the whole LDS of a CU

// The epilogue of a work item, through LDS: every wave writes its output
// fragments (the epilogue's bf16 values: SwiGLU of the two tables, or the one
// table rounded) into an image of the tile's route rows, OUT outputs each,
// and the workgroup then stores every route row as 16-byte pieces, 8 lanes a
// 128-byte line, so each line of the output is written whole by one
// instruction, with the non-temporal hint (the rows are read once, by the
// next kernel).  Stored straight from the MFMA layout (16 route rows x 32
// bytes an instruction) with ordinary stores, each output line reached the
// L2 as 32-byte pieces from four instructions of two waves, and the layer's
// output writes slowed the weight stream that runs beside them: against a
// timing variant whose stores stay in L2, T=2048 prefill was 7 % (bf16) and
// 15 % (FP8 mode) slower.  Whole lines with the hint recover most of that
// (T=2048 layer -2..-3 %, FP8 mode -8 %, T=8192 Zipf -2 %); whole lines
// without it, or the hint on the scattered stores, do not.  Output column
// of fragment (wave, rg, lane): n_item + wave * RGS * 16 + rg * 16 +
// (lane / 16) * 4 .. + 3.  The caller has waited for its last direct-to-LDS
// loads; the first barrier waits for every wave's last reads of the rings.
template <int NCG, int RGS, int TABLES, int EPI, int WAVES>
__device__ __forceinline__ void store_tile_lines(const GroupedGemmArgs& a, uint8_t* lds,
                                                 const f32x4 (&acc)[TABLES][RGS][NCG], const int (&orow)[NCG],
                                                 int live, int wave, int lane, int64_t n_item) {
  static_assert(EPI == kEpiSwiglu || EPI == kEpiStoreBf16, "the prefill epilogues store bf16");
  constexpr int OUT = WAVES * RGS * 16;  // outputs of one route row in this work item
  constexpr int ROWS = NCG * 16;
  constexpr int PITCH = OUT * 2 + 16;    // staged row bytes: +16 puts a fragment's 16 rows in distinct banks
  constexpr int LPR = OUT * 2 / 16;      // 16-byte pieces of a route row
  static_assert(ROWS * PITCH + ROWS * 4 <= kPrefillLds, "the staged tile fits the LDS");
  static_assert((LPR & (LPR - 1)) == 0, "pieces per row: a power of two");
  const int lrow = lane & 15, lgrp = lane >> 4;
  int* const srow = reinterpret_cast<int*>(lds + ROWS * PITCH);
  __syncthreads();  // every wave is done with the rings
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
    for (int rg = 0; rg < RGS; ++rg) {
      const f32x4& g = acc[0][rg][cg];
      const f32x4& u = acc[TABLES - 1][rg][cg];
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[j] = EPI == kEpiSwiglu ? swiglu_bf16(round_to_bf16(g[j]), round_to_bf16(u[j])) : g[j];
      *reinterpret_cast<u32x2*>(lds + (cg * 16 + lrow) * PITCH + (wave * RGS * 16 + rg * 16 + lgrp * 4) * 2) =
          u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  if (wave == 0 && lgrp == 0) {
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) srow[cg * 16 + lrow] = (int)out_row(a, cg * 16 + lrow, live, orow[cg]);
  }
  __syncthreads();
  if constexpr (EPI == kEpiSwiglu && OUT % kScaleBlock == 0) {
    if (a.outq != nullptr) {
      // the rows quantised for the FP8 down projection: 16 lanes a (route row,
      // 128-wide block), 8 values a lane, as launch_quantize_rows_fp8 does on
      // the stored bf16 rows (quantize_block16_fp8); codes as whole 128-byte
      // lines, scales block-major by output row
      constexpr int NB = OUT / kScaleBlock;
      const int l16 = lane & 15;
      for (int i = wave * 4 + (lane >> 4); i < ROWS * NB; i += WAVES * 4) {
        const int r = i / NB, b = i % NB;
        const u32x4 v = *reinterpret_cast<const u32x4*>(lds + r * PITCH + (b * kScaleBlock + 8 * l16) * 2);
        float f[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f[2 * j] = bf16_bits_to_f32(v[j] & 0xFFFFu);
          f[2 * j + 1] = bf16_bits_to_f32(v[j] >> 16);
        }
        uint32_t lo, hi;
        const float scale = quantize_block16_fp8(f, lo, hi);
        const int o = srow[r];
        if (o >= 0) {
          __builtin_nontemporal_store(u32x2{lo, hi},
                                      reinterpret_cast<u32x2*>(a.outq + (int64_t)o * a.ldo + n_item + b * kScaleBlock +
                                                               8 * l16));
          if (l16 == 0) a.outq_scale[(n_item / kScaleBlock + b) * a.out_rows + o] = scale;
        }
      }
      return;
    }
  }
  uint16_t* const out = static_cast<uint16_t*>(a.out) + n_item;
  for (int i = wave * 64 + lane; i < ROWS * LPR; i += WAVES * 64) {
    const int r = i / LPR, part = i % LPR;
    const int o = srow[r];
    if (o >= 0)
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(lds + r * PITCH + part * 16),
                                  reinterpret_cast<u32x4*>(out + (int64_t)o * a.ldo + part * 8));
  }
}

// Ring depths of one column-group variant, within 160 KB of LDS: SW weight
// blocks of BLOCK bytes (every wave's rows of the stripe) and SX activation
// stages of XLOADS 1 KB loads per wave (NCG x 16 rows x 256 B, rounded up to
// whole loads; the rows past NCG x 16 are loaded out of range and never read).
// The weight stream is what HBM latency has to be hidden for.  Iteration kb
// issues weight block kb + LA:
//   * 32 KB blocks (256-row stripes): SW = 3 or 4 slots, LA = SW - 1, so
//     SW - 1 blocks (64-96 KB per CU) stay in flight while one is consumed;
//   * 64 KB blocks (tall, 512-row stripes): SW = 2 slots and early refill
//     (LA = 2): a wave reads its rows of block kb into registers before the
//     barrier, so the slot is refilled with block kb + 2 during kb, and two
//     blocks (128 KB per CU) stay in flight.  Only tiles of <= 64 routes
//     leave room for two full activation stages beside the 128 KB ring.
template <int NCG, int WAVES, int BLOCK>
struct PrefillRings {
  static constexpr bool TALL = BLOCK > kStripeBlockBytes;
  static constexpr int XLOADS = (NCG * 4 + WAVES - 1) / WAVES;
  static constexpr int XSTAGE = XLOADS * WAVES * 1024;
  static constexpr int SW = TALL ? 2 : (XSTAGE <= 8192 ? 4 : 3);
  static constexpr int SX = TALL ? 2 : (XSTAGE <= 16384 ? 4 : 2);
  static constexpr int LA = TALL ? 2 : SW - 1;
};

// Wide tiles of the bf16 kernel: 129 .. 256 routes (9 .. 16 column groups).
// Every decoded weight byte then feeds twice the MFMAs of a 128-route tile,
// which halves the decode VALU per MFMA on hot experts.  A whole K block of
// 256 activation rows (64 KB) does not fit beside the weight ring twice, so
// the activation ring holds half blocks (64 K values, 128 B a row: the
// block's MFMA steps 0-1 and 2-3) in two stages, with a barrier per half
// block; the weight ring is the narrow variants' (3 blocks of 32 KB).  Each
// 1 KB load covers 8 rows x 128 B, chunk c of row r in slot c ^ row_swizzle(r).
constexpr int kBMWide = 256;                // routes per tile of the bf16 kernel's plan
// Slot swizzle of 128-byte rows read as 16 rows x one chunk per lane group
// where the four lane groups read chunks 2 g + j (the FP8 kernel's 32-byte
// operands, the wide half stages' B fragments): (r % 8) alone leaves these
// reads 2-way bank-conflicted (measured: 1.5 x the LDS cycles); flipping the
// low slot bit for rows 8 .. 15 of every 16 makes them conflict-free.  (The
// weight rows of the bf16 kernel, read as chunks g and 4 + g, are
// conflict-free with r % 8 and keep it.)
__device__ __forceinline__ int row_swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }
constexpr int kHalfRowBytes = kScaleBlock;  // one staged activation row of a half K block (bf16)
// Half-stage rings: SW weight blocks of BLOCK bytes (3 of 32 KB, or 2 of 64 KB
// with early refill) and two half stages.
template <int NCG, int WAVES, int BLOCK>
struct PrefillWideRings {
  static constexpr bool TALL = BLOCK > kStripeBlockBytes;
  static constexpr int SW = TALL ? 2 : 3;
  static constexpr int XLOADS = (NCG * 2 + WAVES - 1) / WAVES;  // 1 KB loads per wave per half stage
  static constexpr int HSTAGE = XLOADS * WAVES * 1024;
};
constexpr int kOutOfRange = 0x40000000;  // buffer offset beyond every descriptor's range: reads nothing, returns zeros

// Loads a wave has issued after the later of block kb's activation and weight
// loads, up to the barrier of iteration kb, when iteration i issues the
// activations of block i + SX - 1 and then the weights of block i + LA.
constexpr int prefill_pending(int la, int sx, int xloads, int wloads) {
  return sx - 1 < la ? wloads + (sx - 2) * (xloads + wloads) : (la - 1) * (xloads + wloads);
}

template <int TABLES, int RG, int WAVES, int EPI>
__global__ __launch_bounds__(64 * WAVES, 1) void prefill_gemm_kernel(const GroupedGemmArgs a) {
  static_assert(EPI != kEpiWeighted, "the layer's route weights are applied by the combine, not here");
  constexpr int BN = WAVES * RG * 16;  // weight rows per table per work item
  constexpr int GROUPS = TABLES * RG;  // 16-row weight groups of one wave
  constexpr int WLOADS = GROUPS * 2;   // 1 KB weight loads per wave per K block
  constexpr int WAVE_BLOCK = GROUPS * 2048;  // e4m3 bytes of one wave's rows per K block
  constexpr int BLOCK = WAVES * WAVE_BLOCK;  // e4m3 bytes of the work item's weight rows per K block
  static_assert(BLOCK == kStripeBlockBytes || BLOCK == kTallBlockBytes, "256- or 512-row stripes");
  // [SW][WAVES][GROUPS][16 rows][128 B] weight ring, then [SX][NCG * 16 rows][256 B] activation ring
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int stripes = a.n / BN;
  const int total = stripes * healthy_listings(a);
  const int item = xcd_item(blockIdx.x, total);
  if (item < 0 || item >= total) return;
  // work-item scalars are workgroup-uniform: readfirstlane keeps them (and the
  // addresses derived from them) in scalar registers
  ItemTile it;
  if (!item_expert(a, item / stripes, it)) return;
  const int e = it.e, t0 = it.t0, nt = it.nt;
  int stripe, tile;
  item_of_expert<BLOCK == kStripeBlockBytes ? kTileBlock : 2 * kTileBlock>(item - stripes * t0, stripes, nt, stripe,
                                                                          tile);
  item_place(a, tile, it);
  // On tall stripes with wide tiles listed twice, an expert's listings are
  // pairs (its wide tiles, the second listing taking the stripe's second
  // half), then at most one narrow tile: whether this item is a wide listing,
  // and of which half, follows from its place among the expert's nt listings
  // (checked against the tile's route count below).
  int wide_half = -1;
  if constexpr (BLOCK > kStripeBlockBytes) {
    if (a.wide_twice != 0 && !((nt & 1) && tile == nt - 1)) wide_half = tile & 1;
  }
  tile += t0;
  if (stripe < 0 || stripe >= stripes || tile >= a.max_tiles) return;
  // A wide tile listed twice: on tall stripes each listing takes one 256-row
  // half of the stripe, as predicted above; 256-row stripes take the whole
  // stripe on the first listing and skip the second.
  const bool listing_ok = BLOCK == kStripeBlockBytes
                              ? it.half == 0
                              : (wide_half < 0 ? it.live <= kBM && it.half == 0
                                               : it.live > kBM && it.half == wide_half);
  // A consistent plan always passes; a corrupt one computes nothing instead of
  // reading out of bounds.
  if (it.live <= 0 || it.live > kBMWide || it.r0 + it.live > a.rows || !listing_ok) return;
  const int r0 = (int)it.r0;
  const int live = it.live;

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int lrow = lane & 15;
  const int lgrp = lane >> 4;
  const int N = a.n;
  const int K = a.k;
  const int KB = K / kScaleBlock;
  const int n0 = stripe * BN + wave * RG * 16;

  // Weight group g of this wave: table g / RG, rows n0 + (g % RG) * 16 .. +15.
  // Load h of a group brings its rows 8h .. 8h+7 as whole 128-byte lines (lane
  // l: row 8h + l/8), straight into LDS; the lane fetches chunk (l%8) ^ (l/8),
  // so slot s of row r holds chunk s ^ (r % 8) and the MFMA-layout reads below
  // (16 rows, one chunk each) hit distinct banks.  Block scales: one per lane
  // (lane kb holds block kb; K <= 64 blocks), picked per block with v_readlane.
  __amdgpu_buffer_rsrc_t wrsrc[GROUPS];
  float sreg[GROUPS];
#pragma unroll
  for (int g = 0; g < GROUPS; ++g) {
    const int t = g / RG, rg = g % RG;
    const uint8_t* wb = t == 0 ? a.w0 : a.w1;
    const float* sb = t == 0 ? a.s0 : a.s1;
    wrsrc[g] = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(wb + ((size_t)e * N + n0 + rg * 16) * (size_t)K), (short)0, 16 * K, kBufferFormat);
    const float* srow = sb + ((size_t)e * (N / kScaleBlock) + (n0 + rg * 16) / kScaleBlock) * KB;
    sreg[g] = lane < KB ? srow[lane] : 0.0f;
  }
  const int woff = (lane >> 3) * K + (((lane & 7) ^ (lane >> 3)) << 4);
  uint8_t* const wring = lds + wave * WAVE_BLOCK;  // ring slot s at + s * BLOCK
  // A half stripe of a tall stripe (wide listings): half h is rows
  // h * BN / 2 .. (h + 1) * BN / 2 - 1 of each table of the stripe, so its
  // outputs are one contiguous run of BN / 2 columns; RH row groups per table
  // and GH weight groups a wave, group gl being table gl / RH, rows
  // h * BN / 2 + wave * RH * 16 + (gl % RH) * 16 .. +15 (own descriptors and
  // block scales); its ring has 32 KB slots, the wave's rows of slot s at
  // lds + wave * GH * 2 KB + s * 32 KB.
  constexpr int RH = RG > 1 ? RG / 2 : 1;
  constexpr int GH = TABLES * RH;
  uint8_t* const hring = lds + wave * GH * 2048;
  __amdgpu_buffer_rsrc_t hrsrc[GH];
  float hscale[GH];
  // Weight blocks 0 and 1 (slots 0 and 1 of the variant's ring) go out before
  // the variant is chosen: their HBM latency covers the row-id loads that the
  // activation loads wait for.
  if (wide_half < 0) {
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int g = 0; g < GROUPS; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          load_lds_16<kNonTemporal>(wrsrc[g], wring + blk * BLOCK + (2 * g + h) * 1024,
                                    blk < KB ? woff + 8 * h * K : kOutOfRange, blk < KB ? blk * kScaleBlock : 0);
  } else if constexpr (BLOCK > kStripeBlockBytes) {
#pragma unroll
    for (int gl = 0; gl < GH; ++gl) {
      const int t = gl / RH;
      const int rows = stripe * BN + wide_half * (BN / 2) + wave * RH * 16 + (gl % RH) * 16;
      const uint8_t* wb = t == 0 ? a.w0 : a.w1;
      const float* sb = t == 0 ? a.s0 : a.s1;
      hrsrc[gl] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wb + ((size_t)e * N + rows) * (size_t)K),
                                                    (short)0, 16 * K, kBufferFormat);
      const float* srow = sb + ((size_t)e * (N / kScaleBlock) + rows / kScaleBlock) * KB;
      hscale[gl] = lane < KB ? srow[lane] : 0.0f;
    }
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int gl = 0; gl < GH; ++gl)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          load_lds_16<kNonTemporal>(hrsrc[gl], hring + blk * kStripeBlockBytes + (2 * gl + h) * 1024,
                                    blk < KB ? woff + 8 * h * K : kOutOfRange, blk < KB ? blk * kScaleBlock : 0);
  }
  const int ncg = (live + 15) >> 4;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), (short)0, (int)(a.x_rows * K * 2), kBufferFormat);

  // One variant per column-group count (1 .. 8 groups of 16 routes, 1 .. 4 on
  // tall stripes; the half-stage variants below take the rest): the
  // activation stage, the ring depths, the MFMA loop and the accumulators are
  // compile-time, and each variant ends in its own epilogue.
  auto run = [&](auto ncg_tag) {
    constexpr int NCG = decltype(ncg_tag)::value;
    f32x4 acc[TABLES][RG][NCG];
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) acc[t][rg][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
    using Rings = PrefillRings<NCG, WAVES, BLOCK>;
    constexpr int SW = Rings::SW;
    constexpr int SX = Rings::SX;
    constexpr int LA = Rings::LA;          // weight blocks looked ahead
    constexpr int XLOADS = Rings::XLOADS;  // 1 KB activation loads per wave per K block
    constexpr int XSTAGE = Rings::XSTAGE;
    static_assert(XSTAGE >= NCG * 16 * kRowBytes, "activation stage holds the tile's rows");
    static_assert(SW * BLOCK + SX * XSTAGE <= kPrefillLds, "LDS budget");
    static_assert(SW >= 2 && LA >= 2 && LA <= SW, "weight blocks 0 and 1 are in flight before the variant is chosen");
    constexpr int PENDING = prefill_pending(LA, SX, XLOADS, WLOADS);
    static_assert(PENDING >= 0 && PENDING < 64, "vmcnt range");
    uint8_t* const xring = lds + SW * BLOCK;  // stage s at + s * XSTAGE

    // activation rows this lane loads: instruction i covers rows 4 * (wave *
    // XLOADS + i) + lane / 16; the lane fetches the chunk whose slot is lane % 16
    int xoff[XLOADS];
#pragma unroll
    for (int i = 0; i < XLOADS; ++i) {
      const int row = 4 * (wave * XLOADS + i) + lgrp;
      const int r = r0 + (row < live ? row : 0);  // padding rows repeat a live row; their columns are dropped
      int64_t phys = a.x_row_ids ? a.x_row_ids[r] / a.x_row_div : r;
      phys = phys < 0 ? 0 : (phys >= a.x_rows ? a.x_rows - 1 : phys);
      xoff[i] = row < NCG * 16 ? (int)(phys * K * 2) + ((lrow ^ (row & 15)) << 4) : kOutOfRange;
    }
    // Blocks past the last one are issued out of range (no memory traffic, zeros
    // into a slot nobody reads), so every iteration issues the same loads and
    // the wait count stays exact.
    auto issue_x = [&](int blk) {
      uint8_t* st = xring + (blk % SX) * XSTAGE + wave * XLOADS * 1024;
      const bool in = blk < KB;
#pragma unroll
      for (int i = 0; i < XLOADS; ++i)
        load_lds_16(xrsrc, st + i * 1024, in ? xoff[i] : kOutOfRange, in ? blk * kRowBytes : 0);
    };
    auto issue_w = [&](int blk) {
      uint8_t* st = wring + (blk % SW) * BLOCK;
      const bool in = blk < KB;
#pragma unroll
      for (int g = 0; g < GROUPS; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          load_lds_16<kNonTemporal>(wrsrc[g], st + (2 * g + h) * 1024, in ? woff + 8 * h * K : kOutOfRange,
                      in ? blk * kScaleBlock : 0);
    };
    // Load j of iteration kb's loads (the activations of block kb + SX - 1,
    // then the weights of block kb + LA), in that order.  The iteration's
    // XLOADS + WLOADS loads are spread over its MFMA steps instead of issued
    // together after the barrier: eight waves issuing ~60 loads at once stall
    // on the address path (measured: prefill layer -2.4 % at T=2048, -4.6 % at
    // T=8192 Zipf).  The wait counts are unchanged: every load of iteration kb
    // is still issued inside it, in the same order.
    auto issue_load = [&](int j, int kb) {
      if (j < XLOADS) {
        const int blk = kb + SX - 1;
        const bool in = blk < KB;
        load_lds_16(xrsrc, xring + (blk % SX) * XSTAGE + wave * XLOADS * 1024 + j * 1024,
                    in ? xoff[j] : kOutOfRange, in ? blk * kRowBytes : 0);
      } else if (j < XLOADS + WLOADS) {
        const int blk = kb + LA, g = (j - XLOADS) >> 1, h = (j - XLOADS) & 1;
        const bool in = blk < KB;
        load_lds_16<kNonTemporal>(wrsrc[g], wring + (blk % SW) * BLOCK + (2 * g + h) * 1024,
                                  in ? woff + 8 * h * K : kOutOfRange, in ? blk * kScaleBlock : 0);
      }
    };
    static_assert(XLOADS + WLOADS <= 4 * GROUPS, "one load per (step, weight group) of a block at most");

    // output rows of this lane's route columns, loaded ahead of the streams so
    // the epilogue waits for no load (the layer's route weights are applied by
    // the combine, not here)
    int orow[NCG];
    load_out_rows(a, r0, live, lrow, orow);

    // prologue: the issue schedule's iterations -P .. -1
    constexpr int P = SX - 1 > LA ? SX - 1 : LA;
#pragma unroll
    for (int i = -P; i < 0; ++i) {
      if (i + SX - 1 >= 0) issue_x(i + SX - 1);
      if (i + LA >= 2) issue_w(i + LA);  // blocks 0 and 1 went out first
    }
    for (int kb = 0; kb < KB; ++kb) {
      // this wave's loads of block kb have landed; after the barrier everyone's
      // have, and everyone is done with block kb - 1, whose slots are refilled now.
      // Block 0 waits for every prologue load (weights 0 and 1 were issued ahead
      // of the schedule); from block 1 on the schedule's count holds.
      if (kb == 0)
        wait_loads<0>();
      else
        wait_loads<PENDING>();

      const uint8_t* wl = wring + (kb % SW) * BLOCK;
      const uint8_t* xl = xring + (kb % SX) * XSTAGE;
      // this wave's rows in MFMA A layout: lane l gets row l % 16, chunks l/16
      // and 4 + l/16 (K = g*16 .. +15 and 64 + g*16 .. +15 of the block).  The
      // weight ring is this wave's own, so its rows can be read as soon as its
      // own loads have landed, before the barrier: the reads complete while the
      // wave waits there (T=2048 layer -0.6 %, T=8192 Zipf -2 %).
      u32x4 wbits[GROUPS][2];
#pragma unroll
      for (int g = 0; g < GROUPS; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          wbits[g][h] =
              *reinterpret_cast<const u32x4*>(wl + g * 2048 + lrow * 128 + (((lgrp + 4 * h) ^ (lrow & 7)) << 4));
      // after the barrier every wave's activation rows of block kb have landed
      // and every wave is done with block kb - 1, whose slots are refilled below
      barrier();
      // tall stripes refill the slot just read (block kb + 2): its reads must
      // have returned their data first
      if constexpr (Rings::TALL) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      float sc[GROUPS];
#pragma unroll
      for (int g = 0; g < GROUPS; ++g)
        sc[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sreg[g]), kb));
      // Four 32-wide K steps, software-pipelined inside the wave: while the
      // MFMAs of step q run on the matrix core, the VALU decodes step q + 1's
      // A operands and the LDS delivers its B fragments.  Issue is in order, so
      // the source order is the schedule: per weight group its MFMAs (the
      // first group's interleaved with the next step's B reads) followed by its
      // share of the next decode,
      // fenced with scheduling barriers (the compiler would otherwise gather
      // the decode into one block and run the VALU and the matrix core in turns).
      auto decode_group = [&](int q, int g) -> bf16x8 {
        const u32x4 w = wbits[g][q >> 1];
        return (q & 1) ? decode_fp8x8(w.z, w.w, sc[g]) : decode_fp8x8(w.x, w.y, sc[g]);
      };
      auto read_b1 = [&](int q, int cg) -> bf16x8 {
        // B fragment of route row i for step q: logical chunk 2g + (q & 1) + 8 (q >> 1)
        const int i = cg * 16 + lrow;
        return as_bf16x8(*reinterpret_cast<const u32x4*>(
            xl + i * kRowBytes + (((2 * lgrp + (q & 1) + 8 * (q >> 1)) ^ (i & 15)) << 4)));
      };
      auto read_b = [&](int q, bf16x8 (&B)[NCG]) {
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) B[cg] = read_b1(q, cg);
      };
      bf16x8 A[2][GROUPS];
      bf16x8 B[2][NCG];
      read_b(0, B[0]);
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) A[0][g] = decode_group(0, g);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cur = q & 1;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < GROUPS; ++g) {
          issue_load(q * GROUPS + g, kb);
          // the next step's B fragments are read one per MFMA of the first
          // group (not all at once: NCG reads per wave in one burst queue up in
          // the LDS behind the other waves'; T=8192 Zipf layer -5 %)
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) {
            acc[g / RG][g % RG][cg] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[cur][g], B[cur][cg], acc[g / RG][g % RG][cg], 0, 0, 0);
            if (g == 0 && q < 3) B[cur ^ 1][cg] = read_b1(q + 1, cg);
            __builtin_amdgcn_sched_barrier(0);
          }
          __builtin_amdgcn_sched_barrier(0);
          if (q < 3) A[cur ^ 1][g] = decode_group(q + 1, g);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    wait_all_loads();  // the rings are idle: the epilogue reuses the LDS

    // Epilogue: lane holds rows n .. n+3 of route column cg*16 + lrow.
    store_tile_lines<NCG, RG, TABLES, EPI, WAVES>(a, lds, acc, orow, live, wave, lane, (int64_t)stripe * BN);
  };

  // Tiles in half-block activation stages: the wide tiles (NCG = 10, 12, 14
  // or 16 column groups; an odd count runs the next even variant with one
  // padding group) and, on tall stripes, tiles of 5 .. 8 groups, whose full
  // activation blocks do not fit beside the 128 KB weight ring twice.  Per K
  // block: the wave's weight rows decoded once, as in the narrow variants,
  // and two half-block passes over the tile's routes, each behind its own
  // barrier.  Same MFMA sequence per output (steps 0..3 of every block in
  // order), so the results equal the narrow variants' bit for bit.
  //
  // SUB = 2: a wide tile on tall stripes takes one 256-row half of the stripe
  // (RS = RG / 2 row groups per table, 32 KB blocks in a 3-slot ring; all
  // 512 rows' accumulators would not fit in registers): the half its listing
  // names, the other listing taking the other half.
  //
  // Loads, in issue order: weight blocks 0 and 1, activation half 0; then in
  // half h of block kb: activation half 2 kb + h + 1 (the stage freed by this
  // half's barrier), then half h of weight block kb + 2's loads (its slot is
  // block kb - 1's, done before this block's first barrier; with two slots it
  // is block kb's own, whose rows the wave read into registers before that
  // barrier).  So at each barrier at most the other half's weight loads
  // (WHALF) may still be in flight: the activation half about to be read, and
  // every weight block before the next one, have landed.
  auto run_halves = [&](auto ncg_tag, auto sub_tag) {
    constexpr int NCG = decltype(ncg_tag)::value;
    constexpr int SUB = decltype(sub_tag)::value;
    static_assert(NCG > 4 && NCG <= kBMWide / 16, "half-stage variants: 5 .. 16 column groups");
    static_assert(SUB == 1 || (SUB == 2 && RG % 2 == 0), "one stripe or two halves of it");
    constexpr int RS = RG / SUB;              // 16-row groups per table of a sub-stripe
    constexpr int GS = TABLES * RS;           // weight groups of one wave in a sub-stripe
    constexpr int SBLOCK = WAVES * GS * 2048; // e4m3 bytes of a sub-stripe's K block
    using Rings = PrefillWideRings<NCG, WAVES, SBLOCK>;
    constexpr int SW = Rings::SW;
    constexpr int XLOADS = Rings::XLOADS;
    constexpr int HSTAGE = Rings::HSTAGE;
    constexpr int WHALF = GS;                 // weight loads per half block (2 per group and block)
    static_assert(HSTAGE >= NCG * 16 * kHalfRowBytes, "half stage holds the tile's rows");
    static_assert(SW * SBLOCK + 2 * HSTAGE <= kPrefillLds, "LDS budget");
    static_assert(SW >= 2, "weight blocks 0 and 1 fill the first two slots");
    static_assert(WHALF < 64, "vmcnt range");
    uint8_t* const xring = lds + SW * SBLOCK;  // half stage hb at + (hb & 1) * HSTAGE
    uint8_t* const sring = lds + wave * GS * 2048;  // this wave's weight slot s at + s * SBLOCK

    // activation rows this lane loads: instruction i covers rows 8 * (wave *
    // XLOADS + i) + lane / 8; the lane fetches the chunk whose slot is lane % 8
    int xoff[XLOADS];
#pragma unroll
    for (int i = 0; i < XLOADS; ++i) {
      const int row = 8 * (wave * XLOADS + i) + (lane >> 3);
      const int r = r0 + (row < live ? row : 0);  // padding rows repeat a live row; their columns are dropped
      int64_t phys = a.x_row_ids ? a.x_row_ids[r] / a.x_row_div : r;
      phys = phys < 0 ? 0 : (phys >= a.x_rows ? a.x_rows - 1 : phys);
      xoff[i] = row < NCG * 16 ? (int)(phys * K * 2) + (((lane & 7) ^ row_swizzle(row)) << 4) : kOutOfRange;
    }
    // load j of activation half hb (out of range past the last half)
    auto issue_xh = [&](int j, int hb) {
      const bool in = hb < 2 * KB;
      load_lds_16(xrsrc, xring + (hb & 1) * HSTAGE + (wave * XLOADS + j) * 1024, in ? xoff[j] : kOutOfRange,
                  in ? hb * kHalfRowBytes : 0);
    };
    int orow[NCG];
    load_out_rows(a, r0, live, lrow, orow);

    {
      // the sub-stripe's weight groups: the whole stripe's (SUB = 1), or the
      // half stripe's (their blocks 0 and 1 went out above in this layout)
      const int ss = SUB == 1 ? 0 : wide_half;
      __amdgpu_buffer_rsrc_t wsub[GS];
      float ssc[GS];
#pragma unroll
      for (int gl = 0; gl < GS; ++gl) {
        if constexpr (SUB == 1) {
          wsub[gl] = wrsrc[gl];
          ssc[gl] = sreg[gl];
        } else {
          wsub[gl] = hrsrc[gl];
          ssc[gl] = hscale[gl];
        }
      }
      // load j of half `part` of weight block blk's loads (group l / 2, rows 8 (l % 2) ..)
      auto issue_wh = [&](int j, int blk, int part) {
        const int l = part * WHALF + j, g = l >> 1, h = l & 1;
        const bool in = blk < KB;
        load_lds_16<kNonTemporal>(wsub[g], sring + (blk % SW) * SBLOCK + (2 * g + h) * 1024,
                                  in ? woff + 8 * h * K : kOutOfRange, in ? blk * kScaleBlock : 0);
      };
      static_assert(SUB == 1 ? SBLOCK == BLOCK : (SBLOCK == kStripeBlockBytes && RS == RH && GS == GH),
                    "blocks 0 and 1 were issued in this ring's layout");

      f32x4 acc[TABLES][RS][NCG];
#pragma unroll
      for (int t = 0; t < TABLES; ++t)
#pragma unroll
        for (int rg = 0; rg < RS; ++rg)
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) acc[t][rg][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
      for (int j = 0; j < XLOADS; ++j) issue_xh(j, 0);

      for (int kb = 0; kb < KB; ++kb) {
        if (kb == 0)
          wait_loads<0>();
        else
          wait_loads<WHALF>();
        // the wave's own weight rows of block kb (MFMA A layout, as in the
        // narrow variants), read before the barrier
        const uint8_t* wl = sring + (kb % SW) * SBLOCK;
        u32x4 wbits[GS][2];
#pragma unroll
        for (int g = 0; g < GS; ++g)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            wbits[g][h] =
                *reinterpret_cast<const u32x4*>(wl + g * 2048 + lrow * 128 + (((lgrp + 4 * h) ^ (lrow & 7)) << 4));
        barrier();
        // two slots: this block's slot is refilled in this block, so the
        // reads above must have returned their data first
        if constexpr (Rings::TALL) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        float sc[GS];
#pragma unroll
        for (int g = 0; g < GS; ++g)
          sc[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ssc[g]), kb));
        auto decode_group = [&](int q, int g) -> bf16x8 {
          const u32x4 w = wbits[g][q >> 1];
          return (q & 1) ? decode_fp8x8(w.z, w.w, sc[g]) : decode_fp8x8(w.x, w.y, sc[g]);
        };
        bf16x8 A[2][GS];  // step q's operands in A[q & 1]

        // Half H of block kb: MFMA steps 2H and 2H + 1 over the half stage in
        // slot H (half 2 kb + H), positions p = step-in-half x NCG + column group.
        auto half_pass = [&](auto half_tag) {
          constexpr int H = decltype(half_tag)::value;
          constexpr int P = 2 * NCG;
          constexpr int D = 4;                      // B fragments read ahead
          constexpr int NL = XLOADS + WHALF;        // loads of this half
          static_assert(NL <= P, "every load of the half has a position");
          const uint8_t* xl = xring + H * HSTAGE;
          bf16x8 Bf[P];
          auto read_b = [&](int p) {
            const int q = p / NCG, i = (p % NCG) * 16 + lrow;
            Bf[p] = as_bf16x8(*reinterpret_cast<const u32x4*>(xl + i * kHalfRowBytes +
                                                               (((2 * lgrp + q) ^ row_swizzle(lrow)) << 4)));
          };
#pragma unroll
          for (int p = 0; p < D; ++p) read_b(p);
          if constexpr (H == 0) {
#pragma unroll
            for (int g = 0; g < GS; ++g) A[0][g] = decode_group(0, g);
          }
#pragma unroll
          for (int p = 0; p < P; ++p) {
            const int q = 2 * H + p / NCG, cg = p % NCG;
            __builtin_amdgcn_sched_barrier(0);
            // the next step's operands, one weight group at a time
            if (q < 3) {
#pragma unroll
              for (int g = 0; g < GS; ++g)
                if (cg == g * NCG / GS) A[(q + 1) & 1][g] = decode_group(q + 1, g);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (p + D < P) read_b(p + D);
            // the half's loads, one per position from its first on (issued as
            // early as their slots allow: T=8192 Zipf down -2.5 % against
            // spreading them over the half)
#pragma unroll
            for (int l = 0; l < NL; ++l)
              if (p == l) {
                if (l < XLOADS)
                  issue_xh(l, 2 * kb + H + 1);
                else
                  issue_wh(l - XLOADS, kb + 2, H);
              }
#pragma unroll
            for (int g = 0; g < GS; ++g)
              acc[g / RS][g % RS][cg] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[q & 1][g], Bf[p], acc[g / RS][g % RS][cg], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
        };
        half_pass(std::integral_constant<int, 0>{});
        // this wave's loads of activation half 2 kb + 1 have landed; after the
        // barrier everyone's have, and everyone is done with half 2 kb - 1
        wait_loads<WHALF>();
        barrier();
        half_pass(std::integral_constant<int, 1>{});
      }
      wait_all_loads();  // the rings are idle: the epilogue reuses the LDS

      store_tile_lines<NCG, RS, TABLES, EPI, WAVES>(a, lds, acc, orow, live, wave, lane,
                                                    (int64_t)stripe * BN + ss * (BN / SUB));
    }
  };
  using I = std::integral_constant<int, 1>;
  if constexpr (BLOCK > kStripeBlockBytes) {
    // tall stripes: full activation blocks up to 4 column groups, half blocks
    // above, wide tiles as two sub-stripes
    using I2 = std::integral_constant<int, 2>;
    switch (ncg) {
      case 1: run(std::integral_constant<int, 1>{}); break;
      case 2: run(std::integral_constant<int, 2>{}); break;
      case 3: run(std::integral_constant<int, 3>{}); break;
      case 4: run(std::integral_constant<int, 4>{}); break;
      case 5: run_halves(std::integral_constant<int, 5>{}, I{}); break;
      case 6: run_halves(std::integral_constant<int, 6>{}, I{}); break;
      case 7: run_halves(std::integral_constant<int, 7>{}, I{}); break;
      case 8: run_halves(std::integral_constant<int, 8>{}, I{}); break;
      case 9:
      case 10: run_halves(std::integral_constant<int, 10>{}, I2{}); break;
      case 11:
      case 12: run_halves(std::integral_constant<int, 12>{}, I2{}); break;
      case 13:
      case 14: run_halves(std::integral_constant<int, 14>{}, I2{}); break;
      default: run_halves(std::integral_constant<int, 16>{}, I2{}); break;
    }
  } else {
    switch (ncg) {
      case 1: run(std::integral_constant<int, 1>{}); break;
      case 2: run(std::integral_constant<int, 2>{}); break;
      case 3: run(std::integral_constant<int, 3>{}); break;
      case 4: run(std::integral_constant<int, 4>{}); break;
      case 5: run(std::integral_constant<int, 5>{}); break;
      case 6: run(std::integral_constant<int, 6>{}); break;
      case 7: run(std::integral_constant<int, 7>{}); break;
      case 8: run(std::integral_constant<int, 8>{}); break;
      case 9:
      case 10: run_halves(std::integral_constant<int, 10>{}, I{}); break;
      case 11:
      case 12: run_halves(std::integral_constant<int, 12>{}, I{}); break;
      case 13:
      case 14: run_halves(std::integral_constant<int, 14>{}, I{}); break;
      default: run_halves(std::integral_constant<int, 16>{}, I{}); break;
    }
  }
}

// ---------------------------------------------------------------------------
// Native FP8 mode: activations quantised per (row, 128-wide K block) to e4m3
// with an FP32 scale (amax / 448), weights used as stored.  Per K block and
// 16 x 16 output tile one v_mfma_scale_f32_16x16x128_f8f6f4 (unit E8M0 scales)
// computes the e4m3 x e4m3 block product exactly in FP32, and the FP32 tile
// accumulator takes it times (weight block scale x activation block scale).
// Same work order, activation ring and weight transpose as the bf16 kernel;
// no decode, half the activation bytes.  Tall stripes where N allows them, as
// in the bf16 kernel (512 weight rows a work item, a two-slot ring refilled
// early); their activation block scales are held in registers, the rings
// filling the LDS (T=2048 FP8 layer -2.3 %, T=8192 Zipf -2..4 %).
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x8 join_i32x8(const u32x4& lo, const u32x4& hi) {
  const i32x4 l = __builtin_bit_cast(i32x4, lo);
  const i32x4 h = __builtin_bit_cast(i32x4, hi);
  return __builtin_shufflevector(l, h, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Ring depths of the FP8 kernel: SW weight blocks (32 KB) and SX activation
// stages of XLOADS 1 KB loads per wave (NCG x 16 rows x 128 e4m3 bytes,
// rounded up to whole loads), each with a 256-byte activation-scale slice per
// wave (waves 0 and 1 hold the tile's 128 FP32 block scales).
template <int NCG, int WAVES>
struct Fp8Rings {
  static constexpr int XLOADS = (NCG * 2 + WAVES - 1) / WAVES;
  static constexpr int XSTAGE = XLOADS * WAVES * 1024;
  static constexpr int SW = 3;
  static constexpr int SX = XLOADS == 1 ? 4 : 3;
};

template <int TABLES, int RG, int WAVES, int EPI>
__global__ __launch_bounds__(64 * WAVES, 1) void prefill_gemm_fp8_kernel(const GroupedGemmArgs a) {
  static_assert(EPI != kEpiWeighted, "the layer's route weights are applied by the combine, not here");
  constexpr int BN = WAVES * RG * 16;
  constexpr int GROUPS = TABLES * RG;
  constexpr int WLOADS = GROUPS * 2;
  constexpr int WAVE_BLOCK = GROUPS * 2048;
  constexpr int BLOCK = WAVES * WAVE_BLOCK;
  constexpr bool TALL = BLOCK > kStripeBlockBytes;
  static_assert(BLOCK == kStripeBlockBytes || BLOCK == kTallBlockBytes, "256- or 512-row stripes");
  static_assert(WAVES >= 2, "two waves load the activation scales");
  constexpr int ROWB = kScaleBlock;  // e4m3 bytes of one activation row per K block
  constexpr int SSTAGE = WAVES * 256;  // activation-scale slices of one stage
  // [SW][WAVES][GROUPS][16 rows][128 B] weight ring, [SX][rows][128 B] activation
  // ring, [SX][128] FP32 activation-scale ring
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int stripes = a.n / BN;
  const int R = TALL ? 1 : stripe_run_of(a);
  const int runs = (stripes + R - 1) / R;
  const int total = runs * healthy_listings(a);
  const int item = xcd_item(blockIdx.x, total);
  if (item < 0 || item >= total) return;
  ItemTile it;
  if (!item_expert(a, item / runs, it)) return;
  const int e = it.e, t0 = it.t0, nt = it.nt;
  int run, tile;
  item_of_expert<kTileBlockFp8>(item - runs * t0, runs, nt, run, tile);
  item_place(a, tile, it);
  tile += t0;
  if (run < 0 || run >= runs || tile >= a.max_tiles) return;
  // A consistent plan always passes; a corrupt one computes nothing instead of
  // reading out of bounds.
  if (it.half != 0 || it.live <= 0 || it.live > kBM || it.r0 + it.live > a.rows) return;
  const int r0 = (int)it.r0;
  const int live = it.live;
  const int s0 = run * R;                // the run's first stripe
  const int nr = min(R, stripes - s0);   // and its stripe count
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int lrow = lane & 15;
  const int lgrp = lane >> 4;
  const int N = a.n;
  const int K = a.k;
  const int KB = K / kScaleBlock;

  // Weight group g of stripe s: table g / RG, rows s * BN + wave * RG * 16 +
  // (g % RG) * 16 .. +15, as in the bf16 kernel (direct-to-LDS, chunk c of row
  // r in slot c ^ row_swizzle(r): its 32-byte A reads are chunks 2 g, 2 g + 1);
  // its block scales, lane kb holding block kb.
  auto weight_rsrc = [&](int s, int g) {
    const int n0 = s * BN + wave * RG * 16 + (g % RG) * 16;
    const uint8_t* wb = g / RG == 0 ? a.w0 : a.w1;
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(uniform_ptr(wb + ((size_t)e * N + n0) * (size_t)K)), (short)0, 16 * K, kBufferFormat);
  };
  constexpr int MR = TALL ? 1 : kMaxStripeRun;
  float sreg[MR][GROUPS];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
      const int n0 = (s0 + (r < nr ? r : 0)) * BN + wave * RG * 16 + (g % RG) * 16;
      const float* sb = g / RG == 0 ? a.s0 : a.s1;
      const float* srow = sb + ((size_t)e * (N / kScaleBlock) + n0 / kScaleBlock) * KB;
      sreg[r][g] = r < nr && lane < KB ? srow[lane] : 0.0f;
    }
  // load h of a group brings rows 8 h .. 8 h + 7: lane l row 8 h + l / 8
  const int woff[2] = {(lane >> 3) * K + (((lane & 7) ^ row_swizzle(lane >> 3)) << 4),
                       (8 + (lane >> 3)) * K + (((lane & 7) ^ row_swizzle(8 + (lane >> 3))) << 4)};
  uint8_t* const wring = lds + wave * WAVE_BLOCK;  // ring slot s at + s * 32 KB
  // the first stripe's weight blocks 0 and 1 go out before the row ids are
  // read, as in the bf16 kernel
  {
    __amdgpu_buffer_rsrc_t w0r[GROUPS];
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) w0r[g] = weight_rsrc(s0, g);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int g = 0; g < GROUPS; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          load_lds_16<kNonTemporal>(w0r[g], wring + blk * BLOCK + (2 * g + h) * 1024,
                                    blk < KB ? woff[h] : kOutOfRange, blk < KB ? blk * kScaleBlock : 0);
  }
  const int ncg = (live + 15) >> 4;
  auto phys_row = [&](int row) -> int64_t {
    const int r = r0 + (row < live ? row : 0);  // padding rows repeat a live row; their columns are dropped
    int64_t phys = a.x_row_ids ? a.x_row_ids[r] / a.x_row_div : r;
    return phys < 0 ? 0 : (phys >= a.x_rows ? a.x_rows - 1 : phys);
  };
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.xq), (short)0, (int)(a.x_rows * K), kBufferFormat);
  // activation block scales, block-major by sorted position ([K / 128][rows]):
  // waves 0 and 1 load tile rows 64 w + lane of each block (4 bytes a lane,
  // one contiguous 256-byte run a wave; padding rows repeat row 0); the other
  // waves issue the same load out of range into their own slices, so that
  // every wave's wait count is the same
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.xscale), (short)0, (int)(KB * a.rows * 4), kBufferFormat);
  const int srow = 64 * wave + lane;
  [[maybe_unused]] const int soff = wave < 2 ? 4 * (r0 + (srow < live ? srow : 0)) : kOutOfRange;  // 256-row stripes
  const int sstride = a.rows * 4;  // bytes between the scales of consecutive blocks

  auto run_tile = [&](auto ncg_tag) {
    constexpr int NCG = decltype(ncg_tag)::value;
    using Rings = Fp8Rings<NCG, WAVES>;
    constexpr int SW = Rings::SW;
    constexpr int SX = Rings::SX;
    constexpr int XLOADS = Rings::XLOADS;
    constexpr int XSTAGE = Rings::XSTAGE;
    static_assert(XSTAGE >= NCG * 16 * ROWB, "activation stage holds the tile's rows");
    static_assert(SW * kStripeBlockBytes + SX * (XSTAGE + SSTAGE) <= kPrefillLds, "LDS budget");
    static_assert(SW == 3, "weight blocks 0 and 1 are in flight before the variant is chosen");
    constexpr int PENDING = prefill_pending(SW - 1, SX, XLOADS + 1, WLOADS);
    static_assert(PENDING >= 0 && PENDING < 64, "vmcnt range");
    constexpr int LOADS = XLOADS + 1 + WLOADS;  // ring loads per wave per K block
    uint8_t* const xring = lds + SW * kStripeBlockBytes;
    uint8_t* const sring = xring + SX * XSTAGE;

    // activation rows: instruction i covers rows 8 * (wave * XLOADS + i) + lane / 8,
    // 128 bytes each; chunk c of row r lands in slot c ^ row_swizzle(r)
    int xoff[XLOADS];
#pragma unroll
    for (int i = 0; i < XLOADS; ++i) {
      const int row = 8 * (wave * XLOADS + i) + (lane >> 3);
      xoff[i] = row < NCG * 16 ? (int)(phys_row(row) * K) + (((lane & 7) ^ row_swizzle(row)) << 4) : kOutOfRange;
    }
    int orow[NCG];  // as in the bf16 kernel: output rows loaded ahead of the streams
    load_out_rows(a, r0, live, lrow, orow);
    // prologue: the activations and scales of blocks 0 .. SX - 2
#pragma unroll
    for (int blk = 0; blk < SX - 1; ++blk) {
      const bool in = blk < KB;
      uint8_t* st = xring + blk * XSTAGE + wave * XLOADS * 1024;
#pragma unroll
      for (int i = 0; i < XLOADS; ++i)
        load_lds_16(xrsrc, st + i * 1024, in ? xoff[i] : kOutOfRange, in ? blk * ROWB : 0);
#if defined(__HIP_DEVICE_COMPILE__)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          srsrc, (__attribute__((address_space(3))) void*)(sring + blk * SSTAGE + wave * 256), 4,
          in ? soff : kOutOfRange, in ? blk * sstride : 0, 0, 0);
#endif
    }

    // The run's stripes share the tile: one continuous ring, block kb of
    // stripe r being block r * KB + kb of the ring.  Its slot and stage are
    // stepped once per block; iteration kb refills the slot and stage of block
    // kb - 1 (freed by its barrier) with the activations and scales of block
    // kb + SX - 1 and the weights of block kb + SW - 1, which near a stripe's
    // end are the next stripe's first blocks (the same activation rows, the
    // next stripe's weights), so the next stripe starts with its blocks in
    // flight and the epilogue overlaps them.
    int ws = 0, xs = 0;
    for (int r = 0; r < nr; ++r) {
      const bool more = r + 1 < nr;
      __amdgpu_buffer_rsrc_t wcur[GROUPS];
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) wcur[g] = weight_rsrc(s0 + r, g);
      // the stripe's block scales are sreg[0] (shifted down after each stripe:
      // a runtime index would put the array in scratch memory)
      float sr[GROUPS];
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) sr[g] = sreg[0][g];
      f32x4 acc[TABLES][RG][NCG];
#pragma unroll
      for (int t = 0; t < TABLES; ++t)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) acc[t][rg][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

      // Load j of iteration kb while every block it loads is this stripe's.
      auto issue_own = [&](int j, int kb, int wsf, int xsf) {
        if (j < XLOADS) {
          load_lds_16(xrsrc, xring + xsf * XSTAGE + wave * XLOADS * 1024 + j * 1024, xoff[j], (kb + SX - 1) * ROWB);
        } else if (j == XLOADS) {
#if defined(__HIP_DEVICE_COMPILE__)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              srsrc, (__attribute__((address_space(3))) void*)(sring + xsf * SSTAGE + wave * 256), 4, soff,
              (kb + SX - 1) * sstride, 0, 0);
#endif
        } else if (j < LOADS) {
          const int g = (j - XLOADS - 1) >> 1, h = (j - XLOADS - 1) & 1;
          load_lds_16<kNonTemporal>(wcur[g], wring + wsf * kStripeBlockBytes + (2 * g + h) * 1024, woff[h],
                                    (kb + SW - 1) * kScaleBlock);
        }
      };
      // The same near the stripe's end: a block past its last is the next
      // stripe's (more) or else out of range (no traffic, zeros into a slot
      // nobody reads before the workgroup ends).
      auto issue_end = [&](int j, int kb, int wsf, int xsf) {
        if (j <= XLOADS) {
          const int xb = kb + SX - 1;
          const bool go = xb < KB || more;
          const int blk = xb < KB ? xb : xb - KB;
          if (j < XLOADS) {
            load_lds_16(xrsrc, xring + xsf * XSTAGE + wave * XLOADS * 1024 + j * 1024, go ? xoff[j] : kOutOfRange,
                        go ? blk * ROWB : 0);
          } else {
#if defined(__HIP_DEVICE_COMPILE__)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                srsrc, (__attribute__((address_space(3))) void*)(sring + xsf * SSTAGE + wave * 256), 4,
                go ? soff : kOutOfRange, go ? blk * sstride : 0, 0, 0);
#endif
          }
        } else if (j < LOADS) {
          const int g = (j - XLOADS - 1) >> 1, h = (j - XLOADS - 1) & 1;
          const int wb = kb + SW - 1;
          const bool own = wb < KB;
          const bool go = own || more;
          // (the stripe is selected, not the descriptor: a select between two
          // descriptors goes through scratch memory)
          load_lds_16<kNonTemporal>(weight_rsrc(own ? s0 + r : s0 + r + 1, g),
                                    wring + wsf * kStripeBlockBytes + (2 * g + h) * 1024,
                                    go ? woff[h] : kOutOfRange, go ? (own ? wb : wb - KB) * kScaleBlock : 0);
        }
      };

      auto kstep = [&](int kb, auto issue) {
        if (r == 0 && kb == 0)
          wait_loads<0>();  // block 0: every prologue load
        else
          wait_loads<PENDING>();
        const int wsf = ws == 0 ? SW - 1 : ws - 1;
        const int xsf = xs == 0 ? SX - 1 : xs - 1;
        const uint8_t* wl = wring + ws * kStripeBlockBytes;
        const uint8_t* xl = xring + xs * XSTAGE;
        const float* sl = reinterpret_cast<const float*>(sring + xs * SSTAGE);
        // A: lane l gets row l % 16, chunks 2 (l/16) and 2 (l/16) + 1 (32 e4m3
        // values); the wave's own weight rows are read before the barrier, as in
        // the bf16 kernel
        i32x8 wv[GROUPS];
#pragma unroll
        for (int g = 0; g < GROUPS; ++g)
          wv[g] = join_i32x8(
              *reinterpret_cast<const u32x4*>(wl + g * 2048 + lrow * 128 + (((2 * lgrp) ^ row_swizzle(lrow)) << 4)),
              *reinterpret_cast<const u32x4*>(wl + g * 2048 + lrow * 128 + (((2 * lgrp + 1) ^ row_swizzle(lrow)) << 4)));
        barrier();
        float sw[GROUPS];
#pragma unroll
        for (int g = 0; g < GROUPS; ++g)
          sw[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sr[g]), kb));
        // B fragment and activation scale of column group cg, read one group
        // ahead of the MFMAs that use them (T=8192 Zipf FP8 layer -7 %)
        auto read_bv = [&](int cg) -> i32x8 {
          const int i = cg * 16 + lrow;
          const uint8_t* rowp = xl + i * ROWB;
          return join_i32x8(*reinterpret_cast<const u32x4*>(rowp + (((2 * lgrp) ^ row_swizzle(i)) << 4)),
                            *reinterpret_cast<const u32x4*>(rowp + (((2 * lgrp + 1) ^ row_swizzle(i)) << 4)));
        };
        i32x8 bnext = read_bv(0);
        float sxnext = sl[lrow];
        // the iteration's loads, spread over its column groups (all issued before its end)
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
#pragma unroll
          for (int j = cg * LOADS / NCG; j < (cg + 1) * LOADS / NCG; ++j) issue(j, kb, wsf, xsf);
          const i32x8 bv = bnext;
          const float sx = sxnext;
          if (cg + 1 < NCG) {
            bnext = read_bv(cg + 1);
            sxnext = sl[(cg + 1) * 16 + lrow];
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int g = 0; g < GROUPS; ++g) {
            const f32x4 p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wv[g], bv, f32x4{0.f, 0.f, 0.f, 0.f},
                                                                             0, 0, 0, 127, 0, 127);
            const float f = sw[g] * sx;
            f32x4 c = acc[g / RG][g % RG][cg];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) c[jj] = __builtin_fmaf(p[jj], f, c[jj]);
            acc[g / RG][g % RG][cg] = c;
          }
        }
        ws = ws + 1 == SW ? 0 : ws + 1;
        xs = xs + 1 == SX ? 0 : xs + 1;
      };
      const int kmain = KB - (SX > SW ? SX : SW) + 1;  // blocks whose loads are all this stripe's
      int kb = 0;
      for (; kb < kmain; ++kb) kstep(kb, issue_own);
      for (; kb < KB; ++kb) kstep(kb, issue_end);

      int64_t orow_ok[NCG];
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) orow_ok[cg] = out_row(a, cg * 16 + lrow, live, orow[cg]);
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
          store_fragment_at<TABLES, EPI>(a, orow_ok[cg], 1.0f, (s0 + r) * BN + wave * RG * 16 + rg * 16 + lgrp * 4,
                                         acc[0][rg][cg], acc[TABLES - 1][rg][cg]);
#pragma unroll
      for (int j = 0; j + 1 < MR; ++j)
#pragma unroll
        for (int g = 0; g < GROUPS; ++g) sreg[j][g] = sreg[j + 1][g];
    }
    wait_all_loads();  // no load may still target LDS when the workgroup ends
  };
  // Tall stripes (512 weight rows a work item, 4 weight groups a wave; one
  // stripe a work item): the weight ring is two 64 KB slots refilled early
  // (as in the bf16 kernel), the activation ring two stages, and the tile's
  // activation block scales go to registers -- lane l holds routes l and
  // 64 + l of the next block, loaded one block ahead -- because the rings
  // fill the 160 KB of LDS; a column group's scales reach its lanes by
  // ds_bpermute.
  auto run_tall = [&](auto ncg_tag) {
    constexpr int NCG = decltype(ncg_tag)::value;
    constexpr int SX = 2;
    constexpr int XLOADS = (NCG * 2 + WAVES - 1) / WAVES;
    constexpr int XSTAGE = XLOADS * WAVES * 1024;
    constexpr int SL = NCG > 4 ? 2 : 1;  // scale registers per lane and block
    constexpr int XL = XLOADS + SL;      // activation-side loads per block
    constexpr int LOADS = XL + WLOADS;
    static_assert(XSTAGE >= NCG * 16 * ROWB, "activation stage holds the tile's rows");
    static_assert(2 * BLOCK + SX * XSTAGE <= kPrefillLds, "LDS budget");
    constexpr int PENDING = prefill_pending(2, SX, XL, WLOADS);
    static_assert(PENDING >= 0 && PENDING < 64, "vmcnt range");
    uint8_t* const xring = lds + 2 * BLOCK;
    int xoff[XLOADS];
#pragma unroll
    for (int i = 0; i < XLOADS; ++i) {
      const int row = 8 * (wave * XLOADS + i) + (lane >> 3);
      xoff[i] = row < NCG * 16 ? (int)(phys_row(row) * K) + (((lane & 7) ^ row_swizzle(row)) << 4) : kOutOfRange;
    }
    int orow[NCG];
    load_out_rows(a, r0, live, lrow, orow);
    int soffs[SL];
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      const int rr = 64 * j + lane;
      soffs[j] = 4 * (r0 + (rr < live ? rr : 0));
    }
    float sx_next[SL];
    // prologue: block 0's activations and scales (weights 0 and 1 went out first)
#pragma unroll
    for (int i = 0; i < XLOADS; ++i) load_lds_16(xrsrc, xring + wave * XLOADS * 1024 + i * 1024, xoff[i], 0);
#pragma unroll
    for (int j = 0; j < SL; ++j)
      sx_next[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srsrc, soffs[j], 0, 0));

    f32x4 acc[TABLES][RG][NCG];
#pragma unroll
    for (int t = 0; t < TABLES; ++t)
#pragma unroll
      for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) acc[t][rg][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
    __amdgpu_buffer_rsrc_t wcur[GROUPS];
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) wcur[g] = weight_rsrc(s0, g);
    float sr[GROUPS];
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) sr[g] = sreg[0][g];

    // load j of iteration kb: the activations of block kb + 1, its scales, the
    // weights of block kb + 2 (into the slot of block kb, read before the barrier)
    auto issue = [&](int j, int kb) {
      if (j < XLOADS) {
        const int blk = kb + 1;
        const bool in = blk < KB;
        load_lds_16(xrsrc, xring + (blk & 1) * XSTAGE + wave * XLOADS * 1024 + j * 1024, in ? xoff[j] : kOutOfRange,
                    in ? blk * ROWB : 0);
      } else if (j < XL) {
        const int blk = kb + 1;
        const bool in = blk < KB;
        sx_next[j - XLOADS] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(srsrc, in ? soffs[j - XLOADS] : kOutOfRange,
                                                        in ? blk * sstride : 0, 0));
      } else if (j < LOADS) {
        const int blk = kb + 2, g = (j - XL) >> 1, h = (j - XL) & 1;
        const bool in = blk < KB;
        load_lds_16<kNonTemporal>(wcur[g], wring + (kb & 1) * BLOCK + (2 * g + h) * 1024,
                                  in ? woff[h] : kOutOfRange, in ? blk * kScaleBlock : 0);
      }
    };
    for (int kb = 0; kb < KB; ++kb) {
      if (kb == 0)
        wait_loads<0>();
      else
        wait_loads<PENDING>();
      float sxc[SL];
#pragma unroll
      for (int j = 0; j < SL; ++j) sxc[j] = sx_next[j];
      const uint8_t* wl = wring + (kb & 1) * BLOCK;
      const uint8_t* xl = xring + (kb & 1) * XSTAGE;
      i32x8 wv[GROUPS];
#pragma unroll
      for (int g = 0; g < GROUPS; ++g)
        wv[g] = join_i32x8(
            *reinterpret_cast<const u32x4*>(wl + g * 2048 + lrow * 128 + (((2 * lgrp) ^ row_swizzle(lrow)) << 4)),
            *reinterpret_cast<const u32x4*>(wl + g * 2048 + lrow * 128 + (((2 * lgrp + 1) ^ row_swizzle(lrow)) << 4)));
      barrier();
      // the slot just read is refilled in this iteration: its reads must have returned
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      float sw[GROUPS];
#pragma unroll
      for (int g = 0; g < GROUPS; ++g)
        sw[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sr[g]), kb));
      auto read_bv = [&](int cg) -> i32x8 {
        const int i = cg * 16 + lrow;
        const uint8_t* rowp = xl + i * ROWB;
        return join_i32x8(*reinterpret_cast<const u32x4*>(rowp + (((2 * lgrp) ^ row_swizzle(i)) << 4)),
                          *reinterpret_cast<const u32x4*>(rowp + (((2 * lgrp + 1) ^ row_swizzle(i)) << 4)));
      };
      auto read_sx = [&](int cg) -> float {
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(((cg & 3) * 16 + lrow) * 4,
                                                                      __builtin_bit_cast(int, sxc[cg >> 2])));
      };
      i32x8 bnext = read_bv(0);
      float sxnext = read_sx(0);
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
#pragma unroll
        for (int j = cg * LOADS / NCG; j < (cg + 1) * LOADS / NCG; ++j) issue(j, kb);
        const i32x8 bv = bnext;
        const float sx = sxnext;
        if (cg + 1 < NCG) {
          bnext = read_bv(cg + 1);
          sxnext = read_sx(cg + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < GROUPS; ++g) {
          const f32x4 pr = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wv[g], bv, f32x4{0.f, 0.f, 0.f, 0.f},
                                                                            0, 0, 0, 127, 0, 127);
          const float f = sw[g] * sx;
          f32x4 c = acc[g / RG][g % RG][cg];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) c[jj] = __builtin_fmaf(pr[jj], f, c[jj]);
          acc[g / RG][g % RG][cg] = c;
        }
      }
    }
    wait_all_loads();  // the rings are idle: the epilogue reuses the LDS
    store_tile_lines<NCG, RG, TABLES, EPI, WAVES>(a, lds, acc, orow, live, wave, lane, (int64_t)s0 * BN);
  };
  if constexpr (TALL) {
    switch (ncg) {
      case 1: run_tall(std::integral_constant<int, 1>{}); break;
      case 2: run_tall(std::integral_constant<int, 2>{}); break;
      case 3: run_tall(std::integral_constant<int, 3>{}); break;
      case 4: run_tall(std::integral_constant<int, 4>{}); break;
      case 5: run_tall(std::integral_constant<int, 5>{}); break;
      case 6: run_tall(std::integral_constant<int, 6>{}); break;
      case 7: run_tall(std::integral_constant<int, 7>{}); break;
      default: run_tall(std::integral_constant<int, 8>{}); break;
    }
  } else {
    switch (ncg) {
      case 1: run_tile(std::integral_constant<int, 1>{}); break;
      case 2: run_tile(std::integral_constant<int, 2>{}); break;
      case 3: run_tile(std::integral_constant<int, 3>{}); break;
      case 4: run_tile(std::integral_constant<int, 4>{}); break;
      case 5: run_tile(std::integral_constant<int, 5>{}); break;
      case 6: run_tile(std::integral_constant<int, 6>{}); break;
      case 7: run_tile(std::integral_constant<int, 7>{}); break;
      default: run_tile(std::integral_constant<int, 8>{}); break;
    }
  }
}

template <int TABLES, int RG, int WAVES, int EPI>
hipError_t launch_prefill_fp8(const GroupedGemmArgs& a, hipStream_t stream) {
  constexpr int BN = WAVES * RG * 16;
  static std::atomic<uint64_t> lds_set{0};
  const hipError_t err =
      allow_full_lds(reinterpret_cast<const void*>(prefill_gemm_fp8_kernel<TABLES, RG, WAVES, EPI>), lds_set);
  if (err != hipSuccess) return err;
  constexpr bool TALL = WAVES * TABLES * RG * 2048 > kStripeBlockBytes;
  const int64_t R = TALL ? 1 : stripe_run_of(a);
  const int64_t items = (a.n / BN + R - 1) / R * a.max_tiles;
  const int64_t grid = prefill_grid(items);
  label_grouped_gemm(a, TABLES, a.tile_rows, BN, "_e4m3");
  return launch_kernel(prefill_gemm_fp8_kernel<TABLES, RG, WAVES, EPI>, dim3((unsigned)grid), dim3(64 * WAVES),
                       (size_t)kPrefillLds, stream, a);
}
template <int TABLES, int RG, int WAVES, int EPI>
hipError_t launch_prefill(const GroupedGemmArgs& a, hipStream_t stream) {
  constexpr int BN = WAVES * RG * 16;
  static std::atomic<uint64_t> lds_set{0};
  const hipError_t err =
      allow_full_lds(reinterpret_cast<const void*>(prefill_gemm_kernel<TABLES, RG, WAVES, EPI>), lds_set);
  if (err != hipSuccess) return err;
  const int64_t items = (int64_t)(a.n / BN) * a.max_tiles;  // one stripe per item (a.stripe_run unused)
  const int64_t grid = prefill_grid(items);
  label_grouped_gemm(a, TABLES, a.tile_rows, BN, "");
  return launch_kernel(prefill_gemm_kernel<TABLES, RG, WAVES, EPI>, dim3((unsigned)grid), dim3(64 * WAVES),
                       (size_t)kPrefillLds, stream, a);
}
}  // namespace

// Weight rows per table per work item of the prefill kernels (tall stripes
// of prefill_tall_bn rows where the GEMM args allow them and N is a multiple).
int prefill_bn(int tables) { return tables == 2 ? 8 * 16 : 8 * 32; }
int prefill_tall_bn(int tables) { return tables == 2 ? 8 * 32 : 8 * 64; }

int prefill_stripe_run(int tables) { return tables == 2 ? kRunGateUp : kRunDown; }


int prefill_wide_tile_rows() { return kBMWide; }

// The prefill kernels hold one block scale per lane (K <= 64 blocks of 128).
bool prefill_fits(int64_t n, int64_t k, int tables) {
  return n % prefill_bn(tables) == 0 && k % kScaleBlock == 0 && k / kScaleBlock <= 64;
}
// Their activation buffer offsets are 32-bit: rows x K bf16 must stay below 2 GiB.
bool prefill_rows_fit(int64_t x_rows, int64_t k) { return x_rows > 0 && x_rows * k * 2 <= INT32_MAX; }

bool prefill_quantizes_output(const GroupedGemmArgs& a, int tables, int epilogue) {
  return a.xq != nullptr && tables == 2 && epilogue == kEpiSwiglu && a.tall != 0 && a.n % prefill_tall_bn(2) == 0 &&
         prefill_fits(a.n, a.k, 2) && prefill_rows_fit(a.x_rows, a.k);
}
hipError_t launch_grouped_gemm_prefill(const GroupedGemmArgs& a, int tables, int epilogue, hipStream_t stream) {
  if (a.max_tiles <= 0) return hipSuccess;
  if (a.tile_desc == nullptr || (reinterpret_cast<uintptr_t>(a.tile_desc) & 15) != 0 || a.tile_rows <= 0)
    return hipErrorInvalidValue;
  // the FP8 kernel's tiles: at most 128 routes, each listed once
  if (a.xq != nullptr && (a.tile_rows > kBM || a.wide_twice != 0)) return hipErrorInvalidValue;
  if (!prefill_fits(a.n, a.k, tables) || !prefill_rows_fit(a.x_rows, a.k)) return hipErrorInvalidValue;
  if ((a.outq != nullptr) != (a.outq_scale != nullptr)) return hipErrorInvalidValue;
  if (a.outq != nullptr && !prefill_quantizes_output(a, tables, epilogue)) return hipErrorInvalidValue;
  if (a.xq != nullptr) {
    if (a.xscale == nullptr) return hipErrorInvalidValue;
    if (tables == 2 && epilogue == kEpiSwiglu)
      return a.tall && a.n % prefill_tall_bn(2) == 0 ? launch_prefill_fp8<2, 2, 8, kEpiSwiglu>(a, stream)
                                                     : launch_prefill_fp8<2, 1, 8, kEpiSwiglu>(a, stream);
    if (tables == 1 && epilogue == kEpiStoreBf16)
      return a.tall && a.n % prefill_tall_bn(1) == 0 ? launch_prefill_fp8<1, 4, 8, kEpiStoreBf16>(a, stream)
                                                     : launch_prefill_fp8<1, 2, 8, kEpiStoreBf16>(a, stream);
    return hipErrorInvalidValue;
  }
  // Tall stripes (512 weight rows a work item) wherever N allows them and the
  // work list fits them: tiles of at most 128 routes, or wider tiles listed
  // once per stripe half.
  const bool tall_list = a.tall != 0 && ((a.tile_rows > 0 && a.tile_rows <= kBM) || a.wide_twice != 0);
  if (tables == 2 && epilogue == kEpiSwiglu)
    return tall_list && a.n % prefill_tall_bn(2) == 0 ? launch_prefill<2, 2, 8, kEpiSwiglu>(a, stream)
                                                      : launch_prefill<2, 1, 8, kEpiSwiglu>(a, stream);
  if (tables == 1 && epilogue == kEpiStoreBf16)
    return tall_list && a.n % prefill_tall_bn(1) == 0 ? launch_prefill<1, 4, 8, kEpiStoreBf16>(a, stream)
                                                      : launch_prefill<1, 2, 8, kEpiStoreBf16>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace glm_moe
