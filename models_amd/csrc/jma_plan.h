// Decode launch planning and the index formulas of the decode split exchange, shared by the host
// runtime (jma_runtime.cpp), the kernels (jma_kernels.hip) and a CPU bounds check
// (tests/plan_check.cpp); and the launch planning of the quantized projections (jma_quant.hip,
// checked by tests/qmat_check.cpp). Plain C++: no HIP types, so it also builds with g++ alone.
#pragma once

#include <stdint.h>

#include <algorithm>

#if defined(__HIPCC__)
#define JMA_HD __host__ __device__ inline
#else
#define JMA_HD inline
#endif

namespace jma {

// Rows handled by one launch when their (sequence, position) pairs are passed as kernel
// arguments; larger batches are split into several launches by the runtime.
constexpr int kMaxRows = 128;
// Waves per decode workgroup at head dimension dk: the waves of one workgroup share a split and
// combine in LDS. Two waves per SIMD hide each other's instruction latency; at dk = 256 two tile
// buffers take half the register file, so one wave per SIMD.
constexpr int decode_waves(int dk) { return dk >= 256 ? 4 : 8; }
// Most splits one decode row may be cut into when the decode kernel reduces them itself (the
// reducing workgroup loads every split's partial); and when a separate reduce_kernel does
// (partials in part_acc / part_ml, reduced by one workgroup per head and 64 output elements).
constexpr int kMaxSplits = 32;
constexpr int kMaxWideSplits = 1024;
// Query heads one decode workgroup serves (the 16 MFMA columns); partial buffers reserve this
// many head slots per work item.
constexpr int kHeadSlots = 16;
// Fewest K/V bytes a decode split streams when the planner chooses its size (plan_decode).
constexpr uint64_t kMinSplitBytes = 96 * 1024;

// Storage block (slots) of the transposed V layout, and of the K tiles.
JMA_HD int v_block(bool f16) { return f16 ? 32 : 16; }

// K layout inside one (sequence, layer, kv head) region of cap * key_length elements: blocks of
// B = v_block slots, each stored as key_length / W column panels of B rows x W elements, where a
// panel row is 64 bytes (W = 32 f16 or 16 f32 elements). One matrix-core operand load of a tile
// (16 or 32 rows x 64 bytes across a wave) is then 1 KB of contiguous memory; row-major rows
// would spread it over 16 separate 64-byte pieces, which a compute unit issues 2-3x slower. A
// key length that is not a multiple of W keeps the rows whole (W = key_length).
JMA_HD uint32_t k_panel(uint32_t key_length, bool f16) {
  const uint32_t w = f16 ? 32u : 16u;
  return key_length % w == 0 ? w : key_length;
}
// Element offset of K element e of slot `slot` in its region.
JMA_HD uint64_t k_index(uint32_t slot, uint32_t e, uint32_t key_length, bool f16) {
  const uint32_t b = (uint32_t)v_block(f16), w = k_panel(key_length, f16);
  return (uint64_t)(slot - slot % b) * key_length + (uint64_t)(e / w) * (b * w) +
         (uint64_t)(slot % b) * w + e % w;
}

JMA_HD uint32_t first_visible(uint32_t position, uint32_t window) {
  // LlamaConfig.attentionStartPosition, causal branch (llama/LlamaConfig.java:184-195).
  return (window == 0 || position + 1 <= window) ? 0u : position + 1 - window;
}

// First work item of the group (row, rest = kv head * head groups + head group) whose ns splits
// are items item0 .. item0 + ns - 1. ns_uniform > 0: every row has ns_uniform splits; else row
// `row` starts at item_start_row.
JMA_HD uint64_t group_item0(uint32_t ns_uniform, uint32_t item_start_row, uint32_t row,
                            uint32_t hkv, uint32_t hgroups, uint32_t rest, uint32_t ns) {
  return ns_uniform ? ((uint64_t)row * hkv * hgroups + rest) * ns
                    : (uint64_t)item_start_row + (uint64_t)rest * ns;
}

// Arrival-ticket counter of a group: [row][kv head][head group].
JMA_HD uint64_t group_counter(uint32_t row, uint32_t hkv, uint32_t kvh, uint32_t hgroups, uint32_t hg) {
  return ((uint64_t)row * hkv + kvh) * hgroups + hg;
}

// Fused exchange: float index of element e (e < dv; e = dv is m, dv + 1 is l) of head slot hs of
// work item `item`; each (item, head slot) holds dv + 4 floats.
JMA_HD uint64_t fused_part_float(uint64_t item, uint32_t hs, uint32_t dv, uint32_t e) {
  return (item * kHeadSlots + hs) * (dv + 4) + e;
}
// Separate reduction: element e of head slot hs of item in part_acc, and its (m, l) in part_ml.
// With column slices, the slices of one head group write their columns into a single DV-wide
// item: the item of (row, kv head, head group, split) in the plan without slices, which is the
// group's virtual item numbering with `hgroups` / slices groups and the row's first item / slices
// (every row holds slices times the items it would hold unsliced). reduce_kernel reads it as an
// unsliced plan's.
JMA_HD uint64_t sep_item(uint32_t ns_uniform, uint32_t item_start_row, uint32_t row, uint32_t hkv,
                         uint32_t hgroups, uint32_t slices, uint32_t kvh, uint32_t hg, uint32_t ns,
                         uint32_t split) {
  const uint32_t hgr = hgroups / slices;
  return group_item0(ns_uniform, item_start_row / slices, row, hkv, hgr, kvh * hgr + hg, ns) + split;
}
JMA_HD uint64_t sep_acc_float(uint64_t item, uint32_t hs, uint32_t dv, uint32_t e) {
  return (item * kHeadSlots + hs) * dv + e;
}
JMA_HD uint64_t sep_ml_float(uint64_t item, uint32_t hs) { return (item * kHeadSlots + hs) * 2; }

// Split plan of one decode launch of `count` <= kMaxRows rows at positions[]: every workgroup
// streams tiles_per_split tiles, at least tiles_per_wave per wave, raised until the launch is near
// target_blocks workgroups and no row needs more than kMaxSplits splits (the decode kernel then
// reduces the splits itself). When that cap would leave the launch with fewer than a quarter of
// the target workgroups (few long rows: one sequence at a long context with few KV heads), rows
// are cut wider, up to kMaxWideSplits splits, and reduce_kernel combines them (`separate`); a
// context running separate kernels (`unfused`) always does.
//
// Column slices: at head dim 256 or 512 a launch of few workgroups (short rows: a sliding-window
// layer) cuts each head's value columns among `slices` = 4 workgroups, each computing q.K over its
// tiles and V and the output for a quarter of the columns. That gives four times the workgroups,
// each streaming K and a quarter of V (instead of all of V), with a quarter of the partials to
// exchange per split. The slices are virtual head groups: `hgroups` is head groups x slices. At
// head dim 512 a plan takes four slices when the sliced launch stays within half the target,
// else none (two slices, which read K twice, measured 27.5 against 22.6 us for one row at
// 32 704 positions); wide plans' slices share the separate reduction's items (sep_item).
struct DecodePlan {
  uint32_t hgroups = 0, slices = 1, tiles_per_split = 0, total_items = 0, max_splits = 0, ns_uniform = 0;
  bool any_split = false, separate = false;
  uint32_t nsplit[kMaxRows] = {};
  uint32_t item_start[kMaxRows + 1] = {};
  uint64_t part_f_bytes = 0, counter_bytes = 0, acc_bytes = 0, ml_bytes = 0;
};

inline DecodePlan plan_decode(uint32_t count, const uint32_t* positions, uint32_t window,
                              uint32_t hkv, uint32_t group, int dk, int dv, bool f16,
                              int target_blocks, int tiles_per_wave, bool unfused,
                              int min_split_tiles = 0) {
  DecodePlan p;
  const uint32_t blk = (uint32_t)v_block(f16);
  p.hgroups = (group + kHeadSlots - 1) / kHeadSlots;
  uint32_t ntiles[kMaxRows];
  uint64_t units = 0;
  uint32_t max_tiles = 0;
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t pos = positions[i];
    const uint32_t first = first_visible(pos, window);
    ntiles[i] = pos / blk - first / blk + 1;
    max_tiles = std::max(max_tiles, ntiles[i]);
    units += (uint64_t)ntiles[i] * hkv * p.hgroups;
  }
  const uint64_t target = (uint64_t)std::max(target_blocks, 1);
  const uint64_t tile_bytes = (uint64_t)blk * (uint64_t)(dk + dv) * (f16 ? 2u : 4u);
  uint64_t tps = min_split_tiles > 0 ? (uint64_t)min_split_tiles
                                     : (uint64_t)decode_waves(dk) * (uint64_t)std::max(tiles_per_wave, 1);
  // Every split streams at least kMinSplitBytes: a split's exchange (its partial stored, polled and
  // combined) costs about as much as streaming that many bytes through one compute unit, so
  // smaller splits add exchange work without saving time. One tile per wave already streams that
  // much at head dim 128 and above; at 64 and below the split takes more tiles (C2, d 64: 12
  // tiles, 11 splits, 7.6 against 8.1 us per launch with 8 tiles, 17 splits).
  if (min_split_tiles == 0) tps = std::max<uint64_t>(tps, (kMinSplitBytes + tile_bytes - 1) / tile_bytes);
  const uint64_t base_tps = tps;
  tps = std::max<uint64_t>(tps, (units + target - 1) / target);
  const uint64_t tps_fused = std::max<uint64_t>(tps, (max_tiles + kMaxSplits - 1) / kMaxSplits);
  bool wide = false;
  if (tps_fused > tps && !unfused) {
    uint64_t fused_items = 0;
    for (uint32_t i = 0; i < count; ++i)
      fused_items += (ntiles[i] + tps_fused - 1) / tps_fused * hkv * p.hgroups;
    wide = fused_items * 4 < target;
  }
  tps = wide ? std::max<uint64_t>(tps, (max_tiles + kMaxWideSplits - 1) / kMaxWideSplits)
             : tps_fused;
  // Short rows: a launch of few workgroups (under an eighth of the target) that each stream more
  // than 64 KB waits on the per-CU load issue rate (~64 KB per us), so it takes half the tiles
  // per split (at least one per two waves) and twice the workgroups, as long as each extra
  // split's partial (dv + 4 floats per query head, read back by the reducer) stays within 2 KB.
  const uint64_t part_bytes = (uint64_t)std::min<uint32_t>(group, kHeadSlots) * (dv + 4) * 4;
  if (min_split_tiles == 0 && !wide && tps == base_tps && tps >= 2 && tps * tile_bytes > 65536 &&
      part_bytes <= 2048 && (max_tiles + tps / 2 - 1) / (tps / 2) <= (uint64_t)kMaxSplits) {
    uint64_t few = 0;
    for (uint32_t i = 0; i < count; ++i) few += (ntiles[i] + tps - 1) / tps * hkv * p.hgroups;
    if (few * 8 < target) tps /= 2;
  }
  // Column slices (above): fused plans of at most one tile per wave at head dim 256 (the sliced
  // instance keeps one tile buffer) whose sliced launch stays within half the target; at 512, four
  // slices under the same rule.
  if (!unfused && dk == dv &&
      (dk == 512 || (!wide && dk == 256 && tps <= (uint64_t)decode_waves(dk)))) {
    uint64_t n = 0;
    for (uint32_t i = 0; i < count; ++i) n += (ntiles[i] + tps - 1) / tps * hkv * p.hgroups;
    if (n * 4 * 2 <= target) {
      p.slices = 4;
      p.hgroups *= 4;
    }
  }
  p.tiles_per_split = (uint32_t)tps;
  uint32_t items = 0;
  bool uniform = true;
  for (uint32_t i = 0; i < count; ++i) {
    p.item_start[i] = items;
    p.nsplit[i] = (uint32_t)((ntiles[i] + tps - 1) / tps);
    p.any_split |= p.nsplit[i] > 1;
    uniform &= p.nsplit[i] == p.nsplit[0];
    p.max_splits = std::max(p.max_splits, p.nsplit[i]);
    items += p.nsplit[i] * hkv * p.hgroups;
  }
  p.item_start[count] = items;
  p.total_items = items;
  p.ns_uniform = uniform ? p.nsplit[0] : 0u;
  p.separate = p.any_split && (unfused || wide);
  if (p.separate) {
    p.acc_bytes = (uint64_t)items / p.slices * kHeadSlots * dv * 4;
    p.ml_bytes = (uint64_t)items / p.slices * kHeadSlots * 2 * 4;
  } else if (p.any_split) {
    p.part_f_bytes = (uint64_t)items * kHeadSlots * (dv / p.slices + 4) * 4;
    p.counter_bytes = (uint64_t)count * hkv * p.hgroups * 4;
  }
  return p;
}

// ---------------------------------------------------------------- split prefill units
//
// Work items of a prefill launch whose units (kernel 3b's stripes, kernel 3c's stripe pairs) run
// last-first (the longest causal ranges first), the trailing split_units of them as two items each
// (they come first), one per half of the unit's kv tiles [t0, t1); the first half is kPairLead
// tiles shorter (at least one tile; a split unit has two or more). Shared by the kernels, their
// launches (grid size) and a CPU check that every unit's tiles are covered exactly once.
constexpr uint32_t kPairLead = 2;  // tiles by which a split unit's first half is the shorter

struct SplitItem {
  uint32_t unit, half;
  bool split;
};
JMA_HD uint64_t split_items(uint32_t units, uint32_t split_units) {
  return (uint64_t)units + split_units;
}
JMA_HD SplitItem split_item(uint32_t units, uint32_t split_units, uint32_t item) {
  SplitItem r;
  r.split = item < 2 * split_units;
  r.half = r.split ? item & 1u : 0u;
  r.unit = units - 1 - (r.split ? item / 2 : item - split_units);
  return r;
}
// The item's tiles [tb, te) of its unit's [t0, t1).
JMA_HD void split_range(uint32_t t0, uint32_t t1, const SplitItem& it, uint32_t& tb, uint32_t& te) {
  const uint32_t n = t1 - t0;
  const uint32_t lead = n < kPairLead ? n : kPairLead;
  const uint32_t first = (n - lead) / 2 > 1u ? (n - lead) / 2 : 1u;
  const uint32_t tm = t0 + first;
  tb = it.split && it.half != 0u ? tm : t0;
  te = it.split && it.half == 0u ? tm : t1;
}

// ---------------------------------------------------------------- quantized projections
//
// Launch planning of the block-quantized projections (jma_quant.hip), shared by the runtime and a
// CPU bounds check (tests/qmat_check.cpp). A launch serves every matrix of one weight format:
// workgroup (x, y) takes rows_per_tile rows of one matrix (tiles in matrix order) and the
// activation rows y * group_rows .. + group_rows - 1, which pass through its LDS chunk rows at a
// time while the tile's weight blocks stay in its registers or caches.

// backend-native's weight codes (RS:150-161): 0 Q4_0, 1 Q8_0, 2 Q4_K, 3 Q6_K, 4 Q5_K, 5 Q5_0.
JMA_HD bool qmat_kquant(uint32_t fmt) { return fmt == 2 || fmt == 3 || fmt == 4; }
JMA_HD uint32_t qmat_block_elems(uint32_t fmt) { return qmat_kquant(fmt) ? 256u : 32u; }
// GGUF block bytes (RS:87-92).
JMA_HD uint32_t qmat_block_bytes(uint32_t fmt) {
  return fmt == 0 ? 18u : fmt == 1 ? 34u : fmt == 2 ? 144u : fmt == 3 ? 210u : fmt == 4 ? 176u : 22u;
}

// Dynamic LDS of one workgroup for `chunk` activation rows: Q8_0 activations, their scales and
// block sums, then the tile's (scale product, integer dot) terms per (activation row, tile row).
JMA_HD uint64_t qmatvec_lds_bytes(uint32_t chunk, uint32_t cols, uint32_t rows_per_tile) {
  const uint64_t K = cols / 32u;
  return ((uint64_t)chunk * cols + 15u) / 16u * 16u + (uint64_t)chunk * K * 8u +
         2u * (uint64_t)chunk * rows_per_tile * (K + 1u) * 4u;
}
// K-quants: Q8_K activations, scales and 16-element sums, then 4 (Q4_K, Q5_K) or 9 (Q6_K)
// floats per (activation row, tile row, 256-block).
JMA_HD uint64_t qkmatvec_lds_bytes(uint32_t fmt, uint32_t chunk, uint32_t cols, uint32_t rows_per_tile) {
  const uint64_t KB = cols / 256u, nt = fmt == 3 ? 9u : 4u;
  return ((uint64_t)chunk * cols + 15u) / 16u * 16u + (uint64_t)chunk * KB * 4u +
         (uint64_t)chunk * (cols / 16u) * 4u + (uint64_t)chunk * rows_per_tile * (KB * nt + 1u) * 4u;
}

constexpr uint64_t kQMatLds = 64u * 1024u;   // dynamic LDS a projection workgroup may take
constexpr uint32_t kQMatMaxChunk = 8;        // activation rows per pass
constexpr uint32_t kQMatTargetBlocks = 1024;  // workgroups a projection launch aims for

// Batches of at least kQGemmMinBatch activation rows run as a register-tiled product
// (qgemm_kernel, qkgemm_kernel, q6gemm_kernel): tiles of kQGemmTile weight rows x kQGemmTile
// activation rows, kQGemmKc 32-element blocks (or one 256-element block) staged per step.
constexpr uint32_t kQGemmMinBatch = 16;
constexpr uint32_t kQGemmTile = 64;
constexpr uint32_t kQGemmKc = 4;

struct QMatPlan {
  uint32_t rows_per_tile = 0, chunk = 0;  // 0: cols too large for one workgroup's LDS
};

// Rows per tile (up to 512 (row, block) terms for the 32-element formats, two per thread; 64 for
// the K-quants, eight threads each) and activation rows per pass, the largest that keep every
// format of the call within kQMatLds.
inline QMatPlan plan_qmat(const uint32_t* formats, uint32_t count, uint32_t cols) {
  QMatPlan p;
  if (count == 0) return p;
  const bool kq = qmat_kquant(formats[0]);
  const uint32_t K = cols / qmat_block_elems(formats[0]);
  if (K == 0) return p;
  auto lds = [&](uint32_t chunk, uint32_t tile) {
    uint64_t m = 0;
    for (uint32_t i = 0; i < count; ++i)
      m = std::max(m, kq ? qkmatvec_lds_bytes(formats[i], chunk, cols, tile)
                         : qmatvec_lds_bytes(chunk, cols, tile));
    return m;
  };
  uint32_t tile = std::max<uint32_t>(1u, std::min<uint32_t>(64u, (kq ? 64u : 512u) / K));
  while (tile > 1 && lds(1, tile) > kQMatLds) tile /= 2;
  if (lds(1, tile) > kQMatLds) return p;
  uint32_t chunk = kQMatMaxChunk;
  while (chunk > 1 && lds(chunk, tile) > kQMatLds) --chunk;
  p.rows_per_tile = tile;
  p.chunk = chunk;
  return p;
}

// Activation rows per workgroup of a launch with `tiles` weight tiles: whole passes, as few as
// keep the launch near kQMatTargetBlocks workgroups (one pass each at decode batches).
JMA_HD uint32_t qmat_group_rows(uint32_t batch, uint32_t chunk, uint32_t tiles) {
  const uint64_t passes = (batch + chunk - 1) / chunk;
  uint64_t per = (passes * tiles + kQMatTargetBlocks - 1) / kQMatTargetBlocks;
  per = per < 1 ? 1 : (per > passes ? passes : per);
  return (uint32_t)(per * chunk);
}

}  // namespace jma
