// Internal interface between the C-ABI runtime (jma_runtime.cpp) and the gfx950 kernels
// (jma_kernels.hip). Not part of the public ABI; include/jmodels_attn.h is.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jma_plan.h"

namespace jma {

// Where one layer's K and V live. K: [sequence][layer][kv head][slot / B][key_length / W][B][W]
// (64-byte column panels per tile of B slots, k_index in jma_plan.h).
// V: [sequence][layer][kv head][slot / B][value_length][B] (B = 32 for f16, 16 for f32), the
// transposed block layout the PV matrix cores read directly; f16 blocks store slot r at
// index 8*((r%16)/4) + 4*(r/16) + r%4 (see perm32 in jma_kernels.hip).
struct KvView {
  void* k;
  void* v;
  uint64_t seq_stride_k, seq_stride_v;  // elements per sequence
  uint64_t layer_off_k, layer_off_v;    // elements from a sequence's base to this layer
  uint32_t cap;                         // physical slots per (sequence, layer, kv head)
  uint32_t ring;                        // 1: slot = position % cap, else slot = position
};

// Rows of one launch. Contiguous rows (one sequence, consecutive positions) have no count limit;
// listed rows are at most kMaxRows.
struct RowList {
  uint32_t count;
  uint32_t contiguous;  // 1: row i is (seq0, start + i); else (seq[i], pos[i])
  uint32_t seq0, start;
  uint32_t seq[kMaxRows];
  uint32_t pos[kMaxRows];
};

// Kernel arguments keep their scalars first so a kernel's opening scalar loads touch a few cache
// lines; the row tables come last and are read only when rows are listed.
struct AppendArgs {
  const float* q;       // [count][num_heads * dk]
  const float* k;       // [count][num_kv_heads * dk]
  const float* v;       // [count][num_kv_heads * dv]
  float* q_out;         // rotated q, f32, nullable
  const float* cos_t;   // [max_positions][pairs], nullable = no RoPE
  const float* sin_t;
  KvView kv;
  uint32_t pairs, neox, num_heads, num_kv_heads, dk, dv;
  uint32_t blocks_per_row;  // 256-thread blocks per row; one thread per element pair
  const float* q_norm_w;    // [dk] QK-norm weights applied before RoPE; null = none
  const float* k_norm_w;
  float norm_eps;
  uint32_t v_norm;          // 1: each v head RMS-normalised without a weight before it is stored
  RowList rows;
};

struct DecodeArgs {
  const float* q;       // [count][num_heads * dk]; rotated unless rope_q
  float* out;           // [count][num_heads * dv]
  float* part_acc;      // [items][16][dv]
  float* part_ml;       // [items][16][2]  (running max in log2 units, sum)
  float* part_f;        // [items][16][dv + 4] partials of the fused reduction (acc, m, l, 2 pad);
                        // every word holds 0xFFFFFFFF (not written) between launches
  uint32_t* counters;   // [rows][kv heads][head groups] arrival tickets, zero between launches;
                        // null = reduce_kernel combines the splits
  const float* k_new;   // [count][num_kv_heads * dk] raw keys to rotate and append; null = none
  const float* v_new;   // [count][num_kv_heads * dv]
  const float* cos_t;   // RoPE factors [max_positions][pairs]; null = no RoPE
  const float* sin_t;
  int* err;             // bit 0: non-finite score seen
  KvView kv;
  void* k_base;         // non-null: the rows are contiguous positions of one sequence, every row
  void* v_base;         // has the same split count, one head group; the layer's K / V base for
                        // that sequence (the kernel then skips the general indexing)
  float qscale;         // score scale * log2(e), folded into q
  // hgroups: virtual head groups per kv head = head groups of <= 16 query heads x slices, where
  // `slices` (1 or 4) cuts the value columns among that many workgroups (short rows at head dim
  // 256 or 512); each virtual group has its own work items, partials and arrival ticket.
  uint32_t num_heads, group, hgroups, window;
  uint32_t slices;
  uint32_t num_kv_heads;
  uint32_t pairs, neox, rope_q;  // rope_q: q is raw and the kernel rotates it
  // QK-norm of a fused decode: per-head RMS-norm weights for raw q (used when rope_q) and the new
  // k rows, applied before RoPE (null = none); v_norm: the new v rows are RMS-normalised without a
  // weight before they are stored.
  const float* q_norm_w;
  const float* k_norm_w;
  float norm_eps;
  uint32_t v_norm;
  uint32_t tiles_per_split;
  uint32_t total_items;
  uint32_t max_splits;  // splits of the row with the most; the grid is (max_splits, kv heads *
                        // head groups, rows)
  uint32_t ns_uniform;  // > 0: every row has this many splits
  uint32_t stream_nt;   // 1: tile loads non-temporal (a listed-rows launch streaming more K/V than
                        // the Infinity Cache could keep)
  RowList rows;
  uint32_t item_start[kMaxRows + 1];
  uint32_t nsplit[kMaxRows];
};

// Kernel arguments travel in the kernarg segment, at most 4 KiB.
static_assert(sizeof(DecodeArgs) <= 4096, "DecodeArgs exceeds the kernel argument limit");

struct PrefillArgs {
  KvView kv;
  const float* q;       // [n][num_heads][dk], rotated
  float* out;           // [n][num_heads][dv]
  int* err;
  float qscale;         // score scale * log2(e)
  uint32_t n, start, seq, window;
  uint32_t num_heads, num_kv_heads, group;
  uint32_t heads_per_stripe;  // query heads of one kv head sharing a stripe's 32 MFMA columns
  uint32_t rows_per_stripe;   // query rows of a stripe; rows * heads <= 32
  uint32_t head_groups;       // ceil(group / heads_per_stripe)
  uint32_t row_blocks;        // set by plan_prefill
  // The split_blocks longest row blocks (they run first) have their kv range cut in two halves,
  // each a workgroup; the later of the two to finish merges them (the tickets count stored
  // states). part: [pair][half][stripe][D / 8 chunks x 64 lanes + 32 columns] float4 words, no
  // initial value; tickets: [pair], zero between launches. The sliced prefills split their units
  // the same way (kernel 3b's stripes, kernel 3c's stripe pairs; planned by plan_prefill_pairs):
  // part [split unit][half][wave][4 kNb + 1][64 lanes] float4 words.
  uint32_t split_blocks;
  float* part;
  uint32_t* tickets;
};

// Launch plan of a prefill: row blocks, split blocks, the pairs of split workgroups and the bytes
// of partial words they need. split_tiles >= 2 splits every block with at least that many kv
// tiles; 0 or 1 never splits; -1 splits the blocks holding more than 1.5x the kv tiles an average
// compute unit (of cus) runs, and at least 48: a split costs a second prologue and an exchange,
// and pays only when the longest blocks would otherwise set the kernel's duration.
struct PrefillPlan {
  uint32_t row_blocks = 0, split_blocks = 0, pairs = 0;
  size_t part_bytes = 0;
};

// Stripes (32-column query groups) and kv groups of one prefill_kernel workgroup at head dim d.
constexpr int prefill_stripes(int d) { return d >= 256 ? 2 : 4; }
constexpr int kPrefillKvGroups = 2;

inline PrefillPlan plan_prefill(const PrefillArgs& a, int dk, int split_tiles, uint32_t cus) {
  if (dk != 32 && dk != 64 && dk != 128 && dk != 256) return PrefillPlan{};
  const uint32_t S = (uint32_t)prefill_stripes(dk);
  PrefillPlan p;
  const uint32_t rows_per_block = S * a.rows_per_stripe;
  p.row_blocks = (a.n + rows_per_block - 1) / rows_per_block;
  const uint64_t per_block = (uint64_t)a.head_groups * a.num_kv_heads;  // workgroups per row block
  auto tiles_of = [&](uint32_t rb) {  // kv tiles row block rb sees
    const uint32_t r0 = rb * rows_per_block, r1 = std::min(r0 + rows_per_block, a.n) - 1;
    const uint32_t w = a.window, p0 = a.start + r0;
    const uint32_t first = (w == 0 || p0 + 1 <= w) ? 0u : p0 + 1 - w;
    return (a.start + r1) / 32 + 1 - first / 32;
  };
  uint32_t min_tiles = (uint32_t)std::max(split_tiles, 2);
  if (split_tiles < 0) {
    // Automatic: a block is split when it holds more than 1.5x the tiles the average compute unit
    // runs, and at least 48 (the exchange of the halves' partials, through device-coherent
    // memory, costs about as much as 12 tiles): otherwise the longest blocks set the duration.
    uint64_t total = 0;
    for (uint32_t rb = 0; rb < p.row_blocks; ++rb) total += tiles_of(rb);
    const uint64_t per_cu = total * per_block / std::max<uint32_t>(cus, 1);
    min_tiles = (uint32_t)std::max<uint64_t>(48, per_cu * 3 / 2 + 1);
    // A grid that fills at most half the compute units also splits every block of 32 or more
    // tiles: a Gemma-3-1B-shaped prefill (4 Q / 1 KV heads, d 256, S 2048: 128 workgroups) took
    // 49.5 us with the rule above, 44.1 with this one (44.2-45.2 splitting from 2, 8 or 16 tiles,
    // 57.1 unsplit); grids of 256 or more workgroups measured best with the rule above.
    if ((uint64_t)p.row_blocks * per_block * 2 <= std::max<uint32_t>(cus, 1)) min_tiles = std::min(min_tiles, 32u);
  }
  if (split_tiles < 0 || split_tiles >= 2) {
    // Split the longest blocks, from the last one down.
    while (p.split_blocks < p.row_blocks && tiles_of(p.row_blocks - 1 - p.split_blocks) >= min_tiles)
      ++p.split_blocks;
  }
  p.pairs = p.split_blocks * (uint32_t)per_block;
  p.part_bytes = (size_t)p.pairs * 2 * (S * ((dk / 8) * 64 + 32) + S * kPrefillKvGroups) * 16;
  return p;
}

// Stripe-pair splits of kernel 3c: one workgroup per compute unit (the stage arrays take 128 KB
// of LDS) and a pair's cost grows with its row, so without splits the longest pairs set the
// duration. split_tiles >= 2 splits the trailing (longest) pairs of at least that many kv tiles;
// 0 or 1 never splits; -1 (automatic) splits every pair of 8 or more tiles when the pairs'
// workgroups fit on the compute units at once (with more, the dispatch already fills the units
// that short pairs free; kernel 3b then splits its stripes of 32 or more tiles, below). Measured on the Gemma 4 full-layer prefill (S 2048, 256 pairs of 1-64
// tiles): 115 us unsplit; every pair of at least 2 tiles split 94.8-95.2 us, of 8 93.4-94.0, of
// 16 97.9, of 48 93.8-95.4, of 64 113. The state exchange costs ~6 us (a timing-only copy
// without it: 88 us with every pair split); the rest of the gap to perfect balance is the extra
// prologues and the shared K/V traffic of a fully occupied device. The same rule on kernel 3b's
// stripes: the C1-shaped f32 prefill (256 stripes of 1-16 tiles) 38 -> 31 us.
constexpr uint32_t kPairPartWords = 33;  // float4 words per lane of a half's state: O^T (8 blocks x 4) and (m, l, lb)
constexpr uint32_t kPairAutoSplitTiles = 8;
struct PairPlan {
  uint32_t split_pairs = 0;
  size_t part_bytes = 0, ticket_bytes = 0;
};

// Waves of a kernel 3b workgroup at head dim d, and the float4 words per lane of one wave's state
// when its stripe is split (O^T slice, then m, l, lb).
constexpr int slice_waves(int d) { return d <= 32 ? 1 : d == 64 ? 2 : d <= 256 ? 4 : 8; }
constexpr uint32_t slice_state_words(int d) { return 4u * (uint32_t)(d / slice_waves(d) / 32) + 1u; }

// The split plan of kernel 3c's stripe pairs (unit_rows = 2 rows_per_stripe) or of kernel 3b's
// single stripes (unit_rows = rows_per_stripe), whose units run last-first: the trailing units
// with enough kv tiles run as two workgroups each (same rule and measurements as above).
inline PairPlan plan_prefill_pairs(const PrefillArgs& a, int split_tiles, uint32_t cus,
                                   uint32_t unit_rows = 0, uint32_t state_bytes_per_half = 0) {
  PairPlan p;
  const uint32_t R = unit_rows ? unit_rows : 2 * a.rows_per_stripe;
  const uint32_t pairs = unit_rows ? a.row_blocks : (a.row_blocks + 1) / 2;
  const uint32_t per = a.head_groups * a.num_kv_heads;  // workgroups per unit
  if (pairs == 0 || per == 0 || split_tiles == 0 || split_tiles == 1) return p;
  uint32_t min_tiles = split_tiles >= 2 ? (uint32_t)split_tiles : kPairAutoSplitTiles;
  if (split_tiles < 0 && (uint64_t)pairs * per > std::max<uint32_t>(cus, 1)) {
    // More units than compute units. Kernel 3c (one workgroup per compute unit) measured slower
    // with any split (Gemma 4 full layer at S 4096: 254 us unsplit, 268-309 split; 16 Q / 2 KV
    // heads at S 2048: 143 us against 143-189); kernel 3b's stripes (several workgroups per
    // compute unit) still gain from splitting their longest (C3's shape in f32, 1640 stripes of
    // 1-64 tiles: 351-353 us unsplit, 337 splitting 32+ tiles, 340 48+, 349 16+).
    if (unit_rows == 0) return p;
    min_tiles = 32;
  }
  auto tiles_of = [&](uint32_t pr) -> uint32_t {  // kv tiles of unit pr (the kernel's t1 - t0)
    const uint32_t r0 = pr * R, r1 = std::min(r0 + R, a.n) - 1;
    const uint32_t w = a.window, p0 = a.start + r0;
    const uint32_t first = (w == 0 || p0 + 1 <= w) ? 0u : p0 + 1 - w;
    return (a.start + r1) / 32 + 1 - first / 32;
  };
  // The trailing units with at least min_tiles (>= 2) tiles.
  uint32_t sp = 0;
  while (sp < pairs && tiles_of(pairs - 1 - sp) >= std::max<uint32_t>(min_tiles, 2)) ++sp;
  p.split_pairs = sp;
  p.part_bytes = (size_t)sp * per * 2 *
                 (state_bytes_per_half ? state_bytes_per_half : 4 * kPairPartWords * 64 * 16);
  p.ticket_bytes = (size_t)sp * per * sizeof(uint32_t);
  return p;
}

// Fixed device scratch of the allocation-free decode entry point: one file-scope array per GPU
// (in jma_kernels.hip), split into the regions a decode launch may need. Every call on a GPU
// shares its GPU's array; the split exchange leaves the exchange regions as it found them
// (tickets zero, partial words not-written), so they are prepared once per device.
struct FixedScratch {
  uint32_t* counters = nullptr;  // arrival tickets, zero between launches
  float* part_f = nullptr;       // fused split partials, every word 0xFFFFFFFF between launches
  float* part_acc = nullptr;     // partials combined by reduce_kernel
  float* part_ml = nullptr;
  float* qrot = nullptr;         // rotated queries of the separate-kernel path
  size_t counters_bytes = 0, part_f_bytes = 0, part_acc_bytes = 0, part_ml_bytes = 0, qrot_bytes = 0;
};
// Looks up the array's device address on `device` (which must be current) the first time it is
// asked for that device, prepares the exchange regions there with fill kernels on `stream` and
// waits for them; later calls return the cached addresses.
hipError_t fixed_scratch(int device, hipStream_t stream, FixedScratch* out);
// Restores the exchange regions of `device`'s array (after a reducer gave up waiting).
hipError_t fixed_scratch_reset(const FixedScratch& s, hipStream_t stream);

inline bool decode_supported(bool f16, int dk, int dv) {
  if (dk != dv) return false;
  if (f16) return dk == 32 || dk == 64 || dk == 128 || dk == 256 || dk == 512;
  return dk == 16 || dk == 32 || dk == 64 || dk == 128 || dk == 256 || dk == 512;
}
inline bool prefill_supported(int dk, int dv) {
  return dk == dv && (dk == 32 || dk == 64 || dk == 128 || dk == 256);
}
// Shapes of the sliced prefills: f32 caches at head dims 32-512 (d-sliced, kernel 3b), f16
// caches at 512 (stripe pairs, kernel 3c).
inline bool prefill_slice_supported(bool f16, int dk, int dv) {
  if (dk != dv) return false;
  return f16 ? dk == 512 : (dk == 32 || dk == 64 || dk == 128 || dk == 256 || dk == 512);
}

hipError_t launch_append(const AppendArgs& a, bool f16, hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, bool f16, int dk, int dv, hipStream_t stream);
hipError_t launch_reduce(const DecodeArgs& a, int dv, hipStream_t stream);
hipError_t launch_prefill(const PrefillArgs& a, int dk, int dv, hipStream_t stream);
// rows_per_stripe x heads_per_stripe columns per stripe, row_blocks = stripes; one stripe per
// workgroup (f32) or two (f16); no split.
hipError_t launch_prefill_slice(const PrefillArgs& a, bool f16, int dk, int dv, hipStream_t stream);

// ---------------------------------------------------------------- block-quantized projections

// Matrices one quantized-projection launch may serve (the reference's grouped calls take up to 16,
// backend-native/src/main/rust/model-kernels/src/lib.rs:96).
constexpr uint32_t kQMaxMatrices = 16;

struct QMatrix {
  const uint8_t* w;      // GGUF blocks: [rows][cols / 32] of qmat_block_bytes(fmt) bytes (Q4_0,
                         // Q8_0, Q5_0), or [rows][cols / 256] (Q4_K, Q5_K, Q6_K)
  float* out;            // [batch][rows]
  const float* addend;   // bias [rows] (addend_mode 1) or residual [batch][rows] (2); may be out
  uint32_t rows, tile0;  // tile0: this matrix's first workgroup
};

struct QMatArgs {
  const float* x;  // activations [batch][cols], 16-byte aligned
  uint32_t batch, cols, blocks, rows_per_tile, count, addend_mode;
  uint32_t chunk;       // activation rows per pass through LDS (plan_qmat)
  uint32_t group_rows;  // activation rows per workgroup along the grid's y (qmat_group_rows)
  QMatrix m[kQMaxMatrices];
};

// fmt: backend-native's code (qmat_kquant: blocks = cols / 256, else cols / 32), every matrix of
// the launch. tiles = sum of ceil(rows / rows_per_tile); the grid is tiles x ceil(batch /
// group_rows).
hipError_t launch_qmatvec(const QMatArgs& a, uint32_t fmt, uint32_t tiles, hipStream_t stream);
// Prefill-sized batches of the 32-element block formats (fmt 0, 1, 5): the activations quantized
// once to q (int8 [batch][cols]) and scales ([batch][cols / 32]), then the register-tiled
// product; tiles = sum of ceil(rows / kQGemmTile), grid tiles x ceil(batch / kQGemmTile).
hipError_t launch_q8_0_quant(const float* x, uint32_t batch, uint32_t cols, int8_t* q,
                             float* scales, hipStream_t stream);
hipError_t launch_qgemm(const QMatArgs& a, uint32_t fmt, uint32_t tiles, const int8_t* aq,
                        const float* as, hipStream_t stream);
// The same for Q4_K (fmt 2), Q6_K (fmt 3) and Q5_K (fmt 4) on Q8_K activations: q int8
// [batch][cols], scales [batch][cols / 256], sums int [batch][cols / 16] (Q6_K reads no sums).
hipError_t launch_q8_k_quant(const float* x, uint32_t batch, uint32_t cols, int8_t* q,
                             float* scales, int* sums, hipStream_t stream);
hipError_t launch_qkgemm(const QMatArgs& a, uint32_t fmt, uint32_t tiles, const int8_t* aq,
                         const float* as, const int* asum, hipStream_t stream);

}  // namespace jma
