// CPU bounds check of the decode launch plans (built with g++ and AddressSanitizer /
// UndefinedBehaviorSanitizer by tests/test_plan_cpu.py). For every configured decode shape it
// plans the launch with the runtime's own planner (models_amd/csrc/jma_plan.h), then walks every
// workgroup of the grid the way decode_kernel and reduce_kernel index their buffers (the same
// index functions) and checks:
//   - every (row, kv head, head group, split) work item is distinct and inside total_items;
//   - a row's splits cover its visible kv tiles exactly once;
//   - every partial word a producer writes or a reducer reads lies inside the planned buffer, the
//     fused exchange within the 32-bit byte offsets its buffer descriptor takes;
//   - arrival-ticket counters lie inside the planned counter buffer;
//   - split counts stay within the fused (32) or separate (1024) caps;
//   - the separate reduction (reduce_kernel) reads only items its row's groups own.
// It also checks the K tile layout (k_index): a bijection of every (slot, element) of a region,
// and the addresses the kernels form for their K loads (decode operand loads, prefill
// direct-to-LDS chunks) name the elements k_index places there, each decode operand load reading
// one contiguous 1 KB run.
// Prints one line per case and "ok" at the end; exits non-zero on the first failed check.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <string>
#include <vector>

#include "jma_plan.h"

using namespace jma;

namespace {

struct Case {
  std::string name;
  std::vector<uint32_t> pos;
  uint32_t window, hkv, group;
  int dk, dv;
  bool f16;
  int target, tiles_per_wave;
  bool unfused;
  uint32_t ring;  // ring capacity of the layer, 0 = linear
  int min_split = 0;  // JMA_DECODE_MIN_SPLIT_TILES (0: the planner's own choice)
};

[[noreturn]] void die(const Case& c, const std::string& what) {
  fprintf(stderr, "FAILED %s: %s\n", c.name.c_str(), what.c_str());
  exit(1);
}

void check(const Case& c) {
  const uint32_t count = (uint32_t)c.pos.size();
  if (count == 0 || count > (uint32_t)kMaxRows) die(c, "row count");
  const DecodePlan p = plan_decode(count, c.pos.data(), c.window, c.hkv, c.group, c.dk, c.dv, c.f16,
                                   c.target, c.tiles_per_wave, c.unfused, c.min_split);
  const uint32_t blk = (uint32_t)v_block(c.f16);
  const uint32_t hgroups = p.hgroups;  // virtual head groups: head groups x column slices
  if (p.slices != 1 && p.slices != 4) die(c, "column slices");
  if (hgroups != (c.group + kHeadSlots - 1) / kHeadSlots * p.slices) die(c, "head groups");
  if (p.slices > 1 && (c.dk < 256 || (c.dk == 256 && (p.separate || p.tiles_per_split > 4))))
    die(c, "column slices outside the sliced instances (fused d 256 one tile per wave, d 512)");
  if (p.part_f_bytes > 0x7FFFFFF0ull) die(c, "fused partials exceed 32-bit buffer offsets");
  std::vector<int> owner(p.total_items, 0);
  // Separate plans: (item, slice) pairs of part_acc, each written by one workgroup.
  std::vector<int> sep_owner(p.separate ? p.total_items : 0, 0);
  const uint64_t part_f_floats = p.part_f_bytes / 4, acc_floats = p.acc_bytes / 4;
  const uint64_t ml_floats = p.ml_bytes / 4, counters = p.counter_bytes / 4;
  for (uint32_t row = 0; row < count; ++row) {
    const uint32_t ns = p.ns_uniform ? p.ns_uniform : p.nsplit[row];
    if (ns != p.nsplit[row]) die(c, "uniform split count differs from the row's");
    if (ns == 0 || ns > p.max_splits) die(c, "split count outside [1, max_splits]");
    if (ns > (uint32_t)(p.separate ? kMaxWideSplits : kMaxSplits)) die(c, "split count above the cap");
    const uint32_t pos = c.pos[row];
    const uint32_t first = first_visible(pos, c.window);
    if (c.ring && pos - first + 1 > c.ring) die(c, "window wider than the ring");
    const uint32_t t_begin = first / blk, t_end = pos / blk + 1;
    std::vector<int> seen(t_end - t_begin, 0);
    for (uint32_t rest = 0; rest < c.hkv * hgroups; ++rest) {
      const uint32_t kvh = rest / hgroups, hgv = rest % hgroups, hg = hgv / p.slices;
      const uint32_t slice = hgv % p.slices;
      const uint32_t nreal = std::min<uint32_t>(kHeadSlots, c.group - hg * kHeadSlots);
      const uint32_t dvs = c.dv / p.slices;  // value columns of the slice
      const uint64_t item0 = group_item0(p.ns_uniform, p.item_start[row], row, c.hkv, hgroups, rest, ns);
      if (item0 + ns > p.total_items) die(c, "group items past total_items");
      if (ns > 1 && !p.separate) {
        const uint64_t gid = group_counter(row, c.hkv, kvh, hgroups, hgv);
        if (gid >= counters) die(c, "arrival ticket outside the counter buffer");
      }
      for (uint32_t split = 0; split < p.max_splits; ++split) {
        if (split >= ns) continue;  // the kernel's early exit for rows with fewer splits
        const uint64_t item = item0 + split;
        if (owner[item]++) die(c, "work item shared by two workgroups");
        const uint32_t s_t0 = t_begin + split * p.tiles_per_split;
        const uint32_t s_t1 = std::min(s_t0 + p.tiles_per_split, t_end);
        if (s_t0 >= s_t1) die(c, "a split without tiles");
        if (rest == 0)
          for (uint32_t t = s_t0; t < s_t1; ++t) seen[t - t_begin]++;
        if (p.slices > 1 && c.dk == 256 && s_t1 - s_t0 > 4) die(c, "sliced d256 split with more than one tile per wave");
        if (ns == 1) continue;
        for (uint32_t hs = 0; hs < nreal; ++hs) {
          if (p.separate) {
            // a slice writes its columns of the head group's item (sep_item)
            const uint64_t it = p.slices == 1 ? item
                                              : sep_item(p.ns_uniform, p.item_start[row], row, c.hkv,
                                                         hgroups, p.slices, kvh, hg, ns, split);
            if (sep_acc_float(it, hs, c.dv, slice * dvs + dvs - 1) >= acc_floats) die(c, "part_acc index");
            if (sep_ml_float(it, hs) + 1 >= ml_floats) die(c, "part_ml index");
            if (hs == 0 && sep_owner[it * p.slices + slice]++) die(c, "part_acc columns written twice");
          } else {
            // producer stores acc quads and the (m, l, pad, pad) word group; the reducer reads
            // the same words of every split of the group
            if (fused_part_float(item, hs, dvs, dvs + 3) >= part_f_floats) die(c, "part_f index");
            if (fused_part_float(item, hs, dvs, dvs + 3) * 4 + 16 > 0x7FFFFFF0ull)
              die(c, "part_f byte offset beyond the buffer descriptor");
          }
        }
      }
      if (p.separate && ns > 1) {
        // reduce_kernel: one workgroup per (row, query head, 64-element chunk) reads the row's
        // group base + split for split < ns
        const uint32_t hgr = hgroups / p.slices;
        const uint64_t base = group_item0(p.ns_uniform, p.item_start[row] / p.slices, row, c.hkv,
                                          hgr, kvh * hgr + hg, ns);
        const uint64_t prod = p.slices == 1 ? item0
                                            : sep_item(p.ns_uniform, p.item_start[row], row, c.hkv,
                                                       hgroups, p.slices, kvh, hg, ns, 0);
        if (base != prod) die(c, "reduce_kernel group base differs from the producers'");
        for (uint32_t hs = 0; hs < nreal; ++hs)
          if (sep_acc_float(base + ns - 1, hs, c.dv, c.dv - 1) >= acc_floats) die(c, "reduce read");
      }
    }
    for (uint32_t t = 0; t < seen.size(); ++t)
      if (seen[t] != 1) die(c, "kv tile " + std::to_string(t_begin + t) + " covered " +
                                   std::to_string(seen[t]) + " times");
  }
  for (uint64_t i = 0; i < p.total_items; ++i)
    if (owner[i] != 1) die(c, "work item " + std::to_string(i) + " not written exactly once");
  if (p.separate) {
    // every (item, slice) of a row with splits is written exactly once, none past the items
    uint64_t written = 0;
    for (uint64_t i = 0; i < sep_owner.size(); ++i) {
      if (sep_owner[i] > 1) die(c, "part_acc columns written twice");
      written += sep_owner[i];
    }
    uint64_t want = 0;
    for (uint32_t row = 0; row < count; ++row)
      if (p.nsplit[row] > 1) want += (uint64_t)p.nsplit[row] * c.hkv * hgroups;
    if (written != want) die(c, "part_acc columns not covered exactly once");
  }
  printf("%-44s rows %3u tiles/split %5u splits <= %4u items %7u slices %u %s %8.1f KiB\n", c.name.c_str(),
         count, p.tiles_per_split, p.max_splits, p.total_items, p.slices,
         p.separate ? "separate" : (p.any_split ? "fused   " : "single  "),
         (double)(p.separate ? p.acc_bytes + p.ml_bytes : p.part_f_bytes) / 1024.0);
}

// Deterministic ragged lengths (a 64-bit LCG), uniform on [lo, hi].
std::vector<uint32_t> ragged(uint32_t n, uint32_t lo, uint32_t hi, uint64_t seed) {
  std::vector<uint32_t> v(n);
  uint64_t x = seed;
  for (uint32_t i = 0; i < n; ++i) {
    x = x * 6364136223846793005ull + 1442695040888963407ull;
    v[i] = lo + (uint32_t)((x >> 33) % (hi - lo + 1));
  }
  return v;
}

std::vector<uint32_t> run(uint32_t start, uint32_t n) {
  std::vector<uint32_t> v(n);
  for (uint32_t i = 0; i < n; ++i) v[i] = start + i;
  return v;
}

void k_fail(const std::string& what) {
  fprintf(stderr, "FAILED K layout: %s\n", what.c_str());
  exit(1);
}

// The prefill kernel's XOR swizzle of 16-byte chunks inside a K tile row (swz_k in
// jma_kernels.hip).
uint32_t swz_k(int d, uint32_t r) {
  if (d >= 128) return (r & 7u) | ((r >> 1) & 8u);
  if (d == 64) return r & 7u;
  return (r >> 1) & 3u;
}

void check_k_layout(uint32_t dk, bool f16, uint32_t cap) {
  const std::string tag = std::string(f16 ? "f16" : "f32") + " dk " + std::to_string(dk);
  std::vector<uint8_t> seen((size_t)cap * dk, 0);
  for (uint32_t slot = 0; slot < cap; ++slot)
    for (uint32_t e = 0; e < dk; ++e) {
      const uint64_t i = k_index(slot, e, dk, f16);
      if (i >= (uint64_t)cap * dk || seen[i]++) k_fail(tag + ": not a bijection");
    }
  const uint32_t blk = (uint32_t)v_block(f16);
  if (dk % (f16 ? 32u : 16u) != 0) return;  // decode and prefill take these widths only
  // Decode operand loads (Tile::load_k): lane (g, c16) of the load (b, c) of the tile at slot0.
  for (uint32_t slot0 = 0; slot0 < cap; slot0 += blk)
    for (uint32_t b = 0; b < (f16 ? 2u : 1u); ++b)
      for (uint32_t c = 0; c < dk / (f16 ? 32u : 16u); ++c) {
        uint64_t lo = ~0ull, hi = 0;
        for (uint32_t lane = 0; lane < 64; ++lane) {
          const uint32_t g = lane >> 4, c16 = lane & 15;
          const uint32_t n = f16 ? 8u : 4u;  // elements per 16-byte load
          const uint64_t a = f16 ? (uint64_t)slot0 * dk + c * 1024 + (16 * b + c16) * 32 + 8 * g
                                 : (uint64_t)slot0 * dk + c * 256 + c16 * 16 + 4 * g;
          for (uint32_t j = 0; j < n; ++j) {
            const uint32_t row = slot0 + 16 * b + c16, e = (f16 ? 32 : 16) * c + n * g + j;
            if (a + j != k_index(row, e, dk, f16)) k_fail(tag + ": decode operand load");
          }
          lo = std::min(lo, a);
          hi = std::max(hi, a + n);
        }
        if ((hi - lo) * (f16 ? 2 : 4) != 1024) k_fail(tag + ": decode operand load not contiguous");
      }
  if (!f16 || dk > 256) return;
  // Prefill direct-to-LDS chunks: chunk c, lane l stages 16 bytes of tile row rk.
  const uint32_t nc = dk / 8;
  for (uint32_t c = 0; c < dk / 16; ++c)
    for (uint32_t lane = 0; lane < 64; ++lane) {
      const uint32_t rk = c * (512 / dk) + lane / nc;
      const uint32_t cc = (lane % nc) ^ swz_k((int)dk, rk);
      const uint64_t off = (cc / 4) * (32 * 32) + rk * 32 + 8 * (cc % 4);
      for (uint32_t j = 0; j < 8; ++j)
        if (off + j != k_index(rk, 8 * cc + j, dk, true)) k_fail(tag + ": prefill chunk");
    }
}

}  // namespace

// Split prefill units (kernels 3b and 3c): the launch's items cover every unit's kv tiles exactly
// once, a split unit's two halves nonempty and adjacent.
void check_split_items(uint32_t units, uint32_t split_units, uint32_t (*tiles)(uint32_t)) {
  std::vector<std::vector<std::pair<uint32_t, uint32_t>>> seen(units);
  const uint64_t n = jma::split_items(units, split_units);
  for (uint32_t item = 0; item < n; ++item) {
    const jma::SplitItem it = jma::split_item(units, split_units, item);
    if (it.unit >= units) k_fail("split item maps past the units");
    const uint32_t t1 = tiles(it.unit) + 3, t0 = 3;
    if (it.split && t1 - t0 < 2) k_fail("split unit with fewer than two tiles");
    uint32_t tb, te;
    jma::split_range(t0, t1, it, tb, te);
    if (!(t0 <= tb && tb < te && te <= t1)) k_fail("empty or out-of-range split half");
    seen[it.unit].push_back({tb, te});
  }
  for (uint32_t u = 0; u < units; ++u) {
    const bool split = u + split_units >= units;
    auto& r = seen[u];
    std::sort(r.begin(), r.end());
    const uint32_t t1 = tiles(u) + 3;
    if (r.size() != (split ? 2u : 1u) || r.front().first != 3 || r.back().second != t1 ||
        (split && r[0].second != r[1].first))
      k_fail("unit " + std::to_string(u) + " not covered exactly once");
  }
}

int main() {
  for (uint32_t units : {1u, 2u, 7u, 64u, 256u, 257u})
    for (uint32_t frac : {0u, 1u, 2u, 4u})
      check_split_items(units, frac == 0 ? 0 : (units * frac + 3) / 4,
                        [](uint32_t u) -> uint32_t { return 2 + u / 3; });
  printf("split prefill items: every unit covered once\n");
  std::vector<Case> cases;
  // BASELINE configs at their configured sizes (one decode row per launch unless listed).
  cases.push_back({"C1 f32 d128 16/8 @512", {512}, 0, 8, 2, 128, 128, false, 512, 1, false, 0});
  for (uint32_t p : {4096u, 4159u, 4223u})
    cases.push_back({"C2 f16 d64 32/8 @" + std::to_string(p), {p}, 0, 8, 4, 64, 64, true, 512, 1, false, 0});
  cases.push_back({"C1 prefill rows (f32, listed)", run(0, 128), 0, 8, 2, 128, 128, false, 512, 1, false, 0});
  cases.push_back({"C4 64 ragged U[256,16384] d128 12/2", ragged(64, 256, 16384, 4), 0, 2, 6, 128, 128, true, 512, 1, false, 0});
  for (uint32_t p : {32704u, 32735u, 32767u}) {
    cases.push_back({"C5 global d256 4/1 @" + std::to_string(p), {p}, 0, 1, 4, 256, 256, true, 512, 1, false, 0});
    cases.push_back({"C5 sliding ring 544 w512 @" + std::to_string(p), {p}, 512, 1, 4, 256, 256, true, 512, 1, false, 544});
  }
  // Split-plan extremes the tests and tuning variables reach.
  cases.push_back({"target 1 (one split per row)", ragged(5, 40, 2048, 13), 0, 2, 4, 64, 64, true, 1, 64, false, 0});
  cases.push_back({"target 4096, 1 tile/wave", ragged(5, 40, 2048, 13), 0, 2, 4, 256, 256, true, 4096, 1, false, 0});
  cases.push_back({"unfused (separate reduction)", ragged(5, 40, 2048, 13), 0, 2, 4, 64, 64, true, 4096, 1, true, 0});
  cases.push_back({"wide: 16383 positions d256 MQA", {16383, 300, 4096}, 0, 1, 4, 256, 256, true, 512, 1, false, 0});
  cases.push_back({"wide: ring 16384 w12000 @20000", {20000}, 12000, 1, 4, 128, 128, true, 512, 1, false, 16384});
  cases.push_back({"two head groups (20 q heads / kv head)", ragged(7, 1, 9000, 3), 0, 2, 20, 128, 128, true, 512, 1, false, 0});
  cases.push_back({"128 rows x 8 kv x 4 head groups, long", ragged(128, 60000, 65535, 9), 0, 8, 64, 128, 128, true, 512, 1, false, 0});
  cases.push_back({"128 rows, target 100000", ragged(128, 544, 544, 1), 0, 8, 4, 256, 256, true, 100000, 1, false, 0});
  cases.push_back({"short rows d128 f16 24/8 @1024 (halved)", {1024}, 0, 8, 3, 128, 128, true, 512, 1, false, 0});
  cases.push_back({"min split tiles 1, ragged d256", ragged(5, 40, 2048, 13), 0, 2, 4, 256, 256, true, 512, 1, false, 0, 1});
  cases.push_back({"min split tiles 2, C5 sliding ring", {32767}, 512, 1, 4, 256, 256, true, 512, 1, false, 544, 2});
  cases.push_back({"min split tiles 1, C5 global (wide)", {32767}, 0, 1, 4, 256, 256, true, 512, 1, false, 0, 1});
  cases.push_back({"single position 0", {0}, 0, 1, 1, 16, 16, false, 512, 1, false, 0});
  cases.push_back({"1M context MQA d128", {1048575}, 0, 1, 8, 128, 128, true, 512, 1, false, 0});
  // Gemma-4 layer shapes: full layers d 512 (2 kv heads, LINEAR), sliding d 256 on a ring of
  // window + chunk that is not a multiple of 32 (stored in round_up(356, 32) = 384 slots).
  cases.push_back({"Gemma-4 full d512 2 sessions", {602, 252}, 0, 2, 4, 512, 512, true, 512, 1, false, 0});
  cases.push_back({"Gemma-4 full d512 f32 8k", {8191}, 0, 2, 16, 512, 512, false, 512, 1, false, 0});
  for (uint32_t p : {4096u, 32704u})
    cases.push_back({"Gemma-4 full d512 8/1 @" + std::to_string(p) + " (wide)", {p}, 0, 1, 8, 512, 512, true, 512, 1, false, 0});
  cases.push_back({"Gemma-4 full d512 ragged 3 rows x 2 groups (wide)", {20000, 5000, 12000}, 0, 1, 20, 512, 512, true, 512, 1, false, 0});
  cases.push_back({"d512 ragged 3 rows x 2 groups, target 8192 (wide, sliced)", {9000, 5000, 7000}, 0, 1, 20, 512, 512, true, 8192, 1, false, 0});
  cases.push_back({"d512 one row @16000 (wide, unsliced)", {16000}, 0, 1, 8, 512, 512, true, 512, 1, false, 0});
  cases.push_back({"d512 ragged 9000/5000/7000 x 2 groups", {9000, 5000, 7000}, 0, 1, 20, 512, 512, true, 512, 1, false, 0});
  cases.push_back({"d512 ragged 9000/5000/7000 x 2 groups, f32", {9000, 5000, 7000}, 0, 1, 20, 512, 512, false, 512, 1, false, 0});
  cases.push_back({"d512 one row @16000, f32", {16000}, 0, 1, 8, 512, 512, false, 512, 1, false, 0});
  cases.push_back({"Gemma-4 sliding ring 356 w256", {602, 252}, 256, 4, 2, 256, 256, true, 512, 1, false, 384});
  for (const Case& c : cases) check(c);
  for (bool f16 : {true, false})
    for (uint32_t dk : {16u, 32u, 48u, 64u, 80u, 128u, 256u, 512u})
      check_k_layout(dk, f16, 96);
  printf("K layout: bijective, kernel K loads match k_index\n");
  printf("ok\n");
  return 0;
}
