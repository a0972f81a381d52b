// Host runtime behind the C ABI declared in include/jmodels_attn.h.
//
// Owns the per-GPU context (stream, error word, scratch), the RoPE tables and the HBM-resident
// KV caches with the reference's bookkeeping: the populated bitmap of KvCache
// (backend-java/src/main/java/com/integrallis/models/backend/purejava/cache/KvCache.java:33, 72,
// 161-173) for LINEAR layers and the positions[] array of LayeredKvCache
// (cache/LayeredKvCache.java:124, 168, 192-197, 212-223) for RING layers. Every export catches
// C++ exceptions and turns them into status codes, like the Rust exports' catch_unwind
// (backend-native/src/main/rust/model-kernels/src/lib.rs:497-584).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cstdlib>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/jmodels_attn.h"
#include "jma_kernels.h"

namespace {

thread_local std::string g_last_error;

struct Failure {
  int32_t status;
  std::string message;
};

[[noreturn]] void fail(int32_t status, const std::string& message) {
  throw Failure{status, message};
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(JMODELS_ATTN_DEVICE_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

template <typename F>
int32_t guard(F&& body) {
  try {
    body();
    return JMODELS_ATTN_OK;
  } catch (const Failure& f) {
    g_last_error = f.message;
    return f.status;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return JMODELS_ATTN_PANIC;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return JMODELS_ATTN_PANIC;
  } catch (...) {
    g_last_error = "unknown exception";
    return JMODELS_ATTN_PANIC;
  }
}

uint64_t round_up(uint64_t x, uint64_t m) { return (x + m - 1) / m * m; }

// Fails with NOT_CAPTURABLE when `stream` is being captured into a graph: a call that would
// allocate, fill or wait there must first run once outside the capture.
void require_not_capturing(hipStream_t stream, const char* what) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  hip_check(hipStreamIsCapturing(stream, &status), "hipStreamIsCapturing");
  if (status != hipStreamCaptureStatusNone)
    fail(JMODELS_ATTN_NOT_CAPTURABLE,
         std::string(what) + " needs more scratch memory than this context holds while its stream "
                             "is being captured; make the same call once outside the capture first");
}

// Grow-only device buffer owned by a context. A buffer it outgrows is retired, not freed, until
// the context is destroyed: graphs captured earlier keep the old address in their kernel
// arguments and may still be replayed. Sizes at least double, so the retired buffers together
// never exceed the current one.
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  std::vector<void*> retired;
  // Growth is refused while `stream` is being captured; otherwise it waits for `stream` (its
  // kernels may still use the old allocation, whose contents callers may copy).
  void reserve(size_t need, hipStream_t stream, const char* what = "scratch") {
    if (need <= bytes) return;
    require_not_capturing(stream, what);
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    const size_t grow = std::max({need, 2 * bytes, (size_t)1 << 16});
    void* fresh = nullptr;
    hip_check(hipMalloc(&fresh, grow), "hipMalloc scratch");
    if (ptr) retired.push_back(ptr);
    ptr = fresh;
    bytes = grow;
  }
  void release() {
    for (void* p : retired) (void)hipFree(p);
    retired.clear();
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
};

// Grows `buf` to `need` bytes; a new allocation has every byte set to `byte` (synchronously, so
// no fill is ever recorded into a caller's graph).
void reserve_filled(DeviceBuffer& buf, size_t need, int byte, hipStream_t stream,
                    const char* what = "scratch") {
  if (need <= buf.bytes) return;
  buf.reserve(need, stream, what);
  hip_check(hipMemsetAsync(buf.ptr, byte, buf.bytes, stream), "fill scratch");
  hip_check(hipStreamSynchronize(stream), "fill scratch");
}

// IEEE binary16 bits -> float, exactly (subnormals normalised, NaN payloads kept as the compiler's
// own half-to-float conversion keeps them), for reading an f16 cache back on the host.
float f16_bits_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
  if (exp == 0x1Fu) {
    bits = sign | 0x7F800000u | (man << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;
  } else {
    exp = 113u;
    while ((man & 0x400u) == 0) {
      man <<= 1;
      --exp;
    }
    bits = sign | (exp << 23) | ((man & 0x3FFu) << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  if (!v || !*v) return fallback;
  return std::atoi(v);
}

}  // namespace

struct jmodels_attn_context {
  int device = 0;
  hipStream_t stream = nullptr;
  int* d_err = nullptr;
  DeviceBuffer part_acc, part_ml, part_f, counters, pf_part, pf_tickets, qrot, stage_q, stage_k, stage_v, stage_out;
  DeviceBuffer qact;                // Q8_0 activations of prefill-sized projections
  DeviceBuffer pp_part, pp_tickets; // split stripe pairs of the head-dim-512 f16 prefill
  int decode_target_blocks = 512;   // workgroups a decode launch aims for (two per CU)
  int tiles_per_wave = 1;           // minimum tiles each decode wave streams
  int min_split_tiles = 0;          // minimum tiles per decode split; 0: waves x tiles_per_wave
  int prefill_split_tiles = -1;     // split prefill row blocks of this many kv tiles; -1: automatic
  uint32_t cus = 256;               // compute units of the device
  bool unfused = false;             // JMA_UNFUSED=1: separate append and reduce kernels
  jma::FixedScratch fixed;          // the device's fixed scratch (allocation-free decode)
};

struct jmodels_attn_rope {
  jmodels_attn_context* ctx = nullptr;
  uint32_t rotary_dim = 0, pairs = 0, max_positions = 0;
  float* d_cos = nullptr;
  float* d_sin = nullptr;
};

struct jmodels_attn_norm {
  jmodels_attn_context* ctx = nullptr;
  uint32_t head_dim = 0;
  float eps = 0.0f;
  float* d_q = nullptr;  // null: q heads are not normalised
  float* d_k = nullptr;
  bool v_rms = false;    // v heads are RMS-normalised without a weight (Gemma 4)
};

struct jmodels_attn_kv {
  jmodels_attn_context* ctx = nullptr;
  uint32_t sequences = 0, layers = 0, max_seq_len = 0, dtype = 0;
  // per layer (LayeredKvCache.LayerSpec, BJ/cache/LayeredKvCache.java:41-64): kv heads, key and
  // value lengths per head
  std::vector<uint32_t> hkv_l, dk_l, dv_l;
  std::vector<uint32_t> ring;      // logical ring capacity per layer, 0 = linear
  std::vector<uint32_t> cap;       // physical slots per layer (a ring's rounded up to 32)
  std::vector<uint64_t> layer_off_k, layer_off_v;
  uint64_t seq_stride_k = 0, seq_stride_v = 0;
  void* d_k = nullptr;
  void* d_v = nullptr;
  uint64_t bytes = 0;
  // host bookkeeping, indexed [sequence * layers + layer]
  std::vector<std::vector<uint64_t>> populated;  // linear layers: bitmap over positions
  std::vector<uint32_t> contiguous_end;          // linear: positions [0, end) all populated
  std::vector<std::vector<int32_t>> positions;   // ring layers: position held by each slot

  bool f16() const { return dtype == JMODELS_ATTN_KV_F16; }
  size_t elem() const { return f16() ? 2 : 4; }
  size_t idx(uint32_t s, uint32_t l) const { return (size_t)s * layers + l; }

  jma::KvView view(uint32_t layer) const {
    jma::KvView v{};
    v.k = d_k;
    v.v = d_v;
    v.seq_stride_k = seq_stride_k;
    v.seq_stride_v = seq_stride_v;
    v.layer_off_k = layer_off_k[layer];
    v.layer_off_v = layer_off_v[layer];
    v.cap = cap[layer];
    v.ring = ring[layer] != 0 ? 1u : 0u;
    return v;
  }

  bool available(uint32_t s, uint32_t l, uint32_t p) const {
    if (ring[l]) {
      const auto& pos = positions[idx(s, l)];
      return pos[p % ring[l]] == (int32_t)p;
    }
    const auto& bits = populated[idx(s, l)];
    return (bits[p >> 6] >> (p & 63)) & 1u;
  }

  void mark(uint32_t s, uint32_t l, uint32_t p) {
    if (ring[l]) {
      positions[idx(s, l)][p % ring[l]] = (int32_t)p;
      return;
    }
    auto& bits = populated[idx(s, l)];
    bits[p >> 6] |= 1ull << (p & 63);
    uint32_t& end = contiguous_end[idx(s, l)];
    while (end < max_seq_len && ((bits[end >> 6] >> (end & 63)) & 1u)) ++end;
  }

  // The reference's checks for reading positions [from, to] of a layer: KvCache.slice /
  // LayeredKvCache.attentionView (cache/KvCache.java:208-230, cache/LayeredKvCache.java:178-197).
  void require_range(uint32_t s, uint32_t l, uint32_t from, uint32_t to_inclusive) const {
    if (ring[l] && to_inclusive - from + 1 > ring[l]) {
      fail(JMODELS_ATTN_OUT_OF_RANGE, "attention range length " +
                                          std::to_string(to_inclusive - from + 1) +
                                          " exceeds ring capacity " + std::to_string(ring[l]));
    }
    if (!ring[l] && to_inclusive < contiguous_end[idx(s, l)]) return;
    for (uint32_t p = from; p <= to_inclusive; ++p) {
      if (!available(s, l, p)) {
        fail(JMODELS_ATTN_UNAVAILABLE, "cache position " + std::to_string(p) + " for layer " +
                                           std::to_string(l) + " of sequence " +
                                           std::to_string(s) + " is not populated");
      }
    }
  }
};

namespace {

void require(bool ok, int32_t status, const std::string& msg) {
  if (!ok) fail(status, msg);
}

void check_ctx(const jmodels_attn_context* ctx) {
  require(ctx != nullptr, JMODELS_ATTN_NULL_POINTER, "context is null");
}

struct LayerCall {
  uint32_t layer, num_heads, group, window, neox;
  uint32_t hkv, dk, dv;  // the layer's kv heads and head lengths
  float scale;
  const jmodels_attn_rope* rope;
  const jmodels_attn_norm* norm;  // null or weights on neither side = no QK-norm
};

LayerCall resolve_layer(const jmodels_attn_kv* kv, const jmodels_attn_layer* p) {
  require(p != nullptr, JMODELS_ATTN_NULL_POINTER, "layer parameters are null");
  require(p->layer < kv->layers, JMODELS_ATTN_OUT_OF_RANGE,
          "layer out of range: " + std::to_string(p->layer));
  LayerCall c{};
  c.layer = p->layer;
  c.hkv = kv->hkv_l[p->layer];
  c.dk = kv->dk_l[p->layer];
  c.dv = kv->dv_l[p->layer];
  require(p->num_heads > 0 && p->num_heads % c.hkv == 0, JMODELS_ATTN_INVALID_SHAPE,
          "num_heads must be a positive multiple of the layer's num_kv_heads");
  c.num_heads = p->num_heads;
  c.group = p->num_heads / c.hkv;
  c.window = p->sliding_window;
  c.neox = p->neox ? 1u : 0u;
  // LlamaForwardPass: scale = (float)(1.0 / Math.sqrt(keyLength)) (llama/LlamaForwardPass.java:1559)
  c.scale = p->scale != 0.0f ? p->scale : (float)(1.0 / sqrt((double)c.dk));
  require(isfinite(c.scale) && c.scale > 0.0f, JMODELS_ATTN_INVALID_SHAPE, "scale must be finite and > 0");
  c.rope = p->rope;
  if (c.rope) {
    require(c.rope->ctx == kv->ctx, JMODELS_ATTN_INVALID_SHAPE, "rope table belongs to another context");
    require(c.rope->rotary_dim <= c.dk, JMODELS_ATTN_INVALID_SHAPE, "rotary_dim exceeds key_length");
  }
  c.norm = p->qk_norm;
  if (c.norm) {
    require(c.norm->ctx == kv->ctx, JMODELS_ATTN_INVALID_SHAPE, "qk-norm belongs to another context");
    require(c.norm->head_dim == c.dk, JMODELS_ATTN_INVALID_SHAPE,
            "qk-norm head_dim differs from key_length");
    require(!c.norm->v_rms || c.norm->head_dim == c.dv, JMODELS_ATTN_INVALID_SHAPE,
            "value norm head_dim differs from value_length");
    if (!c.norm->d_q && !c.norm->d_k && !c.norm->v_rms) c.norm = nullptr;
  }
  return c;
}

void check_rows(const jmodels_attn_kv* kv, const LayerCall& lc, uint32_t count,
                const uint32_t* sequences, const uint32_t* positions) {
  require(count > 0, JMODELS_ATTN_INVALID_SHAPE, "count must be > 0");
  require(sequences && positions, JMODELS_ATTN_NULL_POINTER, "sequences/positions are null");
  for (uint32_t i = 0; i < count; ++i) {
    require(sequences[i] < kv->sequences, JMODELS_ATTN_OUT_OF_RANGE,
            "sequence out of range: " + std::to_string(sequences[i]));
    require(positions[i] < kv->max_seq_len, JMODELS_ATTN_OUT_OF_RANGE,
            "position out of range: " + std::to_string(positions[i]));
    if (lc.rope) {
      require(positions[i] < lc.rope->max_positions, JMODELS_ATTN_OUT_OF_RANGE,
              "position beyond the rope table: " + std::to_string(positions[i]));
    }
  }
  std::vector<uint64_t> keys(count);
  for (uint32_t i = 0; i < count; ++i) keys[i] = ((uint64_t)sequences[i] << 32) | positions[i];
  std::sort(keys.begin(), keys.end());
  require(std::adjacent_find(keys.begin(), keys.end()) == keys.end(), JMODELS_ATTN_INVALID_SHAPE,
          "rows repeat a (sequence, position)");
}

void check_elems(uint64_t have, uint64_t need, const char* what) {
  require(have >= need, JMODELS_ATTN_BUFFER_TOO_SMALL,
          std::string(what) + " holds " + std::to_string(have) + " elements, needs " +
              std::to_string(need));
}

// Rows of one launch. Consecutive positions of one sequence (a single decode row included) use the
// contiguous form, which kernels resolve without reading the row tables.
jma::RowList make_rows(uint32_t count, const uint32_t* sequences, const uint32_t* positions) {
  jma::RowList r{};
  r.count = count;
  bool consecutive = true;
  for (uint32_t i = 1; i < count && consecutive; ++i)
    consecutive = sequences[i] == sequences[0] && positions[i] == positions[0] + i;
  r.contiguous = consecutive ? 1u : 0u;
  r.seq0 = sequences[0];
  r.start = positions[0];
  for (uint32_t i = 0; i < count; ++i) {
    r.seq[i] = sequences[i];
    r.pos[i] = positions[i];
  }
  return r;
}

uint32_t append_blocks_per_row(uint32_t num_heads, uint32_t hkv, uint32_t dk, uint32_t dv) {
  const uint32_t pairs = num_heads * dk / 2 + hkv * dk / 2 + hkv * dv / 2;
  return (pairs + 255) / 256;
}

// ---------------------------------------------------------------- launches

void run_append(jmodels_attn_context* ctx, jmodels_attn_kv* kv, const LayerCall& lc,
                const jma::RowList& rows, const float* q, const float* k, const float* v,
                float* q_out) {
  jma::AppendArgs a{};
  a.kv = kv->view(lc.layer);
  a.q = q;
  a.k = k;
  a.v = v;
  a.q_out = q_out;
  if (lc.rope) {
    a.cos_t = lc.rope->d_cos;
    a.sin_t = lc.rope->d_sin;
    a.pairs = lc.rope->pairs;
  }
  a.neox = lc.neox;
  a.num_heads = lc.num_heads;
  a.num_kv_heads = lc.hkv;
  a.dk = lc.dk;
  a.dv = lc.dv;
  a.blocks_per_row = append_blocks_per_row(lc.num_heads, lc.hkv, lc.dk, lc.dv);
  if (lc.norm) {
    a.q_norm_w = lc.norm->d_q;
    a.k_norm_w = lc.norm->d_k;
    a.norm_eps = lc.norm->eps;
    a.v_norm = lc.norm->v_rms ? 1u : 0u;
  }
  a.rows = rows;
  hip_check(jma::launch_append(a, kv->f16(), ctx->stream), "rope_append launch");
}

// Split planning for one launch of <= kMaxRows rows. Every workgroup of the launch streams
// tiles_per_split tiles: at least tiles_per_wave per wave, raised until the launch is near the
// workgroup target, and high enough that no row needs more than kMaxSplits splits (the decode
// kernel then reduces the splits itself). When that cap would leave the launch with fewer than a
// quarter of the target workgroups (few long rows: one sequence at a long context and few KV
// heads), the rows are cut wider, up to kMaxWideSplits splits, and reduce_kernel combines them
// in a second launch.
// New rows handed to the decode kernel to rotate and append itself (all null: rows are cached).
struct FusedAppend {
  const float* k = nullptr;
  const float* v = nullptr;
  bool rope_q = false;  // q is raw: the kernel applies the layer's QK-norm and RoPE
};

jma::DecodePlan decode_plan(const jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                           const LayerCall& lc, const jma::RowList& rows) {
  return jma::plan_decode(rows.count, rows.pos, lc.window, lc.hkv, lc.group, (int)lc.dk,
                          (int)lc.dv, kv->f16(), ctx->decode_target_blocks, ctx->tiles_per_wave,
                          ctx->unfused, ctx->min_split_tiles);
}

// Refuses (BUFFER_TOO_SMALL) a launch plan whose scratch exceeds the device's fixed array.
void check_fixed_fit(const jma::DecodePlan& plan, const jma::FixedScratch& fixed) {
  auto fits = [&](size_t need, size_t have, const char* what) {
    require(need <= have, JMODELS_ATTN_BUFFER_TOO_SMALL,
            std::string("the launch plan needs ") + std::to_string(need) + " bytes of " + what +
                ", the fixed scratch holds " + std::to_string(have));
  };
  if (plan.separate) {
    fits(plan.acc_bytes, fixed.part_acc_bytes, "split partials");
    fits(plan.ml_bytes, fixed.part_ml_bytes, "split maxima and sums");
  } else if (plan.any_split) {
    fits(plan.part_f_bytes, fixed.part_f_bytes, "split exchange partials");
    fits(plan.counter_bytes, fixed.counters_bytes, "arrival tickets");
  }
}

// fixed: null = the context's grow-only scratch; else the device's fixed scratch. The callers
// check every chunk's plan against it (check_fixed_fit) before they enqueue anything, so a
// refusal leaves the cache and the stream untouched; the check here repeats that.
void run_attend_rows(jmodels_attn_context* ctx, const jmodels_attn_kv* kv, const LayerCall& lc,
                     const jma::RowList& rows, const float* q, float* out,
                     const FusedAppend& fa = FusedAppend(),
                     const jma::FixedScratch* fixed = nullptr) {
  jma::DecodeArgs a{};
  a.kv = kv->view(lc.layer);
  a.q = q;
  a.out = out;
  a.err = ctx->d_err;
  a.qscale = lc.scale * 1.4426950408889634f;
  a.num_heads = lc.num_heads;
  a.group = lc.group;
  a.hgroups = (lc.group + jma::kHeadSlots - 1) / jma::kHeadSlots;
  a.num_kv_heads = lc.hkv;
  a.window = lc.window;
  a.rows = rows;
  a.k_new = fa.k;
  a.v_new = fa.v;
  a.rope_q = fa.rope_q ? 1u : 0u;
  if (lc.rope && (fa.k || fa.rope_q)) {
    a.cos_t = lc.rope->d_cos;
    a.sin_t = lc.rope->d_sin;
    a.pairs = lc.rope->pairs;
  }
  a.neox = lc.neox;
  if (lc.norm) {
    if (fa.rope_q) a.q_norm_w = lc.norm->d_q;
    if (fa.k) {
      a.k_norm_w = lc.norm->d_k;
      a.v_norm = lc.norm->v_rms ? 1u : 0u;
    }
    a.norm_eps = lc.norm->eps;
  }
  const jma::DecodePlan plan = decode_plan(ctx, kv, lc, rows);
  a.tiles_per_split = plan.tiles_per_split;
  a.hgroups = plan.hgroups;  // virtual head groups (head groups x column slices)
  a.slices = plan.slices;
  for (uint32_t i = 0; i <= rows.count; ++i) a.item_start[i] = plan.item_start[i];
  for (uint32_t i = 0; i < rows.count; ++i) a.nsplit[i] = plan.nsplit[i];
  a.max_splits = plan.max_splits;
  a.total_items = plan.total_items;
  a.ns_uniform = plan.ns_uniform;
  const bool uniform = plan.ns_uniform != 0;
  if (uniform && rows.contiguous && a.hgroups == a.slices) {
    const size_t es = kv->f16() ? 2 : 4;
    a.k_base = (char*)a.kv.k + (a.kv.seq_stride_k * rows.seq0 + a.kv.layer_off_k) * es;
    a.v_base = (char*)a.kv.v + (a.kv.seq_stride_v * rows.seq0 + a.kv.layer_off_v) * es;
  } else if (kv->f16()) {
    // A listed-rows launch that streams more K/V than half the 256 MB Infinity Cache loads its
    // tiles non-temporally: those bytes cannot stay cached for the next launch anyway, and
    // bypassing the cache measured ~10% faster on C4 (491 MB: 106 -> 96 us), where plain loads
    // keep a re-read working set (C2's 138 MB across 16 layers) cached between tokens.
    const uint32_t blk = (uint32_t)jma::v_block(true);
    uint64_t bytes = 0;
    for (uint32_t i = 0; i < rows.count; ++i) {
      const uint32_t pos = rows.contiguous ? rows.start + i : rows.pos[i];
      const uint32_t first = jma::first_visible(pos, lc.window);
      bytes += (uint64_t)(pos / blk - first / blk + 1) * blk * lc.hkv * (lc.dk + lc.dv) * 2;
    }
    a.stream_nt = bytes > (uint64_t(128) << 20) ? 1u : 0u;
  }
  if (fixed) check_fixed_fit(plan, *fixed);
  if (plan.separate) {
    const size_t acc_b = plan.acc_bytes, ml_b = plan.ml_bytes;
    // reduce_kernel addresses the partials with 32-bit byte offsets.
    require(acc_b <= 0x7FFFFFF0u && ml_b <= 0x7FFFFFF0u, JMODELS_ATTN_INVALID_SHAPE,
            "decode plan needs more than 2 GiB of split partials (lower JMA_DECODE_TARGET_BLOCKS)");
    if (fixed) {
      a.part_acc = fixed->part_acc;
      a.part_ml = fixed->part_ml;
    } else {
      ctx->part_acc.reserve(acc_b, ctx->stream, "decode partials");
      ctx->part_ml.reserve(ml_b, ctx->stream, "decode partials");
      a.part_acc = (float*)ctx->part_acc.ptr;
      a.part_ml = (float*)ctx->part_ml.ptr;
    }
  } else if (plan.any_split) {
    // Arrival tickets start at zero and every partial word starts not-written; the reducing
    // workgroups restore both, so they are zeroed only when (re)allocated, never inside a launch
    // sequence a caller may capture.
    const size_t part_b = plan.part_f_bytes;
    // The exchange addresses its partials with 32-bit byte offsets (a buffer descriptor).
    require(part_b <= 0x7FFFFFF0u, JMODELS_ATTN_INVALID_SHAPE,
            "decode plan needs more than 2 GiB of split partials (lower JMA_DECODE_TARGET_BLOCKS)");
    if (fixed) {
      a.part_f = fixed->part_f;
      a.counters = fixed->counters;
    } else {
      reserve_filled(ctx->part_f, part_b, 0xFF, ctx->stream, "decode split exchange");
      reserve_filled(ctx->counters, (size_t)jma::kMaxRows * lc.hkv * a.hgroups * sizeof(uint32_t), 0,
                     ctx->stream, "decode split exchange");
      a.part_f = (float*)ctx->part_f.ptr;
      a.counters = (uint32_t*)ctx->counters.ptr;
    }
  }
  hip_check(jma::launch_decode(a, kv->f16(), lc.dk, lc.dv, ctx->stream), "decode launch");
  if (plan.separate) hip_check(jma::launch_reduce(a, lc.dv, ctx->stream), "reduce launch");
}

// The decode kernel normalises (QK-norm, value norm), rotates q and appends the new rows itself
// when its RoPE chunks line up with the rotary pairs (a multiple of 8 pairs) and the context does
// not ask for separate kernels.
bool can_fuse_decode(const jmodels_attn_context* ctx, const LayerCall& lc) {
  if (ctx->unfused) return false;
  return lc.rope == nullptr || lc.rope->pairs % 8 == 0;
}

void run_attend(jmodels_attn_context* ctx, const jmodels_attn_kv* kv, const LayerCall& lc,
                uint32_t count, const uint32_t* sequences, const uint32_t* positions,
                const float* q, float* out, const jma::FixedScratch* fixed = nullptr) {
  const uint64_t qdim = (uint64_t)lc.num_heads * lc.dk;
  const uint64_t odim = (uint64_t)lc.num_heads * lc.dv;
  for (uint32_t base = 0; base < count; base += jma::kMaxRows) {
    const uint32_t n = std::min<uint32_t>(jma::kMaxRows, count - base);
    jma::RowList rows = make_rows(n, sequences + base, positions + base);
    run_attend_rows(ctx, kv, lc, rows, q + base * qdim, out + base * odim, FusedAppend(), fixed);
  }
}

void validate_attend_ranges(const jmodels_attn_kv* kv, const LayerCall& lc, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions) {
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t p = positions[i];
    kv->require_range(sequences[i], lc.layer, jma::first_visible(p, lc.window), p);
  }
}

void append_rows(jmodels_attn_context* ctx, jmodels_attn_kv* kv, const LayerCall& lc,
                 uint32_t count, const uint32_t* sequences, const uint32_t* positions,
                 const float* q, const float* k, const float* v, float* q_out) {
  const uint64_t qdim = (uint64_t)lc.num_heads * lc.dk;
  const uint64_t kdim = (uint64_t)lc.hkv * lc.dk;
  const uint64_t vdim = (uint64_t)lc.hkv * lc.dv;
  // One launch takes up to kMaxRows rows. On a RING layer two rows of one sequence may map to
  // the same device slot (position % the physical capacity); such rows go to separate launches
  // in row order, so the later store wins as with sequential KvCache.store calls.
  const uint32_t ring = kv->ring[lc.layer] ? kv->cap[lc.layer] : 0u;
  std::vector<uint64_t> slots_in_launch;
  uint32_t base = 0;
  while (base < count) {
    uint32_t n = 0;
    slots_in_launch.clear();
    while (base + n < count && n < (uint32_t)jma::kMaxRows) {
      if (ring) {
        const uint64_t key = ((uint64_t)sequences[base + n] << 32) | (positions[base + n] % ring);
        if (std::find(slots_in_launch.begin(), slots_in_launch.end(), key) != slots_in_launch.end())
          break;
        slots_in_launch.push_back(key);
      }
      ++n;
    }
    jma::RowList rows = make_rows(n, sequences + base, positions + base);
    run_append(ctx, kv, lc, rows, q + base * qdim, k + base * kdim, v + base * vdim,
               q_out ? q_out + base * qdim : nullptr);
    base += n;
  }
  for (uint32_t i = 0; i < count; ++i) kv->mark(sequences[i], lc.layer, positions[i]);
}

void check_decode_shape(const jmodels_attn_kv* kv, const LayerCall& lc) {
  require(jma::decode_supported(kv->f16(), (int)lc.dk, (int)lc.dv), JMODELS_ATTN_INVALID_SHAPE,
          "unsupported head dims for decode: key_length " + std::to_string(lc.dk) +
              ", value_length " + std::to_string(lc.dv));
}

// Which kernel runs a causal block of rows: the f16 MFMA prefill (f16 caches, head dims 32-256),
// the sliced prefills (f32 caches at 32-512: head-dim slices; f16 at 512: stripe pairs), else
// the split-K decode kernel over chunks of listed rows.
enum class PrefillPath { kF16, kSlice, kDecodeRows };

PrefillPath prefill_path(const jmodels_attn_kv* kv, const LayerCall& lc) {
  if (kv->f16() && jma::prefill_supported((int)lc.dk, (int)lc.dv)) return PrefillPath::kF16;
  if (jma::prefill_slice_supported(kv->f16(), (int)lc.dk, (int)lc.dv)) return PrefillPath::kSlice;
  return PrefillPath::kDecodeRows;
}

void check_prefill_shape(const jmodels_attn_kv* kv, const LayerCall& lc) {
  if (prefill_path(kv, lc) == PrefillPath::kDecodeRows) check_decode_shape(kv, lc);
}

// Causal attention of rows start .. start+n-1 whose K/V are cached and whose rotated queries are
// q (computeBatchedAttention, llama/LlamaForwardPass.java:1515-1541): row b attends
// [first(start+b), start+b], on the kernel prefill_path picks.
void attend_causal_impl(jmodels_attn_context* ctx, const jmodels_attn_kv* kv, const LayerCall& lc,
                        uint32_t sequence, uint32_t start, uint32_t n, const float* q, float* out) {
  const uint64_t qdim = (uint64_t)lc.num_heads * lc.dk;
  const uint64_t odim = (uint64_t)lc.num_heads * lc.dv;
  const PrefillPath path = prefill_path(kv, lc);
  if (path == PrefillPath::kSlice) {
    jma::PrefillArgs a{};
    a.kv = kv->view(lc.layer);
    a.q = q;
    a.qscale = lc.scale * 1.4426950408889634f;
    a.out = out;
    a.err = ctx->d_err;
    a.n = n;
    a.start = start;
    a.seq = sequence;
    a.window = lc.window;
    a.num_heads = lc.num_heads;
    a.num_kv_heads = lc.hkv;
    a.group = lc.group;
    a.heads_per_stripe = std::min<uint32_t>(lc.group, 32);
    a.rows_per_stripe = 32 / a.heads_per_stripe;
    a.head_groups = (lc.group + a.heads_per_stripe - 1) / a.heads_per_stripe;
    a.row_blocks = (n + a.rows_per_stripe - 1) / a.rows_per_stripe;
    {
      // Split stripe pairs (f16, kernel 3c) or stripes (f32, kernel 3b).
      const uint32_t half_bytes =
          kv->f16() ? 4u * jma::kPairPartWords * 64u * 16u
                    : (uint32_t)jma::slice_waves((int)lc.dk) * jma::slice_state_words((int)lc.dk) * 64u * 16u;
      const jma::PairPlan pp = jma::plan_prefill_pairs(a, ctx->prefill_split_tiles, ctx->cus,
                                                       kv->f16() ? 0u : a.rows_per_stripe, half_bytes);
      const uint32_t split = pp.split_pairs;
      if (split > 0) {
        const size_t per = (size_t)a.head_groups * lc.hkv;
        const size_t part_b = pp.part_bytes;
        // The kernel addresses the halves' states with 32-bit byte offsets.
        require(part_b <= 0x7FFFFFF0u, JMODELS_ATTN_INVALID_SHAPE,
                "prefill pair split needs more than 2 GiB of partial states");
        // No initial value for the states; tickets start at zero and the merging workgroups
        // restore them, so they are zeroed only when (re)allocated.
        ctx->pp_part.reserve(part_b, ctx->stream, "prefill pair split");
        reserve_filled(ctx->pp_tickets, (size_t)split * per * sizeof(uint32_t), 0, ctx->stream,
                       "prefill pair split");
        a.split_blocks = split;
        a.part = (float*)ctx->pp_part.ptr;
        a.tickets = (uint32_t*)ctx->pp_tickets.ptr;
      }
    }
    hip_check(jma::launch_prefill_slice(a, kv->f16(), (int)lc.dk, (int)lc.dv, ctx->stream),
              "prefill launch");
    return;
  }
  if (path == PrefillPath::kF16) {
    jma::PrefillArgs a{};
    a.kv = kv->view(lc.layer);
    a.q = q;
    a.qscale = lc.scale * 1.4426950408889634f;
    a.out = out;
    a.err = ctx->d_err;
    a.n = n;
    a.start = start;
    a.seq = sequence;
    a.window = lc.window;
    a.num_heads = lc.num_heads;
    a.num_kv_heads = lc.hkv;
    a.group = lc.group;
    a.heads_per_stripe = std::min<uint32_t>(lc.group, 32);
    a.rows_per_stripe = 32 / a.heads_per_stripe;
    a.head_groups = (lc.group + a.heads_per_stripe - 1) / a.heads_per_stripe;
    const jma::PrefillPlan plan = jma::plan_prefill(a, (int)lc.dk, ctx->prefill_split_tiles, ctx->cus);
    a.row_blocks = plan.row_blocks;
    a.split_blocks = plan.split_blocks;
    if (plan.pairs > 0) {
      // No initial value for the halves' states; tickets start at zero and the merging
      // workgroups restore them, so they are zeroed only when (re)allocated.
      ctx->pf_part.reserve(plan.part_bytes, ctx->stream, "prefill split exchange");
      reserve_filled(ctx->pf_tickets, (size_t)plan.pairs * sizeof(uint32_t), 0, ctx->stream,
                     "prefill split exchange");
      a.part = (float*)ctx->pf_part.ptr;
      a.tickets = (uint32_t*)ctx->pf_tickets.ptr;
    }
    hip_check(jma::launch_prefill(a, (int)lc.dk, (int)lc.dv, ctx->stream), "prefill launch");
    return;
  }
  check_decode_shape(kv, lc);
  for (uint32_t base = 0; base < n; base += jma::kMaxRows) {
    const uint32_t m = std::min<uint32_t>(jma::kMaxRows, n - base);
    jma::RowList rows{};
    rows.count = m;
    rows.contiguous = 0;
    for (uint32_t i = 0; i < m; ++i) {
      rows.seq[i] = sequence;
      rows.pos[i] = start + base + i;
    }
    run_attend_rows(ctx, kv, lc, rows, q + base * qdim, out + base * odim);
  }
}

// The reference's checks before a causal block of rows reads the cache: every position rows
// start .. start+n-1 see must be available, and a RING layer must hold them all at once.
void validate_causal(const jmodels_attn_kv* kv, const LayerCall& lc, uint32_t sequence,
                     uint32_t start, uint32_t n, bool rows_cached) {
  const uint32_t first = jma::first_visible(start, lc.window);
  if (kv->ring[lc.layer]) {
    // Gemma4KvCache sizes rings as window + prefill chunk (gemma4/Gemma4KvCache.java:39).
    require(start + n - first <= kv->ring[lc.layer], JMODELS_ATTN_OUT_OF_RANGE,
            "prefill chunk plus window exceeds ring capacity " + std::to_string(kv->ring[lc.layer]));
  }
  if (rows_cached) kv->require_range(sequence, lc.layer, first, start + n - 1);
  else if (first < start) kv->require_range(sequence, lc.layer, first, start - 1);
}

void prefill_impl(jmodels_attn_context* ctx, jmodels_attn_kv* kv, const LayerCall& lc,
                  uint32_t sequence, uint32_t start, uint32_t n, const float* q, const float* k,
                  const float* v, float* out) {
  const uint64_t qdim = (uint64_t)lc.num_heads * lc.dk;
  check_prefill_shape(kv, lc);
  validate_causal(kv, lc, sequence, start, n, false);
  ctx->qrot.reserve((size_t)n * qdim * sizeof(float), ctx->stream, "prefill rotated queries");
  // One launch appends every row: consecutive positions of one sequence need no row table.
  jma::RowList rows{};
  rows.count = n;
  rows.contiguous = 1;
  rows.seq0 = sequence;
  rows.start = start;
  run_append(ctx, kv, lc, rows, q, k, v, (float*)ctx->qrot.ptr);
  for (uint32_t i = 0; i < n; ++i) kv->mark(sequence, lc.layer, start + i);
  attend_causal_impl(ctx, kv, lc, sequence, start, n, (const float*)ctx->qrot.ptr, out);
}

int32_t collect_errors(jmodels_attn_context* ctx) {
  hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  int err = 0;
  hip_check(hipMemcpy(&err, ctx->d_err, sizeof(int), hipMemcpyDeviceToHost), "read error word");
  if (err != 0) {
    int zero = 0;
    hip_check(hipMemcpy(ctx->d_err, &zero, sizeof(int), hipMemcpyHostToDevice), "reset error word");
    if (err & 2) {
      // A reducer gave up waiting: tickets and partial words may be left set; clear them.
      for (DeviceBuffer* b : {&ctx->part_f})
        if (b->ptr) hip_check(hipMemset(b->ptr, 0xFF, b->bytes), "reset partials");
      for (DeviceBuffer* b : {&ctx->counters, &ctx->pf_tickets, &ctx->pp_tickets})
        if (b->ptr) hip_check(hipMemset(b->ptr, 0, b->bytes), "reset tickets");
      hip_check(jma::fixed_scratch_reset(ctx->fixed, ctx->stream), "reset fixed scratch");
      fail(JMODELS_ATTN_DEVICE_ERROR, "cross-split reduction timed out waiting for a partial");
    }
    fail(JMODELS_ATTN_NON_FINITE, "softmax input contains NaN or positive infinity");
  }
  return JMODELS_ATTN_OK;
}

void set_device(const jmodels_attn_context* ctx) { hip_check(hipSetDevice(ctx->device), "hipSetDevice"); }

template <typename T>
T* stage(DeviceBuffer& buf, const T* host, uint64_t elems, hipStream_t stream) {
  buf.reserve(elems * sizeof(T), stream);
  if (host)
    hip_check(hipMemcpyAsync(buf.ptr, host, elems * sizeof(T), hipMemcpyHostToDevice, stream),
              "copy to device");
  return (T*)buf.ptr;
}

// One matrix of a quantized projection call.
struct QuantMatrix {
  uint32_t format;
  const void* weights;
  uint64_t bytes;
  uint32_t rows;
  const float* addend;
};

// Checks a quantized projection call the way backend-native checks its batched matmuls
// (RS:1017-1060: null pointers, shape, buffer sizes), then launches it: activation rows in chunks
// that fit one workgroup's LDS, one launch per chunk and weight format.
void quantized_matmul_impl(jmodels_attn_context* ctx, const std::vector<QuantMatrix>& mats,
                           const float* input, uint64_t input_elements, float* output,
                           uint64_t output_elements, uint32_t batch, uint32_t cols,
                           uint32_t addend_mode) {
  check_ctx(ctx);
  require(input != nullptr && output != nullptr, JMODELS_ATTN_NULL_POINTER, "null input or output");
  require(!mats.empty(), JMODELS_ATTN_INVALID_SHAPE, "no matrices");
  // Q4_0 / Q8_0 / Q5_0 take Q8_0 activations (32-element blocks), the K-quants Q8_K (256): one
  // call shares one activation format, as backend-native's grouped calls require (RS:1196-1204).
  const bool kq = jma::qmat_kquant(mats[0].format);
  const uint32_t elems = kq ? 256u : 32u;
  require(batch > 0 && cols > 0 && cols % elems == 0, JMODELS_ATTN_INVALID_SHAPE,
          "batch_size and cols must be > 0 and cols a multiple of " + std::to_string(elems));
  require(addend_mode <= JMODELS_ATTN_ADDEND_RESIDUAL, JMODELS_ATTN_INVALID_SHAPE,
          "unknown addend_mode " + std::to_string(addend_mode));
  require(((uintptr_t)input & 15u) == 0, JMODELS_ATTN_INVALID_SHAPE,
          "input must be 16-byte aligned");
  const uint32_t K = cols / elems;
  uint64_t total_rows = 0;
  for (size_t i = 0; i < mats.size(); ++i) {
    const QuantMatrix& m = mats[i];
    const std::string at = " (matrix " + std::to_string(i) + ")";
    require(m.format <= JMODELS_ATTN_WEIGHTS_Q5_0, JMODELS_ATTN_INVALID_SHAPE,
            "unknown weight format " + std::to_string(m.format) + at);
    require(jma::qmat_kquant(m.format) == kq, JMODELS_ATTN_INVALID_SHAPE,
            "one call mixes 32-element block formats (Q4_0/Q8_0/Q5_0) with K-quants "
            "(Q4_K/Q5_K/Q6_K)" + at);
    require(m.weights != nullptr, JMODELS_ATTN_NULL_POINTER, "null weights" + at);
    require(m.rows > 0, JMODELS_ATTN_INVALID_SHAPE, "rows must be > 0" + at);
    require(((uintptr_t)m.weights & 1u) == 0, JMODELS_ATTN_INVALID_SHAPE,
            "weights must be 2-byte aligned" + at);
    require(addend_mode == 0 || m.addend != nullptr, JMODELS_ATTN_NULL_POINTER, "null addend" + at);
    const uint64_t need = (uint64_t)m.rows * K * jma::qmat_block_bytes(m.format);
    require(m.bytes >= need, JMODELS_ATTN_BUFFER_TOO_SMALL,
            "weights hold " + std::to_string(m.bytes) + " bytes, need " + std::to_string(need) + at);
    total_rows += m.rows;
  }
  require(input_elements >= (uint64_t)batch * cols, JMODELS_ATTN_BUFFER_TOO_SMALL,
          "input holds " + std::to_string(input_elements) + " elements, needs " +
              std::to_string((uint64_t)batch * cols));
  require(output_elements >= (uint64_t)batch * total_rows, JMODELS_ATTN_BUFFER_TOO_SMALL,
          "output holds " + std::to_string(output_elements) + " elements, needs " +
              std::to_string((uint64_t)batch * total_rows));
  // Launches, one per weight format of the call. Prefill-sized batches quantize the activations
  // once into the context's scratch (Q8_0 or Q8_K, whichever the call's formats take) and run the
  // register-tiled product; smaller batches run the matrix-vector kernel, whose workgroups take
  // 8-row passes of their activation rows through LDS (a weight tile read from memory once per
  // workgroup, not once per pass).
  auto gemm_format = [&](uint32_t) { return batch >= jma::kQGemmMinBatch; };
  int8_t* aq = nullptr;
  float* as = nullptr;
  int* asum = nullptr;
  set_device(ctx);
  bool need_gemm = false;
  std::vector<uint32_t> pass_fmts;
  for (const QuantMatrix& m : mats) {
    if (gemm_format(m.format)) need_gemm = true;
    else pass_fmts.push_back(m.format);
  }
  if (need_gemm) {
    const uint64_t q_bytes = ((uint64_t)batch * cols + 255u) & ~(uint64_t)255u;
    const uint64_t s_bytes = ((uint64_t)batch * K * sizeof(float) + 255u) & ~(uint64_t)255u;
    const uint64_t sum_bytes = kq ? (uint64_t)batch * (cols / 16u) * sizeof(int) : 0u;
    ctx->qact.reserve(q_bytes + s_bytes + sum_bytes, ctx->stream, "projection activations");
    aq = (int8_t*)ctx->qact.ptr;
    as = (float*)((char*)ctx->qact.ptr + q_bytes);
    asum = kq ? (int*)((char*)ctx->qact.ptr + q_bytes + s_bytes) : nullptr;
    if (kq)
      hip_check(jma::launch_q8_k_quant(input, batch, cols, aq, as, asum, ctx->stream),
                "activation quantization launch");
    else
      hip_check(jma::launch_q8_0_quant(input, batch, cols, aq, as, ctx->stream),
                "activation quantization launch");
  }
  jma::QMatPlan qp;
  if (!pass_fmts.empty()) {
    qp = jma::plan_qmat(pass_fmts.data(), (uint32_t)pass_fmts.size(), cols);
    require(qp.rows_per_tile > 0, JMODELS_ATTN_INVALID_SHAPE,
            "cols too large for the device projection: " + std::to_string(cols));
  }
  for (uint32_t fmt = 0; fmt <= JMODELS_ATTN_WEIGHTS_Q5_0; ++fmt) {
    const bool gemm = gemm_format(fmt);
    const uint32_t R = gemm ? jma::kQGemmTile : qp.rows_per_tile;
    jma::QMatArgs a{};
    a.x = input;
    a.batch = batch;
    a.cols = cols;
    a.blocks = K;
    a.rows_per_tile = R;
    a.chunk = qp.chunk;
    a.addend_mode = addend_mode;
    uint32_t tiles = 0;
    uint64_t out_off = 0;
    for (const QuantMatrix& m : mats) {
      if (m.format == fmt) {
        jma::QMatrix& q = a.m[a.count++];
        q.w = (const uint8_t*)m.weights;
        q.out = output + out_off;
        q.addend = m.addend;
        q.rows = m.rows;
        q.tile0 = tiles;
        tiles += (m.rows + R - 1) / R;
      }
      out_off += (uint64_t)batch * m.rows;
    }
    if (a.count == 0) continue;
    if (gemm) {
      require((batch + jma::kQGemmTile - 1) / jma::kQGemmTile <= 65535u, JMODELS_ATTN_INVALID_SHAPE,
              "batch_size too large for one projection launch: " + std::to_string(batch));
      if (kq)
        hip_check(jma::launch_qkgemm(a, fmt, tiles, aq, as, asum, ctx->stream), "quantized matmul launch");
      else
        hip_check(jma::launch_qgemm(a, fmt, tiles, aq, as, ctx->stream), "quantized matmul launch");
    } else {
      a.group_rows = jma::qmat_group_rows(batch, qp.chunk, tiles);
      require((batch + a.group_rows - 1) / a.group_rows <= 65535u, JMODELS_ATTN_INVALID_SHAPE,
              "batch_size too large for one projection launch: " + std::to_string(batch));
      hip_check(jma::launch_qmatvec(a, fmt, tiles, ctx->stream), "quantized matmul launch");
    }
  }
}

}  // namespace

// ================================================================ exports

extern "C" {

uint32_t jmodels_attn_abi_version(void) { return JMODELS_ATTN_ABI_VERSION; }

uint64_t jmodels_attn_capabilities(void) {
  return JMODELS_ATTN_CAP_DECODE_F32 | JMODELS_ATTN_CAP_DECODE_F16 | JMODELS_ATTN_CAP_PREFILL_MFMA |
         JMODELS_ATTN_CAP_RAGGED_DECODE | JMODELS_ATTN_CAP_SLIDING_WINDOW |
         JMODELS_ATTN_CAP_RING_LAYERS | JMODELS_ATTN_CAP_DEVICE_POINTERS | JMODELS_ATTN_CAP_QK_NORM |
         JMODELS_ATTN_CAP_VALUE_NORM | JMODELS_ATTN_CAP_QUANT_MATMUL;
}

const char* jmodels_attn_status_name(int32_t status) {
  switch (status) {
    case JMODELS_ATTN_OK: return "OK";
    case JMODELS_ATTN_NULL_POINTER: return "NULL_POINTER";
    case JMODELS_ATTN_INVALID_SHAPE: return "INVALID_SHAPE";
    case JMODELS_ATTN_BUFFER_TOO_SMALL: return "BUFFER_TOO_SMALL";
    case JMODELS_ATTN_PANIC: return "PANIC";
    case JMODELS_ATTN_DEVICE_ERROR: return "DEVICE_ERROR";
    case JMODELS_ATTN_OUT_OF_RANGE: return "OUT_OF_RANGE";
    case JMODELS_ATTN_UNAVAILABLE: return "UNAVAILABLE";
    case JMODELS_ATTN_NON_FINITE: return "NON_FINITE";
    case JMODELS_ATTN_NOT_CAPTURABLE: return "NOT_CAPTURABLE";
    default: return "UNKNOWN";
  }
}

const char* jmodels_attn_last_error(void) { return g_last_error.c_str(); }

jmodels_attn_context* jmodels_attn_context_create(int32_t device) {
  jmodels_attn_context* out = nullptr;
  int32_t st = guard([&] {
    int n = 0;
    hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
    require(device >= 0 && device < n, JMODELS_ATTN_OUT_OF_RANGE, "no such device");
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    require(strncmp(prop.gcnArchName, "gfx950", 6) == 0, JMODELS_ATTN_INVALID_SHAPE,
            std::string("device is not gfx950: ") + prop.gcnArchName);
    hip_check(hipSetDevice(device), "hipSetDevice");
    auto* ctx = new jmodels_attn_context();
    ctx->device = device;
    ctx->decode_target_blocks = std::max(1, env_int("JMA_DECODE_TARGET_BLOCKS", 512));
    ctx->tiles_per_wave = std::max(1, env_int("JMA_DECODE_TILES_PER_WAVE", 1));
    ctx->min_split_tiles = std::max(0, env_int("JMA_DECODE_MIN_SPLIT_TILES", 0));
    ctx->prefill_split_tiles = std::max(-1, env_int("JMA_PREFILL_SPLIT_TILES", -1));
    ctx->cus = (uint32_t)std::max(1, prop.multiProcessorCount);
    ctx->unfused = env_int("JMA_UNFUSED", 0) != 0;
    try {
      hip_check(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate");
      hip_check(hipMalloc(&ctx->d_err, sizeof(int)), "hipMalloc error word");
      hip_check(hipMemset(ctx->d_err, 0, sizeof(int)), "hipMemset error word");
      // The device's fixed scratch: its address, and its exchange regions prepared, once per
      // device (the allocation-free entry point then allocates nothing).
      hip_check(jma::fixed_scratch(device, ctx->stream, &ctx->fixed), "fixed scratch");
    } catch (...) {
      if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
      if (ctx->d_err) (void)hipFree(ctx->d_err);
      delete ctx;
      throw;
    }
    out = ctx;
  });
  return st == JMODELS_ATTN_OK ? out : nullptr;
}

int32_t jmodels_attn_context_destroy(jmodels_attn_context* ctx) {
  if (!ctx) return JMODELS_ATTN_NULL_POINTER;
  return guard([&] {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (DeviceBuffer* b : {&ctx->part_acc, &ctx->part_ml, &ctx->part_f, &ctx->counters, &ctx->pf_part, &ctx->pf_tickets, &ctx->qrot, &ctx->stage_q,
                            &ctx->stage_k, &ctx->stage_v, &ctx->stage_out, &ctx->qact, &ctx->pp_part,
                            &ctx->pp_tickets})
      b->release();
    (void)hipFree(ctx->d_err);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
  });
}

int32_t jmodels_attn_context_synchronize(jmodels_attn_context* ctx) {
  return guard([&] {
    check_ctx(ctx);
    set_device(ctx);
    collect_errors(ctx);
  });
}

int32_t jmodels_attn_context_stream(jmodels_attn_context* ctx, void** stream_out) {
  return guard([&] {
    check_ctx(ctx);
    require(stream_out != nullptr, JMODELS_ATTN_NULL_POINTER, "stream_out is null");
    *stream_out = (void*)ctx->stream;
  });
}

int32_t jmodels_attn_rope_create(jmodels_attn_context* ctx, uint32_t rotary_dim, float theta,
                                 float frequency_scale, const float* frequency_factors,
                                 uint32_t factor_count, uint32_t max_positions,
                                 jmodels_attn_rope** rope_out) {
  return guard([&] {
    check_ctx(ctx);
    require(rope_out != nullptr, JMODELS_ATTN_NULL_POINTER, "rope_out is null");
    *rope_out = nullptr;
    // RotaryTable ctor validation (ops/RotaryTable.java:48-66, 188-192).
    require(rotary_dim > 0 && (rotary_dim & 1) == 0, JMODELS_ATTN_INVALID_SHAPE,
            "rotaryDim must be positive and even: " + std::to_string(rotary_dim));
    require(theta > 0.0f && isfinite(theta), JMODELS_ATTN_INVALID_SHAPE, "theta must be finite and > 0");
    require(frequency_scale > 0.0f && isfinite(frequency_scale), JMODELS_ATTN_INVALID_SHAPE,
            "frequencyScale must be finite and > 0");
    require(max_positions > 0, JMODELS_ATTN_INVALID_SHAPE, "max_positions must be > 0");
    const uint32_t pairs = rotary_dim / 2;
    if (frequency_factors) {
      require(factor_count == pairs, JMODELS_ATTN_INVALID_SHAPE,
              "frequencyFactors must contain " + std::to_string(pairs) + " entries");
      for (uint32_t i = 0; i < pairs; ++i)
        require(frequency_factors[i] > 0.0f && isfinite(frequency_factors[i]),
                JMODELS_ATTN_INVALID_SHAPE, "frequencyFactors must be finite and > 0");
    }
    // RotaryTable: frequencies in double pow (:69-72); fillFactors (:177-186): angle in float,
    // cos/sin in double rounded to float.
    std::vector<float> freq(pairs);
    for (uint32_t p = 0; p < pairs; ++p)
      freq[p] = (float)(1.0 / pow((double)theta, (double)(p * 2) / (double)rotary_dim));
    std::vector<float> cs((size_t)max_positions * pairs), sn((size_t)max_positions * pairs);
    for (uint32_t pos = 0; pos < max_positions; ++pos) {
      const float scaled = (float)pos * frequency_scale;
      for (uint32_t p = 0; p < pairs; ++p) {
        const float divisor = frequency_factors ? frequency_factors[p] : 1.0f;
        const float angle = scaled * freq[p] / divisor;
        cs[(size_t)pos * pairs + p] = (float)cos((double)angle);
        sn[(size_t)pos * pairs + p] = (float)sin((double)angle);
      }
    }
    set_device(ctx);
    auto* rope = new jmodels_attn_rope();
    rope->ctx = ctx;
    rope->rotary_dim = rotary_dim;
    rope->pairs = pairs;
    rope->max_positions = max_positions;
    try {
      const size_t bytes = cs.size() * sizeof(float);
      hip_check(hipMalloc(&rope->d_cos, bytes), "hipMalloc rope");
      hip_check(hipMalloc(&rope->d_sin, bytes), "hipMalloc rope");
      hip_check(hipMemcpy(rope->d_cos, cs.data(), bytes, hipMemcpyHostToDevice), "upload rope");
      hip_check(hipMemcpy(rope->d_sin, sn.data(), bytes, hipMemcpyHostToDevice), "upload rope");
    } catch (...) {
      if (rope->d_cos) (void)hipFree(rope->d_cos);
      if (rope->d_sin) (void)hipFree(rope->d_sin);
      delete rope;
      throw;
    }
    *rope_out = rope;
  });
}

int32_t jmodels_attn_rope_destroy(jmodels_attn_rope* rope) {
  if (!rope) return JMODELS_ATTN_NULL_POINTER;
  return guard([&] {
    (void)hipSetDevice(rope->ctx->device);
    (void)hipStreamSynchronize(rope->ctx->stream);
    (void)hipFree(rope->d_cos);
    (void)hipFree(rope->d_sin);
    delete rope;
  });
}

int32_t jmodels_attn_norm_create(jmodels_attn_context* ctx, uint32_t head_dim, const float* q_weight,
                                 const float* k_weight, float eps, jmodels_attn_norm** norm_out) {
  return jmodels_attn_norm_create_ex(ctx, head_dim, q_weight, k_weight, eps, 0u, norm_out);
}

int32_t jmodels_attn_norm_create_ex(jmodels_attn_context* ctx, uint32_t head_dim,
                                    const float* q_weight, const float* k_weight, float eps,
                                    uint32_t flags, jmodels_attn_norm** norm_out) {
  return guard([&] {
    check_ctx(ctx);
    require(norm_out != nullptr, JMODELS_ATTN_NULL_POINTER, "norm_out is null");
    *norm_out = nullptr;
    require(head_dim > 0 && head_dim <= 4096, JMODELS_ATTN_INVALID_SHAPE, "head_dim must be in [1, 4096]");
    require(isfinite(eps) && eps >= 0.0f, JMODELS_ATTN_INVALID_SHAPE, "eps must be finite and >= 0");
    require((flags & ~JMODELS_ATTN_NORM_VALUE_RMS) == 0, JMODELS_ATTN_INVALID_SHAPE, "unknown norm flags");
    const bool v_rms = (flags & JMODELS_ATTN_NORM_VALUE_RMS) != 0;
    // Gemma4Math.normalizeWithoutWeight rejects eps that is not finite and > 0 (:47-49).
    require(!v_rms || eps > 0.0f, JMODELS_ATTN_INVALID_SHAPE, "value norm eps must be > 0");
    hip_check(hipSetDevice(ctx->device), "hipSetDevice");
    auto* norm = new jmodels_attn_norm();
    norm->ctx = ctx;
    norm->head_dim = head_dim;
    norm->eps = eps;
    norm->v_rms = v_rms;
    const size_t bytes = (size_t)head_dim * sizeof(float);
    try {
      if (q_weight) {
        hip_check(hipMalloc(&norm->d_q, bytes), "hipMalloc qk-norm");
        hip_check(hipMemcpy(norm->d_q, q_weight, bytes, hipMemcpyHostToDevice), "upload q-norm");
      }
      if (k_weight) {
        hip_check(hipMalloc(&norm->d_k, bytes), "hipMalloc qk-norm");
        hip_check(hipMemcpy(norm->d_k, k_weight, bytes, hipMemcpyHostToDevice), "upload k-norm");
      }
    } catch (...) {
      (void)hipFree(norm->d_q);
      (void)hipFree(norm->d_k);
      delete norm;
      throw;
    }
    *norm_out = norm;
  });
}

int32_t jmodels_attn_norm_destroy(jmodels_attn_norm* norm) {
  if (!norm) return JMODELS_ATTN_NULL_POINTER;
  return guard([&] {
    (void)hipSetDevice(norm->ctx->device);
    (void)hipStreamSynchronize(norm->ctx->stream);
    (void)hipFree(norm->d_q);
    (void)hipFree(norm->d_k);
    delete norm;
  });
}

// Creates a cache from per-layer specs (LayeredKvCache(maxSeqLen, LayerSpec[]),
// BJ/cache/LayeredKvCache.java:35-64, 124-156): per layer its kv heads, key and value lengths and
// ring capacity (0 = LINEAR). A RING layer keeps the reference's retention in the host
// bookkeeping (slot = position % ring, a newer position evicts the one ring positions before it)
// while its device storage rounds the ring up to a multiple of 32 slots (the kernels' 32-row
// tiles then never wrap inside a tile); the device slot of a position is position % that
// physical capacity, which holds every position the logical ring retains.
static void create_layered(jmodels_attn_context* ctx, uint32_t sequences, uint32_t num_layers,
                           uint32_t max_seq_len, const jmodels_attn_layer_spec* specs,
                           uint32_t dtype, jmodels_attn_kv** kv_out) {
  check_ctx(ctx);
  require(kv_out != nullptr && specs != nullptr, JMODELS_ATTN_NULL_POINTER, "kv_out or specs is null");
  *kv_out = nullptr;
  require(sequences > 0 && num_layers > 0 && max_seq_len > 0, JMODELS_ATTN_INVALID_SHAPE,
          "cache dimensions must be > 0");
  require(dtype == JMODELS_ATTN_KV_F32 || dtype == JMODELS_ATTN_KV_F16, JMODELS_ATTN_INVALID_SHAPE,
          "dtype must be JMODELS_ATTN_KV_F32 or JMODELS_ATTN_KV_F16");
  auto kv = std::make_unique<jmodels_attn_kv>();
  kv->ctx = ctx;
  kv->sequences = sequences;
  kv->layers = num_layers;
  kv->max_seq_len = max_seq_len;
  kv->dtype = dtype;
  kv->hkv_l.assign(num_layers, 0);
  kv->dk_l.assign(num_layers, 0);
  kv->dv_l.assign(num_layers, 0);
  kv->ring.assign(num_layers, 0);
  kv->cap.assign(num_layers, 0);
  kv->layer_off_k.assign(num_layers, 0);
  kv->layer_off_v.assign(num_layers, 0);
  uint64_t off_k = 0, off_v = 0;
  for (uint32_t l = 0; l < num_layers; ++l) {
    const jmodels_attn_layer_spec& sp = specs[l];
    const std::string at = " (layer " + std::to_string(l) + ")";
    require(sp.num_kv_heads > 0 && sp.key_length > 0 && sp.value_length > 0,
            JMODELS_ATTN_INVALID_SHAPE, "layer dimensions must be > 0" + at);
    require(sp.key_length % 16 == 0 && sp.value_length % 16 == 0, JMODELS_ATTN_INVALID_SHAPE,
            "key_length and value_length must be multiples of 16" + at);
    require(sp.num_kv_heads <= 4096 && sp.key_length <= 4096 && sp.value_length <= 4096,
            JMODELS_ATTN_INVALID_SHAPE, "layer dimensions exceed 4096" + at);
    kv->hkv_l[l] = sp.num_kv_heads;
    kv->dk_l[l] = sp.key_length;
    kv->dv_l[l] = sp.value_length;
    uint32_t r = sp.ring_capacity;
    // LayeredKvCache physicalLimit = min(ringCapacity, maxSeqLen) (cache/LayeredKvCache.java:128-129);
    // a ring at least as long as the context never wraps, so it is stored linearly.
    if (r >= max_seq_len) r = 0;
    kv->ring[l] = r;
    kv->cap[l] = (uint32_t)round_up(r ? r : max_seq_len, 32);
    kv->layer_off_k[l] = off_k;
    kv->layer_off_v[l] = off_v;
    off_k += (uint64_t)sp.num_kv_heads * kv->cap[l] * sp.key_length;
    off_v += (uint64_t)sp.num_kv_heads * kv->cap[l] * sp.value_length;
  }
  kv->seq_stride_k = off_k;
  kv->seq_stride_v = off_v;
  const uint64_t kbytes = off_k * sequences * kv->elem();
  const uint64_t vbytes = off_v * sequences * kv->elem();
  kv->bytes = kbytes + vbytes;
  set_device(ctx);
  hip_check(hipMalloc(&kv->d_k, kbytes), "hipMalloc K cache");
  if (hipMalloc(&kv->d_v, vbytes) != hipSuccess) {
    (void)hipFree(kv->d_k);
    fail(JMODELS_ATTN_DEVICE_ERROR, "hipMalloc V cache failed");
  }
  // Zero fill: rows past a sequence's end are masked, and zeros keep 0 * V finite.
  hip_check(hipMemsetAsync(kv->d_k, 0, kbytes, ctx->stream), "zero K cache");
  hip_check(hipMemsetAsync(kv->d_v, 0, vbytes, ctx->stream), "zero V cache");
  hip_check(hipStreamSynchronize(ctx->stream), "zero cache");
  const size_t n = (size_t)sequences * num_layers;
  kv->populated.resize(n);
  kv->positions.resize(n);
  kv->contiguous_end.assign(n, 0);
  for (uint32_t s = 0; s < sequences; ++s)
    for (uint32_t l = 0; l < num_layers; ++l) {
      if (kv->ring[l]) kv->positions[kv->idx(s, l)].assign(kv->ring[l], -1);
      else kv->populated[kv->idx(s, l)].assign((max_seq_len + 63) / 64, 0);
    }
  *kv_out = kv.release();
}

int32_t jmodels_attn_kv_create(jmodels_attn_context* ctx, uint32_t sequences, uint32_t num_layers,
                               uint32_t max_seq_len, uint32_t num_kv_heads, uint32_t key_length,
                               uint32_t value_length, uint32_t dtype,
                               const uint32_t* ring_capacity, jmodels_attn_kv** kv_out) {
  return guard([&] {
    require(num_layers > 0 && num_layers <= (1u << 20), JMODELS_ATTN_INVALID_SHAPE,
            "num_layers must be in [1, 2^20]");
    std::vector<jmodels_attn_layer_spec> specs(num_layers);
    for (uint32_t l = 0; l < num_layers; ++l)
      specs[l] = jmodels_attn_layer_spec{num_kv_heads, key_length, value_length,
                                         ring_capacity ? ring_capacity[l] : 0u};
    create_layered(ctx, sequences, num_layers, max_seq_len, specs.data(), dtype, kv_out);
  });
}

int32_t jmodels_attn_kv_create_layered(jmodels_attn_context* ctx, uint32_t sequences,
                                       uint32_t num_layers, uint32_t max_seq_len,
                                       const jmodels_attn_layer_spec* specs, uint32_t dtype,
                                       jmodels_attn_kv** kv_out) {
  return guard([&] { create_layered(ctx, sequences, num_layers, max_seq_len, specs, dtype, kv_out); });
}

int32_t jmodels_attn_kv_destroy(jmodels_attn_kv* kv) {
  if (!kv) return JMODELS_ATTN_NULL_POINTER;
  return guard([&] {
    (void)hipSetDevice(kv->ctx->device);
    (void)hipStreamSynchronize(kv->ctx->stream);
    (void)hipFree(kv->d_k);
    (void)hipFree(kv->d_v);
    delete kv;
  });
}

int32_t jmodels_attn_kv_clear(jmodels_attn_kv* kv, int32_t sequence) {
  return guard([&] {
    require(kv != nullptr, JMODELS_ATTN_NULL_POINTER, "kv is null");
    require(sequence < (int32_t)kv->sequences, JMODELS_ATTN_OUT_OF_RANGE, "sequence out of range");
    for (uint32_t s = 0; s < kv->sequences; ++s) {
      if (sequence >= 0 && (uint32_t)sequence != s) continue;
      for (uint32_t l = 0; l < kv->layers; ++l) {
        const size_t i = kv->idx(s, l);
        if (kv->ring[l]) std::fill(kv->positions[i].begin(), kv->positions[i].end(), -1);
        else std::fill(kv->populated[i].begin(), kv->populated[i].end(), 0);
        kv->contiguous_end[i] = 0;
      }
    }
  });
}

int32_t jmodels_attn_kv_discard_from(jmodels_attn_kv* kv, uint32_t sequence, uint32_t position) {
  return guard([&] {
    require(kv != nullptr, JMODELS_ATTN_NULL_POINTER, "kv is null");
    require(sequence < kv->sequences, JMODELS_ATTN_OUT_OF_RANGE, "sequence out of range");
    require(position <= kv->max_seq_len, JMODELS_ATTN_OUT_OF_RANGE,
            "position out of range: " + std::to_string(position));
    for (uint32_t l = 0; l < kv->layers; ++l) {
      const size_t i = kv->idx(sequence, l);
      if (kv->ring[l]) {
        for (auto& p : kv->positions[i])
          if (p >= (int32_t)position) p = -1;
        continue;
      }
      auto& bits = kv->populated[i];
      for (uint32_t p = position; p < kv->max_seq_len; ++p) {
        if ((p & 63) == 0 && p + 64 <= kv->max_seq_len) {
          bits[p >> 6] = 0;
          p += 63;
          continue;
        }
        bits[p >> 6] &= ~(1ull << (p & 63));
      }
      kv->contiguous_end[i] = std::min(kv->contiguous_end[i], position);
    }
  });
}

int32_t jmodels_attn_kv_contains(const jmodels_attn_kv* kv, uint32_t sequence, uint32_t layer,
                                 uint32_t position, int32_t* out) {
  return guard([&] {
    require(kv != nullptr && out != nullptr, JMODELS_ATTN_NULL_POINTER, "null argument");
    require(sequence < kv->sequences, JMODELS_ATTN_OUT_OF_RANGE, "sequence out of range");
    require(layer < kv->layers, JMODELS_ATTN_OUT_OF_RANGE, "layer out of range: " + std::to_string(layer));
    require(position < kv->max_seq_len, JMODELS_ATTN_OUT_OF_RANGE,
            "position out of range: " + std::to_string(position));
    *out = kv->available(sequence, layer, position) ? 1 : 0;
  });
}

int32_t jmodels_attn_kv_store(jmodels_attn_context* ctx, jmodels_attn_kv* kv, uint32_t sequence,
                              uint32_t layer, uint32_t position, const float* key,
                              uint64_t key_elements, const float* value, uint64_t value_elements) {
  return guard([&] {
    check_ctx(ctx);
    require(kv != nullptr && key != nullptr && value != nullptr, JMODELS_ATTN_NULL_POINTER, "null argument");
    require(kv->ctx == ctx, JMODELS_ATTN_INVALID_SHAPE, "cache belongs to another context");
    require(layer < kv->layers, JMODELS_ATTN_OUT_OF_RANGE, "layer out of range: " + std::to_string(layer));
    require(sequence < kv->sequences, JMODELS_ATTN_OUT_OF_RANGE, "sequence out of range");
    require(position < kv->max_seq_len, JMODELS_ATTN_OUT_OF_RANGE,
            "position out of range: " + std::to_string(position));
    const uint32_t hkv = kv->hkv_l[layer], key_len = kv->dk_l[layer], value_len = kv->dv_l[layer];
    const uint64_t kdim = (uint64_t)hkv * key_len, vdim = (uint64_t)hkv * value_len;
    check_elems(key_elements, kdim, "key");
    check_elems(value_elements, vdim, "value");
    set_device(ctx);
    float* dk = stage(ctx->stage_k, key, kdim, ctx->stream);
    float* dv = stage(ctx->stage_v, value, vdim, ctx->stream);
    // q is unused by a store: point it at k with zero query heads' worth of work.
    jma::RowList rows = make_rows(1, &sequence, &position);
    jma::AppendArgs a{};
    a.kv = kv->view(layer);
    a.q = dk;
    a.k = dk;
    a.v = dv;
    a.num_heads = 0;
    a.num_kv_heads = hkv;
    a.dk = key_len;
    a.dv = value_len;
    a.blocks_per_row = append_blocks_per_row(0, hkv, key_len, value_len);
    a.rows = rows;
    hip_check(jma::launch_append(a, kv->f16(), ctx->stream), "store launch");
    hip_check(hipStreamSynchronize(ctx->stream), "store");
    kv->mark(sequence, layer, position);
  });
}

int32_t jmodels_attn_kv_read(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                             uint32_t sequence, uint32_t layer, uint32_t from, uint32_t to,
                             float* keys, uint64_t key_elements, float* values,
                             uint64_t value_elements) {
  return guard([&] {
    check_ctx(ctx);
    require(kv != nullptr, JMODELS_ATTN_NULL_POINTER, "kv is null");
    require(layer < kv->layers, JMODELS_ATTN_OUT_OF_RANGE, "layer out of range: " + std::to_string(layer));
    require(sequence < kv->sequences, JMODELS_ATTN_OUT_OF_RANGE, "sequence out of range");
    require(from <= to && to <= kv->max_seq_len, JMODELS_ATTN_OUT_OF_RANGE,
            "invalid position range: [" + std::to_string(from) + ", " + std::to_string(to) + ")");
    const uint32_t n = to - from;
    const uint32_t hkv = kv->hkv_l[layer], key_len = kv->dk_l[layer], value_len = kv->dv_l[layer];
    const uint64_t kdim = (uint64_t)hkv * key_len, vdim = (uint64_t)hkv * value_len;
    if (keys) check_elems(key_elements, n * kdim, "keys");
    if (values) check_elems(value_elements, n * vdim, "values");
    if (n == 0) return;
    // A ring layer rejects a range wider than its capacity before it looks at positions
    // (LayeredKvCache.attentionView, cache/LayeredKvCache.java:178-197).
    kv->require_range(sequence, layer, from, to - 1);
    set_device(ctx);
    hip_check(hipStreamSynchronize(ctx->stream), "read");
    const size_t es = kv->elem();
    const uint32_t cap = kv->cap[layer];
    const uint32_t blk = (uint32_t)jma::v_block(kv->f16());
    const uint64_t kl = (uint64_t)hkv * cap * key_len, vl = (uint64_t)hkv * cap * value_len;
    std::vector<unsigned char> hk(kl * es), hv(vl * es);
    const unsigned char* kbase = (const unsigned char*)kv->d_k +
                                 (sequence * kv->seq_stride_k + kv->layer_off_k[layer]) * es;
    const unsigned char* vbase = (const unsigned char*)kv->d_v +
                                 (sequence * kv->seq_stride_v + kv->layer_off_v[layer]) * es;
    hip_check(hipMemcpy(hk.data(), kbase, hk.size(), hipMemcpyDeviceToHost), "read K");
    hip_check(hipMemcpy(hv.data(), vbase, hv.size(), hipMemcpyDeviceToHost), "read V");
    auto widen = [&](const unsigned char* src, uint64_t index) -> float {
      if (kv->f16()) {
        uint16_t h;
        memcpy(&h, src + index * 2, 2);
        return f16_bits_to_float(h);
      }
      float f;
      memcpy(&f, src + index * 4, 4);
      return f;
    };
    for (uint32_t p = from; p < to; ++p) {
      const uint32_t slot = kv->ring[layer] ? p % cap : p;
      const uint32_t r = slot % blk, b = slot / blk;
      const uint32_t s = kv->f16() ? 8u * ((r & 15u) >> 2) + 4u * (r >> 4) + (r & 3u) : r;
      for (uint32_t h = 0; h < hkv; ++h) {
        if (keys)
          for (uint32_t d = 0; d < key_len; ++d)
            keys[(uint64_t)(p - from) * kdim + h * key_len + d] =
                widen(hk.data(), (uint64_t)h * cap * key_len + jma::k_index(slot, d, key_len, kv->f16()));
        if (values)
          for (uint32_t d = 0; d < value_len; ++d)
            values[(uint64_t)(p - from) * vdim + h * value_len + d] =
                widen(hv.data(), (uint64_t)h * cap * value_len + ((uint64_t)b * value_len + d) * blk + s);
      }
    }
  });
}

int32_t jmodels_attn_kv_bytes(const jmodels_attn_kv* kv, uint64_t* bytes_out) {
  return guard([&] {
    require(kv != nullptr && bytes_out != nullptr, JMODELS_ATTN_NULL_POINTER, "null argument");
    *bytes_out = kv->bytes;
  });
}

// ---------------------------------------------------------------- attention entry points

static void common_checks(jmodels_attn_context* ctx, const jmodels_attn_kv* kv) {
  check_ctx(ctx);
  require(kv != nullptr, JMODELS_ATTN_NULL_POINTER, "kv is null");
  require(kv->ctx == ctx, JMODELS_ATTN_INVALID_SHAPE, "cache belongs to another context");
}

static int32_t append_entry(bool device, jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, const float* k, uint64_t k_elements,
                            const float* v, uint64_t v_elements, float* q_rotated,
                            uint64_t q_rotated_elements) {
  return guard([&] {
    common_checks(ctx, kv);
    const LayerCall lc = resolve_layer(kv, layer);
    check_rows(kv, lc, count, sequences, positions);
    require(q && k && v, JMODELS_ATTN_NULL_POINTER, "q/k/v are null");
    const uint64_t qn = (uint64_t)count * lc.num_heads * lc.dk;
    check_elems(q_elements, qn, "q");
    check_elems(k_elements, (uint64_t)count * lc.hkv * lc.dk, "k");
    check_elems(v_elements, (uint64_t)count * lc.hkv * lc.dv, "v");
    if (q_rotated) check_elems(q_rotated_elements, qn, "q_rotated");
    set_device(ctx);
    if (device) {
      append_rows(ctx, kv, lc, count, sequences, positions, q, k, v, q_rotated);
      return;
    }
    const float* dq = stage(ctx->stage_q, q, qn, ctx->stream);
    const float* dk = stage(ctx->stage_k, k, (uint64_t)count * lc.hkv * lc.dk, ctx->stream);
    const float* dv = stage(ctx->stage_v, v, (uint64_t)count * lc.hkv * lc.dv, ctx->stream);
    float* dqo = q_rotated ? stage<float>(ctx->stage_out, nullptr, qn, ctx->stream) : nullptr;
    append_rows(ctx, kv, lc, count, sequences, positions, dq, dk, dv, dqo);
    if (q_rotated)
      hip_check(hipMemcpyAsync(q_rotated, dqo, qn * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
                "copy q_rotated");
    collect_errors(ctx);
  });
}

static int32_t attend_entry(bool device, jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, float* out, uint64_t out_elements) {
  return guard([&] {
    common_checks(ctx, kv);
    const LayerCall lc = resolve_layer(kv, layer);
    check_decode_shape(kv, lc);
    check_rows(kv, lc, count, sequences, positions);
    require(q && out, JMODELS_ATTN_NULL_POINTER, "q/out are null");
    const uint64_t qn = (uint64_t)count * lc.num_heads * lc.dk;
    const uint64_t on = (uint64_t)count * lc.num_heads * lc.dv;
    check_elems(q_elements, qn, "q");
    check_elems(out_elements, on, "out");
    validate_attend_ranges(kv, lc, count, sequences, positions);
    set_device(ctx);
    if (device) {
      run_attend(ctx, kv, lc, count, sequences, positions, q, out);
      return;
    }
    const float* dq = stage(ctx->stage_q, q, qn, ctx->stream);
    float* dout = stage<float>(ctx->stage_out, nullptr, on, ctx->stream);
    run_attend(ctx, kv, lc, count, sequences, positions, dq, dout);
    hip_check(hipMemcpyAsync(out, dout, on * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
              "copy out");
    collect_errors(ctx);
  });
}

// fixed: null = the context's grow-only scratch; else the device's fixed scratch (device
// pointers only), with plans that need more refused before anything is enqueued.
static int32_t decode_entry(bool device, jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, const float* k, uint64_t k_elements,
                            const float* v, uint64_t v_elements, float* out,
                            uint64_t out_elements, const jma::FixedScratch* fixed = nullptr) {
  return guard([&] {
    common_checks(ctx, kv);
    const LayerCall lc = resolve_layer(kv, layer);
    check_decode_shape(kv, lc);
    check_rows(kv, lc, count, sequences, positions);
    require(q && k && v && out, JMODELS_ATTN_NULL_POINTER, "q/k/v/out are null");
    const uint64_t qn = (uint64_t)count * lc.num_heads * lc.dk;
    const uint64_t kn = (uint64_t)count * lc.hkv * lc.dk;
    const uint64_t vn = (uint64_t)count * lc.hkv * lc.dv;
    const uint64_t on = (uint64_t)count * lc.num_heads * lc.dv;
    check_elems(q_elements, qn, "q");
    check_elems(k_elements, kn, "k");
    check_elems(v_elements, vn, "v");
    check_elems(out_elements, on, "out");
    // Sessions of one batch must be distinct (LlamaForwardPass.validateSessionBatch,
    // llama/LlamaForwardPass.java:933-960).
    for (uint32_t i = 0; i < count; ++i)
      for (uint32_t j = 0; j < i; ++j)
        require(sequences[i] != sequences[j], JMODELS_ATTN_INVALID_SHAPE, "sessions must be distinct");
    // Everything the new rows will read, except the rows themselves, must already be cached.
    for (uint32_t i = 0; i < count; ++i) {
      const uint32_t p = positions[i];
      const uint32_t first = jma::first_visible(p, lc.window);
      if (kv->ring[lc.layer] && p - first + 1 > kv->ring[lc.layer])
        fail(JMODELS_ATTN_OUT_OF_RANGE, "attention range exceeds ring capacity " +
                                            std::to_string(kv->ring[lc.layer]));
      if (first < p) kv->require_range(sequences[i], lc.layer, first, p - 1);
    }
    if (fixed) {
      // Every launch's plan and the rotated-query buffer are checked against the fixed scratch
      // before anything is enqueued: a refusal appends nothing and marks nothing. Both paths
      // below cut the rows into the same chunks of kMaxRows.
      for (uint32_t base = 0; base < count; base += jma::kMaxRows) {
        const uint32_t n = std::min<uint32_t>(jma::kMaxRows, count - base);
        check_fixed_fit(decode_plan(ctx, kv, lc, make_rows(n, sequences + base, positions + base)),
                        *fixed);
      }
      if (!can_fuse_decode(ctx, lc))
        require(qn * sizeof(float) <= fixed->qrot_bytes, JMODELS_ATTN_BUFFER_TOO_SMALL,
                "the rotated queries need " + std::to_string(qn * sizeof(float)) +
                    " bytes, the fixed scratch holds " + std::to_string(fixed->qrot_bytes));
    }
    set_device(ctx);
    const float* dq = q;
    const float* dk = k;
    const float* dv = v;
    float* dout = out;
    if (!device) {
      dq = stage(ctx->stage_q, q, qn, ctx->stream);
      dk = stage(ctx->stage_k, k, kn, ctx->stream);
      dv = stage(ctx->stage_v, v, vn, ctx->stream);
      dout = stage<float>(ctx->stage_out, nullptr, on, ctx->stream);
    }
    if (can_fuse_decode(ctx, lc)) {
      // One launch per chunk of rows: RoPE, append, attention and the split reduction.
      const uint64_t qdim = (uint64_t)lc.num_heads * lc.dk, kdim = (uint64_t)lc.hkv * lc.dk;
      const uint64_t vdim = (uint64_t)lc.hkv * lc.dv, odim = (uint64_t)lc.num_heads * lc.dv;
      for (uint32_t base = 0; base < count; base += jma::kMaxRows) {
        const uint32_t n = std::min<uint32_t>(jma::kMaxRows, count - base);
        jma::RowList rows = make_rows(n, sequences + base, positions + base);
        FusedAppend fa;
        fa.k = dk + base * kdim;
        fa.v = dv + base * vdim;
        fa.rope_q = lc.rope != nullptr || lc.norm != nullptr;
        run_attend_rows(ctx, kv, lc, rows, dq + base * qdim, dout + base * odim, fa, fixed);
      }
      for (uint32_t i = 0; i < count; ++i) kv->mark(sequences[i], lc.layer, positions[i]);
    } else {
      float* qrot = nullptr;
      if (fixed) {
        qrot = fixed->qrot;  // its size was checked above, before anything was enqueued
      } else {
        ctx->qrot.reserve(qn * sizeof(float), ctx->stream, "decode rotated queries");
        qrot = (float*)ctx->qrot.ptr;
      }
      append_rows(ctx, kv, lc, count, sequences, positions, dq, dk, dv, qrot);
      run_attend(ctx, kv, lc, count, sequences, positions, qrot, dout, fixed);
    }
    if (device) return;
    hip_check(hipMemcpyAsync(out, dout, on * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
              "copy out");
    collect_errors(ctx);
  });
}

static int32_t prefill_entry(bool device, jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                             const jmodels_attn_layer* layer, uint32_t sequence, uint32_t start,
                             uint32_t n, const float* q, uint64_t q_elements, const float* k,
                             uint64_t k_elements, const float* v, uint64_t v_elements,
                             float* out, uint64_t out_elements) {
  return guard([&] {
    common_checks(ctx, kv);
    const LayerCall lc = resolve_layer(kv, layer);
    require(n > 0, JMODELS_ATTN_INVALID_SHAPE, "n must be > 0");
    require(sequence < kv->sequences, JMODELS_ATTN_OUT_OF_RANGE, "sequence out of range");
    require((uint64_t)start + n <= kv->max_seq_len, JMODELS_ATTN_OUT_OF_RANGE,
            "position out of range: " + std::to_string((uint64_t)start + n - 1));
    if (lc.rope)
      require((uint64_t)start + n <= lc.rope->max_positions, JMODELS_ATTN_OUT_OF_RANGE,
              "positions beyond the rope table");
    require(q && k && v && out, JMODELS_ATTN_NULL_POINTER, "q/k/v/out are null");
    const uint64_t qn = (uint64_t)n * lc.num_heads * lc.dk;
    const uint64_t kn = (uint64_t)n * lc.hkv * lc.dk;
    const uint64_t vn = (uint64_t)n * lc.hkv * lc.dv;
    const uint64_t on = (uint64_t)n * lc.num_heads * lc.dv;
    check_elems(q_elements, qn, "q");
    check_elems(k_elements, kn, "k");
    check_elems(v_elements, vn, "v");
    check_elems(out_elements, on, "out");
    set_device(ctx);
    if (device) {
      prefill_impl(ctx, kv, lc, sequence, start, n, q, k, v, out);
      return;
    }
    const float* dq = stage(ctx->stage_q, q, qn, ctx->stream);
    const float* dk = stage(ctx->stage_k, k, kn, ctx->stream);
    const float* dv = stage(ctx->stage_v, v, vn, ctx->stream);
    float* dout = stage<float>(ctx->stage_out, nullptr, on, ctx->stream);
    prefill_impl(ctx, kv, lc, sequence, start, n, dq, dk, dv, dout);
    hip_check(hipMemcpyAsync(out, dout, on * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
              "copy out");
    collect_errors(ctx);
  });
}

static int32_t attend_causal_entry(bool device, jmodels_attn_context* ctx,
                                   const jmodels_attn_kv* kv, const jmodels_attn_layer* layer,
                                   uint32_t sequence, uint32_t start, uint32_t n, const float* q,
                                   uint64_t q_elements, float* out, uint64_t out_elements) {
  return guard([&] {
    common_checks(ctx, kv);
    const LayerCall lc = resolve_layer(kv, layer);
    require(n > 0, JMODELS_ATTN_INVALID_SHAPE, "n must be > 0");
    require(sequence < kv->sequences, JMODELS_ATTN_OUT_OF_RANGE, "sequence out of range");
    require((uint64_t)start + n <= kv->max_seq_len, JMODELS_ATTN_OUT_OF_RANGE,
            "position out of range: " + std::to_string((uint64_t)start + n - 1));
    require(q && out, JMODELS_ATTN_NULL_POINTER, "q/out are null");
    const uint64_t qn = (uint64_t)n * lc.num_heads * lc.dk;
    const uint64_t on = (uint64_t)n * lc.num_heads * lc.dv;
    check_elems(q_elements, qn, "q");
    check_elems(out_elements, on, "out");
    check_prefill_shape(kv, lc);
    validate_causal(kv, lc, sequence, start, n, true);
    set_device(ctx);
    if (device) {
      attend_causal_impl(ctx, kv, lc, sequence, start, n, q, out);
      return;
    }
    const float* dq = stage(ctx->stage_q, q, qn, ctx->stream);
    float* dout = stage<float>(ctx->stage_out, nullptr, on, ctx->stream);
    attend_causal_impl(ctx, kv, lc, sequence, start, n, dq, dout);
    hip_check(hipMemcpyAsync(out, dout, on * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
              "copy out");
    collect_errors(ctx);
  });
}

int32_t jmodels_attn_attend_causal(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t sequence,
                                   uint32_t start, uint32_t n, const float* q,
                                   uint64_t q_elements, float* out, uint64_t out_elements) {
  return attend_causal_entry(false, ctx, kv, layer, sequence, start, n, q, q_elements, out,
                             out_elements);
}

int32_t jmodels_attn_attend_causal_device(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                                          const jmodels_attn_layer* layer, uint32_t sequence,
                                          uint32_t start, uint32_t n, const float* q,
                                          uint64_t q_elements, float* out,
                                          uint64_t out_elements) {
  return attend_causal_entry(true, ctx, kv, layer, sequence, start, n, q, q_elements, out,
                             out_elements);
}

int32_t jmodels_attn_append(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, const float* k, uint64_t k_elements,
                            const float* v, uint64_t v_elements, float* q_rotated,
                            uint64_t q_rotated_elements) {
  return append_entry(false, ctx, kv, layer, count, sequences, positions, q, q_elements, k,
                      k_elements, v, v_elements, q_rotated, q_rotated_elements);
}

int32_t jmodels_attn_attend(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, float* out, uint64_t out_elements) {
  return attend_entry(false, ctx, kv, layer, count, sequences, positions, q, q_elements, out,
                      out_elements);
}

int32_t jmodels_attn_decode(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, const float* k, uint64_t k_elements,
                            const float* v, uint64_t v_elements, float* out,
                            uint64_t out_elements) {
  return decode_entry(false, ctx, kv, layer, count, sequences, positions, q, q_elements, k,
                      k_elements, v, v_elements, out, out_elements);
}

int32_t jmodels_attn_prefill(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                             const jmodels_attn_layer* layer, uint32_t sequence, uint32_t start,
                             uint32_t n, const float* q, uint64_t q_elements, const float* k,
                             uint64_t k_elements, const float* v, uint64_t v_elements,
                             float* out, uint64_t out_elements) {
  return prefill_entry(false, ctx, kv, layer, sequence, start, n, q, q_elements, k, k_elements, v,
                       v_elements, out, out_elements);
}

int32_t jmodels_attn_append_device(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t count,
                                   const uint32_t* sequences, const uint32_t* positions,
                                   const float* q, uint64_t q_elements, const float* k,
                                   uint64_t k_elements, const float* v, uint64_t v_elements,
                                   float* q_rotated, uint64_t q_rotated_elements) {
  return append_entry(true, ctx, kv, layer, count, sequences, positions, q, q_elements, k,
                      k_elements, v, v_elements, q_rotated, q_rotated_elements);
}

int32_t jmodels_attn_attend_device(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t count,
                                   const uint32_t* sequences, const uint32_t* positions,
                                   const float* q, uint64_t q_elements, float* out,
                                   uint64_t out_elements) {
  return attend_entry(true, ctx, kv, layer, count, sequences, positions, q, q_elements, out,
                      out_elements);
}

int32_t jmodels_attn_decode_device(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t count,
                                   const uint32_t* sequences, const uint32_t* positions,
                                   const float* q, uint64_t q_elements, const float* k,
                                   uint64_t k_elements, const float* v, uint64_t v_elements,
                                   float* out, uint64_t out_elements) {
  return decode_entry(true, ctx, kv, layer, count, sequences, positions, q, q_elements, k,
                      k_elements, v, v_elements, out, out_elements);
}

int32_t jmodels_attn_decode_device_noalloc(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                           const jmodels_attn_layer* layer, uint32_t count,
                                           const uint32_t* sequences, const uint32_t* positions,
                                           const float* q, uint64_t q_elements, const float* k,
                                           uint64_t k_elements, const float* v,
                                           uint64_t v_elements, float* out,
                                           uint64_t out_elements) {
  if (!ctx) return JMODELS_ATTN_NULL_POINTER;
  return decode_entry(true, ctx, kv, layer, count, sequences, positions, q, q_elements, k,
                      k_elements, v, v_elements, out, out_elements, &ctx->fixed);
}

int32_t jmodels_attn_prefill_device(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                    const jmodels_attn_layer* layer, uint32_t sequence,
                                    uint32_t start, uint32_t n, const float* q,
                                    uint64_t q_elements, const float* k, uint64_t k_elements,
                                    const float* v, uint64_t v_elements, float* out,
                                    uint64_t out_elements) {
  return prefill_entry(true, ctx, kv, layer, sequence, start, n, q, q_elements, k, k_elements, v,
                       v_elements, out, out_elements);
}

int32_t jmodels_attn_quantized_matmul_device(jmodels_attn_context* ctx, uint32_t format,
                                             const void* weights, uint64_t weight_bytes,
                                             const float* input, uint64_t input_elements,
                                             float* output, uint64_t output_elements,
                                             uint32_t batch_size, uint32_t rows, uint32_t cols,
                                             const float* addend, uint32_t addend_mode) {
  return guard([&] {
    quantized_matmul_impl(ctx, {QuantMatrix{format, weights, weight_bytes, rows, addend}}, input,
                          input_elements, output, output_elements, batch_size, cols, addend_mode);
  });
}

int32_t jmodels_attn_quantized_grouped_matmul_device(
    jmodels_attn_context* ctx, const uint32_t* formats, const void* const* weights,
    const uint64_t* weight_bytes, const uint32_t* rows, uint32_t matrix_count, const float* input,
    uint64_t input_elements, float* output, uint64_t output_elements, uint32_t batch_size,
    uint32_t cols, const float* const* addends, uint32_t addend_mode) {
  return guard([&] {
    require(formats != nullptr && weights != nullptr && weight_bytes != nullptr && rows != nullptr,
            JMODELS_ATTN_NULL_POINTER, "null matrix table");
    require(addend_mode == 0 || addends != nullptr, JMODELS_ATTN_NULL_POINTER, "null addends");
    require(matrix_count >= 1 && matrix_count <= jma::kQMaxMatrices, JMODELS_ATTN_INVALID_SHAPE,
            "matrix_count must be in [1, 16]");
    std::vector<QuantMatrix> mats(matrix_count);
    for (uint32_t i = 0; i < matrix_count; ++i)
      mats[i] = QuantMatrix{formats[i], weights[i], weight_bytes[i], rows[i],
                            addend_mode ? addends[i] : nullptr};
    quantized_matmul_impl(ctx, mats, input, input_elements, output, output_elements, batch_size,
                          cols, addend_mode);
  });
}

}  // extern "C"
