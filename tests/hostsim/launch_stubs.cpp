// The kernel side of libjmodels_attn for the host simulation (tests/hostsim/hip_sim.cpp): every
// launch function of models_amd/csrc/jma_kernels.h, with the runtime's own arguments, names the
// device ranges its kernel reads or writes (the extents follow the kernels' indexing: the layer
// region of the cache for each row's sequence, the partial buffers by the plan's item count, the
// row tables' largest position for the RoPE tables, every projection matrix's weights, outputs
// and addends) and hands them to the simulation, which checks them against the live allocations
// when the launch executes (for a captured launch: at every graph replay). No kernel runs.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "jma_kernels.h"

namespace jma {
namespace {

struct Range {
  const void* p;
  size_t bytes;
  std::string what;
};

struct Launch {
  std::vector<Range> ranges;
};

void check_all(void* arg) {
  for (const Range& r : ((Launch*)arg)->ranges) hipsim_check_range(r.p, r.bytes, r.what.c_str());
}

void drop(void* arg) { delete (Launch*)arg; }

hipError_t submit(hipStream_t stream, const char* kernel, Launch* l) {
  for (Range& r : l->ranges) r.what = std::string(kernel) + ": " + r.what;
  return hipsim_launch(stream, kernel, check_all, l, drop);
}

void add(Launch* l, const void* p, size_t bytes, const char* what) {
  if (p != nullptr && bytes > 0) l->ranges.push_back({p, bytes, what});
}

uint32_t row_seq(const RowList& r, uint32_t i) { return r.contiguous ? r.seq0 : r.seq[i]; }
uint32_t row_pos(const RowList& r, uint32_t i) { return r.contiguous ? r.start + i : r.pos[i]; }

uint32_t max_pos(const RowList& r) {
  uint32_t m = 0;
  for (uint32_t i = 0; i < r.count; ++i) m = std::max(m, row_pos(r, i));
  return m;
}

// The layer region (all kv heads, every slot) of each row's sequence, K and V.
void add_cache(Launch* l, const KvView& kv, const RowList& rows, uint32_t hkv, uint32_t dk,
               uint32_t dv, size_t es) {
  for (uint32_t i = 0; i < rows.count; ++i) {
    const uint64_t s = row_seq(rows, i);
    add(l, (const char*)kv.k + (s * kv.seq_stride_k + kv.layer_off_k) * es, (size_t)hkv * kv.cap * dk * es, "K cache");
    add(l, (const char*)kv.v + (s * kv.seq_stride_v + kv.layer_off_v) * es, (size_t)hkv * kv.cap * dv * es, "V cache");
  }
}

}  // namespace

hipError_t fixed_scratch_reset(const FixedScratch& s, hipStream_t) {
  memset(s.counters, 0, s.counters_bytes);
  memset(s.part_f, 0xFF, s.part_f_bytes);
  return hipSuccess;
}

hipError_t fixed_scratch(int device, hipStream_t stream, FixedScratch* out) {
  // The product's sizes (a file-scope device array there; one allocation kept to the end here).
  static FixedScratch s;
  static bool ready = false;
  if (device != 0) return hipErrorInvalidDevice;
  if (!ready) {
    const size_t c = size_t(64) << 10, f = size_t(16) << 20, acc = size_t(16) << 20,
                 ml = size_t(1) << 20, q = size_t(8) << 20;
    unsigned char* base = nullptr;
    hipError_t e = hipMalloc((void**)&base, c + f + acc + ml + q);
    if (e != hipSuccess) return e;
    s.counters = (uint32_t*)base;
    s.counters_bytes = c;
    s.part_f = (float*)(base + c);
    s.part_f_bytes = f;
    s.part_acc = (float*)(base + c + f);
    s.part_acc_bytes = acc;
    s.part_ml = (float*)(base + c + f + acc);
    s.part_ml_bytes = ml;
    s.qrot = (float*)(base + c + f + acc + ml);
    s.qrot_bytes = q;
    e = fixed_scratch_reset(s, stream);
    if (e != hipSuccess) return e;
    ready = true;
  }
  *out = s;
  return hipSuccess;
}

hipError_t launch_append(const AppendArgs& a, bool f16, hipStream_t stream) {
  Launch* l = new Launch();
  const size_t n = a.rows.count;
  add(l, a.q, n * a.num_heads * a.dk * 4, "q");
  add(l, a.k, n * a.num_kv_heads * a.dk * 4, "k");
  add(l, a.v, n * a.num_kv_heads * a.dv * 4, "v");
  add(l, a.q_out, n * a.num_heads * a.dk * 4, "rotated q");
  add(l, a.cos_t, ((size_t)max_pos(a.rows) + 1) * a.pairs * 4, "cos table");
  add(l, a.sin_t, ((size_t)max_pos(a.rows) + 1) * a.pairs * 4, "sin table");
  add(l, a.q_norm_w, (size_t)a.dk * 4, "q norm");
  add(l, a.k_norm_w, (size_t)a.dk * 4, "k norm");
  add_cache(l, a.kv, a.rows, a.num_kv_heads, a.dk, a.dv, f16 ? 2 : 4);
  return submit(stream, "rope_append_kernel", l);
}

hipError_t launch_decode(const DecodeArgs& a, bool f16, int dk, int dv, hipStream_t stream) {
  if (!decode_supported(f16, dk, dv)) return hipErrorInvalidValue;
  if (a.total_items == 0) return hipSuccess;
  Launch* l = new Launch();
  const size_t n = a.rows.count, es = f16 ? 2 : 4;
  add(l, a.q, n * a.num_heads * dk * 4, "q");
  add(l, a.out, n * a.num_heads * dv * 4, "out");
  add(l, a.k_new, n * a.num_kv_heads * dk * 4, "new k rows");
  add(l, a.v_new, n * a.num_kv_heads * dv * 4, "new v rows");
  add(l, a.cos_t, ((size_t)max_pos(a.rows) + 1) * a.pairs * 4, "cos table");
  add(l, a.sin_t, ((size_t)max_pos(a.rows) + 1) * a.pairs * 4, "sin table");
  add(l, a.q_norm_w, (size_t)dk * 4, "q norm");
  add(l, a.k_norm_w, (size_t)dk * 4, "k norm");
  add(l, a.err, 4, "error word");
  const size_t dvs = (size_t)dv / std::max<uint32_t>(a.slices, 1);
  if (a.counters != nullptr) {
    add(l, a.part_f, (size_t)a.total_items * kHeadSlots * (dvs + 4) * 4, "fused partials");
    add(l, a.counters, n * a.num_kv_heads * a.hgroups * 4, "arrival tickets");
  } else if (a.max_splits > 1) {
    const size_t items = a.total_items / std::max<uint32_t>(a.slices, 1);
    add(l, a.part_acc, items * kHeadSlots * dv * 4, "split partials");
    add(l, a.part_ml, items * kHeadSlots * 2 * 4, "split maxima");
  }
  add_cache(l, a.kv, a.rows, a.num_kv_heads, dk, dv, es);
  if (a.k_base != nullptr) {
    add(l, a.k_base, (size_t)a.num_kv_heads * a.kv.cap * dk * es, "K base");
    add(l, a.v_base, (size_t)a.num_kv_heads * a.kv.cap * dv * es, "V base");
  }
  return submit(stream, "decode_kernel", l);
}

hipError_t launch_reduce(const DecodeArgs& a, int dv, hipStream_t stream) {
  Launch* l = new Launch();
  const size_t items = a.total_items / std::max<uint32_t>(a.slices, 1);
  add(l, a.part_acc, items * kHeadSlots * dv * 4, "split partials");
  add(l, a.part_ml, items * kHeadSlots * 2 * 4, "split maxima");
  add(l, a.out, (size_t)a.rows.count * a.num_heads * dv * 4, "out");
  add(l, a.err, 4, "error word");
  return submit(stream, "reduce_kernel", l);
}

hipError_t launch_prefill(const PrefillArgs& a, int dk, int dv, hipStream_t stream) {
  if (!prefill_supported(dk, dv)) return hipErrorInvalidValue;
  Launch* l = new Launch();
  add(l, a.q, (size_t)a.n * a.num_heads * dk * 4, "q");
  add(l, a.out, (size_t)a.n * a.num_heads * dv * 4, "out");
  add(l, a.err, 4, "error word");
  RowList one{};
  one.count = 1;
  one.contiguous = 1;
  one.seq0 = a.seq;
  add_cache(l, a.kv, one, a.num_kv_heads, dk, dv, 2);
  if (a.split_blocks > 0) {
    const size_t S = (size_t)prefill_stripes(dk);
    const size_t pairs = (size_t)a.split_blocks * a.head_groups * a.num_kv_heads;
    add(l, a.part, pairs * 2 * (S * ((dk / 8) * 64 + 32) + S * kPrefillKvGroups) * 16, "split partials");
    add(l, a.tickets, pairs * 4, "split tickets");
  }
  return submit(stream, "prefill_kernel", l);
}

hipError_t launch_prefill_slice(const PrefillArgs& a, bool f16, int dk, int dv, hipStream_t stream) {
  if (!prefill_slice_supported(f16, dk, dv)) return hipErrorInvalidValue;
  Launch* l = new Launch();
  add(l, a.q, (size_t)a.n * a.num_heads * dk * 4, "q");
  add(l, a.out, (size_t)a.n * a.num_heads * dv * 4, "out");
  add(l, a.err, 4, "error word");
  RowList one{};
  one.count = 1;
  one.contiguous = 1;
  one.seq0 = a.seq;
  add_cache(l, a.kv, one, a.num_kv_heads, dk, dv, f16 ? 2 : 4);
  if (a.split_blocks > 0) {
    const size_t splits = (size_t)a.split_blocks * a.head_groups * a.num_kv_heads;
    const size_t half = f16 ? 4 * kPairPartWords * 64 * 16 : (size_t)slice_waves(dk) * slice_state_words(dk) * 64 * 16;
    add(l, a.part, splits * 2 * half, "split states");
    add(l, a.tickets, splits * 4, "pair split tickets");
  }
  return submit(stream, "prefill_slice_kernel", l);
}

namespace {
void add_matrices(Launch* l, const QMatArgs& a, uint32_t fmt) {
  add(l, a.x, (size_t)a.batch * a.cols * 4, "activations");
  for (uint32_t i = 0; i < a.count; ++i) {
    const QMatrix& m = a.m[i];
    add(l, m.w, (size_t)m.rows * a.blocks * qmat_block_bytes(fmt), "weights");
    add(l, m.out, (size_t)a.batch * m.rows * 4, "output");
    if (a.addend_mode == 1) add(l, m.addend, (size_t)m.rows * 4, "bias");
    if (a.addend_mode == 2) add(l, m.addend, (size_t)a.batch * m.rows * 4, "residual");
  }
}
}  // namespace

hipError_t launch_qmatvec(const QMatArgs& a, uint32_t fmt, uint32_t, hipStream_t stream) {
  Launch* l = new Launch();
  add_matrices(l, a, fmt);
  return submit(stream, "qmatvec_kernel", l);
}

hipError_t launch_q8_0_quant(const float* x, uint32_t batch, uint32_t cols, int8_t* q,
                             float* scales, hipStream_t stream) {
  Launch* l = new Launch();
  add(l, x, (size_t)batch * cols * 4, "activations");
  add(l, q, (size_t)batch * cols, "quantized activations");
  add(l, scales, (size_t)batch * (cols / 32) * 4, "activation scales");
  return submit(stream, "q8_0_quant_kernel", l);
}

hipError_t launch_qgemm(const QMatArgs& a, uint32_t fmt, uint32_t, const int8_t* aq, const float* as,
                        hipStream_t stream) {
  Launch* l = new Launch();
  add_matrices(l, a, fmt);
  add(l, aq, (size_t)a.batch * a.cols, "quantized activations");
  add(l, as, (size_t)a.batch * a.blocks * 4, "activation scales");
  return submit(stream, "qgemm_kernel", l);
}

hipError_t launch_q8_k_quant(const float* x, uint32_t batch, uint32_t cols, int8_t* q,
                             float* scales, int* sums, hipStream_t stream) {
  Launch* l = new Launch();
  add(l, x, (size_t)batch * cols * 4, "activations");
  add(l, q, (size_t)batch * cols, "quantized activations");
  add(l, scales, (size_t)batch * (cols / 256) * 4, "activation scales");
  add(l, sums, (size_t)batch * (cols / 16) * 4, "activation sums");
  return submit(stream, "q8_k_quant_kernel", l);
}

hipError_t launch_qkgemm(const QMatArgs& a, uint32_t fmt, uint32_t, const int8_t* aq, const float* as,
                         const int* asum, hipStream_t stream) {
  Launch* l = new Launch();
  add_matrices(l, a, fmt);
  add(l, aq, (size_t)a.batch * a.cols, "quantized activations");
  add(l, as, (size_t)a.batch * a.blocks * 4, "activation scales");
  if (fmt != 3) add(l, asum, (size_t)a.batch * (a.cols / 16) * 4, "activation sums");
  return submit(stream, "qkgemm_kernel", l);
}

}  // namespace jma
