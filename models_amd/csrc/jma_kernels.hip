// gfx950 (MI355X) kernels for backend-java's grouped-query attention + KV-cache path.
//
//   kernel 1  rope_append_kernel   RoPE on q and k, K/V store into the HBM-resident cache
//   kernel 2  decode_kernel        split-K flash-decoding on MFMA, GQA heads share K/V loads
//   kernel 3  prefill_kernel       causal / sliding-window prefill, f16 MFMA, LDS K/V tiles
//   kernel 4  reduce_kernel        cross-split log-sum-exp reduction
//
// Reference semantics (paths under backend-java/src/main/java/com/integrallis/models/backend/
// purejava/): RoPE pairs and rotation follow TensorOps.rope/ropeNeox (ops/TensorOps.java:
// 1336-1390, 1474-1486); the store follows KvCache.store (cache/KvCache.java:58-73) with f16
// storage equal to its half-precision rounding (:94-100); attention follows
// LlamaForwardPass.groupedQueryAttention (llama/LlamaForwardPass.java:1543-1670): query head h
// reads kv head h / group, scores dot * scale over positions [first, position], softmax, weighted
// V sum.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "jma_kernels.h"

namespace jma {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// Index of slot r (0..31) inside a 32-slot f16 V block. A 16x16x32 MFMA lane (g = lane/16)
// supplies k-slots 8g..8g+7; the score tile gives that lane rows {4g..4g+3, 16+4g..16+4g+3},
// so storing those rows at 8g..8g+7 makes one 16-byte load a ready PV operand.
__device__ __forceinline__ uint32_t perm32(uint32_t r) {
  return 8u * ((r & 15u) >> 2) + 4u * (r >> 4) + (r & 3u);
}

__device__ __forceinline__ uint32_t slot_of(const KvView& kv, uint32_t position) {
  return kv.ring ? position % kv.cap : position;
}

__device__ __forceinline__ uint32_t row_sequence(const RowList& r, uint32_t i) {
  return r.contiguous ? r.seq0 : r.seq[i];
}

__device__ __forceinline__ uint32_t row_position(const RowList& r, uint32_t i) {
  return r.contiguous ? r.start + i : r.pos[i];
}

__device__ __forceinline__ uint32_t first_visible(uint32_t position, uint32_t window) {
  // LlamaConfig.attentionStartPosition, causal branch (llama/LlamaConfig.java:184-195).
  return (window == 0 || position + 1 <= window) ? 0u : position + 1 - window;
}

// ================================================================ kernel 1: RoPE + append

// One RoPE pair rotated exactly as TensorOps.rotatePair / rotateSplitPair compute it
// (ops/TensorOps.java:1474-1486): x0*c - x1*s and x0*s + x1*c, every product and sum rounded on its
// own (no fused multiply-add), so the cached K is bit-identical to the reference's.
__device__ __forceinline__ void rotate_pair(float& x0, float& x1, float c, float s) {
#pragma clang fp contract(off)
  const float a = x0 * c - x1 * s;
  const float b = x0 * s + x1 * c;
  x0 = a;
  x1 = b;
}

// One thread per element pair of a row: a RoPE pair of q or k (or a pass-through pair beyond the
// rotary dims), or two V elements. Every load a thread needs is independent of the others, so a
// row costs one memory round trip.
template <typename KV>
__global__ __launch_bounds__(256) void rope_append_kernel(const AppendArgs a) {
  constexpr bool kF16 = std::is_same<KV, _Float16>::value;
  constexpr uint32_t kBlk = kF16 ? 32u : 16u;
  const uint32_t row = blockIdx.x / a.blocks_per_row;
  const uint32_t w = (blockIdx.x % a.blocks_per_row) * blockDim.x + threadIdx.x;
  const uint32_t half_k = a.dk / 2, half_v = a.dv / 2;
  const uint32_t q_pairs = a.num_heads * half_k;
  const uint32_t k_pairs = a.num_kv_heads * half_k;
  const uint32_t v_pairs = a.num_kv_heads * half_v;
  if (w >= q_pairs + k_pairs + v_pairs) return;
  const uint32_t seq = row_sequence(a.rows, row);
  const uint32_t pos = row_position(a.rows, row);
  const uint32_t slot = slot_of(a.kv, pos);

  if (w < q_pairs + k_pairs) {
    const bool is_q = w < q_pairs;
    const uint32_t wi = is_q ? w : w - q_pairs;
    const uint32_t h = wi / half_k, j = wi % half_k;
    const float* x = is_q ? a.q + ((uint64_t)row * a.num_heads + h) * a.dk
                          : a.k + ((uint64_t)row * a.num_kv_heads + h) * a.dk;
    const bool rotate = a.cos_t != nullptr && j < a.pairs;
    const uint32_t e0 = rotate && a.neox ? j : 2 * j;
    const uint32_t e1 = rotate && a.neox ? j + a.pairs : 2 * j + 1;
    float y0 = x[e0], y1 = x[e1];
    if (rotate) {
      const float c = a.cos_t[(uint64_t)pos * a.pairs + j];
      const float s = a.sin_t[(uint64_t)pos * a.pairs + j];
      rotate_pair(y0, y1, c, s);
    }
    if (is_q) {
      if (a.q_out) {
        float* o = a.q_out + ((uint64_t)row * a.num_heads + h) * a.dk;
        o[e0] = y0;
        o[e1] = y1;
      }
    } else {
      KV* kr = (KV*)a.kv.k + seq * a.kv.seq_stride_k + a.kv.layer_off_k +
               ((uint64_t)h * a.kv.cap + slot) * a.dk;
      kr[e0] = (KV)y0;
      kr[e1] = (KV)y1;
    }
    return;
  }
  const uint32_t wi = w - q_pairs - k_pairs;
  const uint32_t h = wi / half_v, d = 2 * (wi % half_v);
  const float* x = a.v + ((uint64_t)row * a.num_kv_heads + h) * a.dv + d;
  const float v0 = x[0], v1 = x[1];
  const uint32_t blk = slot / kBlk, r = slot % kBlk;
  const uint32_t s = kF16 ? perm32(r) : r;
  KV* vb = (KV*)a.kv.v + seq * a.kv.seq_stride_v + a.kv.layer_off_v +
           (uint64_t)h * a.kv.cap * a.dv + ((uint64_t)blk * a.dv + d) * kBlk + s;
  vb[0] = (KV)v0;
  vb[kBlk] = (KV)v1;
}

hipError_t launch_append(const AppendArgs& a, bool f16, hipStream_t stream) {
  if (a.rows.count == 0) return hipSuccess;
  const dim3 grid(a.rows.count * a.blocks_per_row), block(256);
  if (f16) {
    hipLaunchKernelGGL(rope_append_kernel<_Float16>, grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL(rope_append_kernel<float>, grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

// ================================================================ kernel 2: split-K decode

__device__ __forceinline__ float wave_max_groups(float x) {
  // max over the four 16-lane groups that hold the same query head
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float wave_sum_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// Fragments of one tile (kBlk positions) of K and V for one lane, in matrix-core operand order.
template <typename KV, int DK, int DV>
struct Tile;

template <int DK, int DV>
struct Tile<_Float16, DK, DV> {
  static constexpr uint32_t kBlk = 32;
  half8_t k[2][DK / 32];
  half8_t v[DV / 16];
  __device__ __forceinline__ void load(const _Float16* kb, const _Float16* vb, uint32_t slot0,
                                       int c16, int g) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int c = 0; c < DK / 32; ++c)
        k[b][c] = *(const half8_t*)(kb + (uint64_t)(slot0 + 16 * b + c16) * DK + 32 * c + 8 * g);
    const _Float16* vblk = vb + (uint64_t)(slot0 / kBlk) * DV * kBlk;
#pragma unroll
    for (int n = 0; n < DV / 16; ++n) v[n] = *(const half8_t*)(vblk + (16 * n + c16) * kBlk + 8 * g);
  }
};

template <int DK, int DV>
struct Tile<float, DK, DV> {
  static constexpr uint32_t kBlk = 16;
  float4_t k[DK / 16];
  float4_t v[DV / 16];
  __device__ __forceinline__ void load(const float* kb, const float* vb, uint32_t slot0, int c16,
                                       int g) {
#pragma unroll
    for (int c = 0; c < DK / 16; ++c)
      k[c] = *(const float4_t*)(kb + (uint64_t)(slot0 + c16) * DK + 16 * c + 4 * g);
    const float* vblk = vb + (uint64_t)(slot0 / kBlk) * DV * kBlk;
#pragma unroll
    for (int n = 0; n < DV / 16; ++n) v[n] = *(const float4_t*)(vblk + (16 * n + c16) * kBlk + 4 * g);
  }
};

__device__ __forceinline__ uint64_t pack2(float lo, float hi) {
  return (uint64_t)__float_as_uint(lo) | ((uint64_t)__float_as_uint(hi) << 32);
}

// N consecutive elements e0 .. e0+N-1 of one head, rotated as TensorOps.rope / ropeNeox do. x is
// the head's first element; e0 is a multiple of N and N divides the rotary pair count, so a chunk
// lies wholly in the first half, the second half or the pass-through tail of the head.
template <int N>
__device__ __forceinline__ void rope_chunk(const float* __restrict__ x, uint32_t e0,
                                           const float* __restrict__ cs,
                                           const float* __restrict__ sn, uint32_t pairs,
                                           uint32_t neox, float (&out)[N]) {
  float v[N];
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const float4_t t = *(const float4_t*)(x + e0 + i);
    v[i] = t[0], v[i + 1] = t[1], v[i + 2] = t[2], v[i + 3] = t[3];
  }
  if (cs == nullptr || e0 >= 2 * pairs) {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = v[i];
    return;
  }
  if (!neox) {  // interleaved pairs (2j, 2j+1) sit inside the chunk
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      float a0 = v[i], a1 = v[i + 1];
      rotate_pair(a0, a1, cs[(e0 + i) / 2], sn[(e0 + i) / 2]);
      out[i] = a0, out[i + 1] = a1;
    }
    return;
  }
  const bool lower = e0 < pairs;  // split-half pairs (j, j + pairs)
  const uint32_t j0 = lower ? e0 : e0 - pairs;
  float w[N];
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const float4_t t = *(const float4_t*)(x + (lower ? e0 + pairs : j0) + i);
    w[i] = t[0], w[i + 1] = t[1], w[i + 2] = t[2], w[i + 3] = t[3];
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float a0 = lower ? v[i] : w[i], a1 = lower ? w[i] : v[i];
    rotate_pair(a0, a1, cs[j0 + i], sn[j0 + i]);
    out[i] = lower ? a0 : a1;
  }
}

// One workgroup = one work item (row, kv head, head group of <= 16 query heads, split); its
// kDecodeWaves waves stride over the split's tiles, keeping the next tile's loads in flight while
// the current one is computed, and combine in LDS. Scores are computed as S = K * Q^T on 16-row
// blocks so lane (g, c) holds rows 4g+e of query head c: every lane works on a single head, the
// online-softmax rescale is one factor per lane, and the score registers are already the B
// operand of the PV product O^T = V^T * P.
//
// f16 KV: v_mfma_f32_16x16x32_f16. q and p are split into hi + lo halves (x = hi + lo exactly
// to ~2^-22), so both products run at near-f32 accuracy against the f32 reference.
// f32 KV: v_mfma_f32_16x16x4_f32 with f32 operands throughout.
//
// Decode fuses the other per-token work into this one launch:
//  - RoPE on q (rope_q): each lane rotates the q elements it loads;
//  - the append (k_new/v_new): the workgroup of a row's last split rotates and stores that kv
//    head's new K/V row before any wave loads a tile, so the row's own tile reads it back;
//  - the cross-split reduction (counters): partials are written with device-coherent stores, the
//    last workgroup of a (row, kv head, head group) to arrive reduces them with device-coherent
//    loads and resets the counter. No cache-wide fence is needed: the partials bypass the
//    per-XCD L2s.
template <typename KV, int DK, int DV>
__global__ __launch_bounds__(256) void decode_kernel(const DecodeArgs a) {
  constexpr bool kF16 = std::is_same<KV, _Float16>::value;
  using TileT = Tile<KV, DK, DV>;
  constexpr uint32_t kBlk = TileT::kBlk;
  constexpr int kNs = kF16 ? 8 : 4;   // scores per lane per tile
  constexpr int kNv = DV / 16;        // output fragments per lane
  constexpr int kC = kF16 ? DK / 32 : DK / 16;
  constexpr int kQ = kF16 ? 8 : 4;    // q elements per lane per k-chunk
  __shared__ __attribute__((aligned(16))) float s_acc[kDecodeWaves - 1][16][DV];
  __shared__ __attribute__((aligned(16))) float s_ml[kDecodeWaves - 1][16][2];
  __shared__ uint32_t s_last;

  // Fetch the scalar arguments the prologue needs in one batch: left to itself the compiler
  // loads each right before its use, behind its own wait.
  uint32_t num_heads = a.num_heads, group = a.group, hgroups = a.hgroups, ns_uniform = a.ns_uniform;
  uint32_t rows_contig = a.rows.contiguous, rows_seq0 = a.rows.seq0, rows_start = a.rows.start;
  uint32_t window = a.window, tps = a.tiles_per_split, cap = a.kv.cap, ring = a.kv.ring;
  uint64_t seq_stride_k = a.kv.seq_stride_k, seq_stride_v = a.kv.seq_stride_v;
  uint64_t layer_off_k = a.kv.layer_off_k, layer_off_v = a.kv.layer_off_v;
  asm volatile("" : "+s"(num_heads), "+s"(group), "+s"(hgroups), "+s"(ns_uniform), "+s"(rows_contig),
               "+s"(rows_seq0), "+s"(rows_start), "+s"(window), "+s"(tps), "+s"(cap), "+s"(ring),
               "+s"(seq_stride_k), "+s"(seq_stride_v), "+s"(layer_off_k), "+s"(layer_off_v));

  const uint32_t item = blockIdx.x;
  const uint32_t hkv = num_heads / group;
  uint32_t row, ns, local;
  if (ns_uniform) {
    ns = ns_uniform;
    row = item / (hkv * hgroups * ns);
    local = item - row * hkv * hgroups * ns;
  } else {
    // Count the rows that start at or before this item: independent table loads, one round trip.
    row = 0;
#pragma unroll
    for (uint32_t r = 1; r < kMaxRows; ++r) row += (r < a.rows.count && a.item_start[r] <= item) ? 1u : 0u;
    ns = a.nsplit[row];
    local = item - a.item_start[row];
  }
  const uint32_t split = local % ns;
  const uint32_t rest = local / ns;
  const uint32_t hg = rest % hgroups;
  const uint32_t kvh = rest / hgroups;
  const uint32_t seq = rows_contig ? rows_seq0 : a.rows.seq[row];
  const uint32_t pos = rows_contig ? rows_start + row : a.rows.pos[row];
  const uint32_t first = first_visible(pos, window);
  const uint32_t t_begin = first / kBlk, t_end = pos / kBlk + 1;
  const uint32_t s_t0 = t_begin + split * tps;
  const uint32_t s_t1 = min(s_t0 + tps, t_end);

  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t hl = hg * 16 + c16;
  const bool head_ok = hl < group;
  const uint32_t head = kvh * group + hl;
  const float* qrow = a.q + ((uint64_t)row * num_heads + (head_ok ? head : 0)) * DK;
  const float* cs = a.cos_t ? a.cos_t + (uint64_t)pos * a.pairs : nullptr;
  const float* sn = a.cos_t ? a.sin_t + (uint64_t)pos * a.pairs : nullptr;

  KV* kb = (KV*)a.kv.k + seq * seq_stride_k + layer_off_k + (uint64_t)kvh * cap * DK;
  KV* vb = (KV*)a.kv.v + seq * seq_stride_v + layer_off_v + (uint64_t)kvh * cap * DV;

  // Fused append: the last split of the row holds the new position's tile.
  if (a.k_new != nullptr && split == ns - 1) {
    if (hg == 0) {
      const uint32_t slot = slot_of(a.kv, pos);
      const float* kx = a.k_new + ((uint64_t)row * hkv + kvh) * DK;
      const float* vx = a.v_new + ((uint64_t)row * hkv + kvh) * DV;
      const uint32_t tid = threadIdx.x;
      if (tid < DK / 4) {
        float r[4];
        rope_chunk<4>(kx, 4 * tid, cs, sn, a.pairs, a.neox, r);
#pragma unroll
        for (int i = 0; i < 4; ++i) kb[(uint64_t)slot * DK + 4 * tid + i] = (KV)r[i];
      } else if (tid < DK / 4 + DV / 4) {
        const uint32_t d = 4 * (tid - DK / 4);
        const float4_t x = *(const float4_t*)(vx + d);
        const uint32_t s = kF16 ? perm32(slot % kBlk) : slot % kBlk;
        KV* vp = vb + (uint64_t)(slot / kBlk) * DV * kBlk + (uint64_t)d * kBlk + s;
#pragma unroll
        for (int i = 0; i < 4; ++i) vp[i * kBlk] = (KV)x[i];
      }
      // The stores must land before any wave of this workgroup loads the tile holding them.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
  }

  // Start the first tile's loads before preparing Q.
  uint32_t t = s_t0 + wave;
  TileT cur;
  if (t < s_t1) cur.load(kb, vb, ring ? (t * kBlk) % cap : t * kBlk, c16, g);

  // Q operand (B of S = K Q^T), rotated here when the caller passed raw q.
  const float qs = head_ok ? a.qscale : 0.0f;
  half8_t qhi[kF16 ? kC : 1], qlo[kF16 ? kC : 1];
  float4_t qf[kF16 ? 1 : kC];
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    float x[kQ];
    rope_chunk<kQ>(qrow, (kF16 ? 32 : 16) * c + kQ * g, a.rope_q ? cs : nullptr, sn, a.pairs,
                   a.neox, x);
#pragma unroll
    for (int e = 0; e < kQ; ++e) {
      const float y = x[e] * qs;
      if constexpr (kF16) {
        const _Float16 h = (_Float16)y;
        qhi[c][e] = h;
        qlo[c][e] = (_Float16)(y - (float)h);
      } else {
        qf[c][e] = y;
      }
    }
  }

  float m = -INFINITY, l = 0.0f;
  float4_t acc[kNv];
#pragma unroll
  for (int n = 0; n < kNv; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};
  bool bad = false;

  while (t < s_t1) {
    const uint32_t tn = t + kDecodeWaves;
    TileT next;
    if (tn < s_t1) next.load(kb, vb, ring ? (tn * kBlk) % cap : tn * kBlk, c16, g);
    const uint32_t p0 = t * kBlk;

    float s[kNs];
    if constexpr (kF16) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < kC; ++c) {
          sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[b][c], qhi[c], sc, 0, 0, 0);
          sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[b][c], qlo[c], sc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * b + e] = sc[e];
      }
    } else {
      float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kC; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sc = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[c][e], qf[c][e], sc, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] = sc[e];
    }
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < kNs; ++i) {
      const uint32_t p = kF16 ? p0 + 16 * (i >> 2) + 4 * g + (i & 3) : p0 + 4 * g + i;
      const bool valid = p >= first && p <= pos;
      bad |= valid && (s[i] != s[i] || s[i] == INFINITY);
      s[i] = valid ? s[i] : -INFINITY;
      mt = fmaxf(mt, s[i]);
    }
    mt = wave_max_groups(mt);
    const float mn = fmaxf(m, mt);
    const float mu = mn == -INFINITY ? 0.0f : mn;
    const float alpha = exp2f(m - mu);
    m = mn;
    float p[kNs];
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < kNs; ++i) {
      p[i] = exp2f(s[i] - mu);
      psum += p[i];
    }
    l = l * alpha + psum;
    if constexpr (kF16) {
      half8_t phi, plo;
#pragma unroll
      for (int i = 0; i < kNs; ++i) {
        const _Float16 h = (_Float16)p[i];
        phi[i] = h;
        plo[i] = (_Float16)(p[i] - (float)h);
      }
#pragma unroll
      for (int n = 0; n < kNv; ++n) {
        acc[n] *= alpha;
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.v[n], phi, acc[n], 0, 0, 0);
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.v[n], plo, acc[n], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int n = 0; n < kNv; ++n) {
        acc[n] *= alpha;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.v[n][e], p[e], acc[n], 0, 0, 0);
      }
    }
    cur = next;
    t = tn;
  }

  if (__ballot(bad) != 0 && lane == 0) atomicOr(a.err, 1);
  l = wave_sum_groups(l);

  // Combine the waves of this workgroup in LDS (wave 0 keeps its state in registers).
  if (wave != 0) {
    if (g == 0) {
      s_ml[wave - 1][c16][0] = m;
      s_ml[wave - 1][c16][1] = l;
    }
#pragma unroll
    for (int n = 0; n < kNv; ++n)
      *(float4_t*)&s_acc[wave - 1][c16][16 * n + 4 * g] = acc[n];
  }
  __syncthreads();

  const bool fused = ns > 1 && a.counters != nullptr;
  float* o = a.out + ((uint64_t)row * a.num_heads + head) * DV;
  const uint64_t gid = ((uint64_t)row * hkv + kvh) * a.hgroups + hg;
  if (wave == 0) {
    float mx = m;
#pragma unroll
    for (int w = 0; w < kDecodeWaves - 1; ++w) mx = fmaxf(mx, s_ml[w][c16][0]);
    const float mu = mx == -INFINITY ? 0.0f : mx;
    const float f0 = exp2f(m - mu);
    l *= f0;
#pragma unroll
    for (int n = 0; n < kNv; ++n) acc[n] *= f0;
#pragma unroll
    for (int w = 0; w < kDecodeWaves - 1; ++w) {
      const float fw = exp2f(s_ml[w][c16][0] - mu);
      l += s_ml[w][c16][1] * fw;
#pragma unroll
      for (int n = 0; n < kNv; ++n) acc[n] += *(const float4_t*)&s_acc[w][c16][16 * n + 4 * g] * fw;
    }
    if (ns == 1) {
      if (head_ok) {
        if (l == 0.0f && g == 0) atomicOr(a.err, 1);
        const float inv = 1.0f / l;
#pragma unroll
        for (int n = 0; n < kNv; ++n) *(float4_t*)(o + 16 * n + 4 * g) = acc[n] * inv;
      }
      return;
    }
    float* pa = a.part_acc + ((uint64_t)item * 16 + c16) * DV;
    float* pm = a.part_ml + ((uint64_t)item * 16 + c16) * 2;
    if (!fused) {  // reduce_kernel combines the splits after this launch
#pragma unroll
      for (int n = 0; n < kNv; ++n) *(float4_t*)(pa + 16 * n + 4 * g) = acc[n];
      if (g == 0) {
        pm[0] = mx;
        pm[1] = l;
      }
      return;
    }
    // Kernel 4 fused. Device-coherent (write-through) stores, then wait for them before counting
    // this arrival; the last workgroup of the group to arrive reduces.
#pragma unroll
    for (int n = 0; n < kNv; ++n)
#pragma unroll
      for (int e = 0; e < 4; e += 2)
        __hip_atomic_store((uint64_t*)(pa + 16 * n + 4 * g + e), pack2(acc[n][e], acc[n][e + 1]),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (g == 0) __hip_atomic_store((uint64_t*)pm, pack2(mx, l), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint32_t arrived = 0;
    if (lane == 0)
      arrived = __hip_atomic_fetch_add(&a.counters[gid], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lane == 0) s_last = arrived == ns - 1 ? 1u : 0u;
  }
  if (!fused) return;
  __syncthreads();
  if (s_last == 0) return;
  if (threadIdx.x == 0)
    __hip_atomic_store(&a.counters[gid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // Last arrival. Wave w reduces output fragments w, w + 4, ... over every split. Plain loads are
  // coherent here: the kernel-start acquire invalidated every L2, the writers stored through to
  // memory before counting, and each partial line is read by this workgroup only, so no L2 holds
  // a stale copy. Each batch of splits is loaded in one round trip (indices clamped, weight 0
  // past the last split).
  constexpr int kF = kNv >= kDecodeWaves ? kNv / kDecodeWaves : 1;  // fragments per wave
  constexpr int kS = kMaxSplits / kF < kMaxSplits ? kMaxSplits / kF : kMaxSplits;  // batch
  if (wave >= kNv) return;
  const uint64_t item0 = item - split;
  float2 ml[kMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp)
    ml[sp] = *(const float2*)(a.part_ml + ((item0 + min((uint32_t)sp, ns - 1)) * 16 + c16) * 2);
  float4_t x0[kS][kF];
#pragma unroll
  for (int sp = 0; sp < kS; ++sp) {
    const float* ps = a.part_acc + ((item0 + min((uint32_t)sp, ns - 1)) * 16 + c16) * DV;
#pragma unroll
    for (int f = 0; f < kF; ++f) x0[sp][f] = *(const float4_t*)(ps + 16 * (wave + kDecodeWaves * f) + 4 * g);
  }
  float gm = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) gm = (uint32_t)sp < ns ? fmaxf(gm, ml[sp].x) : gm;
  const float gmu = gm == -INFINITY ? 0.0f : gm;
  float gl = 0.0f;
  float wsp[kMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp) {
    wsp[sp] = (uint32_t)sp < ns ? exp2f(ml[sp].x - gmu) : 0.0f;
    gl += ml[sp].y * wsp[sp];
  }
  float4_t gacc[kF];
#pragma unroll
  for (int f = 0; f < kF; ++f) gacc[f] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < kS; ++sp)
#pragma unroll
    for (int f = 0; f < kF; ++f) gacc[f] += x0[sp][f] * wsp[sp];
#pragma unroll
  for (int b = 1; b < kMaxSplits / kS; ++b) {
    if ((uint32_t)(b * kS) < ns) {
      float4_t x[kS][kF];
#pragma unroll
      for (int u = 0; u < kS; ++u) {
        const float* ps = a.part_acc + ((item0 + min((uint32_t)(b * kS + u), ns - 1)) * 16 + c16) * DV;
#pragma unroll
        for (int f = 0; f < kF; ++f) x[u][f] = *(const float4_t*)(ps + 16 * (wave + kDecodeWaves * f) + 4 * g);
      }
#pragma unroll
      for (int u = 0; u < kS; ++u)
#pragma unroll
        for (int f = 0; f < kF; ++f) gacc[f] += x[u][f] * wsp[b * kS + u];
    }
  }
  if (!head_ok) return;
  if (gl == 0.0f && g == 0 && wave == 0) atomicOr(a.err, 1);
  const float inv = 1.0f / gl;
#pragma unroll
  for (int f = 0; f < kF; ++f) *(float4_t*)(o + 16 * (wave + kDecodeWaves * f) + 4 * g) = gacc[f] * inv;
}

// ================================================================ kernel 4: cross-split reduce

// One wave per (row, query head): out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M) over the
// row's splits (at most kMaxSplits). Every split's partial is loaded before any is used (indices
// past the last split are clamped to it and weighted 0), so the reduction costs one round trip.
template <int DV>
__global__ __launch_bounds__(64) void reduce_kernel(const DecodeArgs a) {
  constexpr int kJ = (DV + 63) / 64;  // output elements per lane
  const uint32_t row = blockIdx.x / a.num_heads;
  const uint32_t head = blockIdx.x % a.num_heads;
  const uint32_t hkv = a.num_heads / a.group;
  const uint32_t ns = a.ns_uniform ? a.ns_uniform : a.nsplit[row];
  if (ns == 1) return;
  const uint32_t row_item = a.ns_uniform ? row * hkv * a.hgroups * ns : a.item_start[row];
  const uint32_t kvh = head / a.group;
  const uint32_t hl = head % a.group;
  const uint32_t hg = hl / 16, c16 = hl % 16;
  const uint64_t base = row_item + ((uint64_t)kvh * a.hgroups + hg) * ns;
  const int lane = threadIdx.x;

  float m[kMaxSplits], lw[kMaxSplits], x[kMaxSplits][kJ];
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) {
    const uint64_t it = base + min((uint32_t)s, ns - 1);
    const float2 ml = *(const float2*)(a.part_ml + (it * 16 + c16) * 2);
    m[s] = ml.x;
    lw[s] = ml.y;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int d = min(lane + 64 * j, DV - 1);
      x[s][j] = a.part_acc[(it * 16 + c16) * DV + d];
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) mx = (uint32_t)s < ns ? fmaxf(mx, m[s]) : mx;
  const float mu = mx == -INFINITY ? 0.0f : mx;
  float l = 0.0f, sum[kJ];
#pragma unroll
  for (int j = 0; j < kJ; ++j) sum[j] = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) {
    const float w = (uint32_t)s < ns ? exp2f(m[s] - mu) : 0.0f;
    l += lw[s] * w;
#pragma unroll
    for (int j = 0; j < kJ; ++j) sum[j] += x[s][j] * w;
  }
  if (l == 0.0f && lane == 0) atomicOr(a.err, 1);
  const float inv = 1.0f / l;
  float* o = a.out + ((uint64_t)row * a.num_heads + head) * DV;
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const int d = lane + 64 * j;
    if (d < DV) o[d] = sum[j] * inv;
  }
}

hipError_t launch_reduce(const DecodeArgs& a, int dv, hipStream_t stream) {
  const dim3 grid(a.rows.count * a.num_heads), block(64);
  switch (dv) {
    case 16: hipLaunchKernelGGL(reduce_kernel<16>, grid, block, 0, stream, a); break;
    case 32: hipLaunchKernelGGL(reduce_kernel<32>, grid, block, 0, stream, a); break;
    case 64: hipLaunchKernelGGL(reduce_kernel<64>, grid, block, 0, stream, a); break;
    case 128: hipLaunchKernelGGL(reduce_kernel<128>, grid, block, 0, stream, a); break;
    case 256: hipLaunchKernelGGL(reduce_kernel<256>, grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

bool decode_supported(bool f16, int dk, int dv) {
  if (dk != dv) return false;
  if (f16) return dk == 32 || dk == 64 || dk == 128 || dk == 256;
  return dk == 16 || dk == 32 || dk == 64 || dk == 128 || dk == 256;
}

template <typename KV>
static hipError_t launch_decode_t(const DecodeArgs& a, int d, hipStream_t stream) {
  const dim3 grid(a.total_items), block(64 * kDecodeWaves);
  switch (d) {
    case 16:
      if constexpr (!std::is_same<KV, _Float16>::value) {
        hipLaunchKernelGGL((decode_kernel<KV, 16, 16>), grid, block, 0, stream, a);
        break;
      }
      return hipErrorInvalidValue;
    case 32: hipLaunchKernelGGL((decode_kernel<KV, 32, 32>), grid, block, 0, stream, a); break;
    case 64: hipLaunchKernelGGL((decode_kernel<KV, 64, 64>), grid, block, 0, stream, a); break;
    case 128: hipLaunchKernelGGL((decode_kernel<KV, 128, 128>), grid, block, 0, stream, a); break;
    case 256: hipLaunchKernelGGL((decode_kernel<KV, 256, 256>), grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, bool f16, int dk, int dv, hipStream_t stream) {
  if (!decode_supported(f16, dk, dv)) return hipErrorInvalidValue;
  if (a.total_items == 0) return hipSuccess;
  return f16 ? launch_decode_t<_Float16>(a, dk, stream) : launch_decode_t<float>(a, dk, stream);
}

// ================================================================ kernel 3: prefill (f16 MFMA)

// Workgroup = (block of rows_per_block query rows, kv head, group of heads_per_block query
// heads); wave w owns 16 query rows of one head. Every wave iterates the same 32-row K/V tiles,
// staged once in LDS per workgroup, so the GQA heads and query rows of the workgroup share each
// HBM read. S^T = K * Q^T per 16-row block puts query columns in lanes, as in decode_kernel.
template <int DK, int DV>
__global__ __launch_bounds__(1024) void prefill_kernel(const PrefillArgs a) {
  constexpr int kC = DK / 32;
  constexpr int kNv = DV / 16;
  constexpr int kKPad = DK + 8;   // halves per LDS K row (16-byte pad against bank conflicts)
  constexpr int kVPad = 32 + 8;   // halves per LDS V^T row
  __shared__ __attribute__((aligned(16))) _Float16 sk[32 * kKPad];
  __shared__ __attribute__((aligned(16))) _Float16 sv[DV * kVPad];

  const uint32_t qt = a.q_tiles - 1 - blockIdx.x;  // longest causal rows first
  const uint32_t kvh = blockIdx.y;
  const uint32_t hz0 = blockIdx.z * a.heads_per_block;
  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t blocks_per_head = a.rows_per_block / 16;
  const uint32_t hz = hz0 + wave / blocks_per_head;
  const uint32_t rb = wave % blocks_per_head;
  const bool wave_head_ok = hz < a.group;
  const uint32_t head = kvh * a.group + (wave_head_ok ? hz : 0);
  const uint32_t t_row = qt * a.rows_per_block + rb * 16 + c16;  // this lane's query row
  const bool row_ok = t_row < a.n;
  const uint32_t qpos = a.start + t_row;
  const uint32_t qfirst = first_visible(qpos, a.window);

  // Query rows of the whole workgroup bound the K/V tiles it visits.
  const uint32_t wg_row0 = qt * a.rows_per_block;
  const uint32_t wg_row1 = min(wg_row0 + a.rows_per_block, a.n) - 1;
  const uint32_t t0 = first_visible(a.start + wg_row0, a.window) / 32;
  const uint32_t t1 = (a.start + wg_row1) / 32 + 1;
  // This wave's rows bound the tiles it computes on.
  const uint32_t w_row0 = qt * a.rows_per_block + rb * 16;
  const uint32_t w_row1 = min(w_row0 + 15, a.n - 1);
  const uint32_t w_first = first_visible(a.start + w_row0, a.window);
  const uint32_t w_last = a.start + w_row1;
  const bool wave_rows_ok = w_row0 < a.n && wave_head_ok;

  // Q operand: this lane's query row, scaled by scale*log2(e) and rounded to f16 in registers.
  half8_t qf[kC];
  const float* qrow = a.q + ((uint64_t)(row_ok ? t_row : 0) * a.num_heads + head) * DK;
  float4_t qv[kC][2];
#pragma unroll
  for (int c = 0; c < kC; ++c) {  // qrow is clamped to a valid row: load unconditionally
    qv[c][0] = *(const float4_t*)(qrow + 32 * c + 8 * g);
    qv[c][1] = *(const float4_t*)(qrow + 32 * c + 8 * g + 4);
  }
  const float qs = (row_ok && wave_head_ok) ? a.qscale : 0.0f;
#pragma unroll
  for (int c = 0; c < kC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[c][e] = (_Float16)(qv[c][e >> 2][e & 3] * qs);

  const _Float16* kb = (const _Float16*)a.kv.k + a.seq * a.kv.seq_stride_k + a.kv.layer_off_k +
                       (uint64_t)kvh * a.kv.cap * DK;
  const _Float16* vb = (const _Float16*)a.kv.v + a.seq * a.kv.seq_stride_v + a.kv.layer_off_v +
                       (uint64_t)kvh * a.kv.cap * DV;

  float m = -INFINITY, l = 0.0f;
  float4_t acc[kNv];
#pragma unroll
  for (int n = 0; n < kNv; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};
  bool bad = false;

  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t p0 = t * 32;
    const uint32_t slot0 = a.kv.ring ? p0 % a.kv.cap : p0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < 32 * DK / 8; i += blockDim.x) {
      const uint32_t r = i / (DK / 8), cc = i % (DK / 8);
      *(half8_t*)&sk[r * kKPad + 8 * cc] = *(const half8_t*)(kb + (uint64_t)(slot0 + r) * DK + 8 * cc);
    }
    const _Float16* vblk = vb + (uint64_t)(slot0 / 32) * DV * 32;
    for (uint32_t i = threadIdx.x; i < DV * 4; i += blockDim.x) {
      const uint32_t d = i / 4, cc = i % 4;
      *(half8_t*)&sv[d * kVPad + 8 * cc] = *(const half8_t*)(vblk + d * 32 + 8 * cc);
    }
    __syncthreads();
    if (!wave_rows_ok || p0 > w_last || p0 + 31 < w_first) continue;

    float s[8];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kC; ++c) {
        const half8_t kf = *(const half8_t*)&sk[(16 * b + c16) * kKPad + 32 * c + 8 * g];
        sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[c], sc, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) s[4 * b + e] = sc[e];
    }
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t p = p0 + 16 * (i >> 2) + 4 * g + (i & 3);
      const bool valid = row_ok && p >= qfirst && p <= qpos;
      bad |= valid && (s[i] != s[i] || s[i] == INFINITY);
      s[i] = valid ? s[i] : -INFINITY;
      mt = fmaxf(mt, s[i]);
    }
    mt = wave_max_groups(mt);
    const float mn = fmaxf(m, mt);
    const float mu = mn == -INFINITY ? 0.0f : mn;
    const float alpha = exp2f(m - mu);
    m = mn;
    float psum = 0.0f;
    half8_t pf;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = exp2f(s[i] - mu);
      psum += p;
      pf[i] = (_Float16)p;
    }
    l = l * alpha + psum;
#pragma unroll
    for (int n = 0; n < kNv; ++n) {
      const half8_t vf = *(const half8_t*)&sv[(16 * n + c16) * kVPad + 8 * g];
      acc[n] *= alpha;
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, acc[n], 0, 0, 0);
    }
  }

  if (__ballot(bad) != 0 && lane == 0) atomicOr(a.err, 1);
  l = wave_sum_groups(l);
  if (!(row_ok && wave_head_ok)) return;
  if (l == 0.0f && g == 0) atomicOr(a.err, 1);
  const float inv = 1.0f / l;
  float* o = a.out + ((uint64_t)t_row * a.num_heads + head) * DV;
#pragma unroll
  for (int n = 0; n < kNv; ++n) *(float4_t*)(o + 16 * n + 4 * g) = acc[n] * inv;
}

bool prefill_supported(int dk, int dv) {
  return dk == dv && (dk == 32 || dk == 64 || dk == 128 || dk == 256);
}

hipError_t launch_prefill(const PrefillArgs& a, int dk, int dv, hipStream_t stream) {
  if (!prefill_supported(dk, dv)) return hipErrorInvalidValue;
  const uint32_t head_blocks = (a.group + a.heads_per_block - 1) / a.heads_per_block;
  const uint32_t num_kv_heads = a.num_heads / a.group;
  const dim3 grid(a.q_tiles, num_kv_heads, head_blocks);
  const dim3 block(64 * a.heads_per_block * (a.rows_per_block / 16));
  switch (dk) {
    case 32: hipLaunchKernelGGL((prefill_kernel<32, 32>), grid, block, 0, stream, a); break;
    case 64: hipLaunchKernelGGL((prefill_kernel<64, 64>), grid, block, 0, stream, a); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<128, 128>), grid, block, 0, stream, a); break;
    case 256: hipLaunchKernelGGL((prefill_kernel<256, 256>), grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace jma
