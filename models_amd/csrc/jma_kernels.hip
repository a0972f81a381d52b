// gfx950 (MI355X) kernels for backend-java's grouped-query attention + KV-cache path.
//
//   kernel 1  rope_append_kernel   RoPE on q and k, K/V store into the HBM-resident cache
//   kernel 2  decode_kernel        split-K flash-decoding on MFMA, GQA heads share K/V loads
//   kernel 3  prefill_kernel       causal / sliding-window prefill, f16 MFMA, LDS K/V tiles
//   kernel 3b prefill_slice_kernel the same for f32 caches, head-dim slices
//   kernel 3c prefill_pair_kernel  the same for f16 caches at head dim 512, stripe pairs
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

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "jma_kernels.h"

namespace jma {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Lambdas over shared state must inline, or the captured state (accumulators included) would be
// spilled to scratch memory.
#define JMA_INL __attribute__((always_inline))
#define JMA_GLOBAL __attribute__((address_space(1)))

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

// QK-norm of one head before RoPE (normalizeHead -> TensorOps.rmsNorm, llama/LlamaForwardPass.java:
// 1672-1676, ops/TensorOps.java:50-58): sumSq of the head in order, rms = (float)sqrt(sumSq / d +
// eps) in double, scale = 1 / rms, element = x * scale * w, each operation rounded on its own.
// Every thread of the head computes the same sum (the head row is in L1), so the result is the
// oracle's bit for bit; it replaces the pair's values y0 = x[e0], y1 = x[e1].
__device__ __forceinline__ float head_rms_scale(const float* x, uint32_t d, float eps) {
#pragma clang fp contract(off)
  float ss = 0.0f;
  for (uint32_t i = 0; i < d; ++i) ss = ss + x[i] * x[i];
  const float rms = (float)sqrt((double)(ss / (float)d + eps));
  return 1.0f / rms;
}

// head_rms_scale for a head dim known at compile time: the head's loads are issued in batches of
// eight 16-byte loads ahead of the in-order sum (the loop above waits for each load in turn).
template <uint32_t D>
__device__ __forceinline__ float head_rms_scale_d(const float* x, float eps) {
#pragma clang fp contract(off)
  constexpr uint32_t kB = D >= 32 ? 8u : D / 4;  // 16-byte loads per batch
  float ss = 0.0f;
#pragma unroll
  for (uint32_t b = 0; b < D / 4; b += kB) {
    float4_t v[kB];
#pragma unroll
    for (uint32_t i = 0; i < kB; ++i) v[i] = *(const float4_t*)(x + 4 * (b + i));
#pragma unroll
    for (uint32_t i = 0; i < kB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = ss + v[i][e] * v[i][e];
  }
  const float rms = (float)sqrt((double)(ss / (float)D + eps));
  return 1.0f / rms;
}

__device__ __forceinline__ void head_rms_norm(const float* x, uint32_t d, const float* w, float eps,
                                              uint32_t e0, uint32_t e1, float& y0, float& y1) {
#pragma clang fp contract(off)
  const float scale = head_rms_scale(x, d, eps);
  y0 = y0 * scale * w[e0];
  y1 = y1 * scale * w[e1];
}

// Unweighted RMS norm of one value head before it is stored (Gemma4Math.normalizeWithoutWeight,
// gemma4/Gemma4Math.java:38-55, applied at gemma4/Gemma4ForwardPass.java:990-996): sumSq of the
// head in order, inverse = (float)(1 / sqrt(sumSq / d + eps)) with the mean and eps added in float
// and the square root and reciprocal in double, element = x * inverse. Every thread of the head
// computes the same sum, so the stored values are the oracle's bit for bit.
__device__ __forceinline__ void value_rms_norm(const float* x, uint32_t d, float eps, float& y0,
                                               float& y1) {
#pragma clang fp contract(off)
  float ss = 0.0f;
  for (uint32_t i = 0; i < d; ++i) ss = ss + x[i] * x[i];
  const float inverse = (float)(1.0 / sqrt((double)(ss / (float)d + eps)));
  y0 = y0 * inverse;
  y1 = y1 * inverse;
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
    const float* nw = is_q ? a.q_norm_w : a.k_norm_w;
    if (nw != nullptr) head_rms_norm(x, a.dk, nw, a.norm_eps, e0, e1, y0, y1);
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
      KV* kr = (KV*)a.kv.k + seq * a.kv.seq_stride_k + a.kv.layer_off_k + (uint64_t)h * a.kv.cap * a.dk;
      kr[k_index(slot, e0, a.dk, kF16)] = (KV)y0;
      kr[k_index(slot, e1, a.dk, kF16)] = (KV)y1;
    }
    return;
  }
  const uint32_t wi = w - q_pairs - k_pairs;
  const uint32_t h = wi / half_v, d = 2 * (wi % half_v);
  const float* vh = a.v + ((uint64_t)row * a.num_kv_heads + h) * a.dv;
  float v0 = vh[d], v1 = vh[d + 1];
  if (a.v_norm) value_rms_norm(vh, a.dv, a.norm_eps, v0, v1);
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

// Cross-lane exchanges in vector ALU instructions rather than LDS permutes (an LDS round trip
// each). v_permlane16_swap with both operands x leaves, in its two results, the rows {0, 0, 2, 2}
// and {1, 1, 3, 3} of x (rows of 16 lanes); v_permlane32_swap leaves rows {0, 1, 0, 1} and
// {2, 3, 2, 3}. Combining the two results pairs every lane with its partner 16 (or 32) lanes
// away, and since a + b == b + a exactly, both partners hold the same bits afterwards.
__device__ __forceinline__ void swap16(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap32(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

__device__ __forceinline__ float wave_max_groups(float x) {
  // max over the four 16-lane groups that hold the same query head
  float a, b;
  swap16(x, a, b);
  x = fmaxf(a, b);
  swap32(x, a, b);
  return fmaxf(a, b);
}

__device__ __forceinline__ float wave_sum_groups(float x) {
  float a, b;
  swap16(x, a, b);
  x = a + b;
  swap32(x, a, b);
  return a + b;
}

// DPP lane exchanges inside groups of 8 consecutive lanes: partner lane i ^ 1, i ^ 2, and
// 7 - i within each half row (which, once the quads hold equal values, pairs quad 0 with quad 1
// as i ^ 4 would); row_mirror pairs the two halves of a row of 16 the same way.
template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppRowMirror = 0x140;  // row_mirror: lane 15 - i within each row of 16
constexpr int kDppRowRor4 = 0x124;    // row_ror:4 (lane i of a row of 16 reads lane (i + 4) % 16)
constexpr int kDppRowRor8 = 0x128;    // row_ror:8

// Fragments of one tile (kBlk positions) of K and V for one lane, in matrix-core operand order.
// K tiles are stored in 64-byte column panels (k_index), so each operand load below reads 1 KB of
// contiguous memory across the wave, like the V loads.
// V: the DVS value columns of one column slice of a DV-wide head (vb points at the slice's first
// column; the block stride is the whole head's). NT: the loads are non-temporal (streamed past the
// caches), for launches that read more K/V than the Infinity Cache could keep anyway.
template <bool NT, typename T>
__device__ __forceinline__ T ld16(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

template <typename KV, int DK, int DV, int DVS, bool NT>
struct Tile;

template <int DK, int DV, int DVS, bool NT>
struct Tile<_Float16, DK, DV, DVS, NT> {
  static constexpr uint32_t kBlk = 32;
  half8_t k[2][DK / 32];
  half8_t v[DVS / 16];
  __device__ __forceinline__ void load_k(const _Float16* kb, uint32_t slot0, int c16, int g) {
    const _Float16* kt = kb + (uint64_t)slot0 * DK;  // slot0 starts a tile
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int c = 0; c < DK / 32; ++c)
        k[b][c] = ld16<NT>((const half8_t*)(kt + c * (32 * 32) + (16 * b + c16) * 32 + 8 * g));
  }
  __device__ __forceinline__ void load_v(const _Float16* vb, uint32_t slot0, int c16, int g) {
    const _Float16* vblk = vb + (uint64_t)(slot0 / kBlk) * DV * kBlk;
#pragma unroll
    for (int n = 0; n < DVS / 16; ++n) v[n] = ld16<NT>((const half8_t*)(vblk + (16 * n + c16) * kBlk + 8 * g));
  }
  __device__ __forceinline__ void load(const _Float16* kb, const _Float16* vb, uint32_t slot0,
                                       int c16, int g) {
    load_k(kb, slot0, c16, g);
    load_v(vb, slot0, c16, g);
  }
};

template <int DK, int DV, int DVS, bool NT>
struct Tile<float, DK, DV, DVS, NT> {
  static constexpr uint32_t kBlk = 16;
  float4_t k[DK / 16];
  float4_t v[DVS / 16];
  __device__ __forceinline__ void load_k(const float* kb, uint32_t slot0, int c16, int g) {
    const float* kt = kb + (uint64_t)slot0 * DK;  // slot0 starts a tile
#pragma unroll
    for (int c = 0; c < DK / 16; ++c)
      k[c] = ld16<NT>((const float4_t*)(kt + c * (16 * 16) + c16 * 16 + 4 * g));
  }
  __device__ __forceinline__ void load_v(const float* vb, uint32_t slot0, int c16, int g) {
    const float* vblk = vb + (uint64_t)(slot0 / kBlk) * DV * kBlk;
#pragma unroll
    for (int n = 0; n < DVS / 16; ++n) v[n] = ld16<NT>((const float4_t*)(vblk + (16 * n + c16) * kBlk + 4 * g));
  }
  __device__ __forceinline__ void load(const float* kb, const float* vb, uint32_t slot0, int c16,
                                       int g) {
    load_k(kb, slot0, c16, g);
    load_v(vb, slot0, c16, g);
  }
};

// v with each 32-bit word ANDed with the matching word of keep.
__device__ __forceinline__ half8_t keep_bits(half8_t v, const uint32_t* keep) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  u32x4_t u = __builtin_bit_cast(u32x4_t, v);
#pragma unroll
  for (int w = 0; w < 4; ++w) u[w] &= keep[w];
  return __builtin_bit_cast(half8_t, u);
}

__device__ __forceinline__ uint64_t pack2(float lo, float hi) {
  return (uint64_t)__float_as_uint(lo) | ((uint64_t)__float_as_uint(hi) << 32);
}

// M consecutive floats from p (M = 2 or a multiple of 4; p aligned to 8 or 16 bytes to match).
template <int M>
__device__ __forceinline__ void load_floats(const float* __restrict__ p, float (&out)[M]) {
  if constexpr (M == 2) {
    const float2 t = *(const float2*)p;
    out[0] = t.x, out[1] = t.y;
  } else {
#pragma unroll
    for (int i = 0; i < M; i += 4) {
      const float4_t t = *(const float4_t*)(p + i);
      out[i] = t[0], out[i + 1] = t[1], out[i + 2] = t[2], out[i + 3] = t[3];
    }
  }
}

// N consecutive elements e0 .. e0+N-1 of one head, rotated as TensorOps.rope / ropeNeox do. x is
// the head's first element; e0 is a multiple of N and N divides the rotary pair count, so a chunk
// lies wholly in the first half, the second half or the pass-through tail of the head. Every
// load (the chunk, its NeoX partner chunk, the factors) is issued before any is used: the chunk
// costs one memory round trip. Lanes in the pass-through tail read factor row entry 0 and keep
// their elements.
template <int N>
__device__ __forceinline__ void rope_chunk(const float* __restrict__ x, uint32_t e0,
                                           const float* __restrict__ cs,
                                           const float* __restrict__ sn, uint32_t pairs,
                                           uint32_t neox, float (&out)[N]) {
  float v[N];
  load_floats<N>(x + e0, v);
  if (cs == nullptr) {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = v[i];
    return;
  }
  const bool rot = e0 < 2 * pairs;
  if (!neox) {  // interleaved pairs (2j, 2j+1) sit inside the chunk
    const uint32_t j = rot ? e0 / 2 : 0u;
    float c[N / 2], sf[N / 2];
    load_floats<N / 2>(cs + j, c);
    load_floats<N / 2>(sn + j, sf);
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      float a0 = v[i], a1 = v[i + 1];
      rotate_pair(a0, a1, c[i / 2], sf[i / 2]);
      out[i] = rot ? a0 : v[i];
      out[i + 1] = rot ? a1 : v[i + 1];
    }
    return;
  }
  const bool lower = e0 < pairs;  // split-half pairs (j, j + pairs)
  const uint32_t j = rot ? (lower ? e0 : e0 - pairs) : 0u;
  float w[N], c[N], sf[N];
  load_floats<N>(x + (lower ? e0 + pairs : e0 - pairs), w);  // the partner chunk, inside the head
  load_floats<N>(cs + j, c);
  load_floats<N>(sn + j, sf);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float a0 = lower ? v[i] : w[i], a1 = lower ? w[i] : v[i];
    rotate_pair(a0, a1, c[i], sf[i]);
    out[i] = rot ? (lower ? a0 : a1) : v[i];
  }
}

// Fused cross-split exchange. Partials live in a float buffer, per (item, head slot) dv acc
// values then m, l and two pad words, where every word not yet written this launch holds
// kClear (0xFFFFFFFF, a NaN bit pattern no arithmetic produces once NaNs are canonicalised):
// each 32-bit word is atomic by itself, so producers and the reducer move them with 16-byte
// device-coherent (sc1) buffer accesses and test every word.
constexpr uint32_t kClear = 0xFFFFFFFFu;
constexpr int kCoherent = 16;  // buffer cache policy bit sc1: coherent across the device's L2s

__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(float* p) {
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, 0x7FFFFFF0, 0x00020000);
}

// The buffer load intrinsic reads memory without side effects, so a reload of an unchanged
// address looks redundant to the compiler; every poll iteration starts with a compiler memory
// barrier (no instruction) so the reloads stay in the loop.
__device__ __forceinline__ void poll_barrier() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ float4_t load_part(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kCoherent);
}

__device__ __forceinline__ float2_t load_part2(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kCoherent);
}

__device__ __forceinline__ void store_part(__amdgpu_buffer_rsrc_t rs, uint32_t off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, kCoherent);
}

__device__ __forceinline__ float canon(float x) {  // any NaN -> the default quiet NaN
  return x != x ? __uint_as_float(0x7FC00000u) : x;
}

__device__ __forceinline__ bool written(float4_t v) {
  return __float_as_uint(v[0]) != kClear && __float_as_uint(v[1]) != kClear &&
         __float_as_uint(v[2]) != kClear && __float_as_uint(v[3]) != kClear;
}

__device__ __forceinline__ float4_t clear4() {
  const float c = __uint_as_float(kClear);
  return float4_t{c, c, c, c};
}

// Writes the not-written pattern back over a word group the reducer has read. Nobody reads it
// again in this launch, and the release at the end of the kernel writes it back to memory
// before the next launch starts, so a plain store suffices: it is acknowledged by the L2
// instead of after a write-through to memory, which shortens the kernel's tail.
__device__ __forceinline__ void clear_part(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(clear4(), rs, off, 0, 0);
}

// Polls of one reducer before it gives up and reports a reduction timeout (error bit 1). Each
// poll waits one memory round trip, so this bounds the wait at seconds; it is reached only if a
// producer of the group never stores, which the ticket order rules out.
constexpr uint32_t kSpinLimit = 1u << 22;

// One workgroup's partial for output elements e .. e+3 of head slot hs: its waves' states
// (s_ml, s_acc) rescaled to their common maximum and summed in wave order. Every multiply-add is
// an explicit fmaf, so the reducer (which keeps its own partial) and a producer (which stores it)
// compute the same bits and the result does not depend on which workgroup reduces. Every LDS
// read is issued before the first use; the weights use v_exp_f32 directly (their arguments are
// <= 0 or -inf, and a weight below 2^-126 contributes nothing).
template <int DV, int W>
__device__ __forceinline__ void wave_partial(const float (*s_acc)[16][DV], const float (*s_ml)[16][2],
                                             uint32_t hs, uint32_t e, float& mx, float& lw,
                                             float4_t& aw) {
  float2 ml[W];
  float4_t x[W];
#pragma unroll
  for (int w = 0; w < W; ++w) {
    ml[w] = *(const float2*)&s_ml[w][hs][0];
    x[w] = *(const float4_t*)&s_acc[w][hs][e];
  }
  mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < W; ++w) mx = fmaxf(mx, ml[w].x);
  const float mu = mx == -INFINITY ? 0.0f : mx;
  lw = 0.0f;
  aw = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float f = __builtin_amdgcn_exp2f(ml[w].x - mu);
    lw = fmaf(ml[w].y, f, lw);
#pragma unroll
    for (int i = 0; i < 4; ++i) aw[i] = fmaf(x[w][i], f, aw[i]);
  }
}

// The reducer's side of the exchange for one group (row, kv head, head group) whose ns <= B
// partials start at item0; this workgroup is split `split`, its own per-wave state in s_acc /
// s_ml. Output quads (4 elements) are taken by SUB consecutive threads each; sub-thread r takes
// the splits r, r + SUB, ... and loads their acc quad and (m, l) word, reloading until no word
// reads kClear (its own split comes from its waves, computed while the loads are in flight).
// The maximum M, the sum L of l * 2^(m - M) and the weighted acc sum are formed per thread in
// split order and meet across the SUB threads in a fixed shuffle tree, so the result does not
// depend on which workgroup reduces. Every word read is set back to kClear; the (m, l) words,
// read by all quads of a head, after a barrier.
template <int B, int SUB, int DV, int W, int OS>
__device__ __forceinline__ void reduce_group(float* part, uint64_t item0, uint32_t ns,
                                             uint32_t split, uint32_t nreal,
                                             const float (*s_acc)[16][DV],
                                             const float (*s_ml)[16][2], float* out, int* err) {
  constexpr uint32_t kT = 64 * W;
  constexpr uint32_t kQ4 = DV / 4;   // quads per head
  constexpr int kI = B / SUB;        // splits one thread takes
  static_assert(SUB == 1 || SUB == 2 || SUB == 4 || SUB == 8, "sub-threads per quad");
  static_assert(kI <= 32, "splits per thread");
  const uint32_t tid = threadIdx.x;
  const uint32_t E4 = nreal * kQ4;
  const __amdgpu_buffer_rsrc_t rs = part_rsrc(part);
  auto base = [&](uint32_t g, uint32_t hs) JMA_INL {  // byte offset of (split g, head slot hs)
    return (uint32_t)(fused_part_float(item0 + g, hs, DV, 0) * 4);
  };
  const uint32_t r = tid % SUB;
  // Words a thread does not need (splits past ns, its own split, quads past the group) are
  // addressed past the buffer's record count: such a load returns 0, which reads as written, and
  // such a store is dropped, so the poll, the sums and the clear-back need no per-split branches.
  constexpr uint32_t kSkip = 0xFFFFFF00u;
  bool timed_out = false;
  for (uint32_t q0 = 0; q0 < E4; q0 += kT / SUB) {
    const uint32_t quad = q0 + tid / SUB;
    const bool qok = quad < E4;
    const uint32_t hs = qok ? quad / kQ4 : 0u, e = qok ? (quad % kQ4) * 4 : 0u;
    uint32_t off_x[kI], off_m[kI];
#pragma unroll
    for (int i = 0; i < kI; ++i) {
      const uint32_t g = r + SUB * i;
      const bool needed = qok && g < ns && g != split;
      const uint32_t w = base(g, hs);
      off_x[i] = needed ? w + e * 4 : kSkip;
      off_m[i] = needed ? w + DV * 4 : kSkip;
    }
    float4_t xv[kI];
    float2_t mv[kI];
#pragma unroll
    for (int i = 0; i < kI; ++i) {
      xv[i] = load_part(rs, off_x[i]);
      mv[i] = load_part2(rs, off_m[i]);
    }
    float mx, lw;  // this workgroup's own partial, while the loads are in flight
    float4_t own;
    wave_partial<DV, W>(s_acc, s_ml, hs, e, mx, lw, own);
    // Keep that work ahead of the first wait for the loads (left alone, the compiler sinks it
    // behind the wait, where it lengthens the reducer's tail).
    asm volatile("" ::"v"(mx), "v"(lw), "v"(own[0]), "v"(own[1]), "v"(own[2]), "v"(own[3]));
    for (uint32_t spin = 0;; ++spin) {
      bool ready = true;
#pragma unroll
      for (int i = 0; i < kI; ++i) ready &= written(xv[i]) && written(float4_t{mv[i][0], mv[i][1], mv[i][0], mv[i][1]});
      if (ready) break;
      if (spin == kSpinLimit) {
        timed_out = true;
        break;
      }
      poll_barrier();
      // Every word again (those already written read the same data).
#pragma unroll
      for (int i = 0; i < kI; ++i) {
        xv[i] = load_part(rs, off_x[i]);
        mv[i] = load_part2(rs, off_m[i]);
      }
    }
    // Per-thread maximum, then the maximum over the quad's SUB threads. Splits past ns weigh
    // 2^-inf = 0 (their words read 0), so every split takes the same code.
    float m_i[kI];
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < kI; ++i) {
      const uint32_t g = r + SUB * i;
      m_i[i] = g == split ? mx : (g < ns ? mv[i][0] : -INFINITY);
      M = fmaxf(M, m_i[i]);
    }
    if constexpr (SUB >= 2) M = fmaxf(M, dpp<kDppXor1>(M));
    if constexpr (SUB >= 4) M = fmaxf(M, dpp<kDppXor2>(M));
    if constexpr (SUB >= 8) M = fmaxf(M, dpp<kDppHalfMirror>(M));
    const float mu = M == -INFINITY ? 0.0f : M;
    float L = 0.0f;
    float4_t X = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kI; ++i) {
      const uint32_t g = r + SUB * i;
      const float wg = __builtin_amdgcn_exp2f(m_i[i] - mu);
      const float lg = g == split ? lw : mv[i][1];
      const float4_t xg = g == split ? own : xv[i];
      L = fmaf(lg, wg, L);
#pragma unroll
      for (int c = 0; c < 4; ++c) X[c] = fmaf(xg[c], wg, X[c]);
    }
    if constexpr (SUB >= 2) {
      L += dpp<kDppXor1>(L);
#pragma unroll
      for (int c = 0; c < 4; ++c) X[c] += dpp<kDppXor1>(X[c]);
    }
    if constexpr (SUB >= 4) {
      L += dpp<kDppXor2>(L);
#pragma unroll
      for (int c = 0; c < 4; ++c) X[c] += dpp<kDppXor2>(X[c]);
    }
    if constexpr (SUB >= 8) {
      L += dpp<kDppHalfMirror>(L);
#pragma unroll
      for (int c = 0; c < 4; ++c) X[c] += dpp<kDppHalfMirror>(X[c]);
    }
    if (qok && r == 0) {
      if (!(L > 0.0f) && e == 0) atomicOr(err, 1);  // all -inf, or a NaN / +inf score
      *(float4_t*)(out + hs * OS + e) = X * __builtin_amdgcn_rcpf(L);  // L >= 1: no denormals
    }
    // Clear-back of the acc words, after the output store.
#pragma unroll
    for (int i = 0; i < kI; ++i) clear_part(rs, off_x[i]);
  }
  __syncthreads();  // every quad of every head has read its (m, l) words
  for (uint32_t k = tid; k < (ns - 1) * nreal; k += kT) {
    const uint32_t o = k / nreal, hs = k % nreal;
    clear_part(rs, base(o + (o >= split ? 1u : 0u), hs) + DV * 4);
  }
  if (timed_out) atomicOr(err, 2);
}

// One workgroup = one work item (row, kv head, head group of <= 16 query heads, split); its
// decode_waves(DK) waves stride over the split's tiles. Scores are computed as S = K * Q^T on 16-row
// blocks so lane (g, c) holds rows 4g+e of query head c: every lane works on a single head, the
// online-softmax rescale is one factor per lane, and the score registers are already the B
// operand of the PV product O^T = V^T * P.
//
// f16 KV: v_mfma_f32_16x16x32_f16. q and p are split into hi + lo halves (x = hi + lo exactly
// to ~2^-22), so both products run at near-f32 accuracy against the f32 reference.
// f32 KV: v_mfma_f32_16x16x4_f32 with f32 operands throughout.
//
// The kernel is bound by memory latency, not bandwidth (a layer-step at 4k context moves a few
// MB), so it is laid out to put as few dependent memory round trips on the critical path as it
// can:
//  - each wave issues the loads of its first two tiles before it loads q, and one tile ahead
//    after that;
//  - RoPE on q (rope_q): each lane rotates the q elements it loads;
//  - the append (k_new/v_new): the workgroups whose last tile holds the new position rotate the
//    new K row and patch it, with the new V row, into the registers of that tile; the head
//    group 0 workgroup also stores the row to the cache, and nobody waits for that store;
//  - the cross-split reduction (counters): every workgroup of a (row, kv head, head group) takes
//    an arrival ticket with one atomic at its start. The last to arrive becomes the reducer:
//    every other workgroup of its group has started by then and so will finish. The others store
//    their partial (acc, m, l) as plain words with device-coherent 16-byte stores and exit
//    without waiting; the reducer reads them back with device-coherent loads, reloading until no
//    word holds the not-written pattern, then writes that pattern back, so every partial word is
//    clear again when the launch ends.
// kOne: the plan gives every wave at most one tile (tiles_per_split <= waves), so the second tile
// buffer is never needed (at head dim 256 two buffers are the whole register file).
// The leading scalar arguments are what the kSimple instance needs to address its first tiles
// (the layer's K / V base for the sequence, the first row's position, the window, tiles per split
// and the slot capacity). The library is built with kernel-argument preloading, so they arrive in
// scalar registers at wave start and the first tile loads do not wait for a kernel-argument
// load; the other instances pass zeros there and read everything from `a`.
template <typename KV, int DK, int DV, int DVS, bool kSimple, bool kOne, bool kNT, bool kPack>
__global__ __launch_bounds__(64 * decode_waves(DK)) void decode_kernel(
    const void* p_kb, const void* p_vb, uint32_t p_start, uint32_t p_window, uint32_t p_tps,
    uint32_t p_cap, uint32_t p_ring, const DecodeArgs a) {
  constexpr bool kF16 = std::is_same<KV, _Float16>::value;
  using TileT = Tile<KV, DK, DV, DVS, kNT>;
  constexpr uint32_t kBlk = TileT::kBlk;
  constexpr int kNs = kF16 ? 8 : 4;   // scores per lane per tile
  constexpr int kNv = DVS / 16;       // output fragments per lane
  // kP (f16 KV, head dim 512, kv groups of at most 8 query heads): the hi and lo halves of q, and
  // of p, share one matrix op as columns j and 8 + j of head j, instead of taking one op each.
  // Each lane pair (j, 8 + j) adds its two partial scores with one row rotation, so both lanes
  // hold the whole score and the same softmax state; column 8 + j of the PV product accumulates
  // the lo halves, added to column j once the tile loop is done. Half the matrix ops per tile.
  constexpr bool kP = kPack && kF16 && DK == 512;
  // Column slices: a workgroup computes DVS of the DV value columns (the whole of q.K, the V
  // columns and output of its slice only). The slices are virtual head groups: `hgroups` counts
  // head groups x kSlices, and a virtual group hgv is head group hgv / kSlices, slice
  // hgv % kSlices, with its own work items, partials and arrival tickets.
  constexpr uint32_t kSlices = DV / DVS;
  constexpr int kC = kF16 ? DK / 32 : DK / 16;
  constexpr int kQ = kF16 ? 8 : 4;    // q elements per lane per k-chunk
  constexpr uint32_t kW = decode_waves(DK);
  // kQLds (head dim 512): the q operands are read from LDS at every tile instead of being held in
  // registers (16 heads x 512 elements as f16 hi + lo would take 128 registers per lane), and the
  // q rows share their LDS with the waves' combine area, which is written only after every wave
  // has left its tile loop.
  constexpr bool kQLds = DK >= 512;
  // q rows in LDS, padded against bank conflicts: f32 KV keeps them as floats (kQRowF per row);
  // f16 KV keeps the f16 hi and lo halves of each element (x = hi + lo to ~2^-22), formed once
  // while staging, in two arrays of kQRowH halves per row.
  constexpr int kQRowF = DK + 4, kQRowH = DK + 8;
  constexpr int kAccFloats = kW * 16 * DVS, kQFloats = kF16 ? 16 * kQRowH : 16 * kQRowF;
  __shared__ __attribute__((aligned(16))) float s_acc_mem[kQLds && kQFloats > kAccFloats ? kQFloats : kAccFloats];
  __shared__ __attribute__((aligned(16))) float s_q_mem[kQLds ? 4 : kQFloats];
  float (*s_acc)[16][DVS] = (float (*)[16][DVS])s_acc_mem;
  float (*s_q)[kQRowF] = (float (*)[kQRowF])(kQLds ? s_acc_mem : s_q_mem);
  _Float16 (*s_qh)[kQRowH] = (_Float16 (*)[kQRowH])(kQLds ? s_acc_mem : s_q_mem);
  _Float16 (*s_ql)[kQRowH] = s_qh + 16;
  __shared__ float s_ml[kW][16][2];
  __shared__ uint32_t s_ticket;
  __shared__ __attribute__((aligned(16))) KV s_new_k[DK];  // the appended row, rotated
  __shared__ KV s_new_v[DV];
  __shared__ float s_qn[16];  // QK-norm scale of each raw q head

  // The grid is (split, kv head * head groups + head group, row). Every scalar argument the
  // kernel uses, the row's own table entries included, is fetched in one batch: left to itself
  // the compiler loads each right before its use, behind its own wait, and a scalar load costs
  // about half a vector memory round trip here. kSimple (contiguous rows of one sequence, equal
  // split counts, one head group) takes its cache base from the host and needs almost no address
  // arithmetic before the first tile load.
  const uint32_t split = blockIdx.x, rest = blockIdx.y, row = blockIdx.z;
  uint32_t num_heads = a.num_heads, group = a.group, hgroups = a.hgroups, hkv = a.num_kv_heads;
  uint32_t ns_uniform = a.ns_uniform, rows_contig = a.rows.contiguous;
  uint32_t rows_seq0 = a.rows.seq0, rows_start = a.rows.start;
  uint32_t window = a.window, tps = a.tiles_per_split, cap = a.kv.cap, ring = a.kv.ring;
  uint32_t pairs = a.pairs, neox = a.neox, rope_q = a.rope_q;
  float qscale = a.qscale;
  // Pointers go through the asm typed as global memory so the loads through them stay global
  // (a generic pointer would turn them into flat loads, which also count against lgkmcnt).
  JMA_GLOBAL const float *g_q = (JMA_GLOBAL const float*)a.q;
  JMA_GLOBAL const float *g_cos = (JMA_GLOBAL const float*)a.cos_t;
  JMA_GLOBAL const float *g_sin = (JMA_GLOBAL const float*)a.sin_t;
  JMA_GLOBAL const float *g_kn = (JMA_GLOBAL const float*)a.k_new;
  JMA_GLOBAL const float *g_vn = (JMA_GLOBAL const float*)a.v_new;
  JMA_GLOBAL uint32_t* g_ctr = (JMA_GLOBAL uint32_t*)a.counters;
  JMA_GLOBAL float* g_out = (JMA_GLOBAL float*)a.out;
  JMA_GLOBAL float* g_tag = (JMA_GLOBAL float*)a.part_f;
  JMA_GLOBAL float* g_pacc = (JMA_GLOBAL float*)a.part_acc;
  JMA_GLOBAL float* g_pml = (JMA_GLOBAL float*)a.part_ml;
  JMA_GLOBAL int* g_err = (JMA_GLOBAL int*)a.err;
  uint32_t ns, item, hg, hgv, slice, kvh, seq, pos, item_row0 = 0;
  KV *kb, *vb;
  if constexpr (kSimple) {
    // Only the preloaded arguments here: the rest are fetched after the first tile loads issue.
    JMA_GLOBAL KV* g_kb = (JMA_GLOBAL KV*)p_kb;
    JMA_GLOBAL KV* g_vb = (JMA_GLOBAL KV*)p_vb;
    asm volatile("" : "+s"(g_kb), "+s"(g_vb), "+s"(p_start), "+s"(p_window), "+s"(p_tps), "+s"(p_cap),
                 "+s"(p_ring));
    rows_start = p_start;
    window = p_window;
    tps = p_tps;
    cap = p_cap;
    ns = 0;
    item = 0;
    hg = 0;
    hgv = rest % kSlices;
    slice = hgv;
    kvh = rest / kSlices;
    seq = 0;
    pos = rows_start + row;
    ring = p_ring;
    hgroups = kSlices;
    kb = (KV*)g_kb + (uint64_t)kvh * cap * DK;
    vb = (KV*)g_vb + (uint64_t)kvh * cap * DV + slice * DVS * TileT::kBlk;
  } else {
    uint32_t r_seq = a.rows.seq[row], r_pos = a.rows.pos[row], r_ns = a.nsplit[row],
             r_item0 = a.item_start[row];
    uint64_t seq_stride_k = a.kv.seq_stride_k, seq_stride_v = a.kv.seq_stride_v;
    uint64_t layer_off_k = a.kv.layer_off_k, layer_off_v = a.kv.layer_off_v;
    JMA_GLOBAL KV *g_k = (JMA_GLOBAL KV*)a.kv.k, *g_v = (JMA_GLOBAL KV*)a.kv.v;
    asm volatile("" : "+s"(num_heads), "+s"(group), "+s"(hgroups), "+s"(hkv), "+s"(ns_uniform),
                 "+s"(rows_contig), "+s"(r_seq), "+s"(r_pos), "+s"(r_ns), "+s"(r_item0),
                 "+s"(rows_seq0), "+s"(rows_start), "+s"(window), "+s"(tps), "+s"(cap), "+s"(ring),
                 "+s"(pairs), "+s"(neox), "+s"(rope_q), "+s"(qscale),
                 "+s"(seq_stride_k), "+s"(seq_stride_v), "+s"(layer_off_k), "+s"(layer_off_v));
    asm volatile("" : "+s"(g_k), "+s"(g_v), "+s"(g_q), "+s"(g_cos), "+s"(g_sin), "+s"(g_kn),
                 "+s"(g_vn), "+s"(g_ctr), "+s"(g_out), "+s"(g_tag), "+s"(g_pacc), "+s"(g_pml),
                 "+s"(g_err));
    ns = ns_uniform ? ns_uniform : r_ns;
    if (split >= ns) return;  // a listed row with fewer splits than the grid's widest row
    item = group_item0(ns_uniform, r_item0, row, hkv, hgroups, rest, ns) + split;
    item_row0 = r_item0;
    hgv = hgroups == 1 ? 0u : rest % hgroups;
    hg = hgv / kSlices;
    slice = hgv % kSlices;
    kvh = hgroups == 1 ? rest : rest / hgroups;
    seq = rows_contig ? rows_seq0 : r_seq;
    pos = rows_contig ? rows_start + row : r_pos;
    kb = (KV*)g_k + seq * seq_stride_k + layer_off_k + (uint64_t)kvh * cap * DK;
    vb = (KV*)g_v + seq * seq_stride_v + layer_off_v + (uint64_t)kvh * cap * DV + slice * DVS * TileT::kBlk;
  }
  const uint32_t first = first_visible(pos, window);
  const uint32_t t_begin = first / kBlk, t_end = pos / kBlk + 1;
  const uint32_t s_t0 = t_begin + split * tps;
  const uint32_t s_t1 = min(s_t0 + tps, t_end);
  // Ring layers: the split's first tile slot, then consecutive tiles wrap at most once (a
  // split spans fewer positions than the ring holds).
  uint32_t slot_base = s_t0 * kBlk;
  if (ring) slot_base %= cap;

  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  auto slot0_of = [&](uint32_t t) JMA_INL {
    const uint32_t x = slot_base + (t - s_t0) * kBlk;
    return ring && x >= cap ? x - cap : x;
  };

  // The first two tiles of this wave are in flight before anything else is loaded (at head
  // dimension 256 the second waits until q is prepared: two tiles are half the register file).
  // At head dimension 512 a tile's K and V never share the registers: K is loaded here, V inside
  // the step once the scores are formed.
  constexpr bool kEarly2 = DK <= 128;
  constexpr bool kSplitKV = DK >= 512;
  auto tile_load = [&](TileT& x, uint32_t tt) JMA_INL {
    if constexpr (kSplitKV) x.load_k(kb, slot0_of(tt), c16, g);
    else x.load(kb, vb, slot0_of(tt), c16, g);
  };
  uint32_t t = s_t0 + wave;
  TileT ta, tb;
  if (t < s_t1) tile_load(ta, t);
  if constexpr (!kOne)
    if (kEarly2 && t + kW < s_t1) tile_load(tb, t + kW);

  if constexpr (kSimple) {
    // The remaining arguments, in one batch, once the first tile loads are issued.
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+s"(num_heads), "+s"(group), "+s"(hkv), "+s"(ns_uniform), "+s"(pairs),
                 "+s"(neox), "+s"(rope_q), "+s"(qscale));
    asm volatile("" : "+s"(g_q), "+s"(g_cos), "+s"(g_sin), "+s"(g_kn), "+s"(g_vn), "+s"(g_ctr),
                 "+s"(g_out), "+s"(g_tag), "+s"(g_pacc), "+s"(g_pml), "+s"(g_err));
    ns = ns_uniform;
    item = group_item0(ns, 0, row, hkv, kSlices, rest, ns) + split;
  }
  const float *q_in = (const float*)g_q, *cos_t = (const float*)g_cos, *sin_t = (const float*)g_sin;
  const float *k_new = (const float*)g_kn, *v_new = (const float*)g_vn;
  uint32_t* counters = (uint32_t*)g_ctr;
  float* out = (float*)g_out;
  float* part_f = (float*)g_tag;
  float* part_acc = (float*)g_pacc;
  float* part_ml = (float*)g_pml;
  int* err = (int*)g_err;

  const bool fused = ns > 1 && counters != nullptr;
  const uint64_t gid = group_counter(row, hkv, kvh, hgroups, hgv);
  // Arrival ticket: its round trip overlaps the tile loads.
  uint32_t ticket = 0;
  if (fused && threadIdx.x == 0)
    ticket = __hip_atomic_fetch_add(&counters[gid], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  const uint32_t hl = hg * 16 + c16;
  const bool head_ok = hl < group;
  // The q operand column of this lane holds a real head (kP: head c16 % 8, hi or lo half).
  const bool qcol_ok = kP ? ((uint32_t)c16 & 7u) + hg * 16 < group : head_ok;
  const float* cs = cos_t ? cos_t + (uint64_t)pos * pairs : nullptr;
  const float* sn = cos_t ? sin_t + (uint64_t)pos * pairs : nullptr;

  // Fused append and q staging. The loads of both (the new K / V row elements with their RoPE
  // factors, then the q elements with theirs) are all issued before any of them is used: a
  // vector-memory wait also waits for every earlier load of the wave, the tile loads included, so
  // using the append's loads before issuing the q loads would put a second memory round trip on
  // the path of the workgroup that appends (and the reducer waits for that workgroup).
  //
  // Append: the new row's tile is the last of the row's last split. One thread per K pair (rotated
  // as rope_append_kernel rotates it) or V element pair, the workgroup's threads taking
  // DK / 2 + DV / 2 pairs in turn (two turns at head dimension 512); the row goes to LDS, from
  // where the wave owning that tile patches it into its registers, and the head group 0
  // workgroup stores it to the cache (the next launches read it there).
  const bool append = k_new != nullptr && split == ns - 1;
  constexpr uint32_t kPairs = DK / 2 + DV / 2;
  constexpr uint32_t kTurns = (kPairs + 64 * kW - 1) / (64 * kW);
  const float* kx = append ? k_new + ((uint64_t)row * hkv + kvh) * DK : nullptr;
  const float* vx = append ? v_new + ((uint64_t)row * hkv + kvh) * DV : nullptr;
  float ax0[kTurns], ax1[kTurns], afc[kTurns], afs[kTurns];
  if (append) {
#pragma unroll
    for (uint32_t turn = 0; turn < kTurns; ++turn) {
      const uint32_t tid = threadIdx.x + turn * 64 * kW;
      afc[turn] = 1.0f;
      afs[turn] = 0.0f;
      if (tid < DK / 2) {
        const uint32_t j = tid;
        const bool rot = cs != nullptr && j < pairs;
        ax0[turn] = kx[rot && neox ? j : 2 * j];
        ax1[turn] = kx[rot && neox ? j + pairs : 2 * j + 1];
        if (cs != nullptr) {
          afc[turn] = cs[rot ? j : 0u];
          afs[turn] = sn[rot ? j : 0u];
        }
      } else if (tid < kPairs) {
        const uint32_t d = 2 * (tid - DK / 2);
        ax0[turn] = vx[d];
        ax1[turn] = vx[d + 1];
      }
    }
  }

  // q of this head group, rotated here when the caller passed raw q, times the score scale,
  // staged in LDS by the whole workgroup: thread k takes RoPE pair k (head k / (DK/2)).
  const uint32_t nreal = min(16u, group - hg * 16);  // query heads of this head group
  constexpr uint32_t kHalf = DK / 2;
  constexpr int kIt = (16 * kHalf + 64 * kW - 1) / (64 * kW);
  const uint32_t nq = nreal * kHalf;
  const bool rope_on = rope_q != 0 && cs != nullptr;
  const float* qg = q_in + ((uint64_t)row * num_heads + kvh * group + hg * 16) * DK;
  float qy0[kIt], qy1[kIt], qfc[kIt], qfs[kIt];
  uint32_t qe0[kIt], qe1[kIt];
  bool qrot[kIt];
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    // Turns past the head group's pairs (fewer than 16 heads) load nothing; within a turn the
    // indices are clamped, so every load is valid.
    const uint32_t k = min(threadIdx.x + 64 * kW * it, nq - 1);
    const uint32_t hs = k / kHalf, j = k % kHalf;
    qrot[it] = rope_on && j < pairs;
    qe0[it] = hs * DK + (qrot[it] && neox ? j : 2 * j);
    qe1[it] = hs * DK + (qrot[it] && neox ? j + pairs : 2 * j + 1);
    qy0[it] = qy1[it] = qfc[it] = qfs[it] = 0.0f;
    if (64 * kW * it < nq) {
      qy0[it] = qg[qe0[it]];
      qy1[it] = qg[qe1[it]];
      if (rope_on) {
        qfc[it] = cs[qrot[it] ? j : 0u];
        qfs[it] = sn[qrot[it] ? j : 0u];
      }
    }
  }

  if (append) {
    const uint32_t slot = ring ? pos % cap : pos;
#pragma unroll
    for (uint32_t turn = 0; turn < kTurns; ++turn) {
      const uint32_t tid = threadIdx.x + turn * 64 * kW;
      if (tid < DK / 2) {
        const uint32_t j = tid;
        const bool rot = cs != nullptr && j < pairs;
        const uint32_t e0 = rot && neox ? j : 2 * j, e1 = rot && neox ? j + pairs : 2 * j + 1;
        float y0 = ax0[turn], y1 = ax1[turn];
        // QK-norm of the head before RoPE, as the append kernel applies it.
        if (a.k_norm_w != nullptr) {
#pragma clang fp contract(off)
          const float sc = head_rms_scale_d<DK>(kx, a.norm_eps);
          y0 = y0 * sc * a.k_norm_w[e0];
          y1 = y1 * sc * a.k_norm_w[e1];
        }
        if (rot) rotate_pair(y0, y1, afc[turn], afs[turn]);
        s_new_k[e0] = (KV)y0;
        s_new_k[e1] = (KV)y1;
        if (hg == 0 && slice == 0) {
          kb[k_index(slot, e0, DK, kF16)] = (KV)y0;
          kb[k_index(slot, e1, DK, kF16)] = (KV)y1;
        }
      } else if (tid < kPairs) {
        const uint32_t d = 2 * (tid - DK / 2);
        float v0 = ax0[turn], v1 = ax1[turn];
        if (a.v_norm != 0u) value_rms_norm(vx, DV, a.norm_eps, v0, v1);
        s_new_v[d] = (KV)v0;
        s_new_v[d + 1] = (KV)v1;
        if (hg == 0 && slice == 0) {  // vb is the unsliced base here
          const uint32_t r = kF16 ? perm32(slot % kBlk) : slot % kBlk;
          KV* vp = vb + (uint64_t)(slot / kBlk) * DV * kBlk + (uint64_t)d * kBlk + r;
          vp[0] = (KV)v0;
          vp[kBlk] = (KV)v1;
        }
      }
    }
  }
  // Lanes of the wave owning the new row's tile that hold that row: K lanes hold tile rows
  // 16b + c16 (f16) or c16 (f32); V lanes hold tile rows by MFMA k-group g.
  const uint32_t t_new = pos / kBlk, r_new = pos % kBlk;
  const bool patch_wave = append && (t_new - s_t0) % kW == (uint32_t)wave;
  const uint32_t v_at = kF16 ? perm32(r_new) : r_new;  // V block index of the new row
  const bool k_lane = patch_wave && (uint32_t)c16 == (r_new & 15u);
  const bool v_lane = patch_wave && (uint32_t)g == v_at / (kF16 ? 8u : 4u);

  {
    // Raw q of a QK-norm layer: each head's scale (one thread per head, the append kernel's
    // arithmetic), then every element times that scale and its weight, before RoPE.
    const float* qw = rope_q != 0 ? (const float*)a.q_norm_w : nullptr;
    if (qw != nullptr) {
      if (threadIdx.x < nreal) s_qn[threadIdx.x] = head_rms_scale_d<DK>(qg + threadIdx.x * DK, a.norm_eps);
      __syncthreads();
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      if (threadIdx.x + 64 * kW * it >= nq) continue;
      float u0 = qy0[it], u1 = qy1[it];
      const uint32_t hs = qe0[it] / DK;
      if (qw != nullptr) {
#pragma clang fp contract(off)
        const float sc = s_qn[hs];
        u0 = u0 * sc * qw[qe0[it] - hs * DK];
        u1 = u1 * sc * qw[qe1[it] - hs * DK];
      }
      if (qrot[it]) rotate_pair(u0, u1, qfc[it], qfs[it]);
      const float x0 = u0 * qscale, x1 = u1 * qscale;
      const uint32_t f0 = qe0[it] - hs * DK, f1 = qe1[it] - hs * DK;
      if constexpr (kF16) {
        const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
        s_qh[hs][f0] = h0;
        s_ql[hs][f0] = (_Float16)(x0 - (float)h0);
        s_qh[hs][f1] = h1;
        s_ql[hs][f1] = (_Float16)(x1 - (float)h1);
      } else {
        s_q[hs][f0] = x0;
        s_q[hs][f1] = x1;
      }
    }
  }
  if constexpr (!kOne)
    if (!kEarly2 && t + kW < s_t1) tile_load(tb, t + kW);
  __syncthreads();  // q (and the appended row) are in LDS

  // Q operand (B of S = K Q^T); the padding head lanes hold zeros. kQLds: formed from LDS at each
  // use by q_chunk instead.
  constexpr int kCR = kQLds ? 1 : kC;  // chunks held in registers
  half8_t qhi[kF16 ? kCR : 1], qlo[kF16 ? kCR : 1];
  float4_t qf[kF16 ? 1 : kCR];
  auto q_chunk = [&](int c, half8_t& hi, half8_t& lo, float4_t& f) JMA_INL {
    if constexpr (kP) {  // hi: the packed operand (column j: hi of head j, 8 + j: its lo)
      const uint32_t hq = (uint32_t)c16 & 7u;
      const _Float16* row = c16 < 8 ? &s_qh[hq][0] : &s_ql[hq][0];
      hi = qcol_ok ? *(const half8_t*)(row + 32 * c + 8 * g) : half8_t{};
      lo = half8_t{};
    } else if constexpr (kF16) {
      hi = head_ok ? *(const half8_t*)&s_qh[c16][32 * c + 8 * g] : half8_t{};
      lo = head_ok ? *(const half8_t*)&s_ql[c16][32 * c + 8 * g] : half8_t{};
    } else {
      f = head_ok ? *(const float4_t*)&s_q[c16][16 * c + 4 * g] : float4_t{0.f, 0.f, 0.f, 0.f};
    }
  };
  if constexpr (!kQLds) {
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      half8_t h, lo;
      float4_t f;
      q_chunk(c, h, lo, f);
      if constexpr (kF16) {
        qhi[c] = h;
        qlo[c] = lo;
      } else {
        qf[c] = f;
      }
    }
  }

  float m = -INFINITY, l = 0.0f;
  float4_t acc[kNv];
#pragma unroll
  for (int n = 0; n < kNv; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto step = [&](TileT cur, uint32_t tt, auto patch) JMA_INL {
    if constexpr (decltype(patch)::value) {
      // The lanes holding the new row take it from LDS: K by whole 16-byte chunks, V by element.
      if constexpr (kF16) {
#pragma unroll
        for (int c = 0; c < kC; ++c) {
          const half8_t x = *(const half8_t*)&s_new_k[32 * c + 8 * g];
          if (r_new < 16) cur.k[0][c] = k_lane ? x : cur.k[0][c];
          else cur.k[1][c] = k_lane ? x : cur.k[1][c];
        }
      } else {
#pragma unroll
        for (int c = 0; c < kC; ++c) {
          const float4_t x = *(const float4_t*)&s_new_k[16 * c + 4 * g];
          cur.k[c] = k_lane ? x : cur.k[c];
        }
      }
    }
    // The new row's V elements: every LDS read is issued before any is used, then each lands in
    // operand element v_at % kQ (the same for the whole workgroup, so one uniform branch picks the
    // element and the selects inside it are branch-free).
    auto patch_v = [&]() JMA_INL {
      KV nv[kNv];
#pragma unroll
      for (int n = 0; n < kNv; ++n) nv[n] = s_new_v[slice * DVS + 16 * n + c16];
      const uint32_t ev = v_at % (uint32_t)kQ;
#pragma unroll
      for (int e = 0; e < kQ; ++e) {
        if ((uint32_t)e == ev) {
#pragma unroll
          for (int n = 0; n < kNv; ++n) cur.v[n][e] = v_lane ? nv[n] : cur.v[n][e];
        }
      }
    };
    if constexpr (decltype(patch)::value && !kSplitKV) patch_v();
    const uint32_t p0 = tt * kBlk;
    // Only the first and last tiles of the visible range hold masked rows. Their value elements
    // (element i of each V operand is the position of score i) are cleared too, through the
    // bit masks vkeep (one per 32-bit word of an operand): a masked slot may hold anything (a
    // discarded tail, an old ring slot, a value that overflowed f16), and 0 * inf would reach the
    // result. The masks depend on positions only, so they are formed ahead of the matrix ops
    // (whose results only take the selects).
    const bool edge = p0 < first || p0 + kBlk - 1 > pos;
    uint32_t okbits = ~0u;
    uint32_t vkeep[4] = {~0u, ~0u, ~0u, ~0u};
    if (edge) {
#pragma unroll
      for (int i = 0; i < kNs; ++i) {
        const uint32_t p = kF16 ? p0 + 16 * (i >> 2) + 4 * g + (i & 3) : p0 + 4 * g + i;
        const bool ok = p >= first && p <= pos;
        okbits &= ok ? ~0u : ~(1u << i);
        if constexpr (kF16) vkeep[i >> 1] &= ok ? ~0u : ((i & 1) ? 0x0000FFFFu : 0xFFFF0000u);
        else vkeep[i] = ok ? ~0u : 0u;
      }
    }
    float s[kNs];
    if constexpr (kF16 && kQLds) {
      // q chunk c is formed once from LDS and serves both 16-row halves of the tile.
      float4_t sc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int c = 0; c < kC; ++c) {
        half8_t qh, ql;
        float4_t unused;
        q_chunk(c, qh, ql, unused);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[b][c], qh, sc[b], 0, 0, 0);
          if constexpr (!kP) sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[b][c], ql, sc[b], 0, 0, 0);
        }
      }
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * b + e] = sc[b][e];
    } else if constexpr (kF16) {
      // The k-chunks accumulate into kNa independent chains per 16-row half (a dependent matrix
      // op waits for its predecessor's result), added at the end.
      constexpr int kNa = kC >= 8 ? 4 : (kC >= 4 ? 2 : 1);
      float4_t sc[2][kNa];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < kNa; ++i) sc[b][i] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kC; ++c)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          sc[b][c % kNa] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[b][c], qhi[c], sc[b][c % kNa], 0, 0, 0);
          if constexpr (!kP)
            sc[b][c % kNa] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.k[b][c], qlo[c], sc[b][c % kNa], 0, 0, 0);
        }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int w = kNa / 2; w >= 1; w /= 2)
#pragma unroll
          for (int i = 0; i < w; ++i) sc[b][i] += sc[b][i + w];
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * b + e] = sc[b][0][e];
      }
    } else {
      constexpr int kNa = kC >= 4 ? 4 : kC;  // independent chains, as above
      float4_t sc[kNa];
#pragma unroll
      for (int i = 0; i < kNa; ++i) sc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kC; ++c) {
        half8_t unused_h, unused_l;
        float4_t qc;
        if constexpr (kQLds) q_chunk(c, unused_h, unused_l, qc);
        else qc = qf[c];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sc[c % kNa] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[c][e], qc[e], sc[c % kNa], 0, 0, 0);
      }
#pragma unroll
      for (int w = kNa / 2; w >= 1; w /= 2)
#pragma unroll
        for (int i = 0; i < w; ++i) sc[i] += sc[i + w];
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] = sc[0][e];
    }
    if constexpr (kP) {  // the hi and lo partial scores of each head meet in lanes j and 8 + j
#pragma unroll
      for (int i = 0; i < kNs; ++i) s[i] += dpp<kDppRowRor8>(s[i]);
    }
    if constexpr (kSplitKV) {  // V of this tile, now that K's registers are free
      cur.load_v(vb, slot0_of(tt), c16, g);
      if constexpr (decltype(patch)::value) patch_v();
    }
    if (edge) {
#pragma unroll
      for (int i = 0; i < kNs; ++i) s[i] = (okbits >> i) & 1u ? s[i] : -INFINITY;
    }
    float mt = s[0];
#pragma unroll
    for (int i = 1; i < kNs; ++i) mt = fmaxf(mt, s[i]);
    mt = wave_max_groups(mt);
    // Lazy rescaling: the reference maximum m moves only when a tile exceeds it by more than
    // 2^8 somewhere in the wave, so the exponentials stay <= 256 and most tiles skip the O
    // rescale. A NaN or +inf score turns l into NaN (exp2 of NaN or of inf - inf), which the
    // final normalisation reports: no per-score check is needed.
    if (__builtin_amdgcn_ballot_w64(mt > m + 8.0f) != 0) {
      const float mn = fmaxf(m, mt);
      const float alpha = __builtin_amdgcn_exp2f(m - (mn == -INFINITY ? 0.0f : mn));
      m = mn;
      l *= alpha;
#pragma unroll
      for (int n = 0; n < kNv; ++n) acc[n] *= alpha;
    }
    const float mu = m == -INFINITY ? 0.0f : m;
    float p[kNs];
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < kNs; ++i) {
      p[i] = __builtin_amdgcn_exp2f(s[i] - mu);
      psum += p[i];
    }
    l += psum;
    if constexpr (kF16) {
      half8_t phi, plo;
#pragma unroll
      for (int i = 0; i < kNs; ++i) {
        const _Float16 h = (_Float16)p[i];
        phi[i] = h;
        plo[i] = (_Float16)(p[i] - (float)h);
      }
      if constexpr (kP) {
        const half8_t pp = c16 < 8 ? phi : plo;  // column j: hi of head j, 8 + j: its lo
#pragma unroll
        for (int n = 0; n < kNv; ++n)
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(keep_bits(cur.v[n], vkeep), pp, acc[n], 0, 0, 0);
      } else {
#pragma unroll
        for (int n = 0; n < kNv; ++n) {
          const half8_t vn = keep_bits(cur.v[n], vkeep);
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vn, phi, acc[n], 0, 0, 0);
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vn, plo, acc[n], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int n = 0; n < kNv; ++n) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(
              __uint_as_float(__float_as_uint(cur.v[n][e]) & vkeep[e]), p[e], acc[n], 0, 0, 0);
      }
    }
  };

  // Two tile buffers in turn: each is reloaded, kW * 2 tiles ahead, as soon as it is consumed.
  // The new row's tile is the last tile of the wave that owns it; that wave takes it after the
  // loop, where its other buffer is dead, and patches the new row in.
  using no_patch = std::integral_constant<bool, false>;
  using with_patch = std::integral_constant<bool, true>;
  const uint32_t t_stop = patch_wave ? t_new : s_t1;
  if constexpr (kOne && DK < 512) {
    // At most one tile per wave (the launch picks this instance only then).
    if (t < t_stop) step(ta, t, no_patch{});
    if (patch_wave) step(ta, t_new, with_patch{});
  } else if constexpr (kOne) {
    // One tile buffer: a further tile of this wave is loaded once the buffer is consumed.
    for (;;) {
      if (t >= t_stop) break;
      step(ta, t, no_patch{});
      t += kW;
      if (t < s_t1) tile_load(ta, t);
    }
    if (patch_wave) step(ta, t_new, with_patch{});
  } else {
    for (;;) {
      if (t >= t_stop) break;
      step(ta, t, no_patch{});
      if (t + 2 * kW < s_t1) tile_load(ta, t + 2 * kW);
      t += kW;
      if (t >= t_stop) break;
      step(tb, t, no_patch{});
      if (t + 2 * kW < s_t1) tile_load(tb, t + 2 * kW);
      t += kW;
    }
    if (patch_wave) {
      if (((t_new - s_t0 - wave) / kW) % 2 == 0) step(ta, t_new, with_patch{});
      else step(tb, t_new, with_patch{});
    }
  }

  l = wave_sum_groups(l);
  if constexpr (kP) {  // column 8 + j holds the lo halves' share of head j's output
#pragma unroll
    for (int n = 0; n < kNv; ++n)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[n][e] += dpp<kDppRowRor8>(acc[n][e]);
  }
  if constexpr (kQLds) __syncthreads();  // every wave is done with the q rows the combine area overlays

  // Every wave publishes its state; then one thread per (head, element) combines the waves.
  if (head_ok) {
    if (g == 0) {
      s_ml[wave][c16][0] = m;
      s_ml[wave][c16][1] = l;
    }
#pragma unroll
    for (int n = 0; n < kNv; ++n) *(float4_t*)&s_acc[wave][c16][16 * n + 4 * g] = acc[n];
  }
  if (fused && threadIdx.x == 0) s_ticket = ticket;
  __syncthreads();

  const bool reducer = fused && s_ticket == ns - 1;
  if (reducer && threadIdx.x == 0)  // every ticket of this launch is taken: reset for the next
    __hip_atomic_store(&counters[gid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t item0 = item - split;
  float* o_grp = out + ((uint64_t)row * num_heads + kvh * group + hg * 16) * DV + slice * DVS;
  if (reducer) {
    // Sub-threads per quad: at least B / 8 (so a thread takes at most 8 splits), all of the
    // workgroup's threads when the head group has few quads.
    constexpr int kSubMax = kW;  // 64 * kW threads over >= 64 quads
    const bool narrow = nreal * (DVS / 4) * kSubMax <= 64 * kW;
    // One quad per thread covers every quad of the group in one poll round; only the four-wave
    // instances (head dim >= 256, one wave per SIMD) have the registers for all its splits.
    const bool one_round = kW == 4 && nreal * (DVS / 4) <= 64 * kW;
    if (ns <= 8) {
      if (narrow) reduce_group<8, kSubMax, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
      else reduce_group<8, 1, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
    } else if (ns <= 16) {
      if (narrow) reduce_group<16, kSubMax, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
      else if (kW == 4 && one_round) reduce_group<16, kW == 4 ? 1 : 2, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
      else reduce_group<16, 2, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
    } else if (ns <= 24) {  // (a thread's split slots past ns still cost poll issue slots)
      if (narrow) reduce_group<24, kSubMax, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
      else if (kW == 4 && one_round) reduce_group<24, kW == 4 ? 1 : 4, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
      else reduce_group<24, 4, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
    } else {
      if (narrow) reduce_group<32, kSubMax, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
      else if (kW == 4 && one_round) reduce_group<32, kW == 4 ? 1 : 4, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
      else reduce_group<32, 4, DVS, kW, DV>(part_f, item0, ns, split, nreal, s_acc, s_ml, o_grp, err);
    }
    return;
  }
  const __amdgpu_buffer_rsrc_t rs = part_rsrc(part_f);
  for (uint32_t j = threadIdx.x; j < nreal * (DVS / 4); j += 64 * kW) {
    const uint32_t hs = j / (DVS / 4), e = (j % (DVS / 4)) * 4;
    float mx, lw;
    float4_t aw;
    wave_partial<DVS, kW>(s_acc, s_ml, hs, e, mx, lw, aw);
    if (ns == 1) {
      if (!(lw > 0.0f) && e == 0) atomicOr(err, 1);  // all -inf, or a NaN / +inf score
      *(float4_t*)(o_grp + hs * DV + e) = aw * __builtin_amdgcn_rcpf(lw);
    } else if (!fused) {  // reduce_kernel combines the splits after this launch
      // Column slices write their columns into the head group's item; (m, l) are the same in
      // every slice (each forms all of q.K), so slice 0 writes them.
      const uint64_t it = kSlices == 1 ? (uint64_t)item
                                       : sep_item(ns_uniform, item_row0, row, hkv, hgroups, kSlices,
                                                  kvh, hg, ns, split);
      *(float4_t*)(part_acc + sep_acc_float(it, hs, DV, slice * DVS + e)) = aw;
      if (e == 0 && slice == 0) {
        part_ml[sep_ml_float(it, hs)] = mx;
        part_ml[sep_ml_float(it, hs) + 1] = lw;
      }
    } else {
      const uint32_t off = (uint32_t)(fused_part_float(item, hs, DVS, 0) * 4);
      store_part(rs, off + e * 4, float4_t{canon(aw[0]), canon(aw[1]), canon(aw[2]), canon(aw[3])});
      if (e == 0) {
        const float c = __uint_as_float(kClear);
        store_part(rs, off + DVS * 4, float4_t{canon(mx), canon(lw), c, c});
      }
    }
  }
}

// ================================================================ kernel 4: cross-split reduce

// Maximum and sum over the 64 lanes of a wave in VALU lane exchanges (DPP inside rows of 16, then
// the row swaps); every lane ends with the result, formed in the same fixed tree.
__device__ __forceinline__ float wave_max64(float x) {
  x = fmaxf(x, dpp<kDppXor1>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppRowMirror>(x));
  return wave_max_groups(x);
}
__device__ __forceinline__ float wave_sum64(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  x += dpp<kDppHalfMirror>(x);
  x += dpp<kDppRowMirror>(x);
  return wave_sum_groups(x);
}

// One workgroup of kWaves waves per (row, query head, chunk of 4 kQ outputs of the head):
// out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M) over the row's splits, up to kMaxNs
// (at most kMaxWideSplits). With 16 outputs per workgroup: 16 waves for more than 256 splits,
// else 4, or 1 for up to 64, each lane taking at most four splits (four waves taking 16 splits
// per lane with 64 outputs measured slower, 14.1 against 12.2 us per C5 global layer-step).
// With kQ = 16, lane (s, q) of wave w takes output quad q of the chunk for splits
// (kWaves i + w) * 4 + s, so every load instruction moves 16 bytes per lane (four splits'
// 256-byte rows, 1 KB); with kQ = 4, 16 split lanes per wave; thread t loads split t's (m, l);
// all loads are issued before any is used (one memory round trip). The workgroup agrees on M
// through DPP and row-swap exchanges and LDS, takes the weights 2^(m_s - M) from the (m, l) staged
// in LDS, sums each lane's splits in order, then the four split lanes in a fixed tree and the
// waves in wave order: the same result on every run for a plan. The leading scalar arguments
// (the partial buffers, the uniform split count, the head counts) arrive preloaded in SGPRs, so
// the loads need no kernel-argument load first; the row tables are read only for listed rows.
template <int DV, int kWaves, int kQ, int kMaxNs = kMaxWideSplits>
__global__ __launch_bounds__(64 * kWaves) void reduce_kernel(const float* p_acc, const float* p_ml,
                                                             uint32_t p_ns, uint32_t p_heads,
                                                             uint32_t p_group, const DecodeArgs a) {
  static_assert(kQ == 4 || kQ == 16, "quads per workgroup");
  constexpr uint32_t kOut = 4 * kQ;                          // outputs per workgroup
  constexpr uint32_t kChunks = (DV + kOut - 1) / kOut;
  constexpr uint32_t kSL = 64 / kQ;                          // split lanes of a quad per wave
  constexpr int kPer = kMaxNs / (kWaves * kSL);              // splits one lane sums at most
  constexpr uint32_t kMl = kMaxNs / (64 * kWaves);           // (m, l) words one thread loads
  static_assert(kPer >= 1 && kMl >= 1 && kPer * kWaves * kSL == kMaxNs && kMl * 64 * kWaves == kMaxNs,
                "the lanes cover kMaxNs splits exactly");
  __shared__ float2 s_ml[kMaxNs];
  __shared__ float s_m[kWaves], s_l[kWaves];
  __shared__ float4_t s_x[kWaves][kQ];
  JMA_GLOBAL const float* g_acc = (JMA_GLOBAL const float*)p_acc;
  JMA_GLOBAL const float* g_ml = (JMA_GLOBAL const float*)p_ml;
  asm volatile("" : "+s"(g_acc), "+s"(g_ml), "+s"(p_ns), "+s"(p_heads), "+s"(p_group));
  const uint32_t chunk = blockIdx.x % kChunks;
  const uint32_t row = blockIdx.x / kChunks / p_heads;
  const uint32_t head = blockIdx.x / kChunks % p_heads;
  const uint32_t hkv = p_heads / p_group;
  const uint32_t hgroups = (p_group + kHeadSlots - 1) / kHeadSlots;
  const uint32_t ns = p_ns ? p_ns : a.nsplit[row];
  if (ns == 1) return;
  const uint32_t kvh = head / p_group;
  const uint32_t hl = head % p_group;
  const uint32_t hg = hl / 16, c16 = hl % 16;
  // (A sliced plan's row starts count its slices' virtual items: see sep_item.)
  const uint64_t base = group_item0(p_ns, p_ns ? 0u : a.item_start[row] / a.slices, row, hkv,
                                    hgroups, kvh * hgroups + hg, ns);
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint32_t sl = lane / kQ, q = lane % kQ;
  const uint32_t e = chunk * kOut + 4 * q;
  const uint32_t el = e < DV ? e : DV - 4;  // lanes past the head load a valid quad
  // Buffer loads with 32-bit byte offsets (the runtime keeps both buffers under 2 GiB). A split
  // past ns is addressed past the record count, where a buffer load returns zeros: every load is
  // issued unconditionally, with no per-split branch (whose join made the compiler wait for the
  // first loads before issuing the rest, two memory round trips instead of one).
  const __amdgpu_buffer_rsrc_t rs_acc = part_rsrc(const_cast<float*>((const float*)g_acc));
  const __amdgpu_buffer_rsrc_t rs_ml = part_rsrc(const_cast<float*>((const float*)g_ml));
  constexpr uint32_t kSkip = 0xFFFFFF00u;

  float2 ml[kMl];
#pragma unroll
  for (uint32_t i = 0; i < kMl; ++i) {
    const uint32_t sp = tid + 64 * kWaves * i;
    const uint32_t off = sp < ns ? (uint32_t)(sep_ml_float(base + sp, c16) * 4) : kSkip;
    const float2_t v = __builtin_amdgcn_raw_buffer_load_b64(rs_ml, off, 0, 0);
    ml[i] = float2{sp < ns ? v[0] : -INFINITY, v[1]};
  }
  float4_t xv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t sp = (i * kWaves + wave) * kSL + sl;
    const uint32_t off = sp < ns ? (uint32_t)(sep_acc_float(base + sp, c16, DV, el) * 4) : kSkip;
    xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rs_acc, off, 0, 0);
  }
  // The output pointer is not preloaded: its argument load is issued here, behind the partial
  // loads, so that it completes under their latency instead of after the last barrier.
  float* out_p = a.out;
  asm volatile("" : "+s"(out_p));

  float mt = -INFINITY;
#pragma unroll
  for (uint32_t i = 0; i < kMl; ++i) {
    const uint32_t sp = tid + 64 * kWaves * i;
    if (sp < ns) s_ml[sp] = ml[i];
    mt = fmaxf(mt, ml[i].x);
  }
  const float mw = wave_max64(mt);
  if (lane == 0) s_m[wave] = mw;
  __syncthreads();
  float M = s_m[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) M = fmaxf(M, s_m[i]);
  const float mu = M == -INFINITY ? 0.0f : M;
  float lsum = 0.0f;
#pragma unroll
  for (uint32_t i = 0; i < kMl; ++i)
    if (tid + 64 * kWaves * i < ns) lsum = fmaf(ml[i].y, __builtin_amdgcn_exp2f(ml[i].x - mu), lsum);
  const float lw = wave_sum64(lsum);

  float4_t X = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t sp = (i * kWaves + wave) * kSL + sl;
    if (sp < ns) {
      const float w = __builtin_amdgcn_exp2f(s_ml[sp].x - mu);
#pragma unroll
      for (int c = 0; c < 4; ++c) X[c] = fmaf(xv[i][c], w, X[c]);
    }
  }
  // The split lanes of quad q: with 16 quads one lane in each row of 16; with 4 quads four lanes
  // 4 apart in every row, summed by row rotations first.
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if constexpr (kQ == 4) {
      X[c] += dpp<kDppRowRor4>(X[c]);
      X[c] += dpp<kDppRowRor8>(X[c]);
    }
    X[c] = wave_sum_groups(X[c]);
  }
  if (sl == 0) s_x[wave][q] = X;
  if (lane == 0) s_l[wave] = lw;
  __syncthreads();
  if (wave != 0 || sl != 0) return;
  float lt = 0.0f;
  float4_t xt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    lt += s_l[i];
    xt += s_x[i][q];
  }
  if (!(lt > 0.0f) && q == 0 && chunk == 0) atomicOr(a.err, 1);  // all -inf, NaN or +inf
  if (e < DV) *(float4_t*)(out_p + ((uint64_t)row * p_heads + head) * DV + e) = xt * __builtin_amdgcn_rcpf(lt);
}

// Workgroups of 16 outputs when 64-output ones would leave most compute units idle (few rows
// and heads: a long-context layer), else 64.
template <int DV>
static void launch_reduce_t(const DecodeArgs& a, hipStream_t stream) {
  const uint32_t wide_groups = a.rows.count * a.num_heads * ((DV + 63) / 64);
  if (wide_groups < 128 && DV >= 16) {
    const dim3 grid(a.rows.count * a.num_heads * ((DV + 15) / 16));
    // As few waves as cover the splits with four loads per lane: fewer waves to start and to
    // synchronise (one row at 32 704 positions, 256 splits: 22.6 -> 21.8 us per d-512 layer-step).
    if (a.max_splits <= 64)
      hipLaunchKernelGGL((reduce_kernel<DV, 1, 4, 64>), grid, dim3(64), 0, stream, a.part_acc,
                         a.part_ml, a.ns_uniform, a.num_heads, a.group, a);
    else if (a.max_splits <= 256)
      hipLaunchKernelGGL((reduce_kernel<DV, 4, 4, 256>), grid, dim3(256), 0, stream, a.part_acc,
                         a.part_ml, a.ns_uniform, a.num_heads, a.group, a);
    else
      hipLaunchKernelGGL((reduce_kernel<DV, 16, 4>), grid, dim3(1024), 0, stream, a.part_acc, a.part_ml,
                         a.ns_uniform, a.num_heads, a.group, a);
  } else {
    hipLaunchKernelGGL((reduce_kernel<DV, 16, 16>), dim3(wide_groups), dim3(1024), 0, stream, a.part_acc,
                       a.part_ml, a.ns_uniform, a.num_heads, a.group, a);
  }
}

hipError_t launch_reduce(const DecodeArgs& a, int dv, hipStream_t stream) {
  switch (dv) {
    case 16: launch_reduce_t<16>(a, stream); break;
    case 32: launch_reduce_t<32>(a, stream); break;
    case 64: launch_reduce_t<64>(a, stream); break;
    case 128: launch_reduce_t<128>(a, stream); break;
    case 256: launch_reduce_t<256>(a, stream); break;
    case 512: launch_reduce_t<512>(a, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ================================================================ fixed scratch

// The allocation-free decode entry point's scratch: a file-scope device array (each GPU the
// library runs on holds its own copy until the process ends). Host code never uses the array's
// name as an address: fixed_scratch() resolves the device address with hipGetSymbolAddress once
// per device and hands out that pointer.
constexpr size_t kFixedCounterBytes = size_t(64) << 10;
constexpr size_t kFixedPartFBytes = size_t(16) << 20;
constexpr size_t kFixedPartAccBytes = size_t(16) << 20;
constexpr size_t kFixedPartMlBytes = size_t(1) << 20;
constexpr size_t kFixedQrotBytes = size_t(8) << 20;
constexpr size_t kFixedBytes =
    kFixedCounterBytes + kFixedPartFBytes + kFixedPartAccBytes + kFixedPartMlBytes + kFixedQrotBytes;
static __device__ __align__(256) unsigned char scratch[kFixedBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_fixed_mutex;
static FixedScratch g_fixed[kMaxDevices];
static bool g_fixed_ready[kMaxDevices];

__global__ __launch_bounds__(256) void fill_words_kernel(uint32_t* p, uint32_t value, uint64_t words) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += (uint64_t)gridDim.x * 256)
    p[i] = value;
}

static hipError_t fill_words(void* p, uint32_t value, size_t bytes, hipStream_t stream) {
  const uint64_t words = bytes / 4;
  const uint32_t blocks = (uint32_t)std::min<uint64_t>((words + 255) / 256, 2048);
  hipLaunchKernelGGL(fill_words_kernel, dim3(blocks), dim3(256), 0, stream, (uint32_t*)p, value, words);
  return hipGetLastError();
}

hipError_t fixed_scratch_reset(const FixedScratch& s, hipStream_t stream) {
  hipError_t e = fill_words(s.counters, 0u, s.counters_bytes, stream);
  if (e == hipSuccess) e = fill_words(s.part_f, 0xFFFFFFFFu, s.part_f_bytes, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  return e;
}

hipError_t fixed_scratch(int device, hipStream_t stream, FixedScratch* out) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_fixed_mutex);
  if (!g_fixed_ready[device]) {
    unsigned char* base = nullptr;
    hipError_t e = hipGetSymbolAddress((void**)&base, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    FixedScratch s;
    s.counters = (uint32_t*)base;
    s.counters_bytes = kFixedCounterBytes;
    s.part_f = (float*)(base + kFixedCounterBytes);
    s.part_f_bytes = kFixedPartFBytes;
    s.part_acc = (float*)(base + kFixedCounterBytes + kFixedPartFBytes);
    s.part_acc_bytes = kFixedPartAccBytes;
    s.part_ml = (float*)(base + kFixedCounterBytes + kFixedPartFBytes + kFixedPartAccBytes);
    s.part_ml_bytes = kFixedPartMlBytes;
    s.qrot = (float*)(base + kFixedCounterBytes + kFixedPartFBytes + kFixedPartAccBytes + kFixedPartMlBytes);
    s.qrot_bytes = kFixedQrotBytes;
    e = fixed_scratch_reset(s, stream);
    if (e != hipSuccess) return e;
    g_fixed[device] = s;
    g_fixed_ready[device] = true;
  }
  *out = g_fixed[device];
  return hipSuccess;
}


template <typename KV, bool kSimple, bool kNT, bool kPack>
static hipError_t launch_decode_t(const DecodeArgs& a, int d, hipStream_t stream) {
  const dim3 grid(a.max_splits, a.num_kv_heads * a.hgroups, a.rows.count), block(64 * decode_waves(d));
  // Preloaded leading arguments of the kSimple instance (zeros for the general one).
  const void* kb = kSimple ? a.k_base : nullptr;
  const void* vb = kSimple ? a.v_base : nullptr;
  const uint32_t start = kSimple ? a.rows.start : 0u, window = kSimple ? a.window : 0u;
  const uint32_t tps = kSimple ? a.tiles_per_split : 0u, cap = kSimple ? a.kv.cap : 0u;
  const uint32_t ring = kSimple ? a.kv.ring : 0u;
  switch (d) {
    case 16:
      if constexpr (!std::is_same<KV, _Float16>::value) {
        hipLaunchKernelGGL((decode_kernel<KV, 16, 16, 16, kSimple, false, kNT, false>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a);
        break;
      }
      return hipErrorInvalidValue;
    case 32: hipLaunchKernelGGL((decode_kernel<KV, 32, 32, 32, kSimple, false, kNT, false>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a); break;
    case 64: hipLaunchKernelGGL((decode_kernel<KV, 64, 64, 64, kSimple, false, kNT, false>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a); break;
    case 128: hipLaunchKernelGGL((decode_kernel<KV, 128, 128, 128, kSimple, false, kNT, false>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a); break;
    case 256:
      if (a.slices == 4) {  // short rows: four 64-column slices, at most one tile per wave
        hipLaunchKernelGGL((decode_kernel<KV, 256, 256, 64, kSimple, true, kNT, false>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a);
        break;
      }
      // One tile per wave (the long-context plans cut this fine) needs one tile buffer only.
      if (a.tiles_per_split <= (uint32_t)decode_waves(256))
        hipLaunchKernelGGL((decode_kernel<KV, 256, 256, 256, kSimple, true, kNT, false>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a);
      else
        hipLaunchKernelGGL((decode_kernel<KV, 256, 256, 256, kSimple, false, kNT, false>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a);
      break;
    case 512:
      if (a.slices == 4) {  // short rows: four 128-column slices
        hipLaunchKernelGGL((decode_kernel<KV, 512, 512, 128, kSimple, true, kNT, kPack>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a);
        break;
      }
      // One tile buffer always: a tile is the whole register budget of a wave at this width.
      hipLaunchKernelGGL((decode_kernel<KV, 512, 512, 512, kSimple, true, kNT, kPack>), grid, block, 0, stream, kb, vb, start, window, tps, cap, ring, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, bool f16, int dk, int dv, hipStream_t stream) {
  if (!decode_supported(f16, dk, dv)) return hipErrorInvalidValue;
  if (a.total_items == 0) return hipSuccess;
  const bool simple = a.k_base != nullptr;
  if (f16) {
    // Head dim 512 with groups of at most 8 query heads per kv head takes the packed hi / lo
    // columns (measured: 4k context 12.8 -> 12.0 us, 32k 28.6 -> 28.2; at head dims 64 and 256 the
    // extra row rotations cost more than the halved matrix ops save).
    if (a.group <= 8 && dk == 512) {
      if (simple) return launch_decode_t<_Float16, true, false, true>(a, dk, stream);
      return a.stream_nt ? launch_decode_t<_Float16, false, true, true>(a, dk, stream)
                         : launch_decode_t<_Float16, false, false, true>(a, dk, stream);
    }
    if (simple) return launch_decode_t<_Float16, true, false, false>(a, dk, stream);
    return a.stream_nt ? launch_decode_t<_Float16, false, true, false>(a, dk, stream)
                       : launch_decode_t<_Float16, false, false, false>(a, dk, stream);
  }
  return simple ? launch_decode_t<float, true, false, false>(a, dk, stream)
                : launch_decode_t<float, false, false, false>(a, dk, stream);
}

// ================================================================ kernel 3: prefill (f16 MFMA)

// v_mfma_f32_32x32x16_f16 operand layouts, lane l, j = l % 32, h = l / 32:
//   A[i][k]: i = j, k = 8h + e (e < 8)      B[k][c]: c = j, k = 8h + e
//   D[i][c]: c = j, i = 8(e/4) + 4h + e%4 (e < 16)
// Prefill computes S^T = K Q^T. The 32 MFMA columns are (query row, query head) pairs of one kv
// head, so every query head of a GQA group shares each K/V operand; the 32 MFMA rows are the
// slots of a 32-slot kv tile. A-row i reads tile slot swap34(i) (bits 3 and 4 exchanged): then
// the eight scores a lane holds for kv half b are exactly the slots a V^T operand finds at
// positions 16b+8h .. 16b+8h+7 of a perm32-ordered V block, so exponentiated scores feed the PV
// MFMA from registers and each V^T operand is one 16-byte LDS read.
namespace pf {

__device__ __forceinline__ uint32_t swap34(uint32_t i) {
  return (i & ~24u) | ((i & 8u) << 1) | ((i & 16u) >> 1);
}

// 16 bytes per lane from global memory straight into LDS (lane i's at lds + 16 i): a buffer load
// over the rows at `base`, the lane's byte offset in a vector register and the tile's in a scalar
// one. (The descriptor has a constant record count and is made here, at the use: otherwise the
// compiler builds it in vector registers and wraps every load in a uniformity loop.)
__device__ __forceinline__ void dma16(const void* base, _Float16* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFF0, 0x00020000),
      (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// Tile slot of score register e in lane half h.
__device__ __forceinline__ uint32_t score_slot(int e, int h) {
  return 16u * ((e >> 2) & 1) + 8u * (e >> 3) + 4u * h + (e & 3);
}

// XOR swizzles of 16-byte chunks inside the LDS tiles, so that the lanes of one LDS read cycle,
// which read the same chunk column of different rows, hit different banks.
template <int D>
__device__ __forceinline__ uint32_t swz_k(uint32_t r) {
  if constexpr (D >= 128) return (r & 7u) | ((r >> 1) & 8u);
  else if constexpr (D == 64) return r & 7u;
  else return (r >> 1) & 3u;
}
__device__ __forceinline__ uint32_t swz_v(uint32_t r) { return ((r >> 1) ^ (r >> 2)) & 3u; }

// Combine a value across the two lane halves (lanes l and l ^ 32 hold the same column).
__device__ __forceinline__ float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef float float16_t __attribute__((ext_vector_type(16)));

// Calls f(integral_constant<int, i>) for i = 0 .. N-1 (compile-time indices keep register
// arrays in registers).
template <int N, typename F, int I = 0>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, F, I + 1>(static_cast<F&&>(f));
  }
}

// Stripes (32-column query groups) and kv groups of one workgroup per head dimension.
template <int D> struct Shape { static constexpr int S = prefill_stripes(D), Q = kPrefillKvGroups; };

}  // namespace pf

// Finish of one half of a split row block. Each wave holds kCQ finished O^T chunks of its stripe
// (chunks c0 .. c0 + kCQ - 1, unnormalised: weighted by 2^(m_r - M) over the kv groups) and its
// columns' (M, L). a.tickets[pair] counts the halves' stored states. A half that finds the other's
// state stored merges at once; otherwise it stores its words ((M, L) once per stripe, by the
// stripe's wave of kv group 0; device-coherent, acknowledged) and takes a ticket, and the one that
// then finds the count at 1 merges: exactly one half merges, with no wait, and resets the ticket.
// The merge combines the halves in half order, (O0 e0 + O1 e1) / (L0 e0 + L1 e1) with
// e_h = 2^(M_h - max), so the result does not depend on which half merges. Every wave of the
// workgroup calls this (the decisions are uniform).
template <int D, int S, int kWaves, int kCQ>
__device__ __forceinline__ void split_exchange(const PrefillArgs& a, uint32_t pair, uint32_t half,
                                               int s, uint32_t c0, bool post_ml, int lane, int j, int h,
                                               bool col_ok, uint32_t crow, uint32_t head, float m,
                                               float l, const float4_t (&v)[kCQ]) {
  constexpr int kC = D / 8;  // float4 chunks of O^T per lane and stripe
  const __amdgpu_buffer_rsrc_t rs = part_rsrc(a.part);
  auto base = [&](uint32_t hf) JMA_INL {
    return (uint32_t)((((uint64_t)pair * 2 + hf) * S + s) * (kC * 64 + 32) * 16);
  };
  __shared__ uint32_t s_tk;
  if (threadIdx.x == 0) s_tk = __hip_atomic_load(&a.tickets[pair], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_tk == 0u) {
    const uint32_t b = base(half);
#pragma unroll
    for (int i = 0; i < kCQ; ++i) store_part(rs, b + ((c0 + i) * 64 + lane) * 16, v[i]);
    if (post_ml && h == 0) store_part(rs, b + (kC * 64 + j) * 16, float4_t{m, l, 0.0f, 0.0f});
    // The stores are acknowledged (visible device-wide) before the ticket is taken.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      s_tk = __hip_atomic_fetch_add(&a.tickets[pair], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_tk == 0u) return;  // the other half merges
  }
  if (threadIdx.x == 0) __hip_atomic_store(&a.tickets[pair], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t ob = base(1 - half);
  float4_t x[kCQ];
#pragma unroll
  for (int i = 0; i < kCQ; ++i) x[i] = load_part(rs, ob + ((c0 + i) * 64 + lane) * 16);
  const float4_t mlv = load_part(rs, ob + (kC * 64 + j) * 16);
  const float m0 = half == 0 ? m : mlv[0], l0 = half == 0 ? l : mlv[1];
  const float m1 = half == 0 ? mlv[0] : m, l1 = half == 0 ? mlv[1] : l;
  const float M = fmaxf(m0, m1);
  const float e0 = m0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0 - M);
  const float e1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
  const float L = fmaf(l1, e1, l0 * e0);
  if (__ballot(col_ok && !(L > 0.0f && L < INFINITY)) != 0 && lane == 0) atomicOr(a.err, 1);
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  float* const orow = a.out + ((uint64_t)crow * a.num_heads + head) * D + 4 * h;
#pragma unroll
  for (int i = 0; i < kCQ; ++i) {
    const uint32_t c = c0 + i;
    const float4_t v0 = half == 0 ? v[i] : x[i], v1 = half == 0 ? x[i] : v[i];
    float4_t r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = fmaf(v1[e], e1, v0[e] * e0) * inv;
    if (col_ok) *(float4_t*)(orow + 32 * (c >> 2) + 8 * (c & 3)) = r;
  }
}

// Workgroup = (kv head, head group, block of S stripes). A stripe is R query rows x Gz query heads
// = 32 MFMA columns (R * Gz <= 32). Wave (s, q) owns stripe s and the kv tiles t0+q, t0+q+Q, ...
// of the block's causal range: the Q waves of a stripe split its kv range, and the S waves of a kv
// group share every K/V tile, which direct-to-LDS loads stage ahead of use.
//
// Each wave runs a two-tile software pipeline: step k computes the scores of tile k+1 on the
// matrix cores while the vector units exponentiate tile k, then accumulates tile k's PV while the
// maximum of tile k+1 is taken. K and V stream one tile apart (K(k+1) and V(k) are read in step k,
// K(k+2) and V(k+1) are loaded), so two LDS stages hold everything and one barrier per step
// separates reuse from loads.
//
// Softmax keeps a per-column reference maximum m and rescales the accumulators only when a tile
// maximum exceeds it by more than 8 (log2 units), so exponentials stay <= 256 and most steps skip
// the rescale; the final normalisation divides by the sum of the same (f16-rounded) exponentials,
// so the result is the softmax of the reference up to f16 rounding of q, k, v and p.
// Up to D = 128 the kernel fits 256 registers per lane (two waves per SIMD), which also keeps
// the matrix-op results in ordinary vector registers (no accumulation-register copies per tile).
template <int D>
__global__ __launch_bounds__(64 * pf::Shape<D>::S * pf::Shape<D>::Q)
__attribute__((amdgpu_waves_per_eu(D >= 256 ? 1 : 2))) void prefill_kernel(const PrefillArgs a) {
  using namespace pf;
  constexpr int S = Shape<D>::S, Q = Shape<D>::Q;
  constexpr int kWaves = S * Q;
  constexpr int kKS = D / 16;                    // k-steps of QK^T
  constexpr int kNb = D / 32;                    // 32-row dv blocks of O^T
  constexpr int kT = 32 * D;                     // halves of one K tile (or one V^T tile)
  constexpr int kChunks = D / 16;                // 1 KB chunks per K (or V) tile
  constexpr int kCPW = (kChunks + S - 1) / S;    // chunks of a tile one wave of its group loads
  constexpr int kNC = D / 8;                     // 16-byte chunks per K row
  constexpr int kC = 4 * kNb;                    // float4 chunks of O^T held per lane
  static_assert(Q == 1 || Q == 2 || Q == 4, "kv groups per stripe");
  // T tiles per barrier. An LDS array holds, for each kv group, T consecutive K tiles and T V
  // tiles. Two arrays alternate: barrier-step m reads array (m + 1) mod 2 — K tiles Tm+1 .. Tm+T
  // and V tiles Tm .. Tm+T-1, so step k = Tm + j reads K(k+1) and V(k) from sub-slot j — while
  // step k loads K(k+T+1) and V(k+T) into sub-slot j of array m mod 2. As distinct variables,
  // the compiler sees that the loads in flight do not alias the reads and adds no waits for them.
  // Two tiles per barrier halve the per-barrier costs (the wait for the slowest wave, the first
  // LDS read after it); at d = 256 two arrays of one tile already take 128 KB.
  constexpr int T = D >= 256 ? 1 : 2;
  constexpr int kArr = 2 * T * Q * kT;           // halves per LDS array
  __shared__ __attribute__((aligned(16))) _Float16 lx[kArr];
  __shared__ __attribute__((aligned(16))) _Float16 ly[kArr];
  __shared__ float2 s_ml[kWaves][32];

  // Kv heads vary fastest: consecutive workgroups land on different XCDs, so each XCD's L2 keeps
  // the K/V of few kv heads. Row blocks run last-first (longest causal ranges first); the
  // split_blocks longest come first as two halves each.
  const uint32_t n_split_items = 2 * a.split_blocks * a.head_groups * a.num_kv_heads;
  const bool split = blockIdx.x < n_split_items;
  const uint32_t b_item = split ? blockIdx.x : blockIdx.x - n_split_items;
  const uint32_t kvh = b_item % a.num_kv_heads;
  const uint32_t rest = b_item / a.num_kv_heads;
  const uint32_t hz = rest % a.head_groups;
  const uint32_t half = split ? (rest / a.head_groups) % 2 : 0u;
  const uint32_t rank = split ? rest / a.head_groups / 2 : a.split_blocks + rest / a.head_groups;
  const uint32_t rb = a.row_blocks - 1 - rank;
  const uint32_t pair = (rank * a.head_groups + hz) * a.num_kv_heads + kvh;
  __shared__ uint32_t s_rerun;  // set when the block needs the robust pass
  if (threadIdx.x == 0) s_rerun = 0u;
  const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int s = wave % S, q = wave / S;
  const uint32_t R = a.rows_per_stripe, Gz = a.heads_per_stripe;

  const uint32_t b_row0 = rb * S * R;
  const uint32_t b_row1 = min(b_row0 + S * R, a.n) - 1;
  const uint32_t row0 = b_row0 + s * R;
  const bool stripe_ok = row0 < a.n;
  const uint32_t row_last = min(row0 + R - 1, a.n - 1);

  // This lane's column; padding columns alias a valid row and head and are never stored.
  const uint32_t cr = min((uint32_t)j / Gz, R - 1);
  const uint32_t hz_head = hz * Gz + (uint32_t)j % Gz;
  const bool col_ok = stripe_ok && (uint32_t)j < R * Gz && row0 + cr < a.n && hz_head < a.group;
  const uint32_t crow = min(row0 + cr, a.n - 1);
  const uint32_t head = kvh * a.group + min(hz_head, a.group - 1);
  const uint32_t cpos = a.start + crow;
  const uint32_t cfirst = first_visible(cpos, a.window);

  // Kv tiles of the block (of its half, for a split block), and the part of them this wave's
  // stripe sees.
  const uint32_t bt0 = first_visible(a.start + b_row0, a.window) / 32;
  const uint32_t bt1 = (a.start + b_row1) / 32 + 1;
  // The first half is a little shorter (split_range), so it usually stores its state while the
  // second still computes, and the second merges without storing its own.
  SplitItem si;
  si.split = split;
  si.half = half;
  si.unit = rb;
  uint32_t t0, t1;
  split_range(bt0, bt1, si, t0, t1);
  const uint32_t steps = (t1 - t0 + Q - 1) / Q;
  const uint32_t w_last = a.start + row_last;
  const uint32_t w_first_early = first_visible(a.start + row0, a.window);
  const uint32_t w_first_late = first_visible(w_last, a.window);

  const _Float16* kbase = (const _Float16*)a.kv.k + a.seq * a.kv.seq_stride_k + a.kv.layer_off_k +
                          (uint64_t)kvh * a.kv.cap * D;
  const _Float16* vbase = (const _Float16*)a.kv.v + a.seq * a.kv.seq_stride_v + a.kv.layer_off_v +
                          (uint64_t)kvh * a.kv.cap * D;
  // Byte offsets inside a tile of the 16 bytes this lane stages per chunk. A direct-to-LDS load
  // writes lane i's 16 bytes at chunk base + 16 i, so the LDS swizzle is applied on the global side.
  uint32_t koff[kCPW], voff[kCPW];
#pragma unroll
  for (int i = 0; i < kCPW; ++i) {
    const uint32_t c = s + S * i;
    const uint32_t rk = c * (512 / D) + lane / kNC;
    // 16-byte chunk cc of tile row rk sits in column panel cc / 4 of the tile (k_index).
    const uint32_t cc = (lane % kNC) ^ swz_k<D>(rk);
    koff[i] = 2 * ((cc / 4) * (32 * 32) + rk * 32 + 8 * (cc % 4));
    const uint32_t rv = c * 16 + lane / 4;
    voff[i] = 2 * (rv * 32 + 8 * ((lane % 4) ^ swz_v(rv)));
  }
  // Whether every column of the stripe sees all of step k's tile (no mask needed). A tile at or
  // past t1 (the last step of a kv group, or the other half's range of a split block) is masked.
  auto full = [&](uint32_t k) JMA_INL {
    const uint32_t p0 = 32 * (t0 + k * Q + q);
    return p0 + 31 <= a.start + row0 && p0 >= w_first_late && p0 < 32 * t1;
  };
  // Byte offset (in the kv head's rows) of step k's tile. A step past the group's last tile loads
  // that tile again (its scores are masked), and a group without tiles loads slot 0, so every
  // wave issues the same number of loads each step. Positions of a non-ring cache are below its
  // capacity, and a ring holds the whole visible range, so one conditional subtraction wraps.
  const bool g_has = t0 + q < t1;
  const uint32_t g_last = g_has ? (t1 - 1 - t0 - q) / Q : 0u;
  const uint32_t cap_bytes = a.kv.cap * (2 * D);
  const uint32_t base_bytes = g_has ? ((32 * (t0 + q)) % a.kv.cap) * (2 * D) : 0u;
  auto tile_off = [&](uint32_t k) JMA_INL {
    const uint32_t x = base_bytes + min(k, g_last) * (32 * Q * 2 * D);
    return x >= cap_bytes ? x - cap_bytes : x;
  };
  // Where sub-slot j of this wave's kv group sits in an LDS array, for K and for V.
  auto k_slot = [&](_Float16* arr, int j) JMA_INL { return arr + (j * Q + q) * kT; };
  auto v_slot = [&](_Float16* arr, int j) JMA_INL { return arr + T * Q * kT + (j * Q + q) * kT; };
  // This wave's chunk i of step k's K tile or V tile into sub-slot j of LDS array `arr`.
  auto dma_k = [&](uint32_t k, _Float16* arr, int j, int i) JMA_INL {
    const uint32_t c = s + S * i;
    if (c >= (uint32_t)kChunks) return;
    pf::dma16(kbase, k_slot(arr, j) + 512 * c, koff[i], tile_off(k));
  };
  auto dma_v = [&](uint32_t k, _Float16* arr, int j, int i) JMA_INL {
    const uint32_t c = s + S * i;
    if (c >= (uint32_t)kChunks) return;
    pf::dma16(vbase, v_slot(arr, j) + 512 * c, voff[i], tile_off(k));
  };
  auto arr_of = [&](auto idx) JMA_INL -> _Float16* {
    return decltype(idx)::value % 2 == 0 ? lx : ly;
  };
  // Waits until at most `outstanding` of this wave's loads are in flight, then barrier. (The
  // barrier is bare: __syncthreads() would also wait for the loads still meant to be in flight.)
  auto wait_barrier = [](auto outstanding) JMA_INL {
    constexpr int n = decltype(outstanding)::value;
    __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  // The first K tile goes out (to sub-slot 0 of array 0) before the Q loads, so the two latencies
  // overlap. A group without tiles loads slot 0 like its later steps: every K stage holds cache
  // data, never stale LDS contents.
#pragma unroll
  for (int i = 0; i < kCPW; ++i) dma_k(0, lx, 0, i);

  // Q^T operands: 8 consecutive dims of this lane's column per k-step, scaled by
  // scale * log2(e) and rounded to f16. A scaled element beyond the f16 range (where the
  // reference's f32 scores stay finite) or infinite is reported like a non-finite score; a NaN
  // element makes its column's scores NaN, which the final normalisation reports.
  half8_t qf[kKS];
  {
    const float* qrow = a.q + ((uint64_t)crow * a.num_heads + head) * D + 8 * h;
    const float qs = col_ok ? a.qscale : 0.0f;
    float qmax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      const float4_t x0 = *(const float4_t*)(qrow + 16 * ks);
      const float4_t x1 = *(const float4_t*)(qrow + 16 * ks + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qmax = fmaxf(qmax, fmaxf(fabsf(x0[e] * qs), fabsf(x1[e] * qs)));
        qf[ks][e] = (_Float16)(x0[e] * qs);
        qf[ks][4 + e] = (_Float16)(x1[e] * qs);
      }
    }
    if (__ballot(col_ok && !(qmax < 65520.0f)) != 0 && lane == 0) atomicOr(a.err, 1);
  }

  // Softmax state, set up by each pass: l accumulates in two chains (l, lb), summed at the end;
  // negm holds -m (0 while m is -inf) in every element: the initial accumulators of each score
  // tile.
  float16_t o[kNb];
  float m, l, lb;
  float16_t negm;
  const uint32_t kr = swap34(j);

  // LDS reads are issued in batches of up to 4 ahead of the matrix ops that consume them: with
  // eight waves and the direct-to-LDS traffic sharing the LDS, one read's latency is several
  // hundred cycles, and a read-use-read chain would serialise on it. (Batches of 8 measured ~1%
  // slower on C3.)
  constexpr int kBatch = kKS < 4 ? kKS : 4;
  // Two passes share the code below. The fast pass masks a partly visible tile through the
  // accumulators its first QK^T op starts from: kMaskFloor (-2^100) at the positions a column
  // does not see (outside [first, position], or past t1), so no score is masked after the matrix
  // ops and masked and unmasked tiles share all the code after the first op. Any score the ops
  // add stays below half the floor (its exponential is 0, and a column maximum under half the
  // floor reads as -inf) as long as the keys there are finite. The cache may hold anything at
  // positions a row does not see (a discarded tail, an old ring slot, a value that overflowed
  // f16), and there an infinite key or value turns the column's state non-finite (-2^100 + inf,
  // 0 * inf). A workgroup whose valid columns end the fast pass with a non-finite state runs its
  // block again in the robust pass, which masks scores after the products (select) and zeroes
  // the value operands at positions no column of the wave sees, so those positions never reach
  // a result, as in the reference; a state still non-finite then is the reference's too.
  constexpr float kMaskFloor = -0x1p100f;
  auto masked_init = [&](uint32_t k) JMA_INL {
    const uint32_t p0 = 32 * (t0 + k * Q + q), pend = 32 * t1;
    float16_t mi;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t p = p0 + score_slot(e, h);
      mi[e] = p >= cfirst && p <= cpos && p < pend ? negm[e] : kMaskFloor;
    }
    return mi;
  };
  // S^T of tile k minus the reference maximum of each column (the accumulators start at -m, or
  // at 0 before the first tile): the tile's exponentials need no subtraction. `issue(i)` runs
  // after the i-th matrix op, to spread loads between them.
  auto qk = [&](const _Float16* sk, uint32_t k, auto robust, auto issue) JMA_INL {
    const bool masked = !decltype(robust)::value && !full(k);
    float16_t mi;
    if (masked) mi = masked_init(k);
    float16_t sc;
#pragma unroll
    for (int ks0 = 0; ks0 < kKS; ks0 += kBatch) {
      half8_t kf[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int ks = ks0 + i;
        kf[i] = *(const half8_t*)(sk + kr * D + 8 * ((2 * ks + h) ^ swz_k<D>(kr)));
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (ks0 + i == 0) {
          if (masked) sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i], qf[0], mi, 0, 0, 0);
          else sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i], qf[0], negm, 0, 0, 0);
        } else {
          sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i], qf[ks0 + i], sc, 0, 0, 0);
        }
        issue(ks0 + i);
      }
    }
    return sc;
  };
  // The per-column maximum of tile k's (shifted) scores, -inf when the column sees none of them.
  // The robust pass masks the scores here (positions outside [first, position] of each column,
  // or past t1, become -inf).
  auto tile_max = [&](float16_t& sc, uint32_t k, auto robust) JMA_INL {
    float tmax = -INFINITY;
    if constexpr (decltype(robust)::value) {
      if (full(k)) {
#pragma unroll
        for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sc[e]);
      } else {
        const uint32_t p0 = 32 * (t0 + k * Q + q), pend = 32 * t1;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t p = p0 + score_slot(e, h);
          const bool ok = p >= cfirst && p <= cpos && p < pend;
          sc[e] = ok ? sc[e] : -INFINITY;
          tmax = fmaxf(tmax, sc[e]);
        }
      }
      return half_max(tmax);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sc[e]);
      tmax = half_max(tmax);
      return tmax < 0.5f * kMaskFloor ? -INFINITY : tmax;
    }
  };
  // Raises the reference maximum when the tile's maximum exceeds it by more than 8 (tmax is the
  // shifted tile's maximum, so the test is tmax > 8; any tile that has a visible score raises it
  // from -inf), and shifts the tile to the new maximum.
  auto rescale = [&](float16_t& sc, float tmax) JMA_INL {
    const bool up = m == -INFINITY ? tmax > -INFINITY : tmax > 8.0f;
    if (__ballot(up) != 0) {
      const float alpha = !up ? 1.0f : (m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(-tmax));
      const float delta = up ? tmax : 0.0f;
      m = up ? (m == -INFINITY ? 0.0f : m) + tmax : m;
#pragma unroll
      for (int e = 0; e < 16; ++e) negm[e] = m == -INFINITY ? 0.0f : -m;
      l *= alpha;
      lb *= alpha;
#pragma unroll
      for (int nb = 0; nb < kNb; ++nb) o[nb] *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] -= delta;
    }
  };
  // Exponentials of a shifted tile, rounded to f16 for the PV product; l sums the rounded values
  // (dot products with (1, 1), f32 accumulation).
  auto exp_tile = [&](const float16_t& sc, half8_t* pf) JMA_INL {
#pragma unroll
    for (int e = 0; e < 16; ++e) pf[e >> 3][e & 7] = (_Float16)__builtin_amdgcn_exp2f(sc[e]);
    const half2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const half2_t pr = {pf[i >> 2][2 * (i & 3)], pf[i >> 2][2 * (i & 3) + 1]};
      if (i & 1) lb = __builtin_amdgcn_fdot2(pr, one, lb, false);
      else l = __builtin_amdgcn_fdot2(pr, one, l, false);
    }
  };
  // O^T += V^T P for tile k. Element t of operand b holds the key of score register 8b + t (the
  // f16 V blocks are stored in that order); the robust pass zeroes the elements at positions no
  // column of this wave sees.
  auto pv = [&](const _Float16* sv, const half8_t* pf, uint32_t k, auto robust) JMA_INL {
    constexpr int kNbB = kBatch / 2;  // dv blocks per batch of reads
    bool keep[2][8];
    if constexpr (decltype(robust)::value) {
      const uint32_t p0 = 32 * (t0 + k * Q + q);
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const uint32_t p = p0 + score_slot(8 * b + t, h);
          keep[b][t] = p >= w_first_early && p <= w_last;
        }
    }
#pragma unroll
    for (int nb0 = 0; nb0 < kNb; nb0 += kNbB) {
      half8_t vf[kNbB][2];
#pragma unroll
      for (int i = 0; i < kNbB; ++i)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const uint32_t vr = 32 * (nb0 + i) + j;
          vf[i][b] = *(const half8_t*)(sv + vr * 32 + 8 * ((2 * b + h) ^ swz_v(vr)));
          if constexpr (decltype(robust)::value) {
#pragma unroll
            for (int t = 0; t < 8; ++t) vf[i][b][t] = keep[b][t] ? vf[i][b][t] : (_Float16)0.0f;
          }
        }
#pragma unroll
      for (int i = 0; i < kNbB; ++i)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          o[nb0 + i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[i][b], pf[b], o[nb0 + i], 0, 0, 0);
    }
  };
  auto no_issue = [](int) JMA_INL {};
  // At D = 256 the accumulators leave no registers for two live score tiles: tile k is finished
  // before tile k+1's scores are computed.
  constexpr bool kOverlap = D <= 128;

  // One pass over the block's tiles (K(0) already on its way to sub-slot 0 of array 0).
  auto run = [&](auto robust) JMA_INL {
#pragma unroll
  for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[nb][e] = 0.0f;
  m = -INFINITY;
  l = 0.0f;
  lb = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) negm[e] = 0.0f;
  // V stages start zeroed: a step whose tile this wave does not see still runs its PV product,
  // with p = 0, and 0 * (anything the stage held) must be 0. Only cache data or zeros ever reach
  // a V stage.
  for (int i = threadIdx.x; i < T * Q * kT / 8; i += 64 * kWaves) {
    *(half8_t*)(lx + T * Q * kT + 8 * i) = half8_t{};
    *(half8_t*)(ly + T * Q * kT + 8 * i) = half8_t{};
  }
  // Prologue: K(0) ready; the loads for barrier-step 0 go out (K(1) .. K(T) and V(0) .. V(T-1)
  // into array 1); scores of step 0 (masked, maximum taken, accumulators scaled for it).
  wait_barrier(std::integral_constant<int, 0>{});
  static_for<T>([&](auto jj) JMA_INL {
    constexpr int jv = decltype(jj)::value;
#pragma unroll
    for (int i = 0; i < kCPW; ++i) {
      dma_k(jv + 1, ly, jv, i);
      dma_v(jv, ly, jv, i);
    }
  });
  // Score tiles alternate between two register sets (even steps finish sa and compute sb). A
  // tile this wave does not see at all, or one that does not exist, is masked completely.
  float16_t sa = qk(k_slot(lx, 0), 0, robust, no_issue), sb;
  rescale(sa, tile_max(sa, 0, robust));

  // Step k (P = k mod 2T, fixed per unrolled copy; sub-step j = P mod T of barrier-step m, whose
  // parity is P / T): after the barrier that opens the barrier-step, K(k+1) and V(k) are ready
  // in array (m + 1) mod 2; K(k+T+1) and V(k+T) are loaded into array m mod 2. Every step runs
  // the same code; only the masking of partly visible tiles and the occasional rescale branch.
  auto step = [&](uint32_t k, auto kp) JMA_INL {
    constexpr int P = decltype(kp)::value;
    constexpr int j = P % T;
    float16_t& scur = P % 2 == 0 ? sa : sb;
    float16_t& snxt = P % 2 == 0 ? sb : sa;
    if constexpr (j == 0) wait_barrier(std::integral_constant<int, 0>{});
    _Float16* const dst = arr_of(std::integral_constant<int, P / T>{});
    _Float16* const src = arr_of(std::integral_constant<int, P / T + 1>{});
    const _Float16* const ksrc = k_slot(src, j);
    const _Float16* const vsrc = v_slot(src, j);
    half8_t pf[2];
    auto spread = [&](int ks) JMA_INL {
      constexpr int kEvery = kKS / kCPW;
      if (ks % kEvery == 0) {
        dma_k(k + T + 1, dst, j, ks / kEvery);
        dma_v(k + T, dst, j, ks / kEvery);
      }
    };
    if constexpr (kOverlap) {
      // QK^T of tile k+1 overlaps the exponentials of tile k.
      snxt = qk(ksrc, k + 1, robust, spread);
      exp_tile(scur, pf);
      pv(vsrc, pf, k, robust);
      // Order: all K and V^T operand reads, then the QK^T matrix ops each followed by a share of
      // the exponentials, then the PV matrix ops.
      __builtin_amdgcn_sched_group_barrier(0x100, kKS + 2 * kNb, 0);
      static_for<kKS>([&](auto) JMA_INL {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
      });
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * kNb, 0);
    } else {
      exp_tile(scur, pf);
      pv(vsrc, pf, k, robust);
      snxt = qk(ksrc, k + 1, robust, spread);
    }
    rescale(snxt, tile_max(snxt, k + 1, robust));
  };
  // (The last copies are guarded inside the loop: remainder copies after it would double the
  // code the register allocator spans and spill.)
  for (uint32_t k = 0; k < steps; k += 2 * T)
    static_for<2 * T>([&](auto pp) JMA_INL {
      if (k + decltype(pp)::value < steps) step(k + decltype(pp)::value, pp);
    });
  };

  run(std::false_type{});
  {
    // A valid column whose state is not finite (NaN or +inf in l, m or the accumulators) asks
    // for the robust pass.
    float osum = 0.0f;
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) osum += o[nb][e];
    const bool bad = col_ok && !(l + lb < INFINITY && m < INFINITY && fabsf(osum) < INFINITY);
    if (__ballot(bad) != 0 && lane == 0) s_rerun = 1u;
  }
  // Every wave's operand reads and tile loads (the last steps still load clamped tiles) are
  // complete before a second pass or the exchange below overwrites the tile stages, since waves
  // leave the loop up to a step apart.
  wait_barrier(std::integral_constant<int, 0>{});
  if (s_rerun != 0u) {
#pragma unroll
    for (int i = 0; i < kCPW; ++i) dma_k(0, lx, 0, i);
    run(std::true_type{});
    wait_barrier(std::integral_constant<int, 0>{});
  }

  // Merge the kv-group partials of each stripe in one LDS exchange: wave q of a stripe finishes
  // the q-th of its O^T chunks. Every wave posts (m, l) and, for each other kv group r, the
  // chunks wave r finishes; then it combines its own chunks (from registers) with the Q - 1
  // posted ones, in kv-group order, weighted by exp2(m_r - M) / L.
  l = half_sum(l + lb);
  constexpr int kCQ = kC / Q;  // chunks one wave finishes
  // Posted chunks of stripe s: [source group][destination slot][kCQ][64 lanes] float4, in lx for
  // even stripes and ly for odd ones (each holds Q * (Q - 1) * kCQ KB <= one LDS array).
  static_assert(Q * (Q - 1) * kCQ * 1024 <= kArr * 2 || Q == 1, "merge exchange exceeds an LDS array");
  float* const xbase = (float*)((s & 1) ? ly : lx) + (s >> 1) * Q * (Q - 1) * kCQ * 256;
  auto xslot = [&](int src, int dst) JMA_INL {  // where src posts the chunks dst finishes
    return xbase + (src * (Q - 1) + (dst < src ? dst : dst - 1)) * kCQ * 256;
  };
  // O^T chunk c (c < kC) of this lane: dims 32(c/4) + 8(c%4) + 4h .. +3 of its column. The part a
  // wave posts or finishes is chosen by a wave-uniform branch so that o[] is indexed statically.
  auto chunk = [&](auto cc) JMA_INL {
    constexpr int c = decltype(cc)::value;
    const float16_t& acc = o[c >> 2];
    return float4_t{acc[4 * (c & 3)], acc[4 * (c & 3) + 1], acc[4 * (c & 3) + 2],
                    acc[4 * (c & 3) + 3]};
  };
  if constexpr (Q > 1) {
    if (h == 0) s_ml[wave][j] = float2{m, l};
    static_for<Q>([&](auto rr) JMA_INL {
      constexpr int r = decltype(rr)::value;
      if (r != q) {
        float* const dst = xslot(q, r);
        static_for<kCQ>([&](auto idx) JMA_INL {
          *(float4_t*)(dst + idx.value * 256 + 4 * lane) =
              chunk(std::integral_constant<int, r * kCQ + decltype(idx)::value>{});
        });
      }
    });
  }
  __syncthreads();
  // Weights of the kv groups of this lane's column: 2^(m_r - M), divided by L unless the block is
  // split (the halves are normalised together).
  float wr[Q];
  float M = m, L = l;
  if constexpr (Q > 1) {
    float mr[Q], lr[Q];
    M = -INFINITY;
#pragma unroll
    for (int r = 0; r < Q; ++r) {
      const float2 v = r == q ? float2{m, l} : s_ml[r * S + s][j];
      mr[r] = v.x;
      lr[r] = v.y;
      M = fmaxf(M, v.x);
    }
    L = 0.0f;
#pragma unroll
    for (int r = 0; r < Q; ++r) {
      wr[r] = mr[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mr[r] - M);
      L = fmaf(lr[r], wr[r], L);
    }
  } else {
    wr[0] = 1.0f;
  }
  if (!split) {
    const bool bad = col_ok && !(L > 0.0f && L < INFINITY);
    if (__ballot(bad) != 0 && lane == 0) atomicOr(a.err, 1);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int r = 0; r < Q; ++r) wr[r] *= inv;
  }
  float4_t fin[kCQ];  // this wave's finished chunks q * kCQ ..
  static_for<Q>([&](auto qq) JMA_INL {
    constexpr int own = decltype(qq)::value;
    if (own == q) {
      static_for<kCQ>([&](auto idx) JMA_INL {
        constexpr int c = own * kCQ + decltype(idx)::value;
        float4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < Q; ++r) {
          const float4_t x = r == own ? chunk(std::integral_constant<int, c>{})
                                      : *(const float4_t*)(xslot(r, own) + idx.value * 256 + 4 * lane);
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = fmaf(x[i], wr[r], v[i]);
        }
        fin[idx.value] = v;
      });
    }
  });
  if (split) {
    split_exchange<D, S, kWaves, kCQ>(a, pair, half, s, (uint32_t)q * kCQ, q == 0, lane, j, h,
                                      col_ok, crow, head, M, L, fin);
    return;
  }
  float* const orow = a.out + ((uint64_t)crow * a.num_heads + head) * D + 4 * h;
#pragma unroll
  for (int i = 0; i < kCQ; ++i) {
    const uint32_t c = (uint32_t)q * kCQ + i;
    if (col_ok) *(float4_t*)(orow + 32 * (c >> 2) + 8 * (c & 3)) = fin[i];
  }
}

// ================================================================ kernel 3b: d-sliced prefill

// Causal / sliding-window prefill for f32 caches (head dims 32..512, on the f32 matrix ops, so
// scores and weighted sums keep f32 products as the reference's do). A workgroup is one stripe
// of 32 (query row, query head) columns of one kv head, as in the f16 kernel, and its W waves cut the head dimension into W slices of DS = D / W: wave w forms the
// partial scores of each kv tile over its DS dims of q and K, the waves add their partial tiles
// through LDS in wave order (so every wave holds the same scores, bit for bit), each runs the
// same online softmax, and wave w accumulates output dims w*DS .. (w+1)*DS - 1 from the same
// dims of V. Registers scale with DS instead of D, and no wave repeats another's matrix work.
// Tiles are read from the cache (L2-resident after the first stripe of a kv head) straight into
// registers, one tile ahead of the one being computed.
//
// Operands (32x32 results: lane (j, h) holds column j, rows 8(e/4) + 4h + e%4 of element e):
//  f32, v_mfma_f32_32x32x2_f32 (A[i][k]: i = j, k = h; B[k][c]: c = j, k = h): S^T = K Q^T with
//    result row i = tile slot i. Lane (j, h) loads K[slot j][8m + 4h .. +3] and q[col j][8m + 4h
//    .. +3] as float4s and gives element t of both to op (m, t), which so adds dims 8m + t and
//    8m + 4 + t. PV: op u (u < 16) takes the lane's own probability u (slot 8(u/4) + 4h + u%4)
//    as its B operand and V^T at the same slots as A, four consecutive slots per float4 load of
//    an f32 V block.
// A split stripe (kernel 3b) or stripe pair (kernel 3c) runs as two workgroups, one per half of
// its kv tiles. Each ends with an online-softmax state per lane of each of its W waves (O^T,
// m, l, lb), kept at [sidx][half][wave][4 kNb + 1 float4 words][64 lanes] in a.part, and
// a.tickets[sidx] counts the states stored. A half that finds the other's state stored merges at
// once (its own never leaves the registers); otherwise it stores its state (device-coherent,
// acknowledged) and takes a ticket, and the one that then finds the count at 1 merges: exactly one
// half merges either way, and it resets the ticket. The merge forms each half's rounded terms
// o 2^(m_h - M) (no fused multiply-add) and adds them, which commutes, so the result does not
// depend on which half merges. Returns whether this workgroup merged (o, m, l, lb then hold the
// pair's state); the other returns false and stores nothing more.
template <int W, int kNb>
__device__ __forceinline__ bool merge_halves(const PrefillArgs& a, uint32_t sidx, uint32_t half, int w,
                                             int lane, pf::float16_t (&o)[kNb], float& m, float& l, float& lb) {
  constexpr uint32_t kWords = 4u * kNb + 1u;
  // The descriptor's record count is the launch's state bytes (the host keeps them < 2 GiB).
  const uint32_t state_bytes = a.split_blocks * a.head_groups * a.num_kv_heads * 2u * W * kWords * 64u * 16u;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(a.part, 0, state_bytes, 0x00020000);
  auto word = [&](uint32_t hh, uint32_t k) JMA_INL {
    return (uint32_t)((((sidx * 2 + hh) * W + (uint32_t)w) * kWords + k) * 64 + (uint32_t)lane) * 16u;
  };
  __shared__ uint32_t s_tk;
  if (threadIdx.x == 0) s_tk = __hip_atomic_load(&a.tickets[sidx], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_tk == 0u) {
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        store_part(rs, word(half, 4 * nb + c), float4_t{o[nb][4 * c], o[nb][4 * c + 1], o[nb][4 * c + 2], o[nb][4 * c + 3]});
    store_part(rs, word(half, 4 * kNb), float4_t{m, l, lb, 0.0f});
    // The stores are acknowledged (visible device-wide) before the ticket is taken.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      s_tk = __hip_atomic_fetch_add(&a.tickets[sidx], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_tk == 0u) return false;
  }
  if (threadIdx.x == 0) __hip_atomic_store(&a.tickets[sidx], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  pf::float16_t ox[kNb];
#pragma unroll
  for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4_t x = load_part(rs, word(1u - half, 4 * nb + c));
#pragma unroll
      for (int i = 0; i < 4; ++i) ox[nb][4 * c + i] = x[i];
    }
  const float4_t mx = load_part(rs, word(1u - half, 4 * kNb));
  {
#pragma clang fp contract(off)
    const float M = fmaxf(m, mx[0]);
    const float aw = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
    const float ax = mx[0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mx[0] - M);
    l = l * aw + mx[1] * ax;
    lb = lb * aw + mx[2] * ax;
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[nb][e] = o[nb][e] * aw + ox[nb][e] * ax;
    m = M;
  }
  return true;
}

template <typename KV, int D, int W>
__global__ __launch_bounds__(64 * W) void prefill_slice_kernel(const PrefillArgs a) {
  using namespace pf;
  static_assert(std::is_same<KV, float>::value, "f32 caches (f16 at head dim 512: kernel 3c)");
  constexpr int DS = D / W;                      // dims of this wave's slice
  constexpr int kNb = DS / 32;                   // 32-row blocks of its O^T slice
  static_assert(D % W == 0 && DS % 32 == 0, "head-dim slices of 32-row blocks");
  constexpr int kKq = DS / 8;                    // K (and q) operand registers per tile
  constexpr int kVq = 4 * kNb;                   // V operand registers per tile
  using Op = float4_t;
  struct Ops {
    Op k[kKq];
    Op v[kVq];
  };
  // Partial score tiles: [tile parity][wave][4 float4 chunks][lane]. Two buffers let one barrier
  // per tile order both the writes before the reads and the reads before the next overwrite.
  __shared__ float4_t s_x[2][W][4][64];

  const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  static_assert(W == slice_waves(D) && slice_state_words(D) == 4 * kNb + 1, "split state layout");
  // Kv heads vary fastest (consecutive workgroups on different XCDs, each XCD's L2 keeping few
  // kv heads); stripes run last-first (longest causal ranges first): items 0 .. 2 split_blocks - 1
  // are the halves of the split stripes (as kernel 3c splits its pairs), the rest one stripe each.
  const uint32_t kvh = blockIdx.x % a.num_kv_heads;
  const uint32_t rest = blockIdx.x / a.num_kv_heads;
  const uint32_t hz = rest % a.head_groups;
  const uint32_t item = rest / a.head_groups;
  const SplitItem si = split_item(a.row_blocks, a.split_blocks, item);
  const bool split = si.split;
  const uint32_t half = si.half, stripe = si.unit;
  const uint32_t sidx = ((split ? item / 2 : 0u) * a.head_groups + hz) * a.num_kv_heads + kvh;
  const uint32_t R = a.rows_per_stripe, Gz = a.heads_per_stripe;
  const uint32_t row0 = stripe * R;
  const uint32_t row_last = min(row0 + R - 1, a.n - 1);
  // This lane's column; padding columns alias a valid row and head and are never stored.
  const uint32_t cr = min((uint32_t)j / Gz, R - 1);
  const uint32_t hz_head = hz * Gz + (uint32_t)j % Gz;
  const bool col_ok = (uint32_t)j < R * Gz && row0 + cr < a.n && hz_head < a.group;
  const uint32_t crow = min(row0 + cr, a.n - 1);
  const uint32_t head = kvh * a.group + min(hz_head, a.group - 1);
  const uint32_t cpos = a.start + crow;
  const uint32_t cfirst = first_visible(cpos, a.window);
  // Positions some column of the stripe sees, [s_first, s_last], and those every column sees,
  // [all_first, all_last] (first_visible does not decrease with the position).
  const uint32_t s_first = first_visible(a.start + row0, a.window);
  const uint32_t s_last = a.start + row_last;
  const uint32_t all_first = first_visible(s_last, a.window);
  const uint32_t all_last = a.start + row0;
  // This workgroup's tiles [t0, t1): the stripe's, or one half of them.
  uint32_t t0, t1;
  split_range(s_first / 32, s_last / 32 + 1, si, t0, t1);

  const KV* const kb = (const KV*)a.kv.k + a.seq * a.kv.seq_stride_k + a.kv.layer_off_k +
                       (uint64_t)kvh * a.kv.cap * D;
  const KV* const vb = (const KV*)a.kv.v + a.seq * a.kv.seq_stride_v + a.kv.layer_off_v +
                       (uint64_t)kvh * a.kv.cap * D;
  // Operands of kv tile t (positions 32t .. 32t+31; a ring's physical capacity is a multiple of
  // 32 and holds the stripe's whole visible range, so the tile is 32 consecutive slots).
  auto load = [&](uint32_t t, Ops& op) JMA_INL {
    const uint64_t slot0 = a.kv.ring ? (32u * t) % a.kv.cap : 32u * t;
    const KV* const kt = kb + slot0 * D;
    const KV* const vt = vb + slot0 * D;
    // K panels of 16 slots x 16 dims (k_index): slot j, dims 8m + 4h .. +3.
#pragma unroll
    for (int i = 0; i < kKq; ++i) {
      const uint32_t m = w * kKq + i;
      op.k[i] = *(const float4_t*)(kt + (uint64_t)(16 * (j / 16)) * D + (m / 2) * 256 +
                                   (j % 16) * 16 + 8 * (m % 2) + 4 * h);
    }
    // V blocks [16 slots][D]: row dv, slots 8c + 4h .. +3 (block c / 2).
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        op.v[4 * nb + c] = *(const float4_t*)(vt + (uint64_t)(c / 2) * 16 * D +
                                              (uint64_t)(32 * (w * kNb + nb) + j) * 16 +
                                              8 * (c % 2) + 4 * h);
  };
  // Tile slot of result element e in lane half h.
  auto slot_of_e = [&](int e) JMA_INL -> uint32_t { return (uint32_t)(8 * (e >> 2) + 4 * h + (e & 3)); };

  Ops cur, nxt;
  if (t0 < t1) load(t0, cur);

  // q operands of this wave's slice, scaled by scale * log2(e).
  Op qf[kKq];
  {
    const float* const qrow = a.q + ((uint64_t)crow * a.num_heads + head) * D;
    const float qs = col_ok ? a.qscale : 0.0f;
#pragma unroll
    for (int i = 0; i < kKq; ++i) {
      const float4_t x = *(const float4_t*)(qrow + 8 * (w * kKq + i) + 4 * h);
#pragma unroll
      for (int t = 0; t < 4; ++t) qf[i][t] = x[t] * qs;
    }
  }

  float16_t o[kNb];
#pragma unroll
  for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[nb][e] = 0.0f;
  float m = -INFINITY, l = 0.0f, lb = 0.0f;

  auto tile = [&](uint32_t t, const Ops& op) JMA_INL {
    // This wave's partial scores over its dims.
    float16_t s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < kKq; ++i)
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) s = __builtin_amdgcn_mfma_f32_32x32x2f32(op.k[i][t4], qf[i][t4], s, 0, 0, 0);
    // Every wave adds the W partial tiles in wave order.
    if constexpr (W > 1) {
      float4_t(*const xb)[4][64] = s_x[t & 1];
#pragma unroll
      for (int c = 0; c < 4; ++c) xb[w][c][lane] = float4_t{s[4 * c], s[4 * c + 1], s[4 * c + 2], s[4 * c + 3]};
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float4_t x = xb[0][c][lane];
#pragma unroll
        for (int r = 1; r < W; ++r) x += xb[r][c][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * c + i] = x[i];
      }
    }
    // Masks: positions outside [first, position] of a column are -inf (after the products, so a
    // non-finite key there never reaches a result).
    const uint32_t p0 = 32 * t;
    if (!(p0 >= all_first && p0 + 31 <= all_last)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t p = p0 + slot_of_e(e);
        s[e] = p >= cfirst && p <= cpos ? s[e] : -INFINITY;
      }
    }
    // Online softmax: the reference maximum m moves only when a tile's maximum exceeds it by
    // more than 8 (log2 units), so exponentials stay <= 256 and most tiles skip the rescale.
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, s[e]);
    tmax = half_max(tmax);
    const bool up = tmax > m + 8.0f;
    if (__ballot(up) != 0) {
      const float alpha = !up ? 1.0f : (m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - tmax));
      m = up ? tmax : m;
      l *= alpha;
      lb *= alpha;
#pragma unroll
      for (int nb = 0; nb < kNb; ++nb) o[nb] *= alpha;
    }
    const float mu = m == -INFINITY ? 0.0f : m;
    // V rows at positions no column of the stripe sees may hold anything (a discarded tail, an
    // old ring slot); their probabilities are 0, and 0 * inf would be NaN, so they are zeroed.
    Ops v = op;
    if (p0 < s_first || p0 + 31 > s_last) {
#pragma unroll
      for (int i = 0; i < kVq; ++i)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const uint32_t p = p0 + (uint32_t)(8 * (i & 3) + 4 * h + x);
          if (p < s_first || p > s_last) v.v[i][x] = 0;
        }
    }
    float p[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = __builtin_amdgcn_exp2f(s[e] - mu);
      if (e & 1) lb += p[e];
      else l += p[e];
    }
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int u = 0; u < 16; ++u)
        o[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(v.v[4 * nb + (u >> 2)][u & 3], p[u], o[nb], 0, 0, 0);
  };

  // Two tiles per iteration, so the two operand sets stay distinct registers.
  for (uint32_t t = t0; t < t1; t += 2) {
    if (t + 1 < t1) load(t + 1, nxt);
    tile(t, cur);
    if (t + 1 >= t1) break;
    if (t + 2 < t1) load(t + 2, cur);
    tile(t + 1, nxt);
  }

  if (split && !merge_halves<W, kNb>(a, sidx, half, w, lane, o, m, l, lb)) return;  // the other merges

  const float L = half_sum(l + lb);
  const bool bad = col_ok && !(L > 0.0f && L < INFINITY);
  if (__ballot(bad) != 0 && lane == 0) atomicOr(a.err, 1);
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  if (col_ok) {
    float* const orow = a.out + ((uint64_t)crow * a.num_heads + head) * D + 4 * h;
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *(float4_t*)(orow + 32 * (w * kNb + nb) + 8 * c) =
            float4_t{o[nb][4 * c], o[nb][4 * c + 1], o[nb][4 * c + 2], o[nb][4 * c + 3]} * inv;
  }
}


// ================================================================ kernel 3c: paired-stripe prefill

// Causal / sliding-window prefill for f16 caches at head dim 512 (Gemma 4 full layers). A
// workgroup is two adjacent stripes of 32 (query row, query head) columns of one kv head, and its
// four waves are (stripe s, head-dim half hf): wave (s, hf) forms stripe s's partial scores over
// dims 256hf .. 256hf+255, the two waves of a stripe add their partial tiles through LDS (a + b
// is the same float either way, so both hold the same scores bit for bit) and run the same
// select-masked online softmax as kernel 3b, and wave (s, hf) accumulates output dims 256hf ..
// 256hf+255 of its stripe. K and V tiles are staged in LDS once for both stripes (kernel 3b read
// each tile into registers once per stripe, and per-CU load issue bounded it), by direct-to-LDS
// loads in kernel 3's layout and swizzles; K and V each alternate between two stage arrays.
//
// Per tile t: QK^T over the wave's half (16 matrix ops, K operands read eight ahead), partial
// tile to LDS, wait for V(t), barrier A; K(t+2) into K(t)'s array; add the partner's partial,
// read the first eight V operands (their latency passes under the softmax), mask, softmax; PV
// (16 matrix ops); wait for K(t+1), barrier B; V(t+2) into V(t)'s array. So each tile is
// loaded about one and a half tiles ahead of use. The pair's tile range is the union of its
// stripes' (adjacent rows, so at most one tile more than either); a tile a stripe does not see is
// masked to -inf entirely and adds nothing. Past the pair's last tile the loads repeat that
// tile, so every wave issues the same loads each step and the load counters count the same.
//
// V rows at positions a stripe does not see are fed to its PV product as loaded (probability 0)
// in the fast pass; a non-finite value there makes the column's state non-finite, and the
// workgroup then runs again in a robust pass that zeroes those operand elements (as the main
// prefill kernel does). The q operands live in the accumulation registers (the matrix ops read
// them there), leaving the vector registers to O^T, the scores and the operands.
//
// One workgroup per compute unit (the four stage arrays take 128 KB of LDS), and a pair's cost
// grows with its row, so the longest pairs would set the duration: the split_blocks longest
// pairs (planned by plan_prefill_pairs) run first as two workgroups each, one per half of the
// pair's kv tiles. Both store their state (O^T, m, l per lane) device-coherent and take a ticket;
// the later one loads the other's state, merges the two online-softmax states (the same products
// and one sum whichever half merges, so the result does not depend on the arrival order), resets
// the ticket and stores the output.
template <int D>
__global__ __launch_bounds__(256) void prefill_pair_kernel(const PrefillArgs a) {
  using namespace pf;
  static_assert(D == 512, "paired stripes at head dim 512");
  constexpr int kHalf = D / 2;      // dims of a wave
  constexpr int kKq = kHalf / 16;   // QK^T k-steps of a wave
  constexpr int kNb = kHalf / 32;   // 32-row blocks of its O^T
  constexpr int kT = 32 * D;        // halves of one K (or V^T) tile
  constexpr int kChunks = D / 16;   // 1 KB chunks per tile
  constexpr int kCPW = kChunks / 4; // chunks of each tile one wave loads
  __shared__ __attribute__((aligned(16))) _Float16 ka[kT];
  __shared__ __attribute__((aligned(16))) _Float16 kb2[kT];
  __shared__ __attribute__((aligned(16))) _Float16 va[kT];
  __shared__ __attribute__((aligned(16))) _Float16 vb2[kT];
  __shared__ float4_t s_x[2][2][4][64];  // partial scores [stripe][half][float4 chunk][lane]

  const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int st = w & 1, hf = w >> 1;
  // Kv heads vary fastest (consecutive workgroups on different XCDs); pairs run last-first
  // (longest causal ranges first): items 0 .. 2 split_blocks - 1 are the halves of the split
  // pairs, the rest one pair each.
  const uint32_t pairs = (a.row_blocks + 1) / 2;
  const uint32_t kvh = blockIdx.x % a.num_kv_heads;
  const uint32_t rest = blockIdx.x / a.num_kv_heads;
  const uint32_t hz = rest % a.head_groups;
  const uint32_t item = rest / a.head_groups;
  const SplitItem si = split_item(pairs, a.split_blocks, item);
  const bool split = si.split;
  const uint32_t half = si.half, pr = si.unit;
  const uint32_t sidx = ((split ? item / 2 : 0u) * a.head_groups + hz) * a.num_kv_heads + kvh;
  const uint32_t stripe = 2 * pr + st;
  const bool stripe_ok = stripe < a.row_blocks;
  const uint32_t R = a.rows_per_stripe, Gz = a.heads_per_stripe;
  // An absent second stripe (odd stripe count) aliases the first and stores nothing.
  const uint32_t row0 = min(stripe, a.row_blocks - 1) * R;
  const uint32_t row_last = min(row0 + R - 1, a.n - 1);
  const uint32_t cr = min((uint32_t)j / Gz, R - 1);
  const uint32_t hz_head = hz * Gz + (uint32_t)j % Gz;
  const bool col_ok = stripe_ok && (uint32_t)j < R * Gz && row0 + cr < a.n && hz_head < a.group;
  const uint32_t crow = min(row0 + cr, a.n - 1);
  const uint32_t head = kvh * a.group + min(hz_head, a.group - 1);
  const uint32_t cpos = a.start + crow;
  const uint32_t cfirst = first_visible(cpos, a.window);
  // Positions some column of the stripe sees, [s_first, s_last], and those every column sees,
  // [all_first, all_last] (first_visible does not decrease with the position).
  const uint32_t s_first = first_visible(a.start + row0, a.window);
  const uint32_t s_last = a.start + row_last;
  const uint32_t all_first = first_visible(s_last, a.window);
  const uint32_t all_last = a.start + row0;
  // The pair's tiles (the same for every wave).
  const uint32_t p_row0 = 2 * pr * R;
  const uint32_t p_last = min(p_row0 + 2 * R - 1, a.n - 1);
  const uint32_t t0 = first_visible(a.start + p_row0, a.window) / 32;
  const uint32_t t1 = (a.start + p_last) / 32 + 1;
  // This workgroup's tiles [tb, te): all of the pair's, or one half. The first half is shorter,
  // so it usually stores its state while the second still computes, and the second merges
  // without storing its own.
  uint32_t tb, te;
  split_range(t0, t1, si, tb, te);

  const _Float16* const kbase = (const _Float16*)a.kv.k + a.seq * a.kv.seq_stride_k + a.kv.layer_off_k +
                                (uint64_t)kvh * a.kv.cap * D;
  const _Float16* const vbase = (const _Float16*)a.kv.v + a.seq * a.kv.seq_stride_v + a.kv.layer_off_v +
                                (uint64_t)kvh * a.kv.cap * D;
  // Byte offsets inside a tile of the 16 bytes this lane stages per chunk (chunk c = w + 4i: K row
  // c, V^T rows 16c .. 16c+15), with kernel 3's swizzles applied on the global side.
  uint32_t koff[kCPW], voff[kCPW];
#pragma unroll
  for (int i = 0; i < kCPW; ++i) {
    const uint32_t c = (uint32_t)w + 4u * i;
    const uint32_t cc = (uint32_t)lane ^ swz_k<D>(c);
    koff[i] = 2 * ((cc / 4) * (32 * 32) + c * 32 + 8 * (cc % 4));
    const uint32_t rv = c * 16 + lane / 4;
    voff[i] = 2 * (rv * 32 + 8 * ((lane % 4) ^ swz_v(rv)));
  }
  // Tile t's K (or V) into the given stage array (t clamped to the workgroup's last tile; a
  // ring's physical capacity is a multiple of 32 and holds the pair's visible range).
  auto tile_bytes = [&](uint32_t t) JMA_INL {
    const uint32_t tt = min(t, te - 1);
    return (a.kv.ring ? (32u * tt) % a.kv.cap : 32u * tt) * (2u * D);
  };
  auto issue_k = [&](uint32_t t, _Float16* kd) JMA_INL {
    const uint32_t off = tile_bytes(t);
#pragma unroll
    for (int i = 0; i < kCPW; ++i) dma16(kbase, kd + 512 * (w + 4 * i), koff[i], off);
  };
  auto issue_v = [&](uint32_t t, _Float16* vd) JMA_INL {
    const uint32_t off = tile_bytes(t);
#pragma unroll
    for (int i = 0; i < kCPW; ++i) dma16(vbase, vd + 512 * (w + 4 * i), voff[i], off);
  };
  // Waits until at most n of this wave's loads are in flight (and its LDS operations are done),
  // then barrier.
  auto wait_barrier = [](auto outstanding) JMA_INL {
    constexpr int n = decltype(outstanding)::value;
    __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  issue_k(tb, ka);
  issue_v(tb, va);
  issue_k(tb + 1, kb2);
  issue_v(tb + 1, vb2);

  // q operands of this wave's half, scaled by scale * log2(e) and rounded to f16; a scaled element
  // beyond the f16 range (where the reference's f32 scores stay finite) is reported like a
  // non-finite score.
  half8_t qf[kKq];
  {
    const float* const qrow = a.q + ((uint64_t)crow * a.num_heads + head) * D;
    const float qs = col_ok ? a.qscale : 0.0f;
    float qmax = 0.0f;
#pragma unroll
    for (int i = 0; i < kKq; ++i) {
      const uint32_t e = 16 * (hf * kKq + i) + 8 * h;
      const float4_t x0 = *(const float4_t*)(qrow + e);
      const float4_t x1 = *(const float4_t*)(qrow + e + 4);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        qmax = fmaxf(qmax, fmaxf(fabsf(x0[t] * qs), fabsf(x1[t] * qs)));
        qf[i][t] = (_Float16)(x0[t] * qs);
        qf[i][4 + t] = (_Float16)(x1[t] * qs);
      }
    }
    if (__ballot(col_ok && !(qmax < 65520.0f)) != 0 && lane == 0) atomicOr(a.err, 1);
    // The q operands stay in the accumulation registers (matrix ops read them there), leaving
    // the vector registers to O^T, the scores and the tile operands.
#pragma unroll
    for (int i = 0; i < kKq; ++i) asm("" : "+a"(qf[i]));
  }

  float16_t o[kNb];
  float m, l, lb;
  const uint32_t kr = swap34(j);
  float4_t(*const x_own)[64] = s_x[st][hf];
  float4_t(*const x_other)[64] = s_x[st][1 - hf];

  // One tile. The fast pass (robust false) feeds V operands as loaded; the robust pass zeroes the
  // elements of positions the stripe does not see (see the end of the kernel).
  auto tile = [&](uint32_t t, _Float16* kd, _Float16* vd, auto robust) JMA_INL {
    // This wave's partial scores over its half, K operands read eight k-steps ahead of the
    // matrix ops that use them (one wave per SIMD: nothing else hides the LDS latency).
    float16_t sc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = 0.0f;
    auto kread = [&](int i) JMA_INL {
      const int ks = hf * kKq + i;
      return *(const half8_t*)(kd + kr * D + 8 * ((2 * ks + h) ^ swz_k<D>(kr)));
    };
    half8_t kf[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) kf[i] = kread(i);
#pragma unroll
    for (int i = 0; i < kKq; ++i) {
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[i % 8], qf[i], sc, 0, 0, 0);
      if (i + 8 < kKq) kf[i % 8] = kread(i + 8);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) x_own[c][lane] = float4_t{sc[4 * c], sc[4 * c + 1], sc[4 * c + 2], sc[4 * c + 3]};
    // V(t) staged: after it this wave issued K(t+1) and V(t+1). Past this barrier every wave is
    // done with K(t), whose array takes K(t+2).
    wait_barrier(std::integral_constant<int, 2 * kCPW>{});
    issue_k(t + 2, kd);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4_t x = x_other[c][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * c + i] += x[i];
    }
    // V operands (2 per 32-row block of O^T): the first eight are read now, so their LDS latency
    // passes under the softmax, the rest eight ahead of the matrix ops that use them.
    auto vaddr = [&](int u) JMA_INL {
      const uint32_t vr = 32 * (hf * kNb + u / 2) + j;
      return (const uint4*)(vd + vr * 32 + 8 * ((2 * (u & 1) + h) ^ swz_v(vr)));
    };
    uint4 vraw[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) vraw[k] = *vaddr(2 * (k % kNb) + k / kNb);
    // Masks: positions outside [first, position] of a column are -inf (after the products, so a
    // non-finite key there never reaches a result).
    const uint32_t p0 = 32 * t;
    if (!(p0 >= all_first && p0 + 31 <= all_last)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t p = p0 + score_slot(e, h);
        sc[e] = p >= cfirst && p <= cpos ? sc[e] : -INFINITY;
      }
    }
    // Online softmax: the reference maximum m moves only when a tile's maximum exceeds it by
    // more than 8 (log2 units), so exponentials stay <= 256 and most tiles skip the rescale.
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sc[e]);
    tmax = half_max(tmax);
    const bool up = tmax > m + 8.0f;
    if (__ballot(up) != 0) {
      const float alpha = !up ? 1.0f : (m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - tmax));
      m = up ? tmax : m;
      l *= alpha;
      lb *= alpha;
#pragma unroll
      for (int nb = 0; nb < kNb; ++nb) o[nb] *= alpha;
    }
    const float mu = m == -INFINITY ? 0.0f : m;
    half8_t pf[2];
#pragma unroll
    for (int e = 0; e < 16; ++e) pf[e >> 3][e & 7] = (_Float16)__builtin_amdgcn_exp2f(sc[e] - mu);
    const half2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const half2_t pr2 = {pf[i >> 2][2 * (i & 3)], pf[i >> 2][2 * (i & 3) + 1]};
      if (i & 1) lb = __builtin_amdgcn_fdot2(pr2, one, lb, false);
      else l = __builtin_amdgcn_fdot2(pr2, one, l, false);
    }
    // Robust pass: element e of V operand b holds position p0 + score_slot(8b + e, h), and the
    // masks clear the elements of positions the stripe does not see at its edge tiles.
    uint32_t vm[2][4];
    if constexpr (decltype(robust)::value) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t q0 = p0 + score_slot(8 * b + 2 * d, h), q1 = p0 + score_slot(8 * b + 2 * d + 1, h);
          vm[b][d] = (q0 < s_first || q0 > s_last ? 0u : 0xFFFFu) | (q1 < s_first || q1 > s_last ? 0u : 0xFFFF0000u);
        }
    }
    // Operand u = 2 nb + b; the ops run b-major (every block's b = 0 op, then every b = 1 op), so
    // the two ops into one accumulator are eight apart and never wait on each other.
#pragma unroll
    for (int k = 0; k < 2 * kNb; ++k) {
      const int u = 2 * (k % kNb) + k / kNb;
      uint4 x = vraw[k % 8];
      if constexpr (decltype(robust)::value) {
        x.x &= vm[u & 1][0];
        x.y &= vm[u & 1][1];
        x.z &= vm[u & 1][2];
        x.w &= vm[u & 1][3];
      }
      o[u / 2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, x), pf[u & 1], o[u / 2], 0, 0, 0);
      if (k + 8 < 2 * kNb) vraw[k % 8] = *vaddr(2 * ((k + 8) % kNb) + (k + 8) / kNb);
    }
    // K(t+1) staged (after it this wave issued V(t+1) and K(t+2)); every wave is past V(t) and
    // the partial tiles, which V(t+2) and the next partials overwrite.
    wait_barrier(std::integral_constant<int, 2 * kCPW>{});
    issue_v(t + 2, vd);
  };
  // One pass over the workgroup's tiles (K(tb), V(tb), K(tb+1), V(tb+1) already on their way).
  auto run = [&](auto robust) JMA_INL {
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[nb][e] = 0.0f;
    m = -INFINITY;
    l = 0.0f;
    lb = 0.0f;
    // K(tb) staged (V(tb), K(tb+1), V(tb+1) may still be in flight).
    wait_barrier(std::integral_constant<int, 3 * kCPW>{});
    for (uint32_t t = tb; t < te; t += 2) {
      tile(t, ka, va, robust);
      if (t + 1 >= te) break;
      tile(t + 1, kb2, vb2, robust);
    }
    // The repeated loads of the last steps land, and every wave is past its last LDS reads,
    // before the arrays are loaded again or the workgroup's LDS is released.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  // V rows at positions no column of a stripe sees may hold anything (a discarded tail, an old
  // ring slot, a value that overflowed f16). Their probabilities are 0, but 0 * inf is NaN, so a
  // non-finite value there turns the column's state non-finite, where the reference never reads
  // that position. A workgroup with a valid column whose state is not finite after the fast pass
  // runs its pair again in the robust pass; a state still non-finite then is the reference's too.
  __shared__ uint32_t s_rerun;
  if (threadIdx.x == 0) s_rerun = 0u;
  run(std::false_type{});
  {
    float osum = 0.0f;
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) osum += o[nb][e];
    const bool bad = col_ok && !(l + lb < INFINITY && m < INFINITY && fabsf(osum) < INFINITY);
    if (__ballot(bad) != 0 && lane == 0) s_rerun = 1u;
  }
  __syncthreads();
  if (s_rerun != 0u) {
    issue_k(tb, ka);
    issue_v(tb, va);
    issue_k(tb + 1, kb2);
    issue_v(tb + 1, vb2);
    run(std::true_type{});
  }

  static_assert(kPairPartWords == 4 * kNb + 1, "a half's state: O^T's float4 words, then (m, l, lb)");
  if (split && !merge_halves<4, kNb>(a, sidx, half, w, lane, o, m, l, lb)) return;  // the other merges

  const float L = half_sum(l + lb);
  const bool bad = col_ok && !(L > 0.0f && L < INFINITY);
  if (__ballot(bad) != 0 && lane == 0) atomicOr(a.err, 1);
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  if (col_ok) {
    float* const orow = a.out + ((uint64_t)crow * a.num_heads + head) * D + 4 * h;
#pragma unroll
    for (int nb = 0; nb < kNb; ++nb)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *(float4_t*)(orow + 32 * (hf * kNb + nb) + 8 * c) =
            float4_t{o[nb][4 * c], o[nb][4 * c + 1], o[nb][4 * c + 2], o[nb][4 * c + 3]} * inv;
  }
}

template <int D>
hipError_t launch_prefill_t(PrefillArgs a, hipStream_t stream) {
  constexpr int S = pf::Shape<D>::S, Q = pf::Shape<D>::Q;
  const uint64_t blocks = ((uint64_t)a.row_blocks + a.split_blocks) * a.head_groups * a.num_kv_heads;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffffu || a.split_blocks > a.row_blocks) return hipErrorInvalidValue;
  if ((uint64_t)a.kv.cap * D * 2 > 0x7fffffffu) return hipErrorInvalidValue;  // 32-bit tile offsets
  if (a.split_blocks > 0 && (a.part == nullptr || a.tickets == nullptr)) return hipErrorInvalidValue;
  hipLaunchKernelGGL((prefill_kernel<D>), dim3((uint32_t)blocks), dim3(64 * S * Q), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int dk, int dv, hipStream_t stream) {
  if (!prefill_supported(dk, dv)) return hipErrorInvalidValue;
  if (a.heads_per_stripe == 0 || a.heads_per_stripe > 32 ||
      a.rows_per_stripe * a.heads_per_stripe > 32 || a.rows_per_stripe == 0 ||
      a.num_kv_heads == 0 || a.num_heads != a.num_kv_heads * a.group)
    return hipErrorInvalidValue;
  switch (dk) {
    case 32: return launch_prefill_t<32>(a, stream);
    case 64: return launch_prefill_t<64>(a, stream);
    case 128: return launch_prefill_t<128>(a, stream);
    case 256: return launch_prefill_t<256>(a, stream);
    default: return hipErrorInvalidValue;
  }
}


template <typename KV, int D, int W>
hipError_t launch_prefill_slice_t(const PrefillArgs& a, hipStream_t stream) {
  // One workgroup per stripe, two per split stripe.
  const uint64_t blocks = split_items(a.row_blocks, a.split_blocks) * a.head_groups * a.num_kv_heads;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffffu) return hipErrorInvalidValue;
  hipLaunchKernelGGL((prefill_slice_kernel<KV, D, W>), dim3((uint32_t)blocks), dim3(64 * W), 0,
                     stream, a);
  return hipGetLastError();
}

hipError_t launch_prefill_slice(const PrefillArgs& a, bool f16, int dk, int dv, hipStream_t stream) {
  if (!prefill_slice_supported(f16, dk, dv)) return hipErrorInvalidValue;
  if (a.heads_per_stripe == 0 || a.heads_per_stripe > 32 || a.rows_per_stripe == 0 ||
      a.rows_per_stripe * a.heads_per_stripe > 32 || a.num_kv_heads == 0 ||
      a.num_heads != a.num_kv_heads * a.group ||
      a.row_blocks != (a.n + a.rows_per_stripe - 1) / a.rows_per_stripe ||
      a.head_groups != (a.group + a.heads_per_stripe - 1) / a.heads_per_stripe)
    return hipErrorInvalidValue;
  if (f16) {
    // Stripe pairs (kernel 3c), split_blocks of them as two workgroups; 32-bit tile byte offsets.
    const uint32_t pairs = (a.row_blocks + 1) / 2;
    const uint64_t blocks = split_items(pairs, a.split_blocks) * a.head_groups * a.num_kv_heads;
    if (blocks == 0) return hipSuccess;
    if (blocks > 0x7fffffffu || (uint64_t)a.kv.cap * 512 * 2 > 0x7fffffffu) return hipErrorInvalidValue;
    if (a.split_blocks > 0) {
      // Every split pair (the trailing ones) has at least two kv tiles; the halves' states fit
      // 32-bit byte offsets.
      const uint32_t pr = pairs - a.split_blocks, R = a.rows_per_stripe;
      const uint32_t r0 = 2 * pr * R, r1 = std::min(r0 + 2 * R, a.n) - 1;
      const uint32_t t0 = first_visible(a.start + r0, a.window) / 32, t1 = (a.start + r1) / 32 + 1;
      const uint64_t part_b = (uint64_t)a.split_blocks * a.head_groups * a.num_kv_heads * 2 * 4 *
                              kPairPartWords * 64 * 16;
      if (a.split_blocks > pairs || a.part == nullptr || a.tickets == nullptr || t1 - t0 < 2 ||
          part_b > 0x7FFFFFF0u)
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL((prefill_pair_kernel<512>), dim3((uint32_t)blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  if (a.split_blocks > 0) {
    // Split stripes (the trailing ones) have at least two kv tiles; the halves' states fit 32-bit
    // byte offsets.
    const uint32_t st = a.row_blocks - a.split_blocks, R = a.rows_per_stripe;
    const uint32_t r0 = st * R, r1 = std::min(r0 + R, a.n) - 1;
    const uint32_t t0 = first_visible(a.start + r0, a.window) / 32, t1 = (a.start + r1) / 32 + 1;
    const uint64_t part_b = (uint64_t)a.split_blocks * a.head_groups * a.num_kv_heads * 2 *
                            slice_waves(dk) * slice_state_words(dk) * 64 * 16;
    if (a.split_blocks > a.row_blocks || a.part == nullptr || a.tickets == nullptr || t1 - t0 < 2 ||
        part_b > 0x7FFFFFF0u)
      return hipErrorInvalidValue;
  }
  switch (dk) {
    case 32: return launch_prefill_slice_t<float, 32, 1>(a, stream);
    case 64: return launch_prefill_slice_t<float, 64, 2>(a, stream);
    case 128: return launch_prefill_slice_t<float, 128, 4>(a, stream);
    case 256: return launch_prefill_slice_t<float, 256, 4>(a, stream);
    case 512: return launch_prefill_slice_t<float, 512, 8>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace jma
