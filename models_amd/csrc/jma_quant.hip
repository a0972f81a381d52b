// GGUF block-quantized matrix-vector products for the projections around attention (the Q/K/V
// projection before the append, llama/LlamaForwardPass.java:1043-1067, and the output projection
// plus residual after it, :1131-1138), on gfx950.
//
// Arithmetic (the definition backend-native's tests hold its Q4_0 kernel to exactly,
// backend-native/src/test/java/com/integrallis/models/backend/nativekernel/
// NativeKernelLibraryTest.java:909-1023): each 32-element block of an activation row is quantized
// to Q8_0 (absmax, inverse 127 / absmax, element = nearest integer of x * inverse by the 1.5 * 2^23
// trick, scale = f16-rounded absmax / 127); each output is the in-order chain over the row's
// blocks of fma(weightScale * activationScale, integer block dot, sum). Integer dots are exact and
// every float operation is the reference's, in its order, so the outputs are the oracle's bit for
// bit.
//
// Work: one 256-thread workgroup per tile of R rows of one matrix. It quantizes the activation
// rows itself into LDS (a few KB at decode sizes: no separate launch), forms every (row, block)
// term of its tile in parallel (coalesced 16-bit weight loads: 18- and 34-byte blocks are only
// 2-byte aligned; 4-element integer dots with v_dot4_i32_i8), then one thread per (activation row,
// output row) runs the block chain from LDS. The bytes are the weights (HBM-bound at large
// shapes); at decode shapes a launch is latency-bound.
#include <hip/hip_runtime.h>

#include "jma_kernels.h"

namespace jma {
namespace {

constexpr uint32_t kQThreads = 256;
typedef short short2_t __attribute__((ext_vector_type(2)));

template <int kCtrl>
__device__ __forceinline__ int dpp_int(int x) {
  return __builtin_amdgcn_mov_dpp(x, kCtrl, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
// Once the quads of 8 consecutive lanes hold equal values, row_half_mirror (lane 7 - i within
// each half row) pairs quad 0 with quad 1 as i ^ 4 would; once those 8-lane groups are equal,
// row_mirror (lane 15 - i within each row of 16) pairs them as i ^ 8 would.
constexpr int kHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// A value of the other row of 16 lanes in a 32-lane group (the lane 16 away): v_permlane16_swap
// with both operands x leaves rows {0, 0, 2, 2} and {1, 1, 3, 3} of x in its two results, so a
// lane of row 0 finds its partner in the second and a lane of row 1 in the first. Symmetric
// combinations of the two results give both partners the same bits without choosing.
__device__ __forceinline__ void rows16(uint32_t x, uint32_t& r0, uint32_t& r1) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  r0 = r[0];
  r1 = r[1];
}

// Sum over the 8 consecutive lanes of a group (exact in integers, so the pairing order is free).
__device__ __forceinline__ int sum8(int x) {
  x += dpp_int<kQuadXor1>(x);
  x += dpp_int<kQuadXor2>(x);
  return x + dpp_int<kHalfMirror>(x);
}

// ggmlNearestInt (NativeKernelLibraryTest.java:1019-1022): x + 1.5 * 2^23 rounds x to an integer
// (nearest, ties to even) in the low mantissa bits.
__device__ __forceinline__ int nearest_int(float v) {
#pragma clang fp contract(off)
  const float s = v + 12582912.0f;
  return (int)(__float_as_uint(s) & 0x007FFFFFu) - 0x00400000;
}

__device__ __forceinline__ float f16_bits_to_float(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Bits 0..3 of x moved to bit 4 of bytes 0..3 (the four shifted copies of x do not overlap, so
// the product has no carries).
__device__ __forceinline__ uint32_t fifth_bits(uint32_t x) { return ((x * 0x00204081u) & 0x01010101u) << 4; }

// Weight block of a format (backend-native's codes: 0 Q4_0, 1 Q8_0, 5 Q5_0): a 16-bit scale,
// then 16 bytes of nibbles (Q4_0), a 32-bit word of fifth bits and 16 bytes of nibbles (Q5_0) or
// 32 int8 (Q8_0), read as 16-bit halves (the blocks are 2-byte aligned only).
template <int FMT>
struct QBlock {
  static constexpr uint32_t kHalves = FMT == 0 ? 9u : FMT == 5 ? 11u : 17u;
  uint32_t h[kHalves];
  __device__ __forceinline__ void load(const uint16_t* rec) {
#pragma unroll
    for (uint32_t i = 0; i < kHalves; ++i) h[i] = rec[i];
  }
  __device__ __forceinline__ uint32_t word(uint32_t j) const { return h[1 + 2 * j] | (h[2 + 2 * j] << 16); }
  // Integer dot of the block with Q8_0 activations aq (8 words of 4 int8) whose element sum is
  // asum. Q4_0: byte i holds element i in its low nibble and element i + 16 in its high one, each
  // offset by 8; the offset is applied as -8 * asum. Q5_0: the same nibbles with bit j of the
  // word at byte 2 as element j's fifth bit, offset by 16 (dot_q5_0_q8_0_row_scalar,
  // backend-native/src/main/rust/model-kernels/src/lib.rs:3204-3252): elements 0..31 as bytes.
  __device__ __forceinline__ int dot(const int* aq, int asum) const {
    int d = 0;
    if constexpr (FMT == 0) {
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t w = word(j);
        d = __builtin_amdgcn_sdot4((int)(w & 0x0F0F0F0Fu), aq[j], d, false);
        d = __builtin_amdgcn_sdot4((int)((w >> 4) & 0x0F0F0F0Fu), aq[4 + j], d, false);
      }
      d -= 8 * asum;
    } else if constexpr (FMT == 5) {
      const uint32_t high = word(0);
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t w = h[3 + 2 * j] | (h[4 + 2 * j] << 16);
        const uint32_t lo = (w & 0x0F0F0F0Fu) | fifth_bits((high >> (4 * j)) & 15u);
        const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | fifth_bits((high >> (16 + 4 * j)) & 15u);
        d = __builtin_amdgcn_sdot4((int)lo, aq[j], d, false);
        d = __builtin_amdgcn_sdot4((int)hi, aq[4 + j], d, false);
      }
      d -= 16 * asum;
    } else {
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j) d = __builtin_amdgcn_sdot4((int)word(j), aq[j], d, false);
    }
    return d;
  }
};

// Q8_0 quantization of one eighth of a 32-element activation block (quantizeInputs,
// NativeKernelLibraryTest.java:998-1017): the four consecutive lanes of a quad each take eight
// elements and meet for the block maximum and the element sum through DPP quad exchanges. The
// block's absolute maximum (NaN skipped) gives inverse = 127 / absmax, each element the nearest
// integer of x * inverse (the reference's 1.5 * 2^23 addition), the scale the f16-rounded
// absmax / 127. All four lanes of a quad must call it together.
__device__ __forceinline__ void q8_0_eighth(const float* xs, uint2& packed, float& scale, int& sum) {
  const float4 x0 = *(const float4*)xs, x1 = *(const float4*)(xs + 4);
  const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  float am = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(xv[i]));  // a NaN element is skipped
  am = fmaxf(am, __int_as_float(dpp_int<kQuadXor1>(__float_as_int(am))));
  am = fmaxf(am, __int_as_float(dpp_int<kQuadXor2>(__float_as_int(am))));
  const float inverse = am == 0.0f ? 0.0f : 127.0f / am;
  uint32_t pk[2] = {0u, 0u};
  int s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float scaled;
    {
#pragma clang fp contract(off)
      scaled = xv[i] * inverse;
    }
    const int q = nearest_int(scaled);
    s += (int)(int8_t)q;
    pk[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
  }
  packed = make_uint2(pk[0], pk[1]);
  s += dpp_int<kQuadXor1>(s);
  s += dpp_int<kQuadXor2>(s);
  sum = s;
  scale = (float)(_Float16)(am / 127.0f);
}

// Q8_K quantization of one thirty-second of a 256-element activation block (eight elements;
// quantize_q8_k_batch, backend-native/src/main/rust/model-kernels/src/lib.rs:3906-3952): the 32
// consecutive lanes of the block find the element of largest magnitude (the first on ties, NaN
// skipped) with shuffles; inverse = -127 / that element, each element min(nearest(inverse * x),
// 127). sum16: the 16-element sum of this lane's pair (valid on even parts); scale: 1 / inverse
// (0 for an all-zero block). All 32 lanes of a block must call it together.
__device__ __forceinline__ void q8_k_part(const float* xs, uint32_t part, uint2& packed, int& sum16,
                                          float& scale) {
  const float4 x0 = *(const float4*)xs, x1 = *(const float4*)(xs + 4);
  const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  float best = 0.0f, bval = 0.0f;
  uint32_t bidx = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float m = fabsf(xv[i]);
    if (m > best) {  // strict: the first of equal magnitudes; a NaN compares false
      best = m;
      bval = xv[i];
      bidx = part * 8u + i;
    }
  }
  // The block maximum over its 32 lanes under the total order (magnitude, then the lower index
  // first): the same winner whatever the pairing, so DPP exchanges within rows of 16, then the
  // two rows of the group through v_permlane16_swap.
  auto take = [&](float ob, float ov, uint32_t oi) {
    if (ob > best || (ob == best && oi < bidx)) {
      best = ob;
      bval = ov;
      bidx = oi;
    }
  };
  auto step = [&](auto ctrl) {
    constexpr int c = decltype(ctrl)::value;
    take(__int_as_float(dpp_int<c>(__float_as_int(best))), __int_as_float(dpp_int<c>(__float_as_int(bval))),
         (uint32_t)dpp_int<c>((int)bidx));
  };
  step(std::integral_constant<int, kQuadXor1>{});
  step(std::integral_constant<int, kQuadXor2>{});
  step(std::integral_constant<int, kHalfMirror>{});
  step(std::integral_constant<int, kRowMirror>{});
  {
    uint32_t b0, b1, v0, v1, i0, i1;
    rows16(__float_as_uint(best), b0, b1);
    rows16(__float_as_uint(bval), v0, v1);
    rows16(bidx, i0, i1);
    const float fb0 = __uint_as_float(b0), fb1 = __uint_as_float(b1);
    const bool second = fb1 > fb0 || (fb1 == fb0 && i1 < i0);
    best = second ? fb1 : fb0;
    bval = __uint_as_float(second ? v1 : v0);
    bidx = second ? i1 : i0;
  }
  int s = 0;
  if (best == 0.0f) {
    packed = make_uint2(0u, 0u);
  } else {
    const float inverse = -127.0f / bval;
    uint32_t pk[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float scaled;
      {
#pragma clang fp contract(off)
        scaled = inverse * xv[i];
      }
      const int q = min(nearest_int(scaled), 127);
      s += (int)(int8_t)q;
      pk[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
    }
    packed = make_uint2(pk[0], pk[1]);
  }
  s += dpp_int<kQuadXor1>(s);  // two threads make one 16-element sum
  sum16 = s;
  scale = best == 0.0f ? 0.0f : 1.0f / (-127.0f / bval);
}

}  // namespace

template <int FMT>
__global__ __launch_bounds__(kQThreads) void qmatvec_kernel(const QMatArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char q_lds[];
  // LDS holds one pass of nc activation rows; the workgroup's rows (blockIdx.y's group) pass
  // through it in turn while the weight tile stays in registers.
  const uint32_t nc = a.chunk, cols = a.cols, K = a.blocks, R = a.rows_per_tile, Kp = K + 1;
  int8_t* act_q = (int8_t*)q_lds;                                   // [nc][cols]
  float* act_scale = (float*)(q_lds + ((nc * cols + 15u) & ~15u));  // [nc][K]
  int* act_sum = (int*)(act_scale + nc * K);                        // [nc][K]
  float* t_scale = (float*)(act_sum + nc * K);                      // [nc][R][Kp]
  float* t_dot = t_scale + nc * R * Kp;                             // [nc][R][Kp]

  uint32_t mi = 0;
  for (uint32_t i = 1; i < a.count; ++i) mi = blockIdx.x >= a.m[i].tile0 ? i : mi;
  const uint8_t* w = a.m[mi].w;
  float* out = a.m[mi].out;
  const float* addend = a.m[mi].addend;
  const uint32_t rows = a.m[mi].rows;
  const uint32_t r0 = (blockIdx.x - a.m[mi].tile0) * R;
  const uint32_t nrows = min(R, rows - r0);
  const uint32_t nunits = nrows * K;
  constexpr uint32_t kRecHalves = QBlock<FMT>::kHalves;  // block bytes / 2
  const uint16_t* wrec = (const uint16_t*)(w + (uint64_t)r0 * K * (2u * kRecHalves));
  const uint32_t tid = threadIdx.x;

  // A thread's first kU units (every unit of a tile of up to 1024 terms) are loaded once, in
  // flight while the first activations are quantized, and serve every pass.
  constexpr uint32_t kU = 4;
  QBlock<FMT> unit[kU];
#pragma unroll
  for (uint32_t i = 0; i < kU; ++i)
    if (tid + i * kQThreads < nunits) unit[i].load(wrec + (uint64_t)(tid + i * kQThreads) * kRecHalves);

  const uint32_t g0 = blockIdx.y * a.group_rows, g1 = min(a.batch, g0 + a.group_rows);
  for (uint32_t b0 = g0; b0 < g1; b0 += nc) {
    const uint32_t nb = min(nc, g1 - b0);
    const float* xb = a.x + (uint64_t)b0 * cols;
    // Q8_0 activations: four threads per 32-element block, eight elements each.
    for (uint32_t t = tid; t < nb * K * 4u; t += kQThreads) {
      const uint32_t b = t / (K * 4u), rem = t % (K * 4u), blk = rem >> 2, qtr = rem & 3u;
      uint2 packed;
      float scale;
      int s;
      q8_0_eighth(xb + (uint64_t)b * cols + blk * 32u + qtr * 8u, packed, scale, s);
      *(uint2*)(act_q + (uint64_t)b * cols + blk * 32u + qtr * 8u) = packed;
      if (qtr == 0) {
        act_scale[b * K + blk] = scale;
        act_sum[b * K + blk] = s;
      }
    }
    __syncthreads();

    // Every (row, block) term of the tile: the scale product and the integer dot, per activation
    // row. Tiles of more than kU * 256 terms (rows over 32768 inputs) load further units in turn.
    auto terms = [&](const QBlock<FMT>& wb, uint32_t u) {
      const uint32_t row = u / K, blk = u % K;
      const float wscale = f16_bits_to_float(wb.h[0]);
      for (uint32_t b = 0; b < nb; ++b) {
        const int* aq = (const int*)(act_q + (uint64_t)b * cols + blk * 32u);
        const int d = wb.dot(aq, act_sum[b * K + blk]);
        const uint32_t at = (b * R + row) * Kp + blk;
        t_scale[at] = wscale * act_scale[b * K + blk];
        t_dot[at] = (float)d;
      }
    };
#pragma unroll
    for (uint32_t i = 0; i < kU; ++i)
      if (tid + i * kQThreads < nunits) terms(unit[i], tid + i * kQThreads);
    for (uint32_t u = tid + kU * kQThreads; u < nunits; u += kQThreads) {
      QBlock<FMT> wb;
      wb.load(wrec + (uint64_t)u * kRecHalves);
      terms(wb, u);
    }
    __syncthreads();

    // One thread per (activation row, output row): sum = fma(scale, dot, sum) over the blocks in
    // order, then the optional bias or residual (one float add, as addOptionalBias and the
    // residual loop do).
    for (uint32_t t = tid; t < nb * nrows; t += kQThreads) {
      const uint32_t b = t / nrows, row = t % nrows;
      const float* ps = t_scale + (b * R + row) * Kp;
      const float* pd = t_dot + (b * R + row) * Kp;
      float sum = 0.0f;
      uint32_t blk = 0;
      for (; blk + 8 <= K; blk += 8) {  // the LDS reads of eight steps ahead of their fma chain
        float sc[8], dt[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = ps[blk + i], dt[i] = pd[blk + i];
#pragma unroll
        for (int i = 0; i < 8; ++i) sum = __builtin_fmaf(sc[i], dt[i], sum);
      }
      for (; blk < K; ++blk) sum = __builtin_fmaf(ps[blk], pd[blk], sum);
      const uint32_t r = r0 + row;
      const uint64_t o = (uint64_t)(b0 + b) * rows + r;
      if (a.addend_mode == 1) sum = sum + addend[r];
      else if (a.addend_mode == 2) sum = sum + addend[o];
      out[o] = sum;
    }
  }
}

// ---------------------------------------------------------------- K-quants (Q4_K, Q5_K, Q6_K)
//
// Q8_K activations (quantize_q8_k_batch, backend-native/src/main/rust/model-kernels/src/lib.rs:
// 3906-3952): per 256-element block, the element of largest magnitude (the first on ties, NaN
// skipped) sets inverse = -127 / max, element = min(nearest(inverse * x), 127), sums of 16
// elements, scale = 1 / inverse. Rows as backend-native's scalar row kernels form them
// (dot_q4_k_q8_k_row_scalar :3410-3459, dot_q5_k_q8_k_row_scalar :3461-3518,
// dot_q6_k_q8_k_row_scalar :3519-3577); the integer parts are exact in any order, so eight
// threads share each (row, block) and only the float chains keep the reference's order. Q5_K is
// Q4_K with a 32-byte array of fifth bits ahead of the nibbles (bit g of byte i: element i of
// group g), so the two share their code and float chain.
template <int FMT>
__global__ __launch_bounds__(kQThreads) void qkmatvec_kernel(const QMatArgs a) {
  constexpr bool kQ45 = FMT == 2 || FMT == 4;          // Q4_K or Q5_K
  constexpr uint32_t kNT = kQ45 ? 4u : 9u;             // floats per (row, block) term
  constexpr uint32_t kBlockBytes = FMT == 2 ? 144u : FMT == 4 ? 176u : 210u;
  extern __shared__ __attribute__((aligned(16))) unsigned char q_lds[];
  // One pass of nc activation rows in LDS at a time (qmatvec_kernel); the tile's weight blocks
  // come from memory in the first pass and from the caches in later ones.
  const uint32_t nc = a.chunk, cols = a.cols, KB = a.blocks, R = a.rows_per_tile;
  const uint32_t rs = KB * kNT + 1;  // floats per (activation row, output row) of terms
  int8_t* act_q = (int8_t*)q_lds;                                   // [nc][cols]
  float* act_scale = (float*)(q_lds + ((nc * cols + 15u) & ~15u));  // [nc][KB]
  int* act_sum = (int*)(act_scale + nc * KB);                       // [nc][cols / 16]
  float* terms = (float*)(act_sum + nc * (cols / 16u));             // [nc][R][rs]

  uint32_t mi = 0;
  for (uint32_t i = 1; i < a.count; ++i) mi = blockIdx.x >= a.m[i].tile0 ? i : mi;
  const uint8_t* w = a.m[mi].w;
  float* out = a.m[mi].out;
  const float* addend = a.m[mi].addend;
  const uint32_t rows = a.m[mi].rows;
  const uint32_t r0 = (blockIdx.x - a.m[mi].tile0) * R;
  const uint32_t nrows = min(R, rows - r0);
  const uint32_t nunits = nrows * KB;
  const uint8_t* wtile = w + (uint64_t)r0 * KB * kBlockBytes;
  const uint32_t tid = threadIdx.x, sub = tid & 7u;

  const uint32_t g0 = blockIdx.y * a.group_rows, g1 = min(a.batch, g0 + a.group_rows);
  for (uint32_t b0 = g0; b0 < g1; b0 += nc) {
    const uint32_t nb = min(nc, g1 - b0);
    const float* xb = a.x + (uint64_t)b0 * cols;
    // Q8_K activations: 32 threads per block, eight consecutive elements each.
    for (uint32_t t = tid; t < nb * KB * 32u; t += kQThreads) {
      const uint32_t b = t / (KB * 32u), blk = (t / 32u) % KB, part = t & 31u;
      uint2 packed;
      int s;
      float scale;
      q8_k_part(xb + (uint64_t)b * cols + blk * 256u + part * 8u, part, packed, s, scale);
      *(uint2*)(act_q + (uint64_t)b * cols + blk * 256u + part * 8u) = packed;
      if ((part & 1u) == 0) act_sum[b * (cols / 16u) + blk * 16u + part / 2u] = s;
      if (part == 0) act_scale[b * KB + blk] = scale;
    }
    __syncthreads();

    // Terms: eight threads per (row, block); every thread of a unit runs the same batch loop.
    for (uint32_t t = tid; t < ((nunits * 8u + 63u) & ~63u); t += kQThreads) {
      const uint32_t u = min(t / 8u, nunits - 1u);  // the last wave's spare lanes repeat a unit
      const bool real = t / 8u < nunits;
      const uint32_t row = u / KB, blk = u % KB;
      const uint8_t* wb = wtile + (uint64_t)u * kBlockBytes;
      if constexpr (kQ45) {
        const uint16_t* h = (const uint16_t*)wb;
        const float wd = f16_bits_to_float(h[0]), wdmin = f16_bits_to_float(h[1]);
        uint32_t scb[12];
#pragma unroll
        for (int i = 0; i < 6; ++i) {
          const uint32_t x = h[2 + i];
          scb[2 * i] = x & 0xFFu;
          scb[2 * i + 1] = x >> 8;
        }
        const uint32_t g = sub;
        const int sc = g < 4 ? (int)(scb[g] & 63u) : (int)((scb[g + 4] & 15u) | ((scb[g - 4] >> 6) << 4));
        const int mn = g < 4 ? (int)(scb[g + 4] & 63u) : (int)((scb[g + 4] >> 4) | ((scb[g] >> 6) << 4));
        // The group's 32 quants as 8 words of 4 bytes: nibbles (Q5_K: plus bit g of each qh byte
        // as the byte's bit 4).
        uint32_t nib[8];
        const uint16_t* qn16 = h + (FMT == 4 ? 24 : 8) + (g >> 1) * 16;
        const uint32_t shift = (g & 1u) * 4u;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          nib[i] = (((uint32_t)qn16[2 * i] | ((uint32_t)qn16[2 * i + 1] << 16)) >> shift) & 0x0F0F0F0Fu;
        if constexpr (FMT == 4) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t qh = (uint32_t)h[8 + 2 * i] | ((uint32_t)h[9 + 2 * i] << 16);
            nib[i] |= ((qh >> g) & 0x01010101u) << 4;
          }
        }
        for (uint32_t b = 0; b < nb; ++b) {
          const int* aq = (const int*)(act_q + (uint64_t)b * cols + blk * 256u + g * 32u);
          int dot = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) dot = __builtin_amdgcn_sdot4((int)nib[i], aq[i], dot, false);
          const int* s16 = act_sum + b * (cols / 16u) + blk * 16u;
          const int qs = sum8(sc * dot), ms = sum8(mn * (s16[2 * g] + s16[2 * g + 1]));
          if (real && sub == 0) {
            const float as = act_scale[b * KB + blk];
            float* tt = terms + (b * R + row) * rs + blk * kNT;
            tt[0] = wd * as;
            tt[1] = (float)qs;
            tt[2] = -(wdmin * as);
            tt[3] = (float)ms;
          }
        }
      } else {
        // Lane class l = sub: elements i, i + 8, i + 16, i + 24 of each 32-run, both halves, all
        // four quarters (ql low / high nibble, qh bit pairs), each times its int8 group scale.
        const int8_t* sc = (const int8_t*)(wb + 192);
        const float wd = (float)__builtin_bit_cast(_Float16, (uint16_t)(wb[208] | (wb[209] << 8)));
        int ql1[8], ql2[8], qhh[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t hf = k >> 2, i = sub + 8u * (k & 3);
          ql1[k] = wb[hf * 64u + i];
          ql2[k] = wb[hf * 64u + 32u + i];
          qhh[k] = wb[128u + hf * 32u + i];
        }
        for (uint32_t b = 0; b < nb; ++b) {
          const int8_t* aq = act_q + (uint64_t)b * cols + blk * 256u;
          int acc = 0;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const uint32_t hf = k >> 2, i = sub + 8u * (k & 3), si = i / 16u;
            const int q1 = ((ql1[k] & 15) | ((qhh[k] & 3) << 4)) - 32;
            const int q2 = ((ql2[k] & 15) | (((qhh[k] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql1[k] >> 4) | (((qhh[k] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql2[k] >> 4) | (((qhh[k] >> 6) & 3) << 4)) - 32;
            const int8_t* aa = aq + hf * 128u;
            acc += sc[hf * 8u + si] * q1 * aa[i];
            acc += sc[hf * 8u + si + 2u] * q2 * aa[i + 32u];
            acc += sc[hf * 8u + si + 4u] * q3 * aa[i + 64u];
            acc += sc[hf * 8u + si + 6u] * q4 * aa[i + 96u];
          }
          if (real) {
            float* tt = terms + (b * R + row) * rs + blk * kNT;
            if (sub == 0) tt[0] = wd * act_scale[b * KB + blk];
            tt[1 + sub] = (float)acc;
          }
        }
      }
    }
    __syncthreads();

    for (uint32_t t = tid; t < nb * nrows; t += kQThreads) {
      const uint32_t b = t / nrows, row = t % nrows;
      const float* tt = terms + (b * R + row) * rs;
      float sum = 0.0f;
      if constexpr (kQ45) {
        for (uint32_t blk = 0; blk < KB; ++blk) {
          sum = __builtin_fmaf(tt[blk * 4], tt[blk * 4 + 1], sum);
          sum = __builtin_fmaf(tt[blk * 4 + 2], tt[blk * 4 + 3], sum);
        }
      } else {
        float ls[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (uint32_t blk = 0; blk < KB; ++blk)
#pragma unroll
          for (int l = 0; l < 8; ++l) ls[l] = __builtin_fmaf(tt[blk * 9], tt[blk * 9 + 1 + l], ls[l]);
#pragma unroll
        for (int l = 0; l < 8; ++l) sum = sum + ls[l];
      }
      const uint32_t r = r0 + row;
      const uint64_t o = (uint64_t)(b0 + b) * rows + r;
      if (a.addend_mode == 1) sum = sum + addend[r];
      else if (a.addend_mode == 2) sum = sum + addend[o];
      out[o] = sum;
    }
  }
}

// ---------------------------------------------------------------- prefill-sized batches (GEMM)
//
// For batches of kQGemmMinBatch activation rows and more, the 32-element block formats (Q4_0,
// Q8_0, Q5_0) run as a register-tiled matrix product: the activations are quantized to Q8_0 once
// (q8_0_quant_kernel, into scratch), then each workgroup computes a tile of kQGemmTile weight
// rows x kQGemmTile activation rows, every thread a 4 x 4 block of outputs. The weight and
// activation blocks of kQGemmKc consecutive 32-element blocks at a time are staged in LDS as
// signed int8 (the weight nibbles with their offset applied, so the integer dot needs no
// correction term) with their f32 scales; each output is the reference's in-order chain of
// fma(weightScale * activationScale, integer block dot, sum) over the blocks, so the results are
// the same bits as the matrix-vector kernel's.

// Q8_0 activations [batch][cols] -> int8 [batch][cols] and f32 scales [batch][cols / 32]; four
// threads per block.
__global__ __launch_bounds__(kQThreads) void q8_0_quant_kernel(const float* x, uint32_t batch,
                                                               uint32_t cols, int8_t* q,
                                                               float* scales) {
  const uint32_t K = cols / 32u;
  const uint64_t units = (uint64_t)batch * K * 4u;
  const uint64_t t = (uint64_t)blockIdx.x * kQThreads + threadIdx.x;
  // The grid covers whole quads (units is a multiple of 4), so the four lanes of a quad are
  // active together for the DPP exchanges.
  if (t >= units) return;
  const uint64_t b = t / (K * 4u);
  const uint32_t rem = (uint32_t)(t % (K * 4u)), blk = rem >> 2, qtr = rem & 3u;
  uint2 packed;
  float scale;
  int s;
  q8_0_eighth(x + b * cols + blk * 32u + qtr * 8u, packed, scale, s);
  *(uint2*)(q + b * cols + blk * 32u + qtr * 8u) = packed;
  if (qtr == 0) scales[b * K + blk] = scale;
}

namespace {

// Each byte of x (below 128) minus the byte `off` (at most 128), as signed bytes: with bit 7 set
// first no byte's subtraction borrows from the next.
__device__ __forceinline__ uint32_t bytes_minus(uint32_t x, uint32_t off4) {
  return ((x | 0x80808080u) - off4) ^ 0x80808080u;
}

// A loaded weight block as 32 signed int8 (8 words, element order) and its f32 scale.
template <int FMT>
__device__ __forceinline__ void gemm_weight_unpack(const QBlock<FMT>& blk, uint32_t (&wd)[8], float& scale) {
  scale = f16_bits_to_float(blk.h[0]);
  if constexpr (FMT == 1) {
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) wd[j] = blk.word(j);
  } else if constexpr (FMT == 0) {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t w = blk.word(j);
      wd[j] = bytes_minus(w & 0x0F0F0F0Fu, 0x08080808u);
      wd[4 + j] = bytes_minus((w >> 4) & 0x0F0F0F0Fu, 0x08080808u);
    }
  } else {
    const uint32_t high = blk.word(0);
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t w = blk.h[3 + 2 * j] | (blk.h[4 + 2 * j] << 16);
      wd[j] = bytes_minus((w & 0x0F0F0F0Fu) | fifth_bits((high >> (4 * j)) & 15u), 0x10101010u);
      wd[4 + j] = bytes_minus(((w >> 4) & 0x0F0F0F0Fu) | fifth_bits((high >> (16 + 4 * j)) & 15u),
                              0x10101010u);
    }
  }
}

}  // namespace

template <int FMT>
__global__ __launch_bounds__(kQThreads, 2) void qgemm_kernel(const QMatArgs a, const int8_t* aq,
                                                             const float* as) {
  constexpr uint32_t T = kQGemmTile, KC = kQGemmKc, kRow = KC * 32u + 16u;  // bytes per LDS row
  __shared__ __attribute__((aligned(16))) int8_t s_w[T * kRow];
  __shared__ __attribute__((aligned(16))) int8_t s_a[T * kRow];
  __shared__ float s_ws[T][KC];
  __shared__ float s_as[T][KC];
  const uint32_t K = a.blocks, cols = a.cols, batch = a.batch;
  uint32_t mi = 0;
  for (uint32_t i = 1; i < a.count; ++i) mi = blockIdx.x >= a.m[i].tile0 ? i : mi;
  const uint8_t* w = a.m[mi].w;
  float* out = a.m[mi].out;
  const float* addend = a.m[mi].addend;
  const uint32_t rows = a.m[mi].rows;
  const uint32_t r0 = (blockIdx.x - a.m[mi].tile0) * T, b0 = blockIdx.y * T;
  const uint32_t tid = threadIdx.x;
  const uint32_t ti = tid / 16u, tj = tid % 16u;  // outputs: weight rows 4 ti.., activation rows 4 tj..
  constexpr uint32_t kRecHalves = QBlock<FMT>::kHalves;
  // Staging unit of this thread: one block (row su / KC, block su % KC of the chunk) of the
  // weight tile and one of the activation tile.
  const uint32_t su_row = tid / KC, su_k = tid % KC;
  static_assert(T * KC == kQThreads, "one staged block per thread and tile");
  const bool w_ok = r0 + su_row < rows, a_ok = b0 + su_row < batch;
  const uint16_t* w_rec = (const uint16_t*)(w + ((uint64_t)min(r0 + su_row, rows - 1) * K) * (2u * kRecHalves));
  const int8_t* a_row = aq + (uint64_t)min(b0 + su_row, batch - 1) * cols;
  const float* as_row = as + (uint64_t)min(b0 + su_row, batch - 1) * K;

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

  // This thread's staging unit of one k-step, as loaded (the weight block still packed). The
  // next step's unit is loaded while the current one is computed, so each step's global loads are
  // in flight during the previous step's dot products instead of ahead of its own.
  struct Stage {
    QBlock<FMT> wb;
    uint4 a0, a1;
    float asc;
    bool w_valid;
  };
  auto load_stage = [&](uint32_t k0, Stage& st) {
    const uint32_t k = k0 + su_k;
    st.a0 = make_uint4(0u, 0u, 0u, 0u);
    st.a1 = st.a0;
    st.asc = 0.0f;
    st.w_valid = k < K && w_ok;
    if (st.w_valid) st.wb.load(w_rec + (uint64_t)k * kRecHalves);
    if (k < K && a_ok) {
      st.a0 = *(const uint4*)(a_row + k * 32u);
      st.a1 = *(const uint4*)(a_row + k * 32u + 16u);
      st.asc = as_row[k];
    }
  };
  Stage st;
  load_stage(0, st);
  for (uint32_t k0 = 0; k0 < K; k0 += KC) {
    {
      uint32_t wd[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
      float wsc = 0.0f;
      if (st.w_valid) gemm_weight_unpack<FMT>(st.wb, wd, wsc);
      uint4* dw = (uint4*)(s_w + su_row * kRow + su_k * 32u);
      dw[0] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      dw[1] = make_uint4(wd[4], wd[5], wd[6], wd[7]);
      uint4* da = (uint4*)(s_a + su_row * kRow + su_k * 32u);
      da[0] = st.a0;
      da[1] = st.a1;
      s_ws[su_row][su_k] = wsc;
      s_as[su_row][su_k] = st.asc;
    }
    __syncthreads();
    if (k0 + KC < K) load_stage(k0 + KC, st);
    const uint32_t kn = min(KC, K - k0);
    for (uint32_t kb = 0; kb < kn; ++kb) {
      uint4 wv[4][2], av[4][2];
      float wsc[4], asc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4* pw = (const uint4*)(s_w + (4u * ti + i) * kRow + kb * 32u);
        wv[i][0] = pw[0];
        wv[i][1] = pw[1];
        wsc[i] = s_ws[4u * ti + i][kb];
        const uint4* pa = (const uint4*)(s_a + (4u * tj + i) * kRow + kb * 32u);
        av[i][0] = pa[0];
        av[i][1] = pa[1];
        asc[i] = s_as[4u * tj + i][kb];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // The block's first dot in the three-operand form with an inline zero accumulator:
          // the accumulating form the compiler picks would need a register cleared first.
          int d;
          asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(d) : "v"((int)wv[i][0].x), "v"((int)av[j][0].x));
          d = __builtin_amdgcn_sdot4((int)wv[i][0].y, (int)av[j][0].y, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][0].z, (int)av[j][0].z, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][0].w, (int)av[j][0].w, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].x, (int)av[j][1].x, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].y, (int)av[j][1].y, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].z, (int)av[j][1].z, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].w, (int)av[j][1].w, d, false);
          float sc;
          {
#pragma clang fp contract(off)
            sc = wsc[i] * asc[j];
          }
          acc[i][j] = __builtin_fmaf(sc, (float)d, acc[i][j]);
        }
    }
    __syncthreads();  // the next chunk overwrites the stages
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t b = b0 + 4u * tj + j;
    if (b >= batch) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = r0 + 4u * ti + i;
      if (r >= rows) continue;
      const uint64_t o = (uint64_t)b * rows + r;
      float v = acc[i][j];
      if (a.addend_mode == 1) v = v + addend[r];
      else if (a.addend_mode == 2) v = v + addend[o];
      out[o] = v;
    }
  }
}

// Q8_K activations [batch][cols] -> int8 [batch][cols], f32 scales [batch][cols / 256] and int
// 16-element sums [batch][cols / 16]; 32 threads per block.
__global__ __launch_bounds__(kQThreads) void q8_k_quant_kernel(const float* x, uint32_t batch,
                                                               uint32_t cols, int8_t* q,
                                                               float* scales, int* sums) {
  const uint32_t KB = cols / 256u;
  const uint64_t units = (uint64_t)batch * KB * 32u;
  const uint64_t t = (uint64_t)blockIdx.x * kQThreads + threadIdx.x;
  if (t >= units) return;  // whole blocks: units is a multiple of 32
  const uint64_t b = t / (KB * 32u);
  const uint32_t blk = (uint32_t)((t / 32u) % KB), part = (uint32_t)(t & 31u);
  uint2 packed;
  int s;
  float scale;
  q8_k_part(x + b * cols + blk * 256u + part * 8u, part, packed, s, scale);
  *(uint2*)(q + b * cols + blk * 256u + part * 8u) = packed;
  if ((part & 1u) == 0) sums[b * (cols / 16u) + blk * 16u + part / 2u] = s;
  if (part == 0) scales[b * KB + blk] = scale;
}

// The register-tiled product of Q4_K (FMT 2) and Q5_K (FMT 4) weights on Q8_K activations, with
// the float order of dot_q4_k_q8_k_row_scalar / dot_q5_k_q8_k_row_scalar (RS:3410-3518): per
// 256-element block the integer sums qsum = sum over groups of scale_g * dot_g and msum = sum of
// min_g * (the group's two 16-element activation sums), then sum = fma(d * as, qsum, sum) and
// sum = fma(-(dmin * as), msum, sum). Tiles of kQGemmTile x kQGemmTile outputs, 4 x 4 per thread,
// one 256-element block staged per step: the quants as bytes (0..31), each row's 6-bit scales and
// mins, d and dmin; the activations' bytes, scale and per-group sums. The integer arithmetic is
// exact in narrow forms: a group's dot is at most 32 x 31 x 128 in magnitude, so scale_g * dot_g
// is a 24-bit multiply-add, and mins (0..63) and group sums (at most 32 x 128) are 16-bit, so msum
// is four v_dot2_i32_i16.
template <int FMT>
__global__ __launch_bounds__(kQThreads, 2) void qkgemm_kernel(const QMatArgs a, const int8_t* aq,
                                                              const float* as, const int* asum) {
  constexpr uint32_t T = kQGemmTile, kRow = 256u + 16u, kBB = FMT == 2 ? 144u : 176u;
  __shared__ __attribute__((aligned(16))) int8_t s_w[T * kRow];
  __shared__ __attribute__((aligned(16))) int8_t s_a[T * kRow];
  __shared__ __attribute__((aligned(16))) int s_sc[T][8];
  __shared__ __attribute__((aligned(16))) int16_t s_mn[T][8];
  __shared__ __attribute__((aligned(16))) int16_t s_gs[T][8];
  __shared__ float s_d[T], s_dm[T], s_as[T];
  const uint32_t KB = a.blocks, cols = a.cols, batch = a.batch;
  uint32_t mi = 0;
  for (uint32_t i = 1; i < a.count; ++i) mi = blockIdx.x >= a.m[i].tile0 ? i : mi;
  const uint8_t* w = a.m[mi].w;
  float* out = a.m[mi].out;
  const float* addend = a.m[mi].addend;
  const uint32_t rows = a.m[mi].rows;
  const uint32_t r0 = (blockIdx.x - a.m[mi].tile0) * T, b0 = blockIdx.y * T;
  const uint32_t tid = threadIdx.x;
  const uint32_t ti = tid / 16u, tj = tid % 16u;
  // Staging: row tid / 4, part tid % 4 (groups 2 part and 2 part + 1: 64 elements).
  const uint32_t su_row = tid / 4u, part = tid % 4u;
  const bool w_ok = r0 + su_row < rows, a_ok = b0 + su_row < batch;
  const uint8_t* w_row = w + (uint64_t)min(r0 + su_row, rows - 1) * KB * kBB;
  const uint64_t arow = min(b0 + su_row, batch - 1);

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

  for (uint32_t kb = 0; kb < KB; ++kb) {
    {
      uint32_t q[16];  // 64 quant bytes: group 2 part, then 2 part + 1
#pragma unroll
      for (int i = 0; i < 16; ++i) q[i] = 0u;
      if (w_ok) {
        const uint16_t* h = (const uint16_t*)(w_row + (uint64_t)kb * kBB);
        const uint16_t* qs = h + (FMT == 4 ? 24 : 8) + part * 16;  // 32 bytes of nibbles
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t x = (uint32_t)qs[2 * i] | ((uint32_t)qs[2 * i + 1] << 16);
          q[i] = x & 0x0F0F0F0Fu;
          q[8 + i] = (x >> 4) & 0x0F0F0F0Fu;
        }
        if constexpr (FMT == 4) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const uint32_t qh = (uint32_t)h[8 + 2 * i] | ((uint32_t)h[9 + 2 * i] << 16);
            q[i] |= ((qh >> (2 * part)) & 0x01010101u) << 4;
            q[8 + i] |= ((qh >> (2 * part + 1)) & 0x01010101u) << 4;
          }
        }
        if (part == 0) {
          s_d[su_row] = f16_bits_to_float(h[0]);
          s_dm[su_row] = f16_bits_to_float(h[1]);
          uint32_t scb[12];
#pragma unroll
          for (int i = 0; i < 6; ++i) {
            scb[2 * i] = h[2 + i] & 0xFFu;
            scb[2 * i + 1] = h[2 + i] >> 8;
          }
#pragma unroll
          for (int g = 0; g < 8; ++g) {
            s_sc[su_row][g] = g < 4 ? (int)(scb[g] & 63u) : (int)((scb[g + 4] & 15u) | ((scb[g - 4] >> 6) << 4));
            s_mn[su_row][g] = (int16_t)(g < 4 ? (scb[g + 4] & 63u) : ((scb[g + 4] >> 4) | ((scb[g] >> 6) << 4)));
          }
        }
      } else if (part == 0) {
        s_d[su_row] = 0.0f;
        s_dm[su_row] = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          s_sc[su_row][g] = 0;
          s_mn[su_row][g] = 0;
        }
      }
      uint4* dw = (uint4*)(s_w + su_row * kRow + part * 64u);
#pragma unroll
      for (int i = 0; i < 4; ++i) dw[i] = make_uint4(q[4 * i], q[4 * i + 1], q[4 * i + 2], q[4 * i + 3]);
      uint4 av[4] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u),
                     make_uint4(0u, 0u, 0u, 0u)};
      int4 sm = make_int4(0, 0, 0, 0);
      float asc = 0.0f;
      if (a_ok) {
        const uint4* pa = (const uint4*)(aq + arow * cols + kb * 256u + part * 64u);
#pragma unroll
        for (int i = 0; i < 4; ++i) av[i] = pa[i];
        sm = *(const int4*)(asum + arow * (cols / 16u) + kb * 16u + part * 4u);
        asc = as[arow * KB + kb];
      }
      uint4* da = (uint4*)(s_a + su_row * kRow + part * 64u);
#pragma unroll
      for (int i = 0; i < 4; ++i) da[i] = av[i];
      s_gs[su_row][2 * part] = (int16_t)(sm.x + sm.y);
      s_gs[su_row][2 * part + 1] = (int16_t)(sm.z + sm.w);
      if (part == 0) s_as[su_row] = asc;
    }
    __syncthreads();
    int qsum[4][4], msum[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) qsum[i][j] = msum[i][j] = 0;
    for (int g = 0; g < 8; ++g) {
      uint4 wv[4][2], avv[4][2];
      int sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4* pw = (const uint4*)(s_w + (4u * ti + i) * kRow + g * 32u);
        wv[i][0] = pw[0];
        wv[i][1] = pw[1];
        sc[i] = s_sc[4u * ti + i][g];
        const uint4* pa = (const uint4*)(s_a + (4u * tj + i) * kRow + g * 32u);
        avv[i][0] = pa[0];
        avv[i][1] = pa[1];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          int d;  // first dot in the zero-accumulator form: no register to clear
          asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(d) : "v"((int)wv[i][0].x), "v"((int)avv[j][0].x));
          d = __builtin_amdgcn_sdot4((int)wv[i][0].y, (int)avv[j][0].y, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][0].z, (int)avv[j][0].z, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][0].w, (int)avv[j][0].w, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].x, (int)avv[j][1].x, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].y, (int)avv[j][1].y, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].z, (int)avv[j][1].z, d, false);
          d = __builtin_amdgcn_sdot4((int)wv[i][1].w, (int)avv[j][1].w, d, false);
          qsum[i][j] += __mul24(sc[i], d);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 m = *(const uint4*)&s_mn[4u * ti + i][0];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 gs = *(const uint4*)&s_gs[4u * tj + j][0];
        int t = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, m.x), __builtin_bit_cast(short2_t, gs.x), 0, false);
        t = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, m.y), __builtin_bit_cast(short2_t, gs.y), t, false);
        t = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, m.z), __builtin_bit_cast(short2_t, gs.z), t, false);
        msum[i][j] = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, m.w), __builtin_bit_cast(short2_t, gs.w), t, false);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float wd = s_d[4u * ti + i], wdm = s_dm[4u * ti + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float asj = s_as[4u * tj + j];
        float d, dm;
        {
#pragma clang fp contract(off)
          d = wd * asj;
          dm = wdm * asj;
        }
        acc[i][j] = __builtin_fmaf(d, (float)qsum[i][j], acc[i][j]);
        acc[i][j] = __builtin_fmaf(-dm, (float)msum[i][j], acc[i][j]);
      }
    }
    __syncthreads();  // the next block overwrites the stages
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t b = b0 + 4u * tj + j;
    if (b >= batch) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = r0 + 4u * ti + i;
      if (r >= rows) continue;
      const uint64_t o = (uint64_t)b * rows + r;
      float v = acc[i][j];
      if (a.addend_mode == 1) v = v + addend[r];
      else if (a.addend_mode == 2) v = v + addend[o];
      out[o] = v;
    }
  }
}

// The register-tiled product of Q6_K weights on Q8_K activations, with the float order of
// dot_q6_k_q8_k_row_scalar (RS:3519-3577): per 256-element block eight integer lane sums (lane l
// takes the elements whose index within their 32-element run is l, l + 8, l + 16 or l + 24, in
// both 128-element halves), then lane_l = fma(d * as, isum_l, lane_l) for l = 0..7; after the last
// block the eight lanes are added in order to 0. One block per step: each weight quant is staged
// with its 16-element sub-block scale applied (16 bits: scale x (quant - 32)) and each activation
// as 16 bits, both in lane-major order (int16 index 32 l + 16 half + 4 run + i / 8 for element
// 128 half + 32 run + i), so a lane's integer sum is 16 v_dot2_i32_i16 over 64 contiguous bytes;
// integer sums are exact in any order. Tiles of kQGemmTile x kQGemmTile outputs, 4 x 4 per thread,
// each output with its eight lane chains.
__global__ __launch_bounds__(kQThreads, 2) void q6gemm_kernel(const QMatArgs a, const int8_t* aq,
                                                              const float* as) {
  constexpr uint32_t T = kQGemmTile, kRow = 256u + 8u, kBB = 210u;  // int16 per staged row
  __shared__ __attribute__((aligned(16))) int16_t s_w[T * kRow];
  __shared__ __attribute__((aligned(16))) int16_t s_a[T * kRow];
  __shared__ float s_d[T], s_as[T];
  const uint32_t KB = a.blocks, cols = a.cols, batch = a.batch;
  uint32_t mi = 0;
  for (uint32_t i = 1; i < a.count; ++i) mi = blockIdx.x >= a.m[i].tile0 ? i : mi;
  const uint8_t* w = a.m[mi].w;
  float* out = a.m[mi].out;
  const float* addend = a.m[mi].addend;
  const uint32_t rows = a.m[mi].rows;
  const uint32_t r0 = (blockIdx.x - a.m[mi].tile0) * T, b0 = blockIdx.y * T;
  const uint32_t tid = threadIdx.x;
  const uint32_t ti = tid / 16u, tj = tid % 16u;
  // Staging: row tid / 4, part tid % 4 = 128-element half (part / 2) and elements i0 .. i0 + 15 of
  // its four 32-element runs (i0 = 16 (part % 2)), which land in dword (8 half + 2 run + part % 2)
  // of each lane's 16.
  const uint32_t su_row = tid / 4u, part = tid % 4u, half = part >> 1, i0 = (part & 1u) * 16u;
  const bool w_ok = r0 + su_row < rows, a_ok = b0 + su_row < batch;
  const uint8_t* w_row = w + (uint64_t)min(r0 + su_row, rows - 1) * KB * kBB;
  const uint64_t arow = min(b0 + su_row, batch - 1);
  uint32_t* const sw_row = (uint32_t*)(s_w + su_row * kRow) + 8u * half + (part & 1u);
  uint32_t* const sa_row = (uint32_t*)(s_a + su_row * kRow) + 8u * half + (part & 1u);

  float acc[4][4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int l = 0; l < 8; ++l) acc[i][j][l] = 0.0f;

  // 16 bytes at a 2-byte aligned address, as four words.
  auto load16 = [](const uint8_t* p, uint32_t (&x)[4]) {
    const uint16_t* h = (const uint16_t*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (uint32_t)h[2 * i] | ((uint32_t)h[2 * i + 1] << 16);
  };
  // Byte t of four words.
  auto byte_of = [](const uint32_t (&x)[4], int t) -> uint32_t { return (x[t >> 2] >> (8 * (t & 3))) & 0xFFu; };

  for (uint32_t kb = 0; kb < KB; ++kb) {
    {
      // Weights: ql bytes i0.. of both 32-byte runs of this half, qh bytes i0.., the four
      // sub-block scales of runs 0..3 (scale index 8 half + i0 / 16 + 2 run), d.
      uint32_t la[4] = {0u, 0u, 0u, 0u}, lb[4] = {0u, 0u, 0u, 0u}, hb[4] = {0u, 0u, 0u, 0u};
      int sc[4] = {0, 0, 0, 0};
      if (w_ok) {
        const uint8_t* blk = w_row + (uint64_t)kb * kBB;
        load16(blk + 64u * half + i0, la);
        load16(blk + 64u * half + 32u + i0, lb);
        load16(blk + 128u + 32u * half + i0, hb);
        const uint16_t* sch = (const uint16_t*)(blk + 192u + 8u * half);  // scales 8 half .. + 7
        uint32_t s8[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) s8[i] = sch[i];
#pragma unroll
        for (int run = 0; run < 4; ++run) {
          // scale byte i0 / 16 + 2 run: word run, low byte when i0 = 0, high byte otherwise
          const uint32_t b = (s8[run] >> (i0 == 0u ? 0 : 8)) & 0xFFu;
          sc[run] = (int)(int8_t)b;
        }
        if (part == 0) s_d[su_row] = f16_bits_to_float(((const uint16_t*)blk)[104]);
      } else if (part == 0) {
        s_d[su_row] = 0.0f;
      }
      // Element i0 + t of run `run`: the low nibble of la (runs 0, 2: low / high nibble) or lb
      // (runs 1, 3), the high bits 2 run of hb; elements t and t + 8 share a lane and fill its
      // dword's low and high halves.
#pragma unroll
      for (int run = 0; run < 4; ++run) {
        const uint32_t(&lo)[4] = (run & 1) ? lb : la;
        const int shift = (run >> 1) * 4;
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          int v[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int t = l + 8 * e;
            const int q = (int)(((byte_of(lo, t) >> shift) & 15u) | (((byte_of(hb, t) >> (2 * run)) & 3u) << 4)) - 32;
            v[e] = w_ok ? sc[run] * q : 0;
          }
          sw_row[16 * l + 2 * run] = ((uint32_t)v[0] & 0xFFFFu) | ((uint32_t)v[1] << 16);
        }
      }
      // Activations: bytes i0 .. i0 + 15 of each 32-element run of this half.
      uint4 av[4] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u),
                     make_uint4(0u, 0u, 0u, 0u)};
      float asc = 0.0f;
      if (a_ok) {
        const int8_t* pa = aq + arow * cols + kb * 256u + 128u * half + i0;
#pragma unroll
        for (int run = 0; run < 4; ++run) av[run] = *(const uint4*)(pa + 32u * run);
        asc = as[arow * KB + kb];
      }
#pragma unroll
      for (int run = 0; run < 4; ++run) {
        const uint32_t x[4] = {av[run].x, av[run].y, av[run].z, av[run].w};
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          const int v0 = (int)(int8_t)byte_of(x, l), v1 = (int)(int8_t)byte_of(x, l + 8);
          sa_row[16 * l + 2 * run] = ((uint32_t)v0 & 0xFFFFu) | ((uint32_t)v1 << 16);
        }
      }
      if (part == 0) s_as[su_row] = asc;
    }
    __syncthreads();
    float dd[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma clang fp contract(off)
        dd[i][j] = s_d[4u * ti + i] * s_as[4u * tj + j];
      }
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      int isum[4][4];
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {  // lane l's 16 dwords, four at a time
        uint4 wv[4], avv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wv[i] = *(const uint4*)(s_w + (4u * ti + i) * kRow + 32u * l + 8u * qd);
          avv[i] = *(const uint4*)(s_a + (4u * tj + i) * kRow + 32u * l + 8u * qd);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            int d;
            if (qd == 0)  // the lane's first dot in the zero-accumulator form: no register to clear
              asm("v_dot2_i32_i16 %0, %1, %2, 0" : "=v"(d) : "v"(wv[i].x), "v"(avv[j].x));
            else
              d = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, wv[i].x), __builtin_bit_cast(short2_t, avv[j].x), isum[i][j], false);
            d = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, wv[i].y), __builtin_bit_cast(short2_t, avv[j].y), d, false);
            d = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, wv[i].z), __builtin_bit_cast(short2_t, avv[j].z), d, false);
            d = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, wv[i].w), __builtin_bit_cast(short2_t, avv[j].w), d, false);
            isum[i][j] = d;
          }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j][l] = __builtin_fmaf(dd[i][j], (float)isum[i][j], acc[i][j][l]);
    }
    __syncthreads();  // the next block overwrites the stages
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t b = b0 + 4u * tj + j;
    if (b >= batch) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = r0 + 4u * ti + i;
      if (r >= rows) continue;
      const uint64_t o = (uint64_t)b * rows + r;
      float v = 0.0f;
#pragma unroll
      for (int l = 0; l < 8; ++l) v = v + acc[i][j][l];
      if (a.addend_mode == 1) v = v + addend[r];
      else if (a.addend_mode == 2) v = v + addend[o];
      out[o] = v;
    }
  }
}

hipError_t launch_q8_k_quant(const float* x, uint32_t batch, uint32_t cols, int8_t* q,
                             float* scales, int* sums, hipStream_t stream) {
  const uint64_t units = (uint64_t)batch * (cols / 256u) * 32u;
  const uint32_t blocks = (uint32_t)((units + kQThreads - 1) / kQThreads);
  hipLaunchKernelGGL(q8_k_quant_kernel, dim3(blocks), dim3(kQThreads), 0, stream, x, batch, cols,
                     q, scales, sums);
  return hipGetLastError();
}

hipError_t launch_qkgemm(const QMatArgs& a, uint32_t fmt, uint32_t tiles, const int8_t* aq,
                         const float* as, const int* asum, hipStream_t stream) {
  const dim3 grid(tiles, (a.batch + kQGemmTile - 1) / kQGemmTile);
  if (fmt == 2)
    hipLaunchKernelGGL(qkgemm_kernel<2>, grid, dim3(kQThreads), 0, stream, a, aq, as, asum);
  else if (fmt == 4)
    hipLaunchKernelGGL(qkgemm_kernel<4>, grid, dim3(kQThreads), 0, stream, a, aq, as, asum);
  else if (fmt == 3)
    hipLaunchKernelGGL(q6gemm_kernel, grid, dim3(kQThreads), 0, stream, a, aq, as);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_q8_0_quant(const float* x, uint32_t batch, uint32_t cols, int8_t* q,
                             float* scales, hipStream_t stream) {
  const uint64_t units = (uint64_t)batch * (cols / 32u) * 4u;
  const uint32_t blocks = (uint32_t)((units + kQThreads - 1) / kQThreads);
  hipLaunchKernelGGL(q8_0_quant_kernel, dim3(blocks), dim3(kQThreads), 0, stream, x, batch, cols,
                     q, scales);
  return hipGetLastError();
}

hipError_t launch_qgemm(const QMatArgs& a, uint32_t fmt, uint32_t tiles, const int8_t* aq,
                        const float* as, hipStream_t stream) {
  const dim3 grid(tiles, (a.batch + kQGemmTile - 1) / kQGemmTile);
  if (fmt == 0)
    hipLaunchKernelGGL(qgemm_kernel<0>, grid, dim3(kQThreads), 0, stream, a, aq, as);
  else if (fmt == 1)
    hipLaunchKernelGGL(qgemm_kernel<1>, grid, dim3(kQThreads), 0, stream, a, aq, as);
  else if (fmt == 5)
    hipLaunchKernelGGL(qgemm_kernel<5>, grid, dim3(kQThreads), 0, stream, a, aq, as);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_qmatvec(const QMatArgs& a, uint32_t fmt, uint32_t tiles, hipStream_t stream) {
  const size_t lds = qmatvec_lds_bytes(a.chunk, a.cols, a.rows_per_tile);
  const dim3 grid(tiles, (a.batch + a.group_rows - 1) / a.group_rows);
  if (fmt == 0)
    hipLaunchKernelGGL(qmatvec_kernel<0>, grid, dim3(kQThreads), lds, stream, a);
  else if (fmt == 1)
    hipLaunchKernelGGL(qmatvec_kernel<1>, grid, dim3(kQThreads), lds, stream, a);
  else if (fmt == 2)
    hipLaunchKernelGGL(qkmatvec_kernel<2>, grid, dim3(kQThreads),
                       qkmatvec_lds_bytes(2, a.chunk, a.cols, a.rows_per_tile), stream, a);
  else if (fmt == 3)
    hipLaunchKernelGGL(qkmatvec_kernel<3>, grid, dim3(kQThreads),
                       qkmatvec_lds_bytes(3, a.chunk, a.cols, a.rows_per_tile), stream, a);
  else if (fmt == 4)
    hipLaunchKernelGGL(qkmatvec_kernel<4>, grid, dim3(kQThreads),
                       qkmatvec_lds_bytes(4, a.chunk, a.cols, a.rows_per_tile), stream, a);
  else if (fmt == 5)
    hipLaunchKernelGGL(qmatvec_kernel<5>, grid, dim3(kQThreads), lds, stream, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace jma
