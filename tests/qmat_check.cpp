// CPU bounds check of the quantized-projection launches (models_amd/csrc/jma_quant.hip), built
// with g++ and AddressSanitizer / UndefinedBehaviorSanitizer by tests/test_plan_cpu.py.
//
// For each call below it routes every weight format the way quantized_matmul_impl does and plans
// its launch with the runtime's own planner (jma_plan.h): prefill-sized batches run the
// register-tiled product (qgemm_kernel, qkgemm_kernel, q6gemm_kernel) in tiles of kQGemmTile rows
// x kQGemmTile activation rows over activations quantized once into scratch; the others run the
// matrix-vector kernels (plan_qmat, qmat_group_rows), whose workgroups take `chunk` activation
// rows per pass. It then walks every workgroup (x, y) of every launch the way the kernels index
// memory: the matrix a workgroup serves (the last with tile0 <= x), its weight blocks, the
// activations (or the quantized activation scratch) it reads, its LDS arrays, and every output,
// bias and residual element it reads or writes. Every access touches an exactly sized heap array,
// so an index past an extent is a sanitizer error; every output element must be written exactly
// once across the call's launches.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <string>
#include <vector>

#include "jma_plan.h"

namespace {

int failures = 0;

void expect(bool ok, const std::string& what) {
  if (!ok) {
    ++failures;
    fprintf(stderr, "FAIL: %s\n", what.c_str());
  }
}

struct Call {
  std::string name;
  std::vector<uint32_t> formats, rows;
  uint32_t batch, cols, addend_mode;
};

// The routing of quantized_matmul_impl.
bool gemm_format(uint32_t, uint32_t batch) { return batch >= jma::kQGemmMinBatch; }

struct Buffers {
  std::vector<uint8_t*> w;
  std::vector<float*> add;
  float* x = nullptr;           // activations [batch][cols]
  int8_t* aq = nullptr;         // quantized activations [batch][cols]
  float* as = nullptr;          // their scales [batch][cols / block]
  int* asum = nullptr;          // Q8_K 16-element sums [batch][cols / 16]
  std::vector<uint8_t> written;  // per output element
};

volatile float sink = 0.0f;

// Launch table of one format: (matrix, first tile, output offset) in matrix order.
struct M { uint32_t idx, tile0; uint64_t out_off; };

std::vector<M> table(const Call& c, uint32_t fmt, uint32_t R, uint32_t& tiles) {
  std::vector<M> ms;
  tiles = 0;
  uint64_t out_off = 0;
  for (uint32_t i = 0; i < c.formats.size(); ++i) {
    if (c.formats[i] == fmt) {
      ms.push_back({i, tiles, out_off});
      tiles += (c.rows[i] + R - 1) / R;
    }
    out_off += (uint64_t)c.batch * c.rows[i];
  }
  return ms;
}

// qgemm_kernel / qkgemm_kernel: each thread stages one weight block and one activation block per
// step (rows clamped to the last valid one and skipped past it), every thread writes 4 x 4 outputs.
// q6gemm_kernel (Q6_K): four threads per row each stage a quarter of the 210-byte block and of the
// 256 activation bytes into lane-major int16 stages.
void walk_gemm(const Call& c, uint32_t fmt, Buffers& B) {
  const bool kq = jma::qmat_kquant(fmt);
  const uint32_t T = jma::kQGemmTile, KB = c.cols / jma::qmat_block_elems(fmt);
  const uint32_t KC = kq ? 1u : jma::kQGemmKc;  // blocks staged per step
  const uint32_t per = kq ? 4u : KC;            // staging threads per row (K-quants: 4 parts)
  const uint32_t kRow = kq ? 256u + 16u : KC * 32u + 16u;
  uint32_t tiles;
  const std::vector<M> ms = table(c, fmt, T, tiles);
  const uint32_t bb = jma::qmat_block_bytes(fmt);
  const uint32_t gy = (c.batch + T - 1) / T;
  expect(gy <= 65535u, c.name + ": product grid rows");
  int8_t* lds = new int8_t[T * kRow];
  constexpr uint32_t kRow6 = 256u + 8u;  // q6gemm_kernel's int16 per staged row
  int16_t* lds16 = new int16_t[T * kRow6];
  for (uint32_t bx = 0; bx < tiles; ++bx) {
    uint32_t mi = 0;
    for (uint32_t i = 1; i < ms.size(); ++i) mi = bx >= ms[i].tile0 ? i : mi;
    const uint32_t idx = ms[mi].idx, rows = c.rows[idx];
    const uint32_t r0 = (bx - ms[mi].tile0) * T;
    expect(r0 < rows, c.name + ": product tile past its matrix");
    for (uint32_t by = 0; by < gy; ++by) {
      const uint32_t b0 = by * T;
      for (uint32_t tid = 0; tid < 256; ++tid) {
        const uint32_t su_row = tid / per, su = tid % per;
        const bool w_ok = r0 + su_row < rows, a_ok = b0 + su_row < c.batch;
        const uint64_t wrow = std::min(r0 + su_row, rows - 1), arow = std::min(b0 + su_row, c.batch - 1);
        if (fmt == 3) {  // q6gemm_kernel: int16 stages of kRow6 halves per row
          const uint32_t half = su >> 1, i0 = (su & 1u) * 16u;
          for (uint32_t k = 0; k < KB; ++k) {
            const uint64_t blk = (wrow * KB + k) * bb;
            if (w_ok) {
              for (uint32_t off : {64u * half + i0, 64u * half + 32u + i0, 128u + 32u * half + i0})
                sink = sink + B.w[idx][blk + off] + B.w[idx][blk + off + 15u];
              sink = sink + B.w[idx][blk + 192u + 8u * half] + B.w[idx][blk + 192u + 8u * half + 7u];
              if (su == 0) sink = sink + B.w[idx][blk + 208u] + B.w[idx][blk + 209u];
            }
            if (a_ok) {
              for (uint32_t run = 0; run < 4; ++run) {
                const uint64_t a0 = arow * c.cols + k * 256u + 128u * half + i0 + 32u * run;
                sink = sink + B.aq[a0] + B.aq[a0 + 15u];
              }
              sink = sink + B.as[arow * KB + k];
            }
            for (uint32_t l = 0; l < 8; ++l)
              for (uint32_t run = 0; run < 4; ++run) {
                const uint32_t dw = su_row * (kRow6 / 2u) + 8u * half + (su & 1u) + 16u * l + 2u * run;
                lds16[2 * dw] = 0;
                lds16[2 * dw + 1] = 0;
              }
          }
          const uint32_t ti = tid / 16, tj = tid % 16;
          for (uint32_t i = 0; i < 4; ++i)
            for (uint32_t l = 0; l < 8; ++l)
              sink = sink + lds16[(4 * ti + i) * kRow6 + 32u * l + 31u] + lds16[(4 * tj + i) * kRow6 + 32u * l];
        }
        for (uint32_t k0 = 0; fmt != 3 && k0 < KB; k0 += KC) {
          const uint32_t k = kq ? k0 : k0 + su;
          if (k < KB && w_ok) sink = sink + B.w[idx][(wrow * KB + k) * bb] + B.w[idx][(wrow * KB + k) * bb + bb - 1];
          if (k < KB && a_ok) {
            const uint64_t a0 = arow * c.cols + k * (kq ? 256u : 32u) + (kq ? su * 64u : 0u);
            sink = sink + B.aq[a0] + B.aq[a0 + (kq ? 63u : 31u)] + B.as[arow * KB + k];
            if (kq) sink = sink + B.asum[arow * (c.cols / 16u) + k * 16u + su * 4u + 3u];
          }
          const uint32_t l0 = su_row * kRow + (kq ? su * 64u : su * 32u);
          lds[l0] = 0;
          lds[l0 + (kq ? 63u : 31u)] = 0;
        }
        const uint32_t ti = tid / 16, tj = tid % 16;
        for (uint32_t i = 0; fmt != 3 && i < 4; ++i)
          sink = sink + lds[(4 * ti + i) * kRow + (kq ? 255u : (KC - 1) * 32u + 31u)] + lds[(4 * tj + i) * kRow];
        for (uint32_t j = 0; j < 4; ++j) {
          const uint32_t b = b0 + 4 * tj + j;
          if (b >= c.batch) continue;
          for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t r = r0 + 4 * ti + i;
            if (r >= rows) continue;
            const uint64_t o = (uint64_t)b * rows + r;
            if (c.addend_mode == 1) sink = sink + B.add[idx][r];
            if (c.addend_mode == 2) sink = sink + B.add[idx][o];
            B.written[ms[mi].out_off + o]++;
          }
        }
      }
    }
  }
  delete[] lds;
  delete[] lds16;
}

// qmatvec_kernel / qkmatvec_kernel: the tile's weight units, the activation rows of each pass,
// the LDS arrays at their largest indices, every output.
void walk_pass(const Call& c, uint32_t fmt, const jma::QMatPlan& qp, Buffers& B) {
  const uint32_t K = c.cols / jma::qmat_block_elems(fmt);
  uint32_t tiles;
  const std::vector<M> ms = table(c, fmt, qp.rows_per_tile, tiles);
  const uint32_t R = qp.rows_per_tile, nc = qp.chunk;
  const uint32_t group_rows = jma::qmat_group_rows(c.batch, nc, tiles);
  const uint32_t gy = (c.batch + group_rows - 1) / group_rows;
  expect(group_rows % nc == 0 && gy <= 65535u, c.name + ": grid rows");
  const bool kq = jma::qmat_kquant(fmt);
  const uint64_t lds = kq ? jma::qkmatvec_lds_bytes(fmt, nc, c.cols, R) : jma::qmatvec_lds_bytes(nc, c.cols, R);
  expect(lds <= jma::kQMatLds, c.name + ": LDS");
  unsigned char* smem = new unsigned char[lds];
  const uint32_t nt = fmt == 3 ? 9u : 4u;
  for (uint32_t bx = 0; bx < tiles; ++bx) {
    uint32_t mi = 0;
    for (uint32_t i = 1; i < ms.size(); ++i) mi = bx >= ms[i].tile0 ? i : mi;
    const uint32_t idx = ms[mi].idx, rows = c.rows[idx];
    const uint32_t r0 = (bx - ms[mi].tile0) * R;
    expect(r0 < rows, c.name + ": tile past its matrix");
    const uint32_t nrows = std::min(R, rows - r0);
    const uint32_t bb = jma::qmat_block_bytes(fmt);
    for (uint32_t u = 0; u < nrows * K; ++u) {
      const uint64_t off = ((uint64_t)r0 * K + u) * bb;
      sink = sink + B.w[idx][off] + B.w[idx][off + bb - 1];
    }
    for (uint32_t by = 0; by < gy; ++by) {
      const uint32_t g0 = by * group_rows, g1 = std::min(c.batch, g0 + group_rows);
      for (uint32_t b0 = g0; b0 < g1; b0 += nc) {
        const uint32_t nb = std::min(nc, g1 - b0);
        for (uint32_t b = 0; b < nb; ++b)
          sink = sink + B.x[(uint64_t)(b0 + b) * c.cols] + B.x[(uint64_t)(b0 + b) * c.cols + c.cols - 1];
        uint64_t top;
        if (!kq) {
          const uint64_t Kp = K + 1;
          const uint64_t act = ((uint64_t)nc * c.cols + 15u) / 16u * 16u;
          top = act + (uint64_t)nc * K * 8u + ((uint64_t)(nb - 1) * R + (nrows - 1)) * Kp * 4u +
                (uint64_t)nc * R * Kp * 4u + K * 4u;  // t_dot[(b * R + row) * Kp + blk]
        } else {
          const uint64_t rs = (uint64_t)K * nt + 1;
          const uint64_t act = ((uint64_t)nc * c.cols + 15u) / 16u * 16u;
          top = act + (uint64_t)nc * K * 4u + (uint64_t)nc * (c.cols / 16u) * 4u +
                (((uint64_t)(nb - 1) * R + (nrows - 1)) * rs + (K - 1) * nt + nt - 1) * 4u + 4u;
        }
        expect(top <= lds, c.name + ": LDS index");
        smem[top - 1] = 0;
        for (uint32_t b = 0; b < nb; ++b)
          for (uint32_t row = 0; row < nrows; ++row) {
            const uint32_t r = r0 + row;
            const uint64_t o = (uint64_t)(b0 + b) * rows + r;
            if (c.addend_mode == 1) sink = sink + B.add[idx][r];
            if (c.addend_mode == 2) sink = sink + B.add[idx][o];
            B.written[ms[mi].out_off + o]++;
          }
      }
    }
  }
  delete[] smem;
}

void walk(const Call& c) {
  const uint32_t n = (uint32_t)c.formats.size();
  const bool kq = jma::qmat_kquant(c.formats[0]);
  const uint32_t K = c.cols / jma::qmat_block_elems(c.formats[0]);
  Buffers B;
  B.w.resize(n);
  B.add.assign(n, nullptr);
  uint64_t total_rows = 0;
  for (uint32_t i = 0; i < n; ++i) {
    B.w[i] = new uint8_t[(uint64_t)c.rows[i] * K * jma::qmat_block_bytes(c.formats[i])];
    if (c.addend_mode == 1) B.add[i] = new float[c.rows[i]];
    if (c.addend_mode == 2) B.add[i] = new float[(uint64_t)c.batch * c.rows[i]];
    total_rows += c.rows[i];
  }
  B.x = new float[(uint64_t)c.batch * c.cols];
  B.aq = new int8_t[(uint64_t)c.batch * c.cols];
  B.as = new float[(uint64_t)c.batch * K];
  B.asum = new int[(uint64_t)c.batch * (c.cols / 16u)];
  B.written.assign(c.batch * total_rows, 0);
  std::vector<uint32_t> pass_fmts;
  for (uint32_t f : c.formats)
    if (!gemm_format(f, c.batch)) pass_fmts.push_back(f);
  jma::QMatPlan qp;
  if (!pass_fmts.empty()) {
    qp = jma::plan_qmat(pass_fmts.data(), (uint32_t)pass_fmts.size(), c.cols);
    expect(qp.rows_per_tile > 0 && qp.chunk >= 1 && qp.chunk <= jma::kQMatMaxChunk, c.name + ": plan");
  }
  std::string how;
  for (uint32_t fmt = 0; fmt <= 5; ++fmt) {
    if (std::find(c.formats.begin(), c.formats.end(), fmt) == c.formats.end()) continue;
    if (gemm_format(fmt, c.batch)) {
      walk_gemm(c, fmt, B);
      how += " fmt " + std::to_string(fmt) + ": product;";
    } else if (qp.rows_per_tile > 0) {
      walk_pass(c, fmt, qp, B);
      how += " fmt " + std::to_string(fmt) + ": " + std::to_string(qp.rows_per_tile) +
             " rows per tile, " + std::to_string(qp.chunk) + " per pass;";
    }
  }
  for (uint64_t i = 0; i < B.written.size(); ++i)
    if (B.written[i] != 1) {
      expect(false, c.name + ": output " + std::to_string(i) + " written " +
                        std::to_string(B.written[i]) + " times");
      break;
    }
  printf("%s (batch %u, cols %u):%s\n", c.name.c_str(), c.batch, c.cols, how.c_str());
  (void)kq;
  for (uint32_t i = 0; i < n; ++i) {
    delete[] B.w[i];
    delete[] B.add[i];
  }
  delete[] B.x;
  delete[] B.aq;
  delete[] B.as;
  delete[] B.asum;
}

}  // namespace

int main() {
  const std::vector<Call> calls = {
      // decode shapes: Llama-3.2-1B Q/K/V and wo, Qwen2 with biases
      {"llama1b qkv decode", {1, 0, 0}, {2048, 512, 512}, 1, 2048, 0},
      {"llama1b wo + residual", {0}, {2048}, 1, 2048, 2},
      {"qwen2 qkv biases", {1, 1, 1}, {896, 128, 128}, 1, 896, 1},
      // prefill-sized grouped calls with biases and residuals (the 200-row shape included)
      {"grouped 200 rows, biases", {1, 0, 0}, {1024, 256, 256}, 200, 1024, 1},
      {"wo 200 rows, residual", {0}, {1024}, 200, 1024, 2},
      {"grouped 2048 rows, biases", {1, 5, 0}, {3072, 1024, 1024}, 2048, 3072, 1},
      {"Q5_K_M 300 rows", {4, 4, 3}, {2048, 512, 512}, 300, 2048, 0},
      {"Q4_K_M 129 rows, residual", {2, 2, 3}, {1536, 256, 256}, 129, 1536, 2},
      {"Q4_K_M 2048 rows, biases", {2, 2, 3}, {3072, 1024, 1024}, 2048, 3072, 1},
      // edges: one block, one row, ragged batches, wide rows, 16 matrices
      {"one block", {0}, {1}, 1, 32, 0},
      {"odd blocks", {5}, {17}, 13, 2080, 1},
      {"wide row", {3}, {64}, 9, 14336, 2},
      {"wide row 32-element", {1}, {64}, 9, 14336, 0},
      {"wide row K-quant product", {2, 4}, {70, 3}, 40, 14336, 1},
      {"sixteen matrices", std::vector<uint32_t>(16, 0), std::vector<uint32_t>(16, 100), 33, 512, 1},
      {"batch 8", {0, 1}, {3072, 3}, 8, 2048, 0},
      {"batch 9", {0, 1}, {3072, 3}, 9, 2048, 0},
      {"batch 16 (product)", {5, 1}, {17, 65}, 16, 2080, 2},
      {"batch 15 (passes)", {5, 1}, {17, 65}, 15, 2080, 2},
      {"ragged product 100 x 200", {0, 5}, {200, 7}, 100, 96, 1},
      {"K-quant product 17 x 65 rows", {4, 2}, {17, 65}, 17, 512, 2},
      {"Q6_K product 33 x 70 rows", {3, 2, 3}, {70, 33, 1}, 33, 768, 1},
      {"wide row Q6_K product", {3}, {65}, 20, 14336, 2},
  };
  for (const Call& c : calls) walk(c);
  if (failures) {
    printf("%d failures\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
