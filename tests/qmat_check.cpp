// CPU bounds check of the quantized-projection launches (models_amd/csrc/jma_quant.hip), built
// with g++ and AddressSanitizer / UndefinedBehaviorSanitizer by tests/test_plan_cpu.py.
//
// For each call below it plans the launches with the runtime's own planner (plan_qmat and
// qmat_group_rows in jma_plan.h, as quantized_matmul_impl does: one launch per weight format,
// tiles in matrix order) and then walks every workgroup (x, y) of every launch the way the
// kernels index memory: the matrix a workgroup serves (the last with tile0 <= x), its weight
// blocks, the activation rows of its passes (y * group_rows ..., `chunk` at a time), its LDS
// arrays and every output, bias and residual element it reads or writes. Every access touches an
// exactly sized heap array, so an index past an extent is a sanitizer error; every output element
// must be written exactly once across the call's launches.
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

// The register-tiled product (qgemm_kernel) of the 32-element block formats at batches of
// kQGemmMinBatch rows and more: the Q8_0 activation scratch [batch][cols] int8 + [batch][K] f32,
// each workgroup's staged weight and activation blocks (one per thread and chunk, rows clamped to
// the last valid one and skipped past it), its LDS rows, and every output it writes.
void walk_gemm(const Call& c) {
  const uint32_t n = (uint32_t)c.formats.size();
  const uint32_t K = c.cols / 32, T = jma::kQGemmTile, KC = jma::kQGemmKc, kRow = KC * 32 + 16;
  std::vector<uint8_t*> w(n);
  std::vector<float*> add(n, nullptr);
  uint64_t total_rows = 0;
  for (uint32_t i = 0; i < n; ++i) {
    w[i] = new uint8_t[(uint64_t)c.rows[i] * K * jma::qmat_block_bytes(c.formats[i])];
    if (c.addend_mode == 1) add[i] = new float[c.rows[i]];
    if (c.addend_mode == 2) add[i] = new float[(uint64_t)c.batch * c.rows[i]];
    total_rows += c.rows[i];
  }
  int8_t* aq = new int8_t[(uint64_t)c.batch * c.cols];
  float* as = new float[(uint64_t)c.batch * K];
  std::vector<uint8_t> written(c.batch * total_rows, 0);
  int8_t* lds = new int8_t[T * kRow];
  volatile int sink = 0;
  for (uint32_t fmt = 0; fmt <= 5; ++fmt) {
    struct M { uint32_t idx, tile0; uint64_t out_off; };
    std::vector<M> ms;
    uint32_t tiles = 0;
    uint64_t out_off = 0;
    for (uint32_t i = 0; i < n; ++i) {
      if (c.formats[i] == fmt) {
        ms.push_back({i, tiles, out_off});
        tiles += (c.rows[i] + T - 1) / T;
      }
      out_off += (uint64_t)c.batch * c.rows[i];
    }
    if (ms.empty()) continue;
    const uint32_t bb = jma::qmat_block_bytes(fmt);
    const uint32_t gy = (c.batch + T - 1) / T;
    expect(gy <= 65535u, c.name + ": gemm grid rows");
    for (uint32_t bx = 0; bx < tiles; ++bx) {
      uint32_t mi = 0;
      for (uint32_t i = 1; i < ms.size(); ++i) mi = bx >= ms[i].tile0 ? i : mi;
      const uint32_t idx = ms[mi].idx, rows = c.rows[idx];
      const uint32_t r0 = (bx - ms[mi].tile0) * T;
      expect(r0 < rows, c.name + ": gemm tile past its matrix");
      for (uint32_t by = 0; by < gy; ++by) {
        const uint32_t b0 = by * T;
        for (uint32_t tid = 0; tid < 256; ++tid) {
          const uint32_t su_row = tid / KC, su_k = tid % KC;
          const bool w_ok = r0 + su_row < rows, a_ok = b0 + su_row < c.batch;
          const uint64_t wrow = std::min(r0 + su_row, rows - 1), arow = std::min(b0 + su_row, c.batch - 1);
          for (uint32_t k0 = 0; k0 < K; k0 += KC) {
            const uint32_t k = k0 + su_k;
            if (k < K && w_ok) sink = sink + w[idx][(wrow * K + k) * bb] + w[idx][(wrow * K + k) * bb + bb - 1];
            if (k < K && a_ok) sink = sink + aq[arow * c.cols + k * 32] + aq[arow * c.cols + k * 32 + 31] + (int)as[arow * K + k];
            lds[su_row * kRow + su_k * 32] = 0;
            lds[su_row * kRow + su_k * 32 + 31] = 0;
          }
          const uint32_t ti = tid / 16, tj = tid % 16;
          for (uint32_t i = 0; i < 4; ++i) sink = sink + lds[(4 * ti + i) * kRow + (KC - 1) * 32 + 31] + lds[(4 * tj + i) * kRow];
          for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t b = b0 + 4 * tj + j;
            if (b >= c.batch) continue;
            for (uint32_t i = 0; i < 4; ++i) {
              const uint32_t r = r0 + 4 * ti + i;
              if (r >= rows) continue;
              const uint64_t o = (uint64_t)b * rows + r;
              if (c.addend_mode == 1) sink = sink + (int)add[idx][r];
              if (c.addend_mode == 2) sink = sink + (int)add[idx][o];
              written[ms[mi].out_off + o]++;
            }
          }
        }
      }
    }
  }
  for (uint64_t i = 0; i < written.size(); ++i)
    if (written[i] != 1) {
      expect(false, c.name + ": gemm output " + std::to_string(i) + " written " +
                        std::to_string(written[i]) + " times");
      break;
    }
  printf("%s: batch %u cols %u, register-tiled product\n", c.name.c_str(), c.batch, c.cols);
  for (uint32_t i = 0; i < n; ++i) {
    delete[] w[i];
    delete[] add[i];
  }
  delete[] aq;
  delete[] as;
  delete[] lds;
}

void walk(const Call& c) {
  const uint32_t n = (uint32_t)c.formats.size();
  if (!jma::qmat_kquant(c.formats[0]) && c.batch >= jma::kQGemmMinBatch) {
    walk_gemm(c);
    return;
  }
  const jma::QMatPlan qp = jma::plan_qmat(c.formats.data(), n, c.cols);
  expect(qp.rows_per_tile > 0 && qp.chunk >= 1 && qp.chunk <= jma::kQMatMaxChunk,
         c.name + ": plan");
  if (qp.rows_per_tile == 0) return;
  const uint32_t elems = jma::qmat_block_elems(c.formats[0]);
  const uint32_t K = c.cols / elems;
  // Exactly sized arrays: the weights of each matrix, the activations, the output of every
  // matrix (matrix after matrix, each [batch][rows]), the biases or residuals.
  std::vector<uint8_t*> w(n);
  std::vector<uint64_t> wbytes(n);
  std::vector<float*> add(n, nullptr);
  uint64_t total_rows = 0;
  for (uint32_t i = 0; i < n; ++i) {
    wbytes[i] = (uint64_t)c.rows[i] * K * jma::qmat_block_bytes(c.formats[i]);
    w[i] = new uint8_t[wbytes[i]];
    if (c.addend_mode == 1) add[i] = new float[c.rows[i]];
    if (c.addend_mode == 2) add[i] = new float[(uint64_t)c.batch * c.rows[i]];
    total_rows += c.rows[i];
  }
  float* x = new float[(uint64_t)c.batch * c.cols];
  float* out = new float[c.batch * total_rows];
  std::vector<uint8_t> written(c.batch * total_rows, 0);
  volatile float sink = 0.0f;
  for (uint32_t fmt = 0; fmt <= 5; ++fmt) {
    // the launch's matrix table, as the runtime fills it
    struct M { uint32_t idx, tile0; uint64_t out_off; };
    std::vector<M> ms;
    uint32_t tiles = 0;
    uint64_t out_off = 0;
    for (uint32_t i = 0; i < n; ++i) {
      if (c.formats[i] == fmt) {
        ms.push_back({i, tiles, out_off});
        tiles += (c.rows[i] + qp.rows_per_tile - 1) / qp.rows_per_tile;
      }
      out_off += (uint64_t)c.batch * c.rows[i];
    }
    if (ms.empty()) continue;
    const uint32_t R = qp.rows_per_tile, nc = qp.chunk;
    const uint32_t group_rows = jma::qmat_group_rows(c.batch, nc, tiles);
    const uint32_t gy = (c.batch + group_rows - 1) / group_rows;
    expect(group_rows % nc == 0 && gy <= 65535u, c.name + ": grid rows");
    // LDS: the kernel's arrays for nc activation rows and R tile rows
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
      // every (row, block) unit of the tile: its whole block
      for (uint32_t u = 0; u < nrows * K; ++u) {
        const uint64_t off = ((uint64_t)r0 * K + u) * bb;
        sink = sink + w[idx][off] + w[idx][off + bb - 1];
      }
      for (uint32_t by = 0; by < gy; ++by) {
        const uint32_t g0 = by * group_rows, g1 = std::min(c.batch, g0 + group_rows);
        for (uint32_t b0 = g0; b0 < g1; b0 += nc) {
          const uint32_t nb = std::min(nc, g1 - b0);
          // activations of the pass, first and last element of each row
          for (uint32_t b = 0; b < nb; ++b)
            sink = sink + x[(uint64_t)(b0 + b) * c.cols] + x[(uint64_t)(b0 + b) * c.cols + c.cols - 1];
          // LDS arrays, at their largest indices of the pass
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
              if (c.addend_mode == 1) sink = sink + add[idx][r];
              if (c.addend_mode == 2) sink = sink + add[idx][o];
              const uint64_t g = ms[mi].out_off + o;
              out[g] = 1.0f;
              written[g]++;
            }
        }
      }
    }
    delete[] smem;
  }
  for (uint64_t i = 0; i < written.size(); ++i)
    if (written[i] != 1) {
      expect(false, c.name + ": output " + std::to_string(i) + " written " +
                        std::to_string(written[i]) + " times");
      break;
    }
  printf("%s: batch %u cols %u, rows per tile %u, %u rows per pass\n", c.name.c_str(), c.batch,
         c.cols, qp.rows_per_tile, qp.chunk);
  for (uint32_t i = 0; i < n; ++i) {
    delete[] w[i];
    delete[] add[i];
  }
  delete[] x;
  delete[] out;
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
      // edges: one block, one row, ragged batches, wide rows, 16 matrices
      {"one block", {0}, {1}, 1, 32, 0},
      {"odd blocks", {5}, {17}, 13, 2080, 1},
      {"wide row", {3}, {64}, 9, 14336, 2},
      {"wide row 32-element", {1}, {64}, 9, 14336, 0},
      {"sixteen matrices", std::vector<uint32_t>(16, 0), std::vector<uint32_t>(16, 100), 33, 512, 1},
      {"batch 8", {0, 1}, {3072, 3}, 8, 2048, 0},
      {"batch 9", {0, 1}, {3072, 3}, 9, 2048, 0},
      {"batch 16 (product)", {5, 1}, {17, 65}, 16, 2080, 2},
      {"batch 15 (passes)", {5, 1}, {17, 65}, 15, 2080, 2},
      {"ragged product 100 x 200", {0, 5}, {200, 7}, 100, 96, 1},
  };
  for (const Call& c : calls) walk(c);
  if (failures) {
    printf("%d failures\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
