// CPU restatement of the reference's native (cpp) backend, af3_kernels (test infrastructure:
// the "cpp" leg of bench.py's CPU baseline). It restates the algorithms of
//   af3_kernels/src/csrc/matrix.cpp:9-129              tiled GEMM, 128 x 128 output tiles, OpenMP
//                                                      over (batch, row tile, column tile), fp32
//                                                      tile accumulator, bias added in fp32
//   af3_kernels/src/csrc/gated_linear_unit.cpp:10-121   per tile: gate and value GEMMs stored in
//                                                      the compute dtype, SiLU, product
//   af3_kernels/src/csrc/dot_product_attention.cpp:17-174  per (batch, head, 128-query block):
//                                                      scores GEMM, bias add rounded to the compute
//                                                      dtype, -1e9 fill, full-key softmax, PV GEMM
//   af3_kernels/src/csrc/triangle_multiplication.cpp:6-73  LayerNorm, tiled projections, mask,
//                                                      sigmoid gate, per-channel contraction, centre
//                                                      LayerNorm, output projection and gate
// with each tile's GEMM done by ATen (at::mm, oneDNN on CPU) in place of LIBXSMM's JIT kernels,
// which are not built here. Tiles, loop nests, dtype boundaries and epilogues follow the cited
// lines.
// The restated algorithms, and parts of the loop structure and local names of
// triangle_multiplication() and softmax_rows(), follow af3_kernels (the reference's
// af3_kernels/src/csrc), which carries this notice:
//
//   BSD 3-Clause License
//
//   Copyright (c) 2025, Xflops
//   All rights reserved.
//
//   Redistribution and use in source and binary forms, with or without
//   modification, are permitted provided that the following conditions are met:
//
//   * Redistributions of source code must retain the above copyright notice, this
//     list of conditions and the following disclaimer.
//
//   * Redistributions in binary form must reproduce the above copyright notice,
//     this list of conditions and the following disclaimer in the documentation
//     and/or other materials provided with the distribution.
//
//   * Neither the name of the copyright holder nor the names of its
//     contributors may be used to endorse or promote products derived from
//     this software without specific prior written permission.
//
//   THIS SOFTWARE IS PROVIDED BY THE COPYRIGHT HOLDERS AND CONTRIBUTORS "AS IS"
//   AND ANY EXPRESS OR IMPLIED WARRANTIES, INCLUDING, BUT NOT LIMITED TO, THE
//   IMPLIED WARRANTIES OF MERCHANTABILITY AND FITNESS FOR A PARTICULAR PURPOSE ARE
//   DISCLAIMED. IN NO EVENT SHALL THE COPYRIGHT HOLDER OR CONTRIBUTORS BE LIABLE
//   FOR ANY DIRECT, INDIRECT, INCIDENTAL, SPECIAL, EXEMPLARY, OR CONSEQUENTIAL
//   DAMAGES (INCLUDING, BUT NOT LIMITED TO, PROCUREMENT OF SUBSTITUTE GOODS OR
//   SERVICES; LOSS OF USE, DATA, OR PROFITS; OR BUSINESS INTERRUPTION) HOWEVER
//   CAUSED AND ON ANY THEORY OF LIABILITY, WHETHER IN CONTRACT, STRICT LIABILITY,
//   OR TORT (INCLUDING NEGLIGENCE OR OTHERWISE) ARISING IN ANY WAY OUT OF THE USE
//   OF THIS SOFTWARE, EVEN IF ADVISED OF THE POSSIBILITY OF SUCH DAMAGE.
#include <torch/extension.h>

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <limits>
#include <vector>

namespace {

// One output tile of x[rows] . w[:, cols] into fp32 (the LIBXSMM kernels' fp32 C tile).
at::Tensor tile_product(const at::Tensor &x, const at::Tensor &w) {
  return at::mm(x, w).to(at::kFloat);
}

// matrix.cpp multiply(): OpenMP over (batch, row tile, column tile); out = T(tile + bias).
at::Tensor tiled_matmul(const at::Tensor &a, const at::Tensor &b, const c10::optional<at::Tensor> &bias,
                        int64_t mb, int64_t nb) {
  TORCH_CHECK(a.dim() == b.dim() && (a.dim() == 2 || a.dim() == 3), "tiled_matmul: rank 2 or 3 operands");
  auto a3 = a.dim() == 2 ? a.unsqueeze(0) : a;
  auto b3 = b.dim() == 2 ? b.unsqueeze(0) : b;
  const int64_t batches = a3.size(0), m = a3.size(1), k = a3.size(2), n = b3.size(2);
  TORCH_CHECK(b3.size(1) == k && b3.size(0) == batches, "tiled_matmul: shapes");
  auto out = at::empty({batches, m, n}, a.options());
  if (batches == 0 || m == 0 || n == 0) return a.dim() == 2 ? out.squeeze(0) : out;
  mb = std::min(mb, m);
  nb = std::min(nb, n);
  const int64_t mt = (m + mb - 1) / mb, nt = (n + nb - 1) / nb;
  at::Tensor bias_f;
  if (bias.has_value()) bias_f = bias->to(at::kFloat).contiguous();
  const bool inference = c10::InferenceMode::is_enabled();
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t batch = 0; batch < batches; ++batch)
    for (int64_t mi = 0; mi < mt; ++mi)
      for (int64_t ni = 0; ni < nt; ++ni) {
        c10::InferenceMode guard(inference);  // thread-local: the workers take the caller's mode
        const int64_t row = mi * mb, col = ni * nb;
        const int64_t h = std::min(mb, m - row), w = std::min(nb, n - col);
        auto tile = tile_product(a3[batch].narrow(0, row, h), b3[batch].narrow(1, col, w));
        if (bias_f.defined()) tile.add_(bias_f.narrow(0, col, w));
        out[batch].narrow(0, row, h).narrow(1, col, w).copy_(tile);
      }
  return a.dim() == 2 ? out.squeeze(0) : out;
}

template <typename T>
void glu_epilogue(const T *gate, const T *value, T *out, int64_t h, int64_t w, int64_t ld_out) {
  for (int64_t r = 0; r < h; ++r)
    for (int64_t c = 0; c < w; ++c) {
      const float a = static_cast<float>(gate[r * w + c]);
      const float sigmoid = a >= 0.0f ? 1.0f / (1.0f + std::exp(-a)) : std::exp(a) / (1.0f + std::exp(a));
      const T activated = T(a * sigmoid);
      out[r * ld_out + c] = T(static_cast<float>(activated) * static_cast<float>(value[r * w + c]));
    }
}

// gated_linear_unit.cpp run_glu(): per (row tile, column tile) two GEMMs stored in T.
at::Tensor gated_linear_unit(const at::Tensor &x, const at::Tensor &weight, int64_t mb, int64_t nb) {
  TORCH_CHECK(x.dim() == 2 && weight.dim() == 2 && weight.size(0) == x.size(1) && weight.size(1) % 2 == 0,
              "gated_linear_unit: x [M, K], weight [K, 2F]");
  const int64_t m = x.size(0), n = weight.size(1) / 2;
  auto out = at::empty({m, n}, x.options());
  if (m == 0 || n == 0) return out;
  mb = std::min(mb, m);
  nb = std::min(nb, n);
  const int64_t mt = (m + mb - 1) / mb, nt = (n + nb - 1) / nb;
  const bool inference = c10::InferenceMode::is_enabled();
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t mi = 0; mi < mt; ++mi)
    for (int64_t ni = 0; ni < nt; ++ni) {
      c10::InferenceMode guard(inference);
      const int64_t row = mi * mb, col = ni * nb;
      const int64_t h = std::min(mb, m - row), w = std::min(nb, n - col);
      auto xs = x.narrow(0, row, h);
      auto gate = at::mm(xs, weight.narrow(1, col, w)).contiguous();
      auto value = at::mm(xs, weight.narrow(1, n + col, w)).contiguous();
      auto dst = out.narrow(0, row, h).narrow(1, col, w);
      if (x.scalar_type() == at::kBFloat16) {
        glu_epilogue(gate.data_ptr<at::BFloat16>(), value.data_ptr<at::BFloat16>(), dst.data_ptr<at::BFloat16>(), h,
                     w, n);
      } else {
        glu_epilogue(gate.data_ptr<float>(), value.data_ptr<float>(), dst.data_ptr<float>(), h, w, n);
      }
    }
  return out;
}

template <typename T>
void softmax_rows(T *scores, int64_t rows, int64_t keys, const float *bias, const int64_t *bias_strides,
                  const bool *mask, const int64_t *mask_strides, int64_t row0, std::vector<float> &exps) {
  for (int64_t r = 0; r < rows; ++r) {
    T *s = scores + r * keys;
    float maximum = -std::numeric_limits<float>::infinity();
    bool has_nan = false;
    for (int64_t j = 0; j < keys; ++j) {
      float value = static_cast<float>(s[j]);
      if (bias) value = static_cast<float>(T(value + bias[(row0 + r) * bias_strides[0] + j * bias_strides[1]]));
      if (mask && !mask[(row0 + r) * mask_strides[0] + j * mask_strides[1]]) value = static_cast<float>(T(-1e9f));
      s[j] = T(value);
      has_nan = has_nan || std::isnan(value);
      maximum = std::max(maximum, value);
    }
    if (has_nan) maximum = std::numeric_limits<float>::quiet_NaN();
    float sum = 0.0f;
    for (int64_t j = 0; j < keys; ++j) {
      exps[j] = std::exp(static_cast<float>(s[j]) - maximum);
      sum += exps[j];
    }
    for (int64_t j = 0; j < keys; ++j) s[j] = T(exps[j] / sum);
  }
}

// dot_product_attention.cpp attend(): q pre-scaled; mask bool and bias fp32 expanded to
// [B, H, Q, K] (any strides; may be undefined).
at::Tensor dot_product_attention(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                                 const c10::optional<at::Tensor> &mask, const c10::optional<at::Tensor> &bias,
                                 int64_t qb) {
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "attention: [B, H, Q/K, D]");
  const int64_t batches = q.size(0), heads = q.size(1), queries = q.size(2), keys = k.size(2);
  auto out = at::empty({batches, heads, queries, v.size(3)}, q.options());
  if (batches * heads * queries == 0) return out;
  qb = std::min(qb, queries);
  const int64_t tiles = (queries + qb - 1) / qb;
  const bool *mask_data = nullptr;
  const float *bias_data = nullptr;
  at::Tensor m, b;
  if (mask.has_value()) {
    m = *mask;
    mask_data = m.data_ptr<bool>();
  }
  if (bias.has_value()) {
    b = *bias;
    bias_data = b.data_ptr<float>();
  }
  const bool bf16 = q.scalar_type() == at::kBFloat16;
  const int threads = std::max(1, omp_get_max_threads());
  std::vector<std::vector<float>> exps(threads, std::vector<float>(keys));
  const bool inference = c10::InferenceMode::is_enabled();
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t batch = 0; batch < batches; ++batch)
    for (int64_t head = 0; head < heads; ++head)
      for (int64_t tile = 0; tile < tiles; ++tile) {
        c10::InferenceMode guard(inference);
        const int64_t row = tile * qb, h = std::min(qb, queries - row);
        auto scores = at::mm(q[batch][head].narrow(0, row, h), k[batch][head].t()).contiguous();
        const float *bp = nullptr;
        const bool *mp = nullptr;
        int64_t bs[2] = {0, 0}, ms[2] = {0, 0};
        if (bias_data) {
          bp = bias_data + batch * b.stride(0) + head * b.stride(1);
          bs[0] = b.stride(2);
          bs[1] = b.stride(3);
        }
        if (mask_data) {
          mp = mask_data + batch * m.stride(0) + head * m.stride(1);
          ms[0] = m.stride(2);
          ms[1] = m.stride(3);
        }
        auto &e = exps[omp_get_thread_num()];
        if (bf16)
          softmax_rows(scores.data_ptr<at::BFloat16>(), h, keys, bp, bs, mp, ms, row, e);
        else
          softmax_rows(scores.data_ptr<float>(), h, keys, bp, bs, mp, ms, row, e);
        out[batch][head].narrow(0, row, h).copy_(at::mm(scores, v[batch][head]));
      }
  return out;
}

// triangle_multiplication.cpp:6-73 with the tiled GEMMs above (weights pre-transposed [C, 2C]
// and [C, C], in the compute dtype).
at::Tensor triangle_multiplication(const at::Tensor &pair, const c10::optional<at::Tensor> &mask, bool outgoing,
                                   const at::Tensor &left_weight, const c10::optional<at::Tensor> &left_bias,
                                   const at::Tensor &projection, const at::Tensor &gate,
                                   const at::Tensor &center_weight, const c10::optional<at::Tensor> &center_bias,
                                   const at::Tensor &output_weight, const at::Tensor &gating_weight, double left_eps,
                                   double center_eps, int64_t block) {
  const int64_t n = pair.size(0), c = pair.size(2);
  auto dtype = projection.scalar_type();
  auto flat = at::layer_norm(pair, {c}, left_weight, left_bias, left_eps, true).to(dtype).contiguous().view({n * n, c});
  at::Tensor contracted;
  {
    auto projected = tiled_matmul(flat, projection, c10::nullopt, block, block).view({n, n, 2 * c}).permute({2, 0, 1});
    if (mask.has_value()) projected.mul_(mask->unsqueeze(0));
    auto gate_values = tiled_matmul(flat, gate, c10::nullopt, block, block).view({n, n, 2 * c}).permute({2, 0, 1});
    projected.mul_(at::sigmoid(gate_values));
    auto interleaved = projected.reshape({c, 2, n, n});
    auto a = interleaved.select(1, 0).contiguous();
    auto b = interleaved.select(1, 1).contiguous();
    auto left = outgoing ? a : b.transpose(1, 2).contiguous();
    auto right = outgoing ? b.transpose(1, 2).contiguous() : a;
    contracted = tiled_matmul(left, right, c10::nullopt, block, block).permute({1, 2, 0});
  }
  auto centered =
      at::layer_norm(contracted, {c}, center_weight, center_bias, center_eps, true).to(dtype).contiguous().view({n * n, c});
  contracted = at::Tensor();
  auto result = tiled_matmul(centered, output_weight, c10::nullopt, block, block);
  auto output_gate = tiled_matmul(flat, gating_weight, c10::nullopt, block, block);
  result.mul_(at::sigmoid(output_gate));
  return result.view({n, n, c});
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("tiled_matmul", &tiled_matmul, "matrix.cpp tiled GEMM", py::arg("a"), py::arg("b"), py::arg("bias"),
        py::arg("mb") = 128, py::arg("nb") = 128);
  m.def("gated_linear_unit", &gated_linear_unit, "gated_linear_unit.cpp", py::arg("x"), py::arg("weight"),
        py::arg("mb") = 128, py::arg("nb") = 128);
  m.def("dot_product_attention", &dot_product_attention, "dot_product_attention.cpp", py::arg("q"), py::arg("k"),
        py::arg("v"), py::arg("mask"), py::arg("bias"), py::arg("qb") = 128);
  m.def("triangle_multiplication", &triangle_multiplication, "triangle_multiplication.cpp");
}
