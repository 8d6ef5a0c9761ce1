// per_group_quant_fp8 for MI355X (gfx950): bf16 x [n_tokens, hidden_size] to e4m3fn codes and one fp32
// dequantization scale per 1 x 128 group, the scales group-major [hidden_size / 128, n_tokens]. Per
// group: amax = max |x| floored at 1e-10, s = amax * fl32(1 / 448), q = e4m3fn(clamp(x * (1 / s),
// +-448)) to nearest even, and s is the stored scale. One HBM pass: a wave covers 8 rows of one group
// (8 lanes a row, 16 values a lane in two 16-byte loads), amax reduced with DPP moves among the lanes
// of a row, codes stored non-temporally, the scales of 8 rows written as 8 consecutive floats.
// Kernel: quant_fp8_1x128_kernel (aklr_amd/csrc/quant.hip) through aklr_per_group_quant_fp8.
#include "entry.h"

namespace {

void run(const at::Tensor& x, at::Tensor& quantized, at::Tensor& scales) {
  TORCH_CHECK(x.dim() == 2 && x.scalar_type() == at::kBFloat16 && x.stride(1) == 1,
              "x: bf16 [n_tokens, hidden_size] with unit column stride");
  const int64_t t = x.size(0), h = x.size(1);
  TORCH_CHECK(quantized.scalar_type() == at::kFloat8_e4m3fn && quantized.sizes() == x.sizes() &&
                  quantized.is_contiguous(),
              "quantized: e4m3fn [n_tokens, hidden_size], contiguous");
  TORCH_CHECK(scales.scalar_type() == at::kFloat && scales.dim() == 2 && scales.size(0) == h / 128 &&
                  scales.size(1) == t && scales.is_contiguous(),
              "scales: fp32 [hidden_size / 128, n_tokens], contiguous");
  aklr_entry::check(aklr_per_group_quant_fp8(x.data_ptr(), x.stride(0), quantized.data_ptr(),
                                             scales.data_ptr<float>(), t, h, aklr_entry::stream_of(x)),
                    "per_group_quant_fp8");
}

}  // namespace

#define TORCH_LIBRARY_EXPAND(ns, m) TORCH_LIBRARY(ns, m)
TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, m) {
  m.def("run(Tensor x, Tensor(a!) quantized, Tensor(b!) scales) -> ()", &run);
}
