// per_group_quant_mxfp8 for MI355X (gfx950): bf16 x [n_tokens, hidden_size] to e4m3fn codes and one
// e8m0 scale per 1 x 32 group, the scales row-major [n_tokens, hidden_size / 32]. Per group the scale
// is the least power of two at or above amax * fl32(1 / 448), amax = max |x| floored at 1e-10 (its
// biased exponent is stored), and each code is x divided by it, clamped to +-448, rounded to the
// nearest even e4m3fn. One HBM pass with the amax reduced by DPP moves among the lanes that share a
// group. Kernel: quant_mxfp8_kernel (aklr_amd/csrc/quant.hip) through aklr_per_group_quant_mxfp8.
#include "entry.h"

namespace {

void run(const at::Tensor& x, at::Tensor& quantized, at::Tensor& scales) {
  TORCH_CHECK(x.dim() == 2 && x.scalar_type() == at::kBFloat16 && x.stride(1) == 1,
              "x: bf16 [n_tokens, hidden_size] with unit column stride");
  const int64_t t = x.size(0), h = x.size(1);
  TORCH_CHECK(quantized.scalar_type() == at::kFloat8_e4m3fn && quantized.sizes() == x.sizes() &&
                  quantized.is_contiguous(),
              "quantized: e4m3fn [n_tokens, hidden_size], contiguous");
  TORCH_CHECK(scales.element_size() == 1 && scales.dim() == 2 && scales.size(0) == t && scales.size(1) == h / 32 &&
                  scales.is_contiguous(),
              "scales: one byte each, [n_tokens, hidden_size / 32], contiguous");
  aklr_entry::check(aklr_per_group_quant_mxfp8(x.data_ptr(), x.stride(0), quantized.data_ptr(),
                                               static_cast<uint8_t*>(scales.data_ptr()), t, h,
                                               aklr_entry::stream_of(x)),
                    "per_group_quant_mxfp8");
}

}  // namespace

#define TORCH_LIBRARY_EXPAND(ns, m) TORCH_LIBRARY(ns, m)
TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, m) {
  m.def("run(Tensor x, Tensor(a!) quantized, Tensor(b!) scales) -> ()", &run);
}
