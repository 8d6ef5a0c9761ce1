// gemm_a4w4_mxfp4 for MI355X (gfx950): out = (a * 2^(a_scale - 127)) @ (b * 2^(b_scale - 127))^T + bias
// with e2m1 a [m, k] and b [n, k] (two values a byte, low nibble first) and one e8m0 scale per 32
// values along k, fp32 accumulation, bf16 or fp16 out (alpha 1, beta 0). Every 128-wide K step of a
// 16 x 16 output tile is one V_MFMA_SCALE_F32_16X16X128_F8F6F4 that applies both e8m0 scales itself,
// accumulating straight into the fp32 result. m <= 32: weight streaming into register rings (K split
// over waves and workgroups, partials summed in split order); m > 32: LDS-tiled 256 x 256 down to
// 128 x 128 tiles through a direct-to-LDS ring with the scale bytes staged beside the codes. Results are
// bitwise reproducible. The layout variant (variant.h): row-major b and scales, or aiter's 16 x 16
// shuffle_weight b with its padded, shuffled scales. Kernels: aklr_amd/csrc/gemm_a4w4.hip through
// aklr_gemm_a4w4_mxfp4.
#include "entry.h"
#include "variant.h"

namespace {

void run(const at::Tensor& a, const at::Tensor& b, const at::Tensor& a_scale, const at::Tensor& b_scale, bool trans_b,
         c10::string_view operand_format, double alpha, double beta, const std::optional<at::Tensor>& bias,
         std::optional<at::ScalarType> out_dtype, at::Tensor& out) {
  TORCH_CHECK(trans_b, "gemm_a4w4_mxfp4: b must be (n, k)");
  TORCH_CHECK(alpha == 1.0 && beta == 0.0, "gemm_a4w4_mxfp4: alpha 1 and beta 0 only");
  TORCH_CHECK(operand_format == (aklr_variant::shuffled ? "none:preshuffled" : "none:none"),
              "gemm_a4w4_mxfp4: operand_format does not match the layout variant");
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2 && a.element_size() == 1 && b.element_size() == 1 && a.is_contiguous() &&
                  b.is_contiguous(),
              "a, b: packed e2m1 bytes, 2-d, contiguous");
  const int64_t m = a.size(0), k = 2 * a.size(1), n = b.size(0), g = k / 32;
  TORCH_CHECK(b.size(1) == a.size(1) && k % 64 == 0 && n % 16 == 0, "b: (n, k / 2) bytes, k % 64 == 0, n % 16 == 0");
  const int64_t sa_rows = aklr_variant::shuffled ? (m + 255) / 256 * 256 : m;
  const int64_t sb_rows = aklr_variant::shuffled ? (n + 255) / 256 * 256 : n;
  const int64_t s_cols = aklr_variant::shuffled ? (g + 7) / 8 * 8 : g;
  TORCH_CHECK(a_scale.element_size() == 1 && a_scale.dim() == 2 && a_scale.size(0) == sa_rows &&
                  a_scale.size(1) == s_cols && a_scale.is_contiguous(),
              "a_scale: e8m0 bytes of the variant's shape, contiguous");
  TORCH_CHECK(b_scale.element_size() == 1 && b_scale.dim() == 2 && b_scale.size(0) == sb_rows &&
                  b_scale.size(1) == s_cols && b_scale.is_contiguous(),
              "b_scale: e8m0 bytes of the variant's shape, contiguous");
  const float* bias_ptr = nullptr;
  if (bias.has_value()) {
    TORCH_CHECK(bias->scalar_type() == at::kFloat && bias->numel() == n && bias->is_contiguous(), "bias: fp32 [n]");
    bias_ptr = bias->data_ptr<float>();
  }
  const at::ScalarType od = out.scalar_type();
  TORCH_CHECK((od == at::kBFloat16 || od == at::kHalf) && (!out_dtype.has_value() || *out_dtype == od),
              "out: bf16 or fp16, of out_dtype when one is given");
  TORCH_CHECK(out.dim() == 2 && out.size(0) == m && out.size(1) == n && out.stride(1) == 1, "out: [m, n]");
  const size_t ws_bytes = aklr_gemm_a4w4_mxfp4_workspace_bytes(m, n, k);
  at::Tensor ws = aklr_entry::scratch(a, ws_bytes);
  aklr_entry::check(
      aklr_gemm_a4w4_mxfp4(static_cast<const uint8_t*>(a.data_ptr()), a.stride(0),
                           static_cast<const uint8_t*>(b.data_ptr()), b.stride(0),
                           static_cast<const uint8_t*>(a_scale.data_ptr()), a_scale.stride(0),
                           static_cast<const uint8_t*>(b_scale.data_ptr()), b_scale.stride(0), bias_ptr,
                           out.data_ptr(), out.stride(0), m, n, k,
                           aklr_variant::shuffled ? AKLR_B_PRESHUFFLE_16x16 : AKLR_B_ROW_MAJOR,
                           aklr_variant::shuffled ? AKLR_SCALES_SHUFFLED : AKLR_SCALES_ROW_MAJOR,
                           od == at::kHalf ? AKLR_OUT_F16 : AKLR_OUT_BF16, ws_bytes ? ws.data_ptr() : nullptr,
                           ws_bytes, aklr_entry::stream_of(a)),
      "gemm_a4w4_mxfp4");
}

}  // namespace

#define TORCH_LIBRARY_EXPAND(ns, m) TORCH_LIBRARY(ns, m)
TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, m) {
  m.def(
      "run(Tensor a, Tensor b, Tensor a_scale, Tensor b_scale, bool trans_b, str operand_format, float alpha, "
      "float beta, Tensor? bias, ScalarType? out_dtype, Tensor(a!) out) -> ()",
      &run);
}
