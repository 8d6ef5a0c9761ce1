// gemm_a8w8_blockwise_scaled for MI355X (gfx950): out = (a * a_scale) @ (b * b_scale)^T + bias with fp8
// a [m, k] and b [n, k], one fp32 scale per 1 x 128 block of a and per 128 x 128 block of b, fp32
// accumulation, bf16 or fp16 out. Each 128-wide K block of each 16 x 16 output tile is one
// V_MFMA_SCALE_F32_16X16X128_F8F6F4 at unit e8m0 scales, folded into the result with one FMA by
// a_scale * b_scale. m <= 128: weight streaming -- each compute wave streams its weight columns from HBM
// into a register ring while a loader wave stages the A blocks in LDS, K split over waves and, where the
// columns alone leave CUs idle, over workgroups (fp32 partials in per-call scratch, summed in split
// order by the last workgroup to arrive). m > 128: 256 x 256 down to 128 x 128 workgroup tiles through
// a 2- to 4-stage LDS ring filled by direct-to-LDS loads, XCD-aware tile order. Results are bitwise
// reproducible. b is row-major or aiter's 16 x 16 shuffle_weight layout; the layout variant
// (variant.h) says how a_scale is stored. A row-major b given as (k, n) (trans_b = false) is first
// transposed into (n, k) scratch of this call. Kernels: aklr_amd/csrc/gemm_a8w8.hip through
// aklr_transpose_b8 and aklr_gemm_a8w8_blockscale.
#include "entry.h"
#include "variant.h"

namespace {

void run(const at::Tensor& a, const at::Tensor& b, const at::Tensor& a_scale, const at::Tensor& b_scale,
         c10::string_view scale_major_mode, bool trans_b, c10::string_view operand_format,
         const std::optional<at::Tensor>& bias, std::optional<at::ScalarType> out_dtype, at::Tensor& out) {
  TORCH_CHECK(trans_b || !aklr_variant::b_preshuffled, "gemm_a8w8_blockwise_scaled: a shuffled b is (n, k)");
  TORCH_CHECK(operand_format == (aklr_variant::b_preshuffled ? "none:preshuffled" : "none:none"),
              "gemm_a8w8_blockwise_scaled: operand_format does not match the layout variant");
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2 && a.is_contiguous() && b.is_contiguous(), "a, b: 2-d, contiguous");
  const at::ScalarType fp8 = a.scalar_type();
  TORCH_CHECK((fp8 == at::kFloat8_e4m3fn || fp8 == at::kFloat8_e5m2) && b.scalar_type() == fp8,
              "a, b: one fp8 dtype");
  const int64_t m = a.size(0), k = a.size(1), n = trans_b ? b.size(0) : b.size(1), kb = k / 128;
  TORCH_CHECK((trans_b ? b.size(1) : b.size(0)) == k && k % 128 == 0 && n % 16 == 0,
              "b: (n, k), or (k, n) when not trans_b; k % 128 == 0, n % 16 == 0");
  const bool mn = scale_major_mode == "MN";
  TORCH_CHECK(mn || scale_major_mode == "K", "scale_major_mode: K or MN");
  // element (i, kb) of a_scale at i * sm + kb * sk
  int64_t sm = kb, sk = 1;
  if (aklr_variant::a_scale_column_major || mn) {
    sm = 1;
    sk = m;
  }
  TORCH_CHECK(a_scale.scalar_type() == at::kFloat && a_scale.is_contiguous() && a_scale.numel() == m * kb,
              "a_scale: fp32, m * k / 128 elements, contiguous");
  TORCH_CHECK(b_scale.scalar_type() == at::kFloat && b_scale.dim() == 2 && b_scale.size(0) == (n + 127) / 128 &&
                  b_scale.size(1) == kb && b_scale.is_contiguous(),
              "b_scale: fp32 [ceil(n / 128), k / 128], contiguous");
  const float* bias_ptr = nullptr;
  if (bias.has_value()) {
    TORCH_CHECK(bias->scalar_type() == at::kFloat && bias->numel() == n && bias->is_contiguous(), "bias: fp32 [n]");
    bias_ptr = bias->data_ptr<float>();
  }
  const at::ScalarType od = out.scalar_type();
  TORCH_CHECK((od == at::kBFloat16 || od == at::kHalf) && (!out_dtype.has_value() || *out_dtype == od),
              "out: bf16 or fp16, of out_dtype when one is given");
  TORCH_CHECK(out.dim() == 2 && out.size(0) == m && out.size(1) == n && out.stride(1) == 1, "out: [m, n]");
  at::Tensor bt = b;  // (n, k)
  if (!trans_b) {
    bt = at::empty({n, k}, b.options());
    aklr_entry::check(aklr_transpose_b8(b.data_ptr(), k, n, b.stride(0), bt.data_ptr(), k, aklr_entry::stream_of(a)),
                      "gemm_a8w8_blockwise_scaled (b transpose)");
  }
  const size_t ws_bytes = aklr_gemm_a8w8_blockscale_workspace_bytes(m, n, k);
  at::Tensor ws = aklr_entry::scratch(a, ws_bytes);
  aklr_entry::check(
      aklr_gemm_a8w8_blockscale(a.data_ptr(), a.stride(0), bt.data_ptr(), aklr_variant::b_preshuffled ? k : bt.stride(0),
                                a_scale.data_ptr<float>(), sm, sk, b_scale.data_ptr<float>(), b_scale.stride(0),
                                bias_ptr, out.data_ptr(), out.stride(0), m, n, k,
                                fp8 == at::kFloat8_e5m2 ? AKLR_FP8_E5M2 : AKLR_FP8_E4M3FN,
                                aklr_variant::b_preshuffled ? AKLR_B_PRESHUFFLE_16x16 : AKLR_B_ROW_MAJOR,
                                od == at::kHalf ? AKLR_OUT_F16 : AKLR_OUT_BF16, ws_bytes ? ws.data_ptr() : nullptr,
                                ws_bytes, aklr_entry::stream_of(a)),
      "gemm_a8w8_blockwise_scaled");
}

}  // namespace

#define TORCH_LIBRARY_EXPAND(ns, m) TORCH_LIBRARY(ns, m)
TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, m) {
  m.def(
      "run(Tensor a, Tensor b, Tensor a_scale, Tensor b_scale, str scale_major_mode, bool trans_b, "
      "str operand_format, Tensor? bias, ScalarType? out_dtype, Tensor(a!) out) -> ()",
      &run);
}
