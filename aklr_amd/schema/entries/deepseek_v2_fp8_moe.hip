// deepseek_v2_fp8_moe for MI355X (gfx950): sglang's DeepseekV2MoE on one rank, the shared expert in the
// last of the experts' slots, as one chain of launches on the caller's stream with no host sync:
// router logits rounded to bf16 (bf16 MFMA), sigmoid scores, grouped top-k (a group scored by its two
// best biased scores; the lower index first among equals), unbiased renormalized weights times
// routed_scaling_factor and the shared slot at weight 1; the rows sorted by expert into 256-, 128- and
// 64-row blocks; each expert's input quantized per 1 x 128 at scale amax / 448 (a division); two
// persistent grouped 128 x 128-block-scaled FP8 GEMMs (gate and up together with silu(gate) * up
// quantized in the epilogue, then down); a combine that sums each token's slots in slot order. The
// layout variant (variant.h): row-major experts or aiter's 16 x 16 shuffle_weight tiles. Kernels:
// aklr_amd/csrc/moe_fp8.hip through aklr_deepseek_v2_fp8_moe.
#include "entry.h"
#include "variant.h"

#include <algorithm>

namespace {

// Tokens per library call: the kernels address the routed rows' activations and intermediates with
// 32-bit byte offsets, and every token's output depends on that token alone, so a larger call runs as
// consecutive calls on row ranges.
int64_t tokens_per_call(int64_t d, int64_t inter, int64_t slots) {
  const int64_t limit = 0x7FFFFFFE;
  return std::min({int64_t{65536}, limit / (2 * d * slots), limit / (inter * slots), limit / d});
}

void run(const at::Tensor& hidden_states, const at::Tensor& router_weight, const at::Tensor& correction_bias,
         const at::Tensor& w1, const at::Tensor& w1_scale, const at::Tensor& w2, const at::Tensor& w2_scale,
         int64_t topk, int64_t num_expert_group, int64_t topk_group, bool renormalize, c10::string_view scoring_func,
         double routed_scaling_factor, std::optional<at::ScalarType> out_dtype, at::Tensor& out) {
  TORCH_CHECK(scoring_func == "sigmoid", "deepseek_v2_fp8_moe: sigmoid scoring only");
  const at::Tensor& x = hidden_states;
  TORCH_CHECK(x.dim() == 2 && x.scalar_type() == at::kBFloat16 && x.is_contiguous(), "hidden_states: bf16 [T, D]");
  const int64_t t = x.size(0), d = x.size(1);
  TORCH_CHECK(router_weight.dim() == 2 && router_weight.size(1) == d && router_weight.scalar_type() == at::kBFloat16 &&
                  router_weight.is_contiguous(),
              "router_weight: bf16 [n_routed, D]");
  const int64_t n_routed = router_weight.size(0);
  TORCH_CHECK(correction_bias.numel() == n_routed && correction_bias.scalar_type() == at::kBFloat16 &&
                  correction_bias.is_contiguous(),
              "correction_bias: bf16 [n_routed]");
  TORCH_CHECK(w1.dim() == 3 && w2.dim() == 3 && w1.size(0) == n_routed + 1 && w2.size(0) == n_routed + 1,
              "w1, w2: [n_routed + 1, ...], the shared expert last");
  const int64_t inter = w2.size(2);
  TORCH_CHECK(w1.size(1) == 2 * inter && w1.size(2) == d && w2.size(1) == d &&
                  w1.scalar_type() == at::kFloat8_e4m3fn && w2.scalar_type() == at::kFloat8_e4m3fn &&
                  w1.is_contiguous() && w2.is_contiguous(),
              "w1: e4m3fn [E, 2 * I, D], w2: e4m3fn [E, D, I]");
  TORCH_CHECK(w1_scale.scalar_type() == at::kFloat && w1_scale.is_contiguous() &&
                  w1_scale.numel() == (n_routed + 1) * (2 * inter / 128) * (d / 128) &&
                  w2_scale.scalar_type() == at::kFloat && w2_scale.is_contiguous() &&
                  w2_scale.numel() == (n_routed + 1) * (d / 128) * (inter / 128),
              "w1_scale, w2_scale: fp32 per 128 x 128 block");
  TORCH_CHECK(out.scalar_type() == at::kBFloat16 && (!out_dtype.has_value() || *out_dtype == at::kBFloat16) &&
                  out.sizes() == x.sizes() && out.is_contiguous(),
              "out: bf16 [T, D]");
  if (t == 0) return;
  const int64_t slots = topk + 1;
  const int64_t most = tokens_per_call(d, inter, slots);
  TORCH_CHECK(most >= 1, "deepseek_v2_fp8_moe: dimensions past the kernels' 32-bit offsets");
  const int64_t first = std::min(t, most);
  const size_t ws_bytes = aklr_moe_fp8_workspace_bytes(first, d, inter, n_routed + 1, slots, n_routed);
  at::Tensor ws = aklr_entry::scratch(x, ws_bytes);
  const int64_t row_bytes = d * 2;
  for (int64_t s = 0; s < t; s += most) {
    const int64_t e = std::min(t, s + most);
    aklr_entry::check(
        aklr_deepseek_v2_fp8_moe(static_cast<const char*>(x.data_ptr()) + s * row_bytes, router_weight.data_ptr(),
                                 correction_bias.data_ptr(), w1.data_ptr(), w1_scale.data_ptr<float>(), w2.data_ptr(),
                                 w2_scale.data_ptr<float>(), e - s, d, inter, n_routed, static_cast<int>(topk),
                                 static_cast<int>(num_expert_group), static_cast<int>(topk_group), renormalize ? 1 : 0,
                                 static_cast<float>(routed_scaling_factor),
                                 aklr_variant::weights_preshuffled ? AKLR_B_PRESHUFFLE_16x16 : AKLR_B_ROW_MAJOR,
                                 static_cast<char*>(out.data_ptr()) + s * row_bytes, ws.data_ptr(), ws_bytes,
                                 aklr_entry::stream_of(x)),
        "deepseek_v2_fp8_moe");
  }
}

}  // namespace

#define TORCH_LIBRARY_EXPAND(ns, m) TORCH_LIBRARY(ns, m)
TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, m) {
  m.def(
      "run(Tensor hidden_states, Tensor router_weight, Tensor correction_bias, Tensor w1, Tensor w1_scale, "
      "Tensor w2, Tensor w2_scale, int topk, int num_expert_group, int topk_group, bool renormalize, "
      "str scoring_func, float routed_scaling_factor, ScalarType? out_dtype, Tensor(a!) out) -> ()",
      &run);
}
