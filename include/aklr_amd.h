/*
 * aklr_amd.h -- C ABI of the MI355X (gfx950) block-scaled low-precision GEMM path.
 *
 * Every entry point takes raw device pointers, element counts and strides, and the HIP stream
 * to launch on. It launches kernels only: it never allocates, frees, synchronizes, or changes
 * the current device. It returns AKLR_OK or a nonzero status (aklr_status_string names it).
 * Entry points are stateless and may be called from any host thread with its own stream.
 *
 * Scratch memory is brought by the caller: ask *_workspace_bytes() for the size and pass a device
 * buffer at least that large (16-byte aligned), with any content -- freshly allocated and never
 * cleared is fine. Its first 128 KiB are split-K arrival words, each tagged with the launch that
 * wrote it (the HSA dispatch id and queue), so a word left by an earlier call, or garbage, counts as
 * empty; the rest holds fp32 partials that the call writes before it reads them. No call depends on
 * what an earlier call left, as the reference's kernel ABI requires of scratch (aklr/ops/README.md:214).
 * Calls that may run at the same time need their own buffers. The library keeps nothing between
 * calls.
 *
 * Each entry point replaces one kernel ABI of the reference (a TORCH_LIBRARY `run(...)` op that
 * AKLR's HipBuilder loads); the citation is on each declaration.
 */
#ifndef AKLR_AMD_H
#define AKLR_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AKLR_AMD_ABI_VERSION 1

/* Status codes. */
enum {
    AKLR_OK = 0,
    AKLR_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, misaligned pointer or stride */
    AKLR_ERR_UNSUPPORTED = 2,      /* a layout/dtype combination no kernel here serves */
    AKLR_ERR_WORKSPACE = 3,        /* workspace smaller than *_workspace_bytes() */
    AKLR_ERR_LAUNCH = 4,           /* hipGetLastError() after the launch was not hipSuccess */
    AKLR_ERR_SCRATCH_LIMIT = 5     /* the plan needs more scratch than a no-allocation entry holds */
};

/* Element types. */
enum { AKLR_FP8_E4M3FN = 0, AKLR_FP8_E5M2 = 1 };
enum { AKLR_OUT_BF16 = 0, AKLR_OUT_F16 = 1 };

/* Weight (b) layouts. PRESHUFFLE_16x16 is aiter shuffle_weight(layout=(16,16)): rows split in
 * tiles of 16, columns in tiles of 32 bytes; tile-major, each tile stored as two 256-byte halves
 * (bytes 0-15 then 16-31 of every row). */
enum { AKLR_B_ROW_MAJOR = 0, AKLR_B_PRESHUFFLE_16x16 = 1 };

/* e8m0 scale layouts for MXFP4. SHUFFLED is aiter shuffle_scale on scales padded with 0x00 to
 * (256-row, 8-column) multiples. */
enum { AKLR_SCALES_ROW_MAJOR = 0, AKLR_SCALES_SHUFFLED = 1 };

int aklr_abi_version(void);
const char* aklr_status_string(int status);

/*
 * Dynamic per-1x128 FP8 quantization.
 * Replaces: per_group_quant_fp8 kernel ABI `run(Tensor x, Tensor(a!) quantized, Tensor(b!) scales)`
 *   (aklr/ops/quant/impls/hip/per_group_quant_fp8_hidden_size7168/1654009925223f46.json:110),
 *   contract aklr/ops/quant/contract.py:17-51, arithmetic aklr/ops/quant/reference.py:9-28.
 * x: bf16 [n_tokens, hidden_size], row stride x_row_stride elements (>= hidden_size).
 * quantized: e4m3fn [n_tokens, hidden_size] contiguous. scales: fp32 [hidden_size/128, n_tokens]
 *   (group-major: element [g, t] at g*n_tokens + t). hidden_size % 128 == 0.
 * Per group: amax = max(|x|) floored at 1e-10; s = amax * fl32(1/448); q = e4m3(clamp(x * (1/s), +-448)).
 */
int aklr_per_group_quant_fp8(const void* x, int64_t x_row_stride, void* quantized, float* scales,
                             int64_t n_tokens, int64_t hidden_size, hipStream_t stream);

/*
 * Dynamic per-1x32 MXFP8 quantization (e4m3fn values, e8m0 scale rounded up to a power of two).
 * Replaces: per_group_quant_mxfp8 kernel ABI `run(Tensor x, Tensor(a!) quantized, Tensor(b!) scales)`
 *   (aklr/ops/quant/impls/hip/per_group_quant_mxfp8_hidden_size7168/8480caae0c25689c.json:110),
 *   contract aklr/ops/quant/contract.py:54-75, arithmetic aklr/ops/quant/reference.py:31-48.
 * scales: uint8 [n_tokens, hidden_size/32] row-major (biased exponent). hidden_size % 32 == 0.
 */
int aklr_per_group_quant_mxfp8(const void* x, int64_t x_row_stride, void* quantized, uint8_t* scales,
                               int64_t n_tokens, int64_t hidden_size, hipStream_t stream);

/*
 * Dynamic MXFP4 quantization of activations (e2m1 codes two per byte, low nibble first; one e8m0
 * scale per 32 values along the row).
 * Replaces: aiter dynamic_mxfp4_quant as restated by aklr/ops/fused_moe/reference.py:21-37 (`_mxfp4`);
 *   AKLR has no kernel ABI for it.
 * quantized: uint8 [n_tokens, hidden_size/2]. scales: e8m0 bytes; scale_layout ROW_MAJOR is
 *   [n_tokens, hidden_size/32]; SHUFFLED is the padded, shuffled aiter layout
 *   [ceil(n_tokens/256)*256, ceil(hidden_size/32/8)*8] (the caller pre-fills nothing: padding bytes
 *   are written as 0x00 by this call). hidden_size % 32 == 0.
 */
int aklr_dynamic_mxfp4_quant(const void* x, int64_t x_row_stride, uint8_t* quantized, uint8_t* scales,
                             int64_t n_tokens, int64_t hidden_size, int scale_layout, hipStream_t stream);

/*
 * 128x128-block-scaled FP8 GEMM: out = (a * a_scale) @ (b * b_scale)^T + bias, fp32 accumulation.
 * Replaces: gemm_a8w8_blockwise_scaled kernel ABI `run(a, b, a_scale, b_scale, scale_major_mode,
 *   trans_b, operand_format, bias, out_dtype, out)` (aklr/ops/gemm/impls/flydsl/
 *   gemm_a8w8_blockwise_scaled_b_shuffled_n4096_k2048/5c97ff66d898f5a1.json entry `run`),
 *   contract aklr/ops/gemm/contract.py:211-308, arithmetic aklr/ops/gemm/reference.py:90-105.
 * a: fp8 [m, k], row stride lda elements. b: fp8, trans_b layout [n, k]: ROW_MAJOR with row stride
 *   ldb, or PRESHUFFLE_16x16 (contiguous, ldb ignored). a and b share fp8_dtype.
 * a_scale: fp32, element (i, kb) at a_scale[i*sa_stride_m + kb*sa_stride_k]; this covers K-major
 *   (stride_m = k/128, stride_k = 1), MN-major and aiter's column-major (stride_m = 1, stride_k = m).
 * b_scale: fp32 [ceil(n/128), k/128], row stride ldbs. bias: fp32 [n] or NULL.
 * out: [m, n] bf16 or f16 (out_dtype), row stride ldo.
 * k % 128 == 0, n % 16 == 0. All pointers 16-byte aligned; lda, ldb, ldo multiples of 16 bytes.
 */
size_t aklr_gemm_a8w8_blockscale_workspace_bytes(int64_t m, int64_t n, int64_t k);
/* Which kernel aklr_gemm_a8w8_blockscale runs (m, n, k) on with weight layout b_layout: 0 the stream
 * kernel (weights streamed into registers, activations through LDS), 1 the LDS-tiled kernel, -1 for
 * invalid sizes (a query for callers that report which kernel serves a call; no counterpart in the
 * reference). */
int aklr_gemm_a8w8_blockscale_kernel(int64_t m, int64_t n, int64_t k, int b_layout);
int aklr_gemm_a8w8_blockscale(const void* a, int64_t lda, const void* b, int64_t ldb, const float* a_scale,
                              int64_t sa_stride_m, int64_t sa_stride_k, const float* b_scale, int64_t ldbs,
                              const float* bias, void* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                              int fp8_dtype, int b_layout, int out_dtype, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/*
 * aklr_gemm_a8w8_blockscale without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture that must not call hipMalloc, tight serving loops, harnesses
 * that forbid allocation). No counterpart in the reference: its kernels take scratch from torch
 * allocations inside the call (aklr/ops/README.md:214).
 * Same arguments, kernels, plans and results (bit for bit) as aklr_gemm_a8w8_blockscale. The split-K
 * scratch is a device array of AKLR_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until
 * the process ends; a plan that needs more (aklr_gemm_a8w8_blockscale_workspace_bytes() larger than
 * that: only m > 128 with few output tiles) returns AKLR_ERR_SCRATCH_LIMIT and launches nothing. Every
 * shape of the DeepSeek-V3 decode and prefill configurations fits. The entry point allocates nothing
 * (it looks the array's address up once per device). Calls on one GPU share the array: calls that may
 * overlap in time (other streams, other host threads) race.
 */
#define AKLR_NOALLOC_SCRATCH_BYTES (48u << 20)
int aklr_gemm_a8w8_blockscale_noalloc(const void* a, int64_t lda, const void* b, int64_t ldb, const float* a_scale,
                                      int64_t sa_stride_m, int64_t sa_stride_k, const float* b_scale, int64_t ldbs,
                                      const float* bias, void* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                                      int fp8_dtype, int b_layout, int out_dtype, hipStream_t stream);

/*
 * The current device's copy of the no-allocation array: *ptr receives its device address and *bytes
 * its size (AKLR_NOALLOC_SCRATCH_BYTES). No counterpart in the reference; it lets a caller of
 * aklr_gemm_a8w8_blockscale_noalloc (one that cannot allocate) see the memory those calls share, e.g.
 * to check that a finished call left no split-K arrival word tagged. Allocates nothing; the same
 * once-per-device address lookup as the entry point's.
 */
int aklr_noalloc_scratch(void** ptr, size_t* bytes);

/*
 * Byte transpose dst[c][r] = src[r][c] for a [rows, cols] matrix of 8-bit codes (row strides src_ld,
 * dst_ld in bytes). It serves gemm_a8w8_blockwise_scaled with trans_b = false, where b is (k, n)
 * (aklr/ops/gemm/contract.py:61-76 `_TRANS_B`, aklr/ops/gemm/reference.py:32-37 `_weight`: b.mT): the
 * host side transposes b into (n, k) scratch of its own and calls aklr_gemm_a8w8_blockscale. No kernel
 * ABI of the reference corresponds to it (none of its recorded kernels takes trans_b = false).
 * rows % 16 == 0, cols % 16 == 0; pointers 16-byte aligned; src_ld >= cols and dst_ld >= rows,
 * multiples of 16.
 */
int aklr_transpose_b8(const void* src, int64_t rows, int64_t cols, int64_t src_ld, void* dst, int64_t dst_ld,
                      hipStream_t stream);

/*
 * Per-1x128 FP8 quantization of bf16 activations fused into the block-scaled FP8 GEMM:
 * out = GEMM(per_group_quant_fp8(x), b), equal bit for bit to aklr_per_group_quant_fp8 followed by
 * aklr_gemm_a8w8_blockscale on its codes and group-major scales (e4m3fn).
 * Replaces: the pair of calls sglang's fp8 block-quant linear makes on this path,
 *   per_group_quant_fp8 (aklr/ops/quant/api.py:8-9) then gemm_a8w8_blockwise_scaled
 *   (aklr/ops/gemm/api.py:32-46), with one launch for m <= 16 (the stream kernel's compute waves
 *   quantize each K block into LDS); larger m runs the two kernels, the codes and scales in the workspace.
 * x: bf16 [m, k], row stride ldx elements (multiple of 8). b, b_scale, bias, out as in
 *   aklr_gemm_a8w8_blockscale. The workspace (aklr_quant_gemm_a8w8_blockscale_workspace_bytes) obeys
 *   the same rules (16-byte aligned, any content).
 */
size_t aklr_quant_gemm_a8w8_blockscale_workspace_bytes(int64_t m, int64_t n, int64_t k);
/* 1 when aklr_quant_gemm_a8w8_blockscale runs (m, n, k) as one launch, 0 when as the two kernels
 * (a query for callers that report which kernel serves a call; no counterpart in the reference). */
int aklr_quant_gemm_a8w8_blockscale_fused(int64_t m, int64_t n, int64_t k);
int aklr_quant_gemm_a8w8_blockscale(const void* x, int64_t ldx, const void* b, int64_t ldb, const float* b_scale,
                                    int64_t ldbs, const float* bias, void* out, int64_t ldo, int64_t m, int64_t n,
                                    int64_t k, int b_layout, int out_dtype, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream);

/*
 * MXFP4 GEMM: out = (a * 2^(a_scale-127)) @ (b * 2^(b_scale-127))^T + bias (alpha 1, beta 0).
 * Replaces: gemm_a4w4_mxfp4 kernel ABI `run(a, b, a_scale, b_scale, trans_b, operand_format, alpha,
 *   beta, bias, out_dtype, out)` (call keys per aklr/core/contract/op.py:511-558; no kernel is
 *   committed in the reference), contract aklr/ops/gemm/contract.py:315-390, arithmetic
 *   aklr/ops/gemm/reference.py:108-122.
 * a: packed e2m1 [m, k/2] bytes (low nibble first), row stride lda bytes. b: [n, k/2] bytes,
 *   ROW_MAJOR (row stride ldb) or PRESHUFFLE_16x16 (contiguous). a_scale, b_scale: e8m0 bytes,
 *   ROW_MAJOR ([rows, k/32], row stride given) or SHUFFLED (padded aiter layout, stride ignored).
 * k % 64 == 0 (k % 128 == 0 is not required), n % 16 == 0.
 */
size_t aklr_gemm_a4w4_mxfp4_workspace_bytes(int64_t m, int64_t n, int64_t k);
int aklr_gemm_a4w4_mxfp4(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb, const uint8_t* a_scale,
                         int64_t lds_a, const uint8_t* b_scale, int64_t lds_b, const float* bias, void* out,
                         int64_t ldo, int64_t m, int64_t n, int64_t k, int b_layout, int scale_layout,
                         int out_dtype, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Grouped DeepSeek FP8 MoE (sglang DeepseekV2MoE.forward_normal on one rank): router logits rounded
 * to bf16, sigmoid scores, grouped top-k (a group scored by its two best biased scores), the shared
 * expert as a last slot at weight 1, each expert down(silu(gate(x)) * up(x)) with both linears
 * 128x128-block-scaled FP8 and their inputs quantized per 1x128 at scale amax / 448 (a division),
 * the slots weighed and summed in slot order.
 * Replaces: deepseek_v2_fp8_moe kernel ABI `run(hidden_states, router_weight, correction_bias, w1,
 *   w1_scale, w2, w2_scale, topk, num_expert_group, topk_group, renormalize, scoring_func,
 *   routed_scaling_factor, out)` (call keys of aklr/plugins/sglang/models/deepseek_v2/contract.py:
 *   188-320, api.py:35-50), arithmetic aklr/plugins/sglang/models/deepseek_v2/reference.py:146-183;
 *   the baseline is aiter fused_moe at per_128x128 (deepseek_v2/baseline.py:113-163).
 * hidden, out: bf16 [tokens, model_dim]. router_weight: bf16 [n_routed, model_dim]. correction_bias:
 *   bf16 [n_routed]. w1: e4m3fn [n_routed + 1, 2 * inter_dim, model_dim] (gate rows, then up rows;
 *   the shared expert last), w1_scale fp32 [n_routed + 1, 2 * inter_dim / 128, model_dim / 128];
 *   w2: e4m3fn [n_routed + 1, model_dim, inter_dim], w2_scale fp32 [n_routed + 1, model_dim / 128,
 *   inter_dim / 128]. w_layout: ROW_MAJOR or PRESHUFFLE_16x16 (per expert). scoring is sigmoid.
 * model_dim, inter_dim multiples of 128 (<= 16384); tokens <= 65536; n_routed <= 1024, divisible by
 *   num_expert_group (<= 64) with >= 2 experts per group; topk <= 63.
 * Workspace: aklr_moe_fp8_workspace_bytes(tokens, model_dim, inter_dim, n_routed + 1, topk + 1,
 *   n_routed); no zeroing needed.
 */
size_t aklr_moe_fp8_workspace_bytes(int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t n_experts,
                                    int64_t slots, int64_t n_router_rows);
int aklr_deepseek_v2_fp8_moe(const void* hidden, const void* router_weight, const void* correction_bias,
                             const void* w1, const float* w1_scale, const void* w2, const float* w2_scale,
                             int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t n_routed, int topk,
                             int num_expert_group, int topk_group, int renormalize, float routed_scaling_factor,
                             int w_layout, void* out, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * The routing step alone: logits bf16 [tokens, n_routed], correction_bias bf16 [n_routed] ->
 * ids int32 [tokens, slots], weights fp32 [tokens, slots], slots = topk (+ 1 with append_shared,
 * which sets slot topk to expert n_routed at weight 1). ids are in descending biased score, the
 * lower index first among equals.
 * Replaces: the grouped top-k of aklr/plugins/sglang/models/deepseek_v2/reference.py:121-143 (with
 *   _with_shared_slot :80-89); the baseline calls sglang/aiter's biased_grouped_topk
 *   (deepseek_v2/baseline.py `_route`).
 */
int aklr_moe_fp8_route(const void* logits, const void* correction_bias, int64_t tokens, int64_t n_routed, int topk,
                       int num_expert_group, int topk_group, int renormalize, float routed_scaling_factor,
                       int append_shared, int32_t* ids, float* weights, hipStream_t stream);

/*
 * The experts on a given routing (every slot, the shared one included): out = sum over slots of
 * weights[t, s] * expert_{ids[t, s]}(hidden[t]); slots whose id is outside [0, n_experts) are skipped.
 * Replaces: aiter fused_moe(hidden, w1, w2, topk_weights, topk_ids, activation=Silu,
 *   quant_type=per_128x128, w1_scale, w2_scale) as called by deepseek_v2/baseline.py:152-163;
 *   arithmetic aklr/plugins/sglang/models/deepseek_v2/reference.py:64-77, :146-160, :178-181.
 * ids int32 / weights fp32 [tokens, slots]; weights as in aklr_deepseek_v2_fp8_moe with n_experts
 *   slots. Workspace: aklr_moe_fp8_workspace_bytes(tokens, model_dim, inter_dim, n_experts, slots, 0).
 */
int aklr_moe_fp8_experts(const void* hidden, int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t n_experts,
                         const int32_t* ids, const float* weights, int64_t slots, const void* w1, const float* w1_scale,
                         const void* w2, const float* w2_scale, int w_layout, void* out, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/*
 * Calibration kernel for the decode roofline (no counterpart in the reference): reads `bytes` from
 * `src` with the decode GEMM's access pattern -- 16-byte non-temporal loads, `unroll` (4 or 8) per lane
 * in flight, `workgroups` workgroups of 256 lanes each streaming one contiguous chunk -- and nothing
 * else, so back-to-back launches time the floor of a kernel that reads that many bytes (launch,
 * first-load latency, stream). bytes = 0 is an empty kernel (the launch floor). sink: uint32
 * [workgroups * 256], written only if the data fold to one particular word.
 */
int aklr_probe_hbm_read(const void* src, int64_t bytes, uint32_t* sink, int workgroups, int unroll,
                        hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AKLR_AMD_H */
