// Dynamic activation quantizers for gfx950: per-1x128 FP8 (fp32 scales, group-major), per-1x32
// MXFP8 (e8m0 scales) and per-1x32 MXFP4 (e2m1 codes, e8m0 scales, row-major or aiter-shuffled).
// All three are HBM-bound: one coalesced pass over x, amax reduced with DPP lane moves inside the
// lanes that share a group, codes and scales written once.
#include "common.h"

AKLR_SCALAR_FP32_BEGIN

namespace aklr {

// ---------------------------------------------------------------------------------------------
// per_group_quant_fp8 (aklr/ops/quant/reference.py:9-28)
// A wave covers 8 rows x one 128-wide group: 8 lanes per row, each lane 16 values as two 16-byte
// loads (elements 8j..8j+7 and 64+8j..64+8j+7), so each load instruction reads 128 contiguous
// bytes per row. A 256-thread workgroup covers the same 8 rows x 4 consecutive groups. Workgroup ids
// run along the row first (group quads fastest): concurrent workgroups then read whole rows rather
// than a narrow column band over many rows. Codes are stored non-temporally (the GEMM reads them
// later, from HBM). Scales [g, t] are group-major, so the 8 lanes j == 0 of a wave write 8
// consecutive floats. (Measured at T = 16384, H = 7168 against row-block-fastest order with plain
// stores: 60.8 vs 75.0 us; a wave per row with 8 chunks in flight ran 69 us, its isolated scale
// writes costing more than the deeper loads gain.)
__device__ __forceinline__ void nt_store8(uint8_t* p, uint32_t a, uint32_t b) {
  const u32x2 v = {a, b};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
}

// NT_LOAD: x streams past the caches (large inputs, read once). Small inputs, a decode step's
// activations, load through them: they are usually still cached from the write that made them (measured
// on the decode step: 0.2920 -> 0.2885 ms; at T = 2048 and 16384, H = 7168 the non-temporal loads are
// 4% faster).
constexpr int64_t kQuantCachedLoadBytes = 8ll << 20;
template <bool NT_LOAD>
__global__ __launch_bounds__(256) void quant_fp8_1x128_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                              uint8_t* __restrict__ q, float* __restrict__ scales,
                                                              int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane >> 3, j = lane & 7;
  const int64_t groups = cols >> 7;
  const int64_t quads = (groups + 3) >> 2;
  const int64_t row = (int64_t)(blockIdx.x / quads) * 8 + r;
  const int64_t g = (int64_t)(blockIdx.x % quads) * 4 + wave;
  if (g >= groups) return;  // whole wave exits together
  const bool active = row < rows;

  u32x4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
  const uint16_t* src = x + row * xs + g * 128;
  if (active) {
    v0 = NT_LOAD ? ld16_nt(src + 8 * j) : ld16(src + 8 * j);
    v1 = NT_LOAD ? ld16_nt(src + 64 + 8 * j) : ld16(src + 64 + 8 * j);
  }
  float f[16];
  const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f[2 * i] = bf16_lo(w[i]);
    f[2 * i + 1] = bf16_hi(w[i]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(f[i]));
  // the 8 lanes of a row are one half DPP row: quad swaps, then the half-row mirror (no LDS permutes)
  amax = fmaxf(amax, dpp_f32<0xB1>(amax));   // quad_perm [1,0,3,2]
  amax = fmaxf(amax, dpp_f32<0x4E>(amax));   // quad_perm [2,3,0,1]
  amax = fmaxf(amax, dpp_f32<0x141>(amax));  // row_half_mirror
  amax = fmaxf(amax, kAmaxFloor);
  const float s = amax * kInv448;   // rounds once to fp32
  const float inv = 1.0f / s;       // IEEE division: correctly rounded (no fast-math in this build)
  if (!active) return;
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = fminf(fmaxf(f[4 * i + 0] * inv, -448.0f), 448.0f);
    float b = fminf(fmaxf(f[4 * i + 1] * inv, -448.0f), 448.0f);
    float c = fminf(fmaxf(f[4 * i + 2] * inv, -448.0f), 448.0f);
    float d = fminf(fmaxf(f[4 * i + 3] * inv, -448.0f), 448.0f);
    o[i] = pack4_e4m3(a, b, c, d);
  }
  uint8_t* dst = q + row * cols + g * 128;
  nt_store8(dst + 8 * j, o[0], o[1]);
  nt_store8(dst + 64 + 8 * j, o[2], o[3]);
  if (j == 0) scales[g * rows + row] = s;
}

// ---------------------------------------------------------------------------------------------
// Groups of 32: 4 lanes per group, 8 values (one 16-byte load) per lane; a wave-wide load covers a
// chunk of 512 values (16 groups, 1 KiB of bf16) of one row. A 256-thread workgroup owns one row:
// wave w takes chunks w, w + 4, ..., in rounds of kChunks32 chunks whose loads are all issued before
// any arithmetic.
constexpr int kChunks32 = 8;

struct Group32 {
  float f[8];
  float amax;  // over the 32 values of the group, shared by its 4 lanes
};

__device__ __forceinline__ Group32 unpack_group32(const u32x4& v) {
  Group32 g;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    g.f[2 * i] = bf16_lo(w[i]);
    g.f[2 * i + 1] = bf16_hi(w[i]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(g.f[i]));
  amax = fmaxf(amax, dpp_f32<0xB1>(amax));  // the group's 4 lanes are one quad: quad_perm [1,0,3,2]
  amax = fmaxf(amax, dpp_f32<0x4E>(amax));  // quad_perm [2,3,0,1]
  g.amax = amax;
  return g;
}

// per_group_quant_mxfp8 (aklr/ops/quant/reference.py:31-48)
__global__ __launch_bounds__(256) void quant_mxfp8_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                          uint8_t* __restrict__ q, uint8_t* __restrict__ scales,
                                                          int64_t rows, int64_t cols) {
  const int64_t row = blockIdx.x;
  const int64_t groups = cols >> 5;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int part = lane & 3;
  const int64_t chunks = (groups + 15) >> 4;
  for (int64_t c0 = w; c0 < chunks; c0 += 4 * kChunks32) {
  u32x4 v[kChunks32];
#pragma unroll
  for (int i = 0; i < kChunks32; ++i) {
    const int64_t g = ((c0 + 4 * i) << 4) + (lane >> 2);
    v[i] = u32x4{0, 0, 0, 0};
    if (c0 + 4 * i < chunks && g < groups) v[i] = ld16_nt(x + row * xs + g * 32 + part * 8);
  }
#pragma unroll
  for (int i = 0; i < kChunks32; ++i) {
    if (c0 + 4 * i >= chunks) break;  // wave-uniform
    const int64_t g = ((c0 + 4 * i) << 4) + (lane >> 2);
    const Group32 gv = unpack_group32(v[i]);
    const float amax = fmaxf(gv.amax, kAmaxFloor);
    const uint32_t raw = __float_as_uint(amax * kInv448);
    const uint32_t e = (raw >> 23) + ((raw & 0x7FFFFFu) != 0u);  // biased exponent rounded up
    // x / 2^(e-127) == x * 2^(127-e) exactly: 127-e is in [-120, 43] for finite bf16 inputs.
    const float mul = __uint_as_float((254u - e) << 23);
    if (g >= groups) continue;
    uint32_t o[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float a = fminf(fmaxf(gv.f[4 * t + 0] * mul, -448.0f), 448.0f);
      float b = fminf(fmaxf(gv.f[4 * t + 1] * mul, -448.0f), 448.0f);
      float c = fminf(fmaxf(gv.f[4 * t + 2] * mul, -448.0f), 448.0f);
      float d = fminf(fmaxf(gv.f[4 * t + 3] * mul, -448.0f), 448.0f);
      o[t] = pack4_e4m3(a, b, c, d);
    }
    nt_store8(q + row * cols + g * 32 + part * 8, o[0], o[1]);
    if (part == 0) scales[row * groups + g] = (uint8_t)e;
  }
  }
}

// e2m1 codes of 8 values already divided by the block scale (|v| <= 6): the nearest grid point of
// {0, .5, 1, 1.5, 2, 3, 4, 6}, ties to the even code, sign kept (also on zero) -- what
// V_CVT_SCALEF32_PK_FP4_F32 computes at scale 1.0, two values per instruction, into the byte `sel`
// (first value in the low nibble). On this GPU it agrees with the comparison rule (codes 0..7 at
// |v| > .25, >= .75, > 1.25, >= 1.75, > 2.5, >= 3.5, > 5) on every bf16 value of magnitude <= 6 in
// either operand; the inputs here are bf16 values times a power of two, so that covers them all.
__device__ __forceinline__ uint32_t e2m1_pack8(const float (&f)[8], float mul) {
  uint32_t p = 0;
  p = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(p, f[0] * mul, f[1] * mul, 1.0f, 0);
  p = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(p, f[2] * mul, f[3] * mul, 1.0f, 1);
  p = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(p, f[4] * mul, f[5] * mul, 1.0f, 2);
  p = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(p, f[6] * mul, f[7] * mul, 1.0f, 3);
  return p;
}

// Byte offset of scale (row, col) in aiter's shuffled e8m0 layout over a [pr, pc] padded matrix:
// split (pr/32, 2, 16, pc/8, 2, 4) permuted (0, 3, 5, 2, 4, 1).
__device__ __forceinline__ int64_t shuffled_scale_offset(int64_t row, int64_t col, int64_t pc) {
  const int64_t r0 = row >> 5, r1 = (row >> 4) & 1, r2 = row & 15;
  const int64_t c0 = col >> 3, c2 = (col >> 2) & 1, c3 = col & 3;
  return ((((r0 * (pc >> 3) + c0) * 4 + c3) * 16 + r2) * 2 + c2) * 2 + r1;
}

// dynamic_mxfp4_quant (aklr/ops/fused_moe/reference.py:21-37). One 256-thread workgroup per row, the
// chunks of the MXFP8 kernel. With a shuffled scale layout the grid also covers the padding
// rows/columns, whose scale bytes are written as 0x00.
__global__ __launch_bounds__(256) void quant_mxfp4_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                          uint8_t* __restrict__ q, uint8_t* __restrict__ scales,
                                                          int64_t rows, int64_t cols, int shuffled,
                                                          int64_t pad_cols) {
  const int64_t row = blockIdx.x;
  const int64_t groups = cols >> 5;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int part = lane & 3;
  const int64_t gcount = shuffled ? pad_cols : groups;
  const int64_t chunks = (gcount + 15) >> 4;
  const bool row_on = row < rows;
  for (int64_t c0 = w; c0 < chunks; c0 += 4 * kChunks32) {
  u32x4 v[kChunks32];
#pragma unroll
  for (int i = 0; i < kChunks32; ++i) {
    const int64_t g = ((c0 + 4 * i) << 4) + (lane >> 2);
    v[i] = u32x4{0, 0, 0, 0};
    if (row_on && c0 + 4 * i < chunks && g < groups) v[i] = ld16_nt(x + row * xs + g * 32 + part * 8);
  }
#pragma unroll
  for (int i = 0; i < kChunks32; ++i) {
    if (c0 + 4 * i >= chunks) break;  // wave-uniform
    const int64_t g = ((c0 + 4 * i) << 4) + (lane >> 2);
    const Group32 gv = unpack_group32(v[i]);
    if (g >= gcount) continue;
    const bool active = row_on && g < groups;
    uint32_t sbyte = 0;
    if (active) {
      const float amax = gv.amax;
      uint32_t packed = 0;
      if (__builtin_isfinite(amax)) {
        int e;
        const float m = frexpf(fmaxf(amax, kAmaxFloor), &e);
        int E = e - 3 + (m > 0.75f ? 1 : 0);
        E = E < -127 ? -127 : (E > 127 ? 127 : E);
        // x / 2^E == x * 2^-E exactly (2^-E is representable for E in [-127, 127]; 2^-127 is the
        // subnormal 0x00400000).
        const float mul = E < 127 ? __uint_as_float((uint32_t)(127 - E) << 23) : __uint_as_float(0x00400000u);
        packed = e2m1_pack8(gv.f, mul);
        sbyte = (uint32_t)(E + 127);
      } else {
        sbyte = 255u;
      }
      __builtin_nontemporal_store(packed, reinterpret_cast<uint32_t*>(q + row * (cols >> 1) + g * 16 + part * 4));
    }
    if (part == 0) {
      if (shuffled)
        scales[shuffled_scale_offset(row, g, pad_cols)] = (uint8_t)sbyte;
      else
        scales[row * groups + g] = (uint8_t)sbyte;
    }
  }
  }
}

}  // namespace aklr

using namespace aklr;

extern "C" int aklr_abi_version(void) { return AKLR_AMD_ABI_VERSION; }

extern "C" const char* aklr_status_string(int status) {
  switch (status) {
    case AKLR_OK: return "ok";
    case AKLR_ERR_INVALID_ARGUMENT: return "invalid argument";
    case AKLR_ERR_UNSUPPORTED: return "unsupported layout or dtype";
    case AKLR_ERR_WORKSPACE: return "workspace too small";
    case AKLR_ERR_LAUNCH: return "kernel launch failed";
    case AKLR_ERR_SCRATCH_LIMIT: return "needs more scratch than the no-allocation entry point holds";
    default: return "unknown status";
  }
}

extern "C" int aklr_per_group_quant_fp8(const void* x, int64_t x_row_stride, void* quantized, float* scales,
                                        int64_t n_tokens, int64_t hidden_size, hipStream_t stream) {
  if (!x || !quantized || !scales) return AKLR_ERR_INVALID_ARGUMENT;
  if (n_tokens < 0 || hidden_size <= 0 || hidden_size % 128 != 0 || x_row_stride < hidden_size ||
      x_row_stride % 8 != 0)
    return AKLR_ERR_INVALID_ARGUMENT;
  if (!aklr_aligned16(x) || !aklr_aligned16(quantized) || (reinterpret_cast<uintptr_t>(scales) & 3u))
    return AKLR_ERR_INVALID_ARGUMENT;
  if (n_tokens == 0) return AKLR_OK;
  const int64_t groups = hidden_size / 128;
  const int64_t blocks = (n_tokens + 7) / 8 * ((groups + 3) / 4);
  if (blocks > 0x7FFFFFFF) return AKLR_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)blocks);
  if (n_tokens * hidden_size * 2 > kQuantCachedLoadBytes)
    hipLaunchKernelGGL(quant_fp8_1x128_kernel<true>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                       x_row_stride, static_cast<uint8_t*>(quantized), scales, n_tokens, hidden_size);
  else
    hipLaunchKernelGGL(quant_fp8_1x128_kernel<false>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                       x_row_stride, static_cast<uint8_t*>(quantized), scales, n_tokens, hidden_size);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

extern "C" int aklr_per_group_quant_mxfp8(const void* x, int64_t x_row_stride, void* quantized,
                                          uint8_t* scales, int64_t n_tokens, int64_t hidden_size,
                                          hipStream_t stream) {
  if (!x || !quantized || !scales) return AKLR_ERR_INVALID_ARGUMENT;
  if (n_tokens < 0 || hidden_size <= 0 || hidden_size % 32 != 0 || x_row_stride < hidden_size ||
      x_row_stride % 8 != 0)
    return AKLR_ERR_INVALID_ARGUMENT;
  if (!aklr_aligned16(x) || !aklr_aligned16(quantized)) return AKLR_ERR_INVALID_ARGUMENT;
  if (n_tokens == 0) return AKLR_OK;
  if (n_tokens > 0x7FFFFFFF) return AKLR_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)n_tokens);
  hipLaunchKernelGGL(quant_mxfp8_kernel, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                     x_row_stride, static_cast<uint8_t*>(quantized), scales, n_tokens, hidden_size);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

extern "C" int aklr_dynamic_mxfp4_quant(const void* x, int64_t x_row_stride, uint8_t* quantized, uint8_t* scales,
                                        int64_t n_tokens, int64_t hidden_size, int scale_layout,
                                        hipStream_t stream) {
  if (!x || !quantized || !scales) return AKLR_ERR_INVALID_ARGUMENT;
  if (n_tokens < 0 || hidden_size <= 0 || hidden_size % 32 != 0 || x_row_stride < hidden_size ||
      x_row_stride % 8 != 0)
    return AKLR_ERR_INVALID_ARGUMENT;
  if (scale_layout != AKLR_SCALES_ROW_MAJOR && scale_layout != AKLR_SCALES_SHUFFLED) return AKLR_ERR_UNSUPPORTED;
  if (!aklr_aligned16(x) || (reinterpret_cast<uintptr_t>(quantized) & 3u)) return AKLR_ERR_INVALID_ARGUMENT;
  if (n_tokens == 0) return AKLR_OK;
  const bool shuffled = scale_layout == AKLR_SCALES_SHUFFLED;
  const int64_t groups = hidden_size / 32;
  const int64_t pad_rows = shuffled ? (n_tokens + 255) / 256 * 256 : n_tokens;
  const int64_t pad_cols = shuffled ? (groups + 7) / 8 * 8 : groups;
  if (pad_rows > 0x7FFFFFFF) return AKLR_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)pad_rows);
  hipLaunchKernelGGL(quant_mxfp4_kernel, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                     x_row_stride, quantized, scales, n_tokens, hidden_size, shuffled ? 1 : 0, pad_cols);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

AKLR_SCALAR_FP32_END
