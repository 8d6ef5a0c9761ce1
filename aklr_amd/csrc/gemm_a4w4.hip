// MXFP4 GEMM for gfx950: out = (a * 2^(a_scale-127)) @ (b * 2^(b_scale-127))^T + bias.
//
// Both operands are e2m1 (two per byte, low nibble first) with one e8m0 scale per 32 values along K.
// V_MFMA_SCALE_F32_16X16X128_F8F6F4 with FP4 on both sides takes exactly that: each lane carries 32
// values of one row (lane group g = lane/16 holds k = 32g..32g+31 of the 128-wide step) and the e8m0
// scale of that row and 32-block, and the atom applies the scales itself. No VALU fold: the MFMA
// accumulates straight into the fp32 result.
//
// * decode (m <= 32): weight streaming, as the FP8 decode kernel -- a workgroup owns 16 columns and a
//   K range, each wave a contiguous K sub-range; fixed-order wave reduction in LDS, then (when K is
//   also split across workgroups) fp32 partials in the caller's workspace summed in split order.
// * tile (m > 32): 128x128 tiles, 4 waves of 64x64, K steps of 256 (128 bytes per row) double-
//   buffered in LDS with the scale bytes staged beside them.
// K % 64 == 0: a K step reaching past K reads zero codes and unit scales there.
#include "common.h"

namespace aklr {

struct Gemm4Args {
  const uint8_t* a;
  int64_t lda;  // bytes
  const uint8_t* b;
  int64_t ldb;
  const uint8_t* sa;
  int64_t lds_a;
  const uint8_t* sb;
  int64_t lds_b;
  const float* bias;
  void* out;
  int64_t ldo;
  int m, n, k;
  int b_pre, scale_shuffled, out_dtype;
  int64_t pc;  // padded scale columns (shuffled layout)
  float* partial;
  int splits;
  int ks_per_split;  // 128-wide K steps per split
};

__device__ __forceinline__ int64_t scale_offset(int64_t row, int64_t col, int shuffled, int64_t ld, int64_t pc) {
  if (!shuffled) return row * ld + col;
  const int64_t r0 = row >> 5, r1 = (row >> 4) & 1, r2 = row & 15;
  const int64_t c0 = col >> 3, c2 = (col >> 2) & 1, c3 = col & 3;
  return ((((r0 * (pc >> 3) + c0) * 4 + c3) * 16 + r2) * 2 + c2) * 2 + r1;
}

__device__ __forceinline__ i32x8 fp4_frag(const u32x4& v) {
  i32x8 r;
  r[0] = (int)v[0]; r[1] = (int)v[1]; r[2] = (int)v[2]; r[3] = (int)v[3];
  r[4] = 0; r[5] = 0; r[6] = 0; r[7] = 0;
  return r;
}

constexpr int kFp4 = 4;

// ---------------------------------------------------------------------------------------------
template <int MT, int NW>
__global__ __launch_bounds__(NW * 64) void gemm4_decode_kernel(Gemm4Args p) {
  __shared__ f32x4 red[(NW - 1) * MT * 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int split = blockIdx.y;
  const int KS = (p.k + 127) >> 7;
  const int ks_base = split * p.ks_per_split;
  const int ks_len = min(p.ks_per_split, KS - ks_base);
  const int chunk = (ks_len + NW - 1) / NW;
  const int ks_begin = ks_base + min(w * chunk, ks_len);
  const int ks_end = ks_base + min((w + 1) * chunk, ks_len);
  const int64_t kbytes = p.k >> 1;
  const int64_t kt32 = kbytes >> 5;
  const int64_t kb32 = p.k >> 5;

  const int64_t col = n0 + li;
  const uint8_t* bp = p.b_pre ? p.b + ((col >> 4) * kt32 + (g >> 1)) * 512 + (g & 1) * 256 + (col & 15) * 16
                              : p.b + col * p.ldb + g * 16;
  const int64_t bstep = p.b_pre ? 1024 : 64;

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int ks = ks_begin; ks < ks_end; ++ks) {
    const bool kin = (int64_t)ks * 64 + g * 16 < kbytes;  // this lane group's 32 values exist
    const int64_t c = (int64_t)ks * 4 + g;                  // scale column (32-block)
    u32x4 bv = {0, 0, 0, 0};
    int bs = 127;
    if (kin) {
      bv = ld16_nt(bp + (int64_t)ks * bstep);
      bs = p.sb[scale_offset(col, c, p.scale_shuffled, p.lds_b, p.pc)];
    }
    const i32x8 bf = fp4_frag(bv);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = mt * 16 + li;
      u32x4 av = {0, 0, 0, 0};
      int as = 127;
      if (kin && row < p.m) {
        av = ld16(p.a + (int64_t)row * p.lda + (int64_t)ks * 64 + g * 16);
        as = p.sa[scale_offset(row, c, p.scale_shuffled, p.lds_a, p.pc)];
      }
      acc[mt] = mfma16x128_scaled<kFp4, 0, 0>(fp4_frag(av), bf, acc[mt], as, bs);
    }
  }
  (void)kb32;

  if (w > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[((w - 1) * MT + mt) * 64 + lane] = acc[mt];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int v = 1; v < NW; ++v)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const f32x4 o = red[((v - 1) * MT + mt) * 64 + lane];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mt][r] += o[r];
    }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mt * 16 + 4 * g + r;
      if (row >= p.m) continue;
      if (p.splits > 1) {
        p.partial[((int64_t)split * p.m + row) * p.n + col] = acc[mt][r];
      } else {
        float v = acc[mt][r];
        if (p.bias) v += p.bias[col];
        store_out(p.out, (int64_t)row * p.ldo + col, v, p.out_dtype);
      }
    }
}

__global__ __launch_bounds__(256) void gemm4_splitk_reduce_kernel(const float* __restrict__ partial, int splits,
                                                                  int m, int n, const float* __restrict__ bias,
                                                                  void* out, int64_t ldo, int out_dtype) {
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const int64_t total = (int64_t)m * n;
  if (idx >= total) return;
  const int row = (int)(idx / n), col = (int)(idx % n);
  f32x4 s = *reinterpret_cast<const f32x4*>(partial + idx);
  for (int sp = 1; sp < splits; ++sp) s += *reinterpret_cast<const f32x4*>(partial + (int64_t)sp * total + idx);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = s[j];
    if (bias) v += bias[col + j];
    store_out(out, (int64_t)row * ldo + col + j, v, out_dtype);
  }
}

// ---------------------------------------------------------------------------------------------
constexpr int kT4M = 128, kT4N = 128;

__device__ __forceinline__ int swz4(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

__global__ __launch_bounds__(256) void gemm4_tile_kernel(Gemm4Args p) {
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][kT4M * 128];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][kT4N * 128];
  __shared__ __attribute__((aligned(16))) uint8_t sSa[2][kT4M * 8];
  __shared__ __attribute__((aligned(16))) uint8_t sSb[2][kT4N * 8];

  const int tiles_m = (p.m + kT4M - 1) / kT4M;
  const int tiles_n = (p.n + kT4N - 1) / kT4N;
  const int pid = (int)xcd_remap(blockIdx.x, gridDim.x);
  constexpr int kGroup = 8;
  const int per_group = kGroup * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroup;
  const int gsize = min(tiles_m - first_m, kGroup);
  const int pm = first_m + (pid % per_group) % gsize;
  const int pn = (pid % per_group) / gsize;
  const int m0 = pm * kT4M, n0 = pn * kT4N;

  const int t = threadIdx.x;
  const int lane = t & 63, w = t >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int wm = w >> 1, wn = w & 1;
  const int64_t kbytes = p.k >> 1;
  const int64_t kt32 = kbytes >> 5;
  const int64_t kb32 = p.k >> 5;
  const int KS = (int)((kbytes + 127) >> 7);  // 256-wide K steps

  const int lc = t & 7, lr = t >> 3;
  u32x4 ra[4], rb[4];
  uint32_t rs[2];  // 8 scale bytes of row/col (t & 127) of A (t < 128) or B (t >= 128)
  auto gload = [&](int ks) {
    const int64_t kofs = (int64_t)ks * 128 + lc * 16;
    const bool kin = kofs < kbytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + lr + 32 * i;
      ra[i] = (kin && row < p.m) ? ld16(p.a + (int64_t)row * p.lda + kofs) : u32x4{0, 0, 0, 0};
    }
    if (p.b_pre) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lin = i * 4096 + t * 16;
        const int rt = lin >> 11, off = lin & 2047;
        const int kt = off >> 9;  // 32-byte column tile within the step
        const int64_t tile_row = (n0 >> 4) + rt;
        const bool ok = (n0 + rt * 16) < p.n && ((int64_t)ks * 4 + kt) < kt32;
        rb[i] = ok ? ld16(p.b + (tile_row * kt32 + (int64_t)ks * 4) * 512 + off) : u32x4{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = n0 + lr + 32 * i;
        rb[i] = (kin && col < p.n) ? ld16(p.b + (int64_t)col * p.ldb + kofs) : u32x4{0, 0, 0, 0};
      }
    }
    const bool is_a = t < 128;
    const int r = (t & 127) + (is_a ? m0 : n0);
    const bool rok = is_a ? r < p.m : r < p.n;
    const uint8_t* sp = is_a ? p.sa : p.sb;
    const int64_t ld = is_a ? p.lds_a : p.lds_b;
    uint32_t w2[2] = {0x7F7F7F7Fu, 0x7F7F7F7Fu};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t c = (int64_t)ks * 8 + j;
      if (rok && c < kb32) {
        const uint32_t byte = sp[scale_offset(r, c, p.scale_shuffled, ld, p.pc)];
        w2[j >> 2] = (w2[j >> 2] & ~(0xFFu << (8 * (j & 3)))) | (byte << (8 * (j & 3)));
      }
    }
    rs[0] = w2[0];
    rs[1] = w2[1];
  };
  auto lstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&sA[st][swz4(lr + 32 * i, lc)]) = ra[i];
    if (p.b_pre) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lin = i * 4096 + t * 16;
        const int rt = lin >> 11, off = lin & 2047;
        const int kt = off >> 9, h = (off >> 8) & 1, r = (off >> 4) & 15;
        *reinterpret_cast<u32x4*>(&sB[st][swz4(rt * 16 + r, kt * 2 + h)]) = rb[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&sB[st][swz4(lr + 32 * i, lc)]) = rb[i];
    }
    uint8_t* dst = t < 128 ? &sSa[st][(t & 127) * 8] : &sSb[st][(t & 127) * 8];
    *reinterpret_cast<u32x2*>(dst) = u32x2{rs[0], rs[1]};
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  gload(0);
  lstore(0);
  __syncthreads();
  for (int ks = 0; ks < KS; ++ks) {
    const int st = ks & 1;
    if (ks + 1 < KS) gload(ks + 1);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      i32x8 bf[4];
      int bsc[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int row = wn * 64 + nt * 16 + li;
        bf[nt] = fp4_frag(*reinterpret_cast<const u32x4*>(&sB[st][swz4(row, s * 4 + g)]));
        bsc[nt] = sSb[st][row * 8 + s * 4 + g];
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = wm * 64 + mt * 16 + li;
        const i32x8 af = fp4_frag(*reinterpret_cast<const u32x4*>(&sA[st][swz4(row, s * 4 + g)]));
        const int asc = sSa[st][row * 8 + s * 4 + g];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = mfma16x128_scaled<kFp4, 0, 0>(af, bf[nt], acc[mt][nt], asc, bsc[nt]);
      }
    }
    if (ks + 1 < KS) lstore(st ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = n0 + wn * 64 + nt * 16 + li;
      if (col >= p.n) continue;
      const float bv = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + mt * 16 + 4 * g + r;
        if (row < p.m) store_out(p.out, (int64_t)row * p.ldo + col, acc[mt][nt][r] + bv, p.out_dtype);
      }
    }
}

// ---------------------------------------------------------------------------------------------
struct Decode4Plan {
  int mt, nw, splits, ks_per_split;
};

static Decode4Plan plan_decode4(int64_t m, int64_t n, int64_t k) {
  Decode4Plan d;
  d.mt = m <= 16 ? 1 : 2;
  const int KS = (int)((k + 127) / 128);
  d.nw = KS < 16 ? 4 : 8;
  const int64_t n_tiles = n / 16;
  int64_t s = (4096 + n_tiles * d.nw - 1) / (n_tiles * d.nw);
  int64_t s_max = KS / (2 * d.nw);
  // partial traffic (8 B per output per split) under ~15% of the weight bytes (k/2 + k/32 per column)
  const int64_t s_traffic = (int64_t)(0.15 * (double)k * 0.53125 / (8.0 * (double)m));
  if (s_traffic < s_max) s_max = s_traffic;
  if (s > s_max) s = s_max;
  if (s < 1) s = 1;
  d.ks_per_split = (int)((KS + s - 1) / s);
  d.splits = (int)((KS + d.ks_per_split - 1) / d.ks_per_split);
  return d;
}

static constexpr int64_t kDecode4MaxM = 32;

}  // namespace aklr

using namespace aklr;

extern "C" size_t aklr_gemm_a4w4_mxfp4_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k < 64 || m > kDecode4MaxM) return 0;
  const Decode4Plan d = plan_decode4(m, n, k);
  return d.splits > 1 ? (size_t)d.splits * (size_t)m * (size_t)n * sizeof(float) : 0;
}

extern "C" int aklr_gemm_a4w4_mxfp4(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb,
                                    const uint8_t* a_scale, int64_t lds_a, const uint8_t* b_scale, int64_t lds_b,
                                    const float* bias, void* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                                    int b_layout, int scale_layout, int out_dtype, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  if (!a || !b || !a_scale || !b_scale || !out) return AKLR_ERR_INVALID_ARGUMENT;
  if (m < 0 || n <= 0 || k <= 0 || k % 64 != 0 || n % 16 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (m > (1 << 20) || n > 262144 || k > 65536) return AKLR_ERR_INVALID_ARGUMENT;
  if (b_layout != AKLR_B_ROW_MAJOR && b_layout != AKLR_B_PRESHUFFLE_16x16) return AKLR_ERR_UNSUPPORTED;
  if (scale_layout != AKLR_SCALES_ROW_MAJOR && scale_layout != AKLR_SCALES_SHUFFLED) return AKLR_ERR_UNSUPPORTED;
  if (out_dtype != AKLR_OUT_BF16 && out_dtype != AKLR_OUT_F16) return AKLR_ERR_UNSUPPORTED;
  if (!aklr_aligned16(a) || !aklr_aligned16(b) || !aklr_aligned16(out)) return AKLR_ERR_INVALID_ARGUMENT;
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 3u)) return AKLR_ERR_INVALID_ARGUMENT;
  if (lda < k / 2 || lda % 16 != 0 || ldo < n || ldo % 8 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (b_layout == AKLR_B_ROW_MAJOR && (ldb < k / 2 || ldb % 16 != 0)) return AKLR_ERR_INVALID_ARGUMENT;
  if (scale_layout == AKLR_SCALES_ROW_MAJOR && (lds_a < k / 32 || lds_b < k / 32)) return AKLR_ERR_INVALID_ARGUMENT;
  if (m == 0) return AKLR_OK;

  Gemm4Args g;
  g.a = a;
  g.lda = lda;
  g.b = b;
  g.ldb = ldb;
  g.sa = a_scale;
  g.lds_a = lds_a;
  g.sb = b_scale;
  g.lds_b = lds_b;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.m = (int)m;
  g.n = (int)n;
  g.k = (int)k;
  g.b_pre = b_layout == AKLR_B_PRESHUFFLE_16x16;
  g.scale_shuffled = scale_layout == AKLR_SCALES_SHUFFLED;
  g.out_dtype = out_dtype;
  g.pc = (k / 32 + 7) / 8 * 8;
  g.partial = nullptr;
  g.splits = 1;
  g.ks_per_split = (int)((k + 127) / 128);

  if (m <= kDecode4MaxM) {
    const Decode4Plan d = plan_decode4(m, n, k);
    g.splits = d.splits;
    g.ks_per_split = d.ks_per_split;
    if (d.splits > 1) {
      const size_t need = (size_t)d.splits * (size_t)m * (size_t)n * sizeof(float);
      if (!workspace || workspace_bytes < need || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
      g.partial = static_cast<float*>(workspace);
    }
    dim3 grid((unsigned)(n / 16), (unsigned)d.splits);
    if (d.mt == 1 && d.nw == 8) hipLaunchKernelGGL((gemm4_decode_kernel<1, 8>), grid, dim3(512), 0, stream, g);
    else if (d.mt == 1) hipLaunchKernelGGL((gemm4_decode_kernel<1, 4>), grid, dim3(256), 0, stream, g);
    else if (d.nw == 8) hipLaunchKernelGGL((gemm4_decode_kernel<2, 8>), grid, dim3(512), 0, stream, g);
    else hipLaunchKernelGGL((gemm4_decode_kernel<2, 4>), grid, dim3(256), 0, stream, g);
    AKLR_LAUNCH_CHECK();
    if (d.splits > 1) {
      const int64_t quads = (m * n) / 4;
      hipLaunchKernelGGL(gemm4_splitk_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                         g.partial, d.splits, g.m, g.n, bias, out, ldo, out_dtype);
      AKLR_LAUNCH_CHECK();
    }
    return AKLR_OK;
  }
  const int tiles = (int)(((m + kT4M - 1) / kT4M) * ((n + kT4N - 1) / kT4N));
  hipLaunchKernelGGL(gemm4_tile_kernel, dim3((unsigned)tiles), dim3(256), 0, stream, g);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}
