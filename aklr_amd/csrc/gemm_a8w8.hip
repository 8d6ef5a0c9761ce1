// 128x128-block-scaled FP8 GEMM for gfx950: out = (a * a_scale) @ (b * b_scale)^T + bias.
//
// Both kernels run one V_MFMA_SCALE_F32_16X16X128_F8F6F4 atom (unit e8m0 scales) per 16x16 output
// tile per 128-wide K block, into a zero accumulator, and fold that partial into the fp32 result
// with one FMA per element: acc += partial * (a_scale[row, kb] * b_scale[n/128, kb]). The fp32 block
// scales are not powers of two, so they cannot ride the MFMA's e8m0 scale operands.
//
// * decode (m <= 128): weight-streaming. A workgroup owns 16*NT output columns and a K range;
//   each wave streams its own contiguous K sub-range of the weight straight from HBM into MFMA
//   operand registers (no LDS), the activations come from L2. Waves are reduced through LDS in
//   wave order; when the K range is split across workgroups too, fp32 partials go to the caller's
//   workspace and a second kernel sums them in split order. Every sum has a fixed order, so
//   results are bitwise reproducible.
// * tile (m > 128): 128x128 workgroup tiles, 4 waves of 64x64, K steps of 128 double-buffered in
//   LDS (16-byte chunks XOR-swizzled by row), a_scale staged in LDS, XCD-aware tile order.
#include "common.h"

namespace aklr {

struct Gemm8Args {
  const uint8_t* a;
  int64_t lda;
  const uint8_t* b;
  int64_t ldb;
  const float* sa;
  int64_t sa_sm, sa_sk;
  const float* sb;
  int64_t ldbs;
  const float* bias;
  void* out;
  int64_t ldo;
  int m, n, k;
  int out_dtype;
  float* partial;  // [splits, m, n] when splits > 1
  int splits;
  int kb_per_split;
};

__device__ __forceinline__ i32x8 cat(const u32x4& lo, const u32x4& hi) {
  i32x8 r;
  r[0] = (int)lo[0]; r[1] = (int)lo[1]; r[2] = (int)lo[2]; r[3] = (int)lo[3];
  r[4] = (int)hi[0]; r[5] = (int)hi[1]; r[6] = (int)hi[2]; r[7] = (int)hi[3];
  return r;
}

// Offset, in a PRESHUFFLE_16x16 weight with kt32 = k/32 column tiles, of the 16 bytes that MFMA lane
// group g (0..3) needs for row `col` and K block kb: k = 16g.. (tile 4kb + g/2, half g%2) and
// k = 64+16g.. (tile 4kb + 2 + g/2). Returns the first; the second is +1024.
__device__ __forceinline__ int64_t preshuffle_frag_offset(int64_t col, int64_t kt32, int kb, int g) {
  return ((col >> 4) * kt32 + (int64_t)kb * 4 + (g >> 1)) * 512 + (g & 1) * 256 + (col & 15) * 16;
}

// ---------------------------------------------------------------------------------------------
// decode
template <int MT, int NT>
struct DecodeFrag {
  i32x8 a[MT];
  i32x8 b[NT];
  float sa[MT][4];
  float sb[NT];
};

template <int MT, int NT, int NW, int FMT, bool PRE>
__global__ __launch_bounds__(NW * 64) void gemm8_decode_kernel(Gemm8Args p) {
  static_assert(NW >= 2, "at least two waves");
  __shared__ f32x4 red[(NW - 1) * MT * NT * 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT;
  const int split = blockIdx.y;
  const int KB = p.k >> 7;
  const int kb_base = split * p.kb_per_split;
  const int kb_len = min(p.kb_per_split, KB - kb_base);
  const int chunk = (kb_len + NW - 1) / NW;
  const int kb_begin = kb_base + min(w * chunk, kb_len);
  const int kb_end = kb_base + min((w + 1) * chunk, kb_len);
  const int64_t kt32 = p.k >> 5;

  const uint8_t* bp[NT];
  bool bval[NT];
  const float* sbp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t col = n0 + nt * 16 + li;
    bval[nt] = (n0 + nt * 16) < p.n;  // n % 16 == 0: validity is uniform per 16-column tile
    if (PRE)
      bp[nt] = p.b + preshuffle_frag_offset(bval[nt] ? col : 0, kt32, 0, g);
    else
      bp[nt] = p.b + (bval[nt] ? col : 0) * p.ldb + g * 16;
    sbp[nt] = p.sb + (int64_t)((bval[nt] ? n0 + nt * 16 : 0) >> 7) * p.ldbs;
  }
  const uint8_t* ap[MT];
  bool aval[MT];
  const float* sap[MT][4];
  bool sval[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 16 + li;
    aval[mt] = row < p.m;
    ap[mt] = p.a + (int64_t)(aval[mt] ? row : 0) * p.lda + g * 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int srow = mt * 16 + 4 * g + r;
      sval[mt][r] = srow < p.m;
      sap[mt][r] = p.sa + (int64_t)(sval[mt][r] ? srow : 0) * p.sa_sm;
    }
  }

  auto load = [&](int kb, DecodeFrag<MT, NT>& f) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      u32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
      if (bval[nt]) {
        if (PRE) {
          lo = ld16_nt(bp[nt] + (int64_t)kb * 2048);
          hi = ld16_nt(bp[nt] + (int64_t)kb * 2048 + 1024);
        } else {
          lo = ld16_nt(bp[nt] + (int64_t)kb * 128);
          hi = ld16_nt(bp[nt] + (int64_t)kb * 128 + 64);
        }
      }
      f.b[nt] = cat(lo, hi);
      f.sb[nt] = bval[nt] ? sbp[nt][kb] : 0.0f;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      u32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
      if (aval[mt]) {
        lo = ld16(ap[mt] + (int64_t)kb * 128);
        hi = ld16(ap[mt] + (int64_t)kb * 128 + 64);
      }
      f.a[mt] = cat(lo, hi);
#pragma unroll
      for (int r = 0; r < 4; ++r) f.sa[mt][r] = sval[mt][r] ? sap[mt][r][(int64_t)kb * p.sa_sk] : 0.0f;
    }
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (kb_begin < kb_end) {
    DecodeFrag<MT, NT> cur, nxt;
    load(kb_begin, cur);
    for (int kb = kb_begin; kb < kb_end; ++kb) {
      if (kb + 1 < kb_end) load(kb + 1, nxt);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          const f32x4 part = mfma16x128<FMT>(cur.a[mt], cur.b[nt], z);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(part[r], cur.sa[mt][r] * cur.sb[nt], acc[mt][nt][r]);
        }
      }
      cur = nxt;
    }
  }

  // Fixed-order reduction over the waves: wave 0 adds waves 1, 2, ... in turn.
  if (w > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) red[(((w - 1) * MT + mt) * NT + nt) * 64 + lane] = acc[mt][nt];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int v = 1; v < NW; ++v)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const f32x4 o = red[(((v - 1) * MT + mt) * NT + nt) * 64 + lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][nt][r] += o[r];
      }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (!bval[nt]) continue;
      const int col = n0 + nt * 16 + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = mt * 16 + 4 * g + r;
        if (row >= p.m) continue;
        if (p.splits > 1) {
          p.partial[((int64_t)split * p.m + row) * p.n + col] = acc[mt][nt][r];
        } else {
          float v = acc[mt][nt][r];
          if (p.bias) v += p.bias[col];
          store_out(p.out, (int64_t)row * p.ldo + col, v, p.out_dtype);
        }
      }
    }
}

// out[row, col] = sum over splits, in split order, of partial[s, row, col] (+ bias[col]).
__global__ __launch_bounds__(256) void gemm8_splitk_reduce_kernel(const float* __restrict__ partial, int splits,
                                                                  int m, int n, const float* __restrict__ bias,
                                                                  void* out, int64_t ldo, int out_dtype) {
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const int64_t total = (int64_t)m * n;
  if (idx >= total) return;
  const int row = (int)(idx / n), col = (int)(idx % n);  // n % 4 == 0: the 4 columns share a row
  f32x4 s = *reinterpret_cast<const f32x4*>(partial + idx);
  for (int sp = 1; sp < splits; ++sp) {
    const f32x4 o = *reinterpret_cast<const f32x4*>(partial + (int64_t)sp * total + idx);
    s += o;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = s[j];
    if (bias) v += bias[col + j];
    store_out(out, (int64_t)row * ldo + col + j, v, out_dtype);
  }
}

// ---------------------------------------------------------------------------------------------
// tile (prefill)
constexpr int kTileM = 128, kTileN = 128;

__device__ __forceinline__ int swz(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

template <int FMT, bool PRE>
__global__ __launch_bounds__(256) void gemm8_tile_kernel(Gemm8Args p) {
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][kTileM * 128];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][kTileN * 128];
  __shared__ __attribute__((aligned(16))) float sSA[2][kTileM];

  const int tiles_m = (p.m + kTileM - 1) / kTileM;
  const int tiles_n = (p.n + kTileN - 1) / kTileN;
  // XCD-aware order (the K splits of one tile are consecutive, so they share an XCD and its L2),
  // then groups of 8 tile-rows so neighbouring tiles share A rows and B columns.
  const int lid = (int)xcd_remap(blockIdx.x, gridDim.x);
  const int pid = lid / p.splits, split = lid % p.splits;
  constexpr int kGroup = 8;
  const int per_group = kGroup * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroup;
  const int gsize = min(tiles_m - first_m, kGroup);
  const int pm = first_m + (pid % per_group) % gsize;
  const int pn = (pid % per_group) / gsize;
  const int m0 = pm * kTileM, n0 = pn * kTileN;

  const int t = threadIdx.x;
  const int lane = t & 63, w = t >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int wm = w >> 1, wn = w & 1;
  const int kb_begin = split * p.kb_per_split;
  const int kb_end = min(p.k >> 7, kb_begin + p.kb_per_split);
  const int64_t kt32 = p.k >> 5;

  // global -> register staging
  const int lc = t & 7, lr = t >> 3;  // chunk and first row this thread moves
  u32x4 ra[4], rb[4];
  float rsa = 0.0f;
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + lr + 32 * i;
      ra[i] = row < p.m ? ld16(p.a + (int64_t)row * p.lda + (int64_t)kb * 128 + lc * 16) : u32x4{0, 0, 0, 0};
    }
    if (PRE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lin = i * 4096 + t * 16;
        const int rt = lin >> 11, off = lin & 2047;
        const int64_t tile_row = (n0 >> 4) + rt;
        rb[i] = (n0 + rt * 16) < p.n ? ld16(p.b + (tile_row * kt32 + (int64_t)kb * 4) * 512 + off)
                                     : u32x4{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = n0 + lr + 32 * i;
        rb[i] = col < p.n ? ld16(p.b + (int64_t)col * p.ldb + (int64_t)kb * 128 + lc * 16) : u32x4{0, 0, 0, 0};
      }
    }
    if (t < kTileM) {
      const int row = m0 + t;
      rsa = row < p.m ? p.sa[(int64_t)row * p.sa_sm + (int64_t)kb * p.sa_sk] : 0.0f;
    }
  };
  auto lstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&sA[st][swz(lr + 32 * i, lc)]) = ra[i];
    if (PRE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lin = i * 4096 + t * 16;
        const int rt = lin >> 11, off = lin & 2047;
        const int kt = off >> 9, h = (off >> 8) & 1, r = (off >> 4) & 15;
        *reinterpret_cast<u32x4*>(&sB[st][swz(rt * 16 + r, kt * 2 + h)]) = rb[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&sB[st][swz(lr + 32 * i, lc)]) = rb[i];
    }
    if (t < kTileM) sSA[st][t] = rsa;
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const float* sbrow = p.sb + (int64_t)(n0 >> 7) * p.ldbs;

  gload(kb_begin);
  lstore(0);
  __syncthreads();
  for (int kb = kb_begin; kb < kb_end; ++kb) {
    const int st = (kb - kb_begin) & 1;
    if (kb + 1 < kb_end) gload(kb + 1);
    const float sb = sbrow[kb];
    i32x8 bf[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int row = wn * 64 + nt * 16 + li;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(&sB[st][swz(row, g)]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(&sB[st][swz(row, 4 + g)]);
      bf[nt] = cat(lo, hi);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int row = wm * 64 + mt * 16 + li;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(&sA[st][swz(row, g)]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(&sA[st][swz(row, 4 + g)]);
      const i32x8 af = cat(lo, hi);
      const f32x4 sa4 = *reinterpret_cast<const f32x4*>(&sSA[st][wm * 64 + mt * 16 + 4 * g]);
      f32x4 s4;
#pragma unroll
      for (int r = 0; r < 4; ++r) s4[r] = sa4[r] * sb;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        const f32x4 part = mfma16x128<FMT>(af, bf[nt], z);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(part[r], s4[r], acc[mt][nt][r]);
      }
    }
    if (kb + 1 < kb_end) lstore(st ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = n0 + wn * 64 + nt * 16 + li;
      if (col >= p.n) continue;
      if (p.splits > 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + wm * 64 + mt * 16 + 4 * g + r;
          if (row < p.m) p.partial[((int64_t)split * p.m + row) * p.n + col] = acc[mt][nt][r];
        }
        continue;
      }
      const float bv = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + mt * 16 + 4 * g + r;
        if (row < p.m) store_out(p.out, (int64_t)row * p.ldo + col, acc[mt][nt][r] + bv, p.out_dtype);
      }
    }
}

// ---------------------------------------------------------------------------------------------
// host-side planning

// m <= kDecodeMaxM streams the weight through the decode kernel; larger m runs the MFMA tile kernel.
static constexpr int64_t kDecodeMaxM = 32;

struct DecodePlan {
  int mt, nw, splits, kb_per_split;
};

static DecodePlan plan_decode(int64_t m, int64_t n, int64_t k) {
  DecodePlan d;
  d.mt = m <= 16 ? 1 : 2;
  const int KB = (int)(k / 128);
  const int64_t n_tiles = (n + 15) / 16;
  // Waves per workgroup: double until ~2048 waves cover the weight (8 per CU), each wave keeping
  // at least 2 K blocks.
  d.nw = 4;
  while (d.nw < 16 && n_tiles * d.nw < 2048 && KB >= 4 * d.nw) d.nw *= 2;
  // Split K across workgroups only when the columns alone give too few waves, keeping at least
  // 2 K blocks per wave and the fp32 partial traffic (8 bytes per output per split) under ~15% of
  // the weight bytes.
  int64_t s = 1;
  if (n_tiles * d.nw < 1024) {
    s = (2048 + n_tiles * d.nw - 1) / (n_tiles * d.nw);
    int64_t s_max = KB / (2 * d.nw);
    const int64_t s_traffic = (int64_t)(0.15 * (double)k / (8.0 * (double)m));
    if (s_traffic < s_max) s_max = s_traffic;
    if (s > s_max) s = s_max;
    if (s < 1) s = 1;
  }
  d.kb_per_split = (int)((KB + s - 1) / s);
  d.splits = (int)((KB + d.kb_per_split - 1) / d.kb_per_split);
  return d;
}

struct TilePlan {
  int tiles, splits, kb_per_split;
};

static TilePlan plan_tile(int64_t m, int64_t n, int64_t k) {
  TilePlan t;
  t.tiles = (int)(((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN));
  const int KB = (int)(k / 128);
  // Split K when the tiles alone leave CUs idle: aim at 2 workgroups per CU (512), keep at least 4
  // K blocks per split, and keep the fp32 partials (8 bytes per output per split, written then
  // summed) within the weight's own bytes.
  int64_t s = 1;
  if (t.tiles < 512) {
    s = (512 + t.tiles - 1) / t.tiles;
    int64_t s_max = KB / 4;
    const int64_t s_traffic = k / (8 * m);
    if (s_traffic < s_max) s_max = s_traffic;
    if (s > s_max) s = s_max;
    if (s < 1) s = 1;
  }
  t.kb_per_split = (int)((KB + s - 1) / s);
  t.splits = (int)((KB + t.kb_per_split - 1) / t.kb_per_split);
  return t;
}

template <int MT, int NW, int FMT, bool PRE>
static void launch_decode(const Gemm8Args& a, const DecodePlan& d, hipStream_t s) {
  dim3 grid((unsigned)((a.n + 15) / 16), (unsigned)d.splits);
  hipLaunchKernelGGL((gemm8_decode_kernel<MT, 1, NW, FMT, PRE>), grid, dim3(NW * 64), 0, s, a);
}

template <int FMT, bool PRE>
static void dispatch_decode(const Gemm8Args& a, const DecodePlan& d, hipStream_t s) {
  if (d.mt == 1) {
    if (d.nw == 16) launch_decode<1, 16, FMT, PRE>(a, d, s);
    else if (d.nw == 8) launch_decode<1, 8, FMT, PRE>(a, d, s);
    else launch_decode<1, 4, FMT, PRE>(a, d, s);
  } else {
    if (d.nw == 16) launch_decode<2, 16, FMT, PRE>(a, d, s);
    else if (d.nw == 8) launch_decode<2, 8, FMT, PRE>(a, d, s);
    else launch_decode<2, 4, FMT, PRE>(a, d, s);
  }
}

template <int FMT, bool PRE>
static void launch_tile(const Gemm8Args& a, const TilePlan& t, hipStream_t s) {
  hipLaunchKernelGGL((gemm8_tile_kernel<FMT, PRE>), dim3((unsigned)(t.tiles * t.splits)), dim3(256), 0, s, a);
}

// Splits and K blocks per split of the kernel that will serve (m, n, k); returns the workspace
// bytes it needs (fp32 partials [splits, m, n] when splits > 1).
static size_t plan_splits(int64_t m, int64_t n, int64_t k, int* splits, int* kb_per_split) {
  if (m <= kDecodeMaxM) {
    const DecodePlan d = plan_decode(m, n, k);
    *splits = d.splits;
    *kb_per_split = d.kb_per_split;
  } else {
    const TilePlan t = plan_tile(m, n, k);
    *splits = t.splits;
    *kb_per_split = t.kb_per_split;
  }
  return *splits > 1 ? (size_t)*splits * (size_t)m * (size_t)n * sizeof(float) : 0;
}

}  // namespace aklr

using namespace aklr;

extern "C" size_t aklr_gemm_a8w8_blockscale_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k < 128) return 0;
  int splits, kps;
  return plan_splits(m, n, k, &splits, &kps);
}

extern "C" int aklr_gemm_a8w8_blockscale(const void* a, int64_t lda, const void* b, int64_t ldb,
                                         const float* a_scale, int64_t sa_stride_m, int64_t sa_stride_k,
                                         const float* b_scale, int64_t ldbs, const float* bias, void* out,
                                         int64_t ldo, int64_t m, int64_t n, int64_t k, int fp8_dtype, int b_layout,
                                         int out_dtype, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
  if (!a || !b || !a_scale || !b_scale || !out) return AKLR_ERR_INVALID_ARGUMENT;
  if (m < 0 || n <= 0 || k <= 0 || k % 128 != 0 || n % 16 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (m > (1 << 20) || n > 262144 || k > 65536) return AKLR_ERR_INVALID_ARGUMENT;
  if (fp8_dtype != AKLR_FP8_E4M3FN && fp8_dtype != AKLR_FP8_E5M2) return AKLR_ERR_UNSUPPORTED;
  if (b_layout != AKLR_B_ROW_MAJOR && b_layout != AKLR_B_PRESHUFFLE_16x16) return AKLR_ERR_UNSUPPORTED;
  if (out_dtype != AKLR_OUT_BF16 && out_dtype != AKLR_OUT_F16) return AKLR_ERR_UNSUPPORTED;
  if (!aklr_aligned16(a) || !aklr_aligned16(b) || !aklr_aligned16(out)) return AKLR_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(a_scale) & 3u) || (reinterpret_cast<uintptr_t>(b_scale) & 3u) ||
      (bias && (reinterpret_cast<uintptr_t>(bias) & 3u)))
    return AKLR_ERR_INVALID_ARGUMENT;
  if (lda < k || lda % 16 != 0 || ldo < n || ldo % 8 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (b_layout == AKLR_B_ROW_MAJOR && (ldb < k || ldb % 16 != 0)) return AKLR_ERR_INVALID_ARGUMENT;
  if (ldbs < k / 128 || sa_stride_m < 0 || sa_stride_k < 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (m == 0) return AKLR_OK;

  Gemm8Args g;
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.b = static_cast<const uint8_t*>(b);
  g.ldb = ldb;
  g.sa = a_scale;
  g.sa_sm = sa_stride_m;
  g.sa_sk = sa_stride_k;
  g.sb = b_scale;
  g.ldbs = ldbs;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.m = (int)m;
  g.n = (int)n;
  g.k = (int)k;
  g.out_dtype = out_dtype;
  g.partial = nullptr;
  const bool pre = b_layout == AKLR_B_PRESHUFFLE_16x16;
  const bool e5 = fp8_dtype == AKLR_FP8_E5M2;

  int splits, kps;
  const size_t need = plan_splits(m, n, k, &splits, &kps);
  g.splits = splits;
  g.kb_per_split = kps;
  if (splits > 1) {
    if (!workspace || workspace_bytes < need || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
    g.partial = static_cast<float*>(workspace);
  }
  if (m <= kDecodeMaxM) {
    const DecodePlan d = plan_decode(m, n, k);
    if (e5) pre ? dispatch_decode<1, true>(g, d, stream) : dispatch_decode<1, false>(g, d, stream);
    else pre ? dispatch_decode<0, true>(g, d, stream) : dispatch_decode<0, false>(g, d, stream);
  } else {
    const TilePlan t = plan_tile(m, n, k);
    if (e5) pre ? launch_tile<1, true>(g, t, stream) : launch_tile<1, false>(g, t, stream);
    else pre ? launch_tile<0, true>(g, t, stream) : launch_tile<0, false>(g, t, stream);
  }
  AKLR_LAUNCH_CHECK();
  if (splits > 1) {
    const int64_t quads = (m * n) / 4;
    hipLaunchKernelGGL(gemm8_splitk_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                       g.partial, splits, g.m, g.n, bias, out, ldo, out_dtype);
    AKLR_LAUNCH_CHECK();
  }
  return AKLR_OK;
}
