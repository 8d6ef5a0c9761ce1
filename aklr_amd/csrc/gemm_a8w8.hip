// 128x128-block-scaled FP8 GEMM for gfx950: out = (a * a_scale) @ (b * b_scale)^T + bias.
//
// Every kernel runs one V_MFMA_SCALE_F32_16X16X128_F8F6F4 atom (unit e8m0 scales) per 16x16 output
// tile per 128-wide K block, into a zero accumulator, and folds that partial into the fp32 result
// with one FMA per element: acc += partial * (a_scale[row, kb] * b_scale[n/128, kb]). The fp32 block
// scales are not powers of two, so they cannot ride the MFMA's e8m0 scale operands.
//
// * skinny (m <= 64): weight streaming. A workgroup owns 16*NT output columns and a K range; each of
//   its waves streams its own contiguous K sub-range of the weight straight from HBM into MFMA
//   operand registers (no LDS), D K-blocks in flight, with the activations from L2. The waves'
//   accumulators are summed in one LDS tile in wave order.
// * tile (m > 64): 128x128 workgroup tiles, 4 waves of 64x64, K steps of 128 double-buffered in
//   LDS (16-byte chunks XOR-swizzled by row), a_scale staged in LDS, XCD-aware tile order.
//
// When K is also split across workgroups, each stores an fp32 partial into the caller's workspace
// and the last workgroup of the output tile to arrive (an agent-scope counter) sums the partials in
// split order and writes the output: one launch, and every sum has a fixed order, so results are
// bitwise reproducible.
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
  unsigned* counters;  // one per output tile when splits > 1
  float* partial;      // [splits, n, round4(m)] when splits > 1
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
// k = 64+16g.. (tile 4kb + 2 + g/2). Returns the first; the second is +1024. The 64 lanes of one
// load read 1 KiB: two runs of 512 contiguous bytes.
__device__ __forceinline__ int64_t preshuffle_frag_offset(int64_t col, int64_t kt32, int kb, int g) {
  return ((col >> 4) * kt32 + (int64_t)kb * 4 + (g >> 1)) * 512 + (g & 1) * 256 + (col & 15) * 16;
}

// ---------------------------------------------------------------------------------------------
// skinny
template <int MT, int NT>
struct SkinnyFrag {
  i32x8 a[MT];
  i32x8 b[NT];
  float sa[MT][4];
  float sb[NT];
};

template <int MT, int NT, int NW, int D, int FMT, bool PRE>
__global__ __launch_bounds__(NW * 64) void gemm8_skinny_kernel(Gemm8Args p) {
  constexpr int T = MT * NT;
  __shared__ f32x4 red[T][64];
  __shared__ unsigned arrive_slot;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: K ranges live in SGPRs
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

  // A and B come through raw buffer loads whose per-block offset is switched off (kOobOffset: zeros,
  // no memory access) past the wave's K range, so the loop below refills its register ring with no
  // branch. Rows past m and column tiles past n read row/tile 0 instead: they only feed output rows
  // and columns that are never stored. B gets one descriptor per 16-column tile (offsets < 16*ldb).
  rsrc_t brs[NT];
  const float* sbp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t c0 = (n0 + nt * 16) < p.n ? n0 + nt * 16 : 0;  // n % 16 == 0: validity per tile
    if (PRE)
      brs[nt] = make_rsrc(p.b + (c0 >> 4) * kt32 * 512, (uint32_t)(kt32 * 512));
    else
      brs[nt] = make_rsrc(p.b + c0 * p.ldb, (uint32_t)(15 * p.ldb + p.k));
    sbp[nt] = p.sb + (c0 >> 7) * p.ldbs;
  }
  const uint32_t b_lane = PRE ? (uint32_t)((g >> 1) * 512 + (g & 1) * 256 + li * 16)
                              : (uint32_t)(li * p.ldb + g * 16);
  // Activation fragments and a_scale are loaded only by lanes whose rows exist: the others get the
  // out-of-range offset (zeros, no request), which for m < 16 removes most of their L2 traffic.
  const rsrc_t ars = make_rsrc(p.a, (uint32_t)((p.m - 1) * p.lda + p.k));
  const rsrc_t sars = make_rsrc(p.sa, (uint32_t)(((p.m - 1) * p.sa_sm + (KB - 1) * p.sa_sk + 1) * 4));
  uint32_t a_lane[MT];
  uint32_t sa_lane[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 16 + li;
    a_lane[mt] = row < p.m ? (uint32_t)(row * p.lda + g * 16) : kOobOffset;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int srow = mt * 16 + 4 * g + r;
      sa_lane[mt][r] = srow < p.m ? (uint32_t)(srow * p.sa_sm * 4) : kOobOffset;
    }
  }
  const uint32_t sa_kstep = (uint32_t)(p.sa_sk * 4);

  auto load = [&](int kb, SkinnyFrag<MT, NT>& f) {
    const bool on = kb < kb_end;
    const int kbc = min(kb, KB - 1);  // b_scale: any valid block (its product with zero data is 0)
    const uint32_t boff = on ? (uint32_t)(PRE ? kb * 2048 : kb * 128) : kOobOffset;
    const uint32_t aoff = on ? (uint32_t)(kb * 128) : kOobOffset;
    const uint32_t soff = on ? (uint32_t)kb * sa_kstep : kOobOffset;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f.b[nt] = cat(buf_ld16<kNt>(brs[nt], b_lane + boff), buf_ld16<kNt>(brs[nt], b_lane + boff + (PRE ? 1024 : 64)));
      f.sb[nt] = sbp[nt][kbc];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f.a[mt] = cat(buf_ld16(ars, a_lane[mt] + aoff), buf_ld16(ars, a_lane[mt] + aoff + 64));
#pragma unroll
      for (int r = 0; r < 4; ++r)
        f.sa[mt][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sars, (int)(sa_lane[mt][r] + soff), 0, 0));
    }
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // D-deep register ring: block kb0 + j lives in f[j]; once consumed, the slot is refilled with block
  // kb0 + j + D. Blocks past kb_end load as zeros, so the last group needs no special case.
  SkinnyFrag<MT, NT> f[D];
#pragma unroll
  for (int j = 0; j < D; ++j) load(kb_begin + j, f[j]);
  for (int kb0 = kb_begin; kb0 < kb_end; kb0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          const f32x4 part = mfma16x128<FMT>(f[j].a[mt], f[j].b[nt], z);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[mt][nt][r] = fmaf(part[r], f[j].sa[mt][r] * f[j].sb[nt], acc[mt][nt][r]);
        }
      load(kb0 + j + D, f[j]);
      __builtin_amdgcn_sched_barrier(0);  // refill slot j before consuming slot j + 1
    }
  }

  // Sum the waves' accumulators in wave order: wave 0 stores, waves 1.. NW-1 add in turn.
  for (int v = 0; v < NW; ++v) {
    if (w == v) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int t = mt * NT + nt;
          red[t][lane] = v == 0 ? acc[mt][nt] : red[t][lane] + acc[mt][nt];
        }
    }
    __syncthreads();
  }

  // Wave w owns tiles t = w, w + NW, ...: it writes the output (one split) or its fp32 partial.
  const int64_t m4 = round4(p.m);
  const int64_t plane = (int64_t)p.n * m4;
  for (int t = w; t < T; t += NW) {
    const int mt = t / NT, nt = t % NT;
    const int c0 = n0 + nt * 16;
    if (c0 >= p.n) continue;
    const f32x4 s = red[t][lane];
    const int col = c0 + li;
    const int row0 = mt * 16 + 4 * g;
    if (p.splits > 1) {
      if (row0 < p.m) store_partial4(partial_rsrc(p.partial, split, plane), (int64_t)col * m4 + row0, s);
      continue;
    }
    const float bv = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (row0 + r < p.m) store_out(p.out, (int64_t)(row0 + r) * p.ldo + col, s[r] + bv, p.out_dtype);
  }
  if (p.splits == 1) return;
  if (!splitk_arrive(p.counters + blockIdx.x, p.splits, &arrive_slot)) return;
  for (int t = w; t < T; t += NW) {
    const int mt = t / NT, nt = t % NT;
    const int c0 = n0 + nt * 16;
    const int row0 = mt * 16 + 4 * g;
    if (c0 >= p.n || row0 >= p.m) continue;
    const int col = c0 + li;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < p.splits; ++sp) v += load_partial4(partial_rsrc(p.partial, sp, plane), (int64_t)col * m4 + row0);
    const float bv = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (row0 + r < p.m) store_out(p.out, (int64_t)(row0 + r) * p.ldo + col, v[r] + bv, p.out_dtype);
  }
}

// ---------------------------------------------------------------------------------------------
// tile
constexpr int kTileM = 128, kTileN = 128;

__device__ __forceinline__ int swz(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

template <int FMT, bool PRE>
__global__ __launch_bounds__(256) void gemm8_tile_kernel(Gemm8Args p) {
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][kTileM * 128];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][kTileN * 128];
  __shared__ __attribute__((aligned(16))) float sSA[2][kTileM];
  __shared__ unsigned arrive_slot;

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

  if (p.splits > 1) {
    const int64_t m4 = round4(p.m);
    const int64_t plane = (int64_t)p.n * m4;
    const rsrc_t prs = partial_rsrc(p.partial, split, plane);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int col = n0 + wn * 64 + nt * 16 + li;
        const int row0 = m0 + wm * 64 + mt * 16 + 4 * g;
        if (col < p.n && row0 < p.m) store_partial4(prs, (int64_t)col * m4 + row0, acc[mt][nt]);
      }
    if (!splitk_arrive(p.counters + pid, p.splits, &arrive_slot)) return;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int col = n0 + wn * 64 + nt * 16 + li;
        const int row0 = m0 + wm * 64 + mt * 16 + 4 * g;
        if (col >= p.n || row0 >= p.m) continue;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < p.splits; ++sp) v += load_partial4(partial_rsrc(p.partial, sp, plane), (int64_t)col * m4 + row0);
        const float bv = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (row0 + r < p.m) store_out(p.out, (int64_t)(row0 + r) * p.ldo + col, v[r] + bv, p.out_dtype);
      }
    return;
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
// host-side planning

// m <= kSkinnyMaxM streams the weight through the skinny kernel; larger m runs the MFMA tile kernel.
static constexpr int64_t kSkinnyMaxM = 64;

struct Plan8 {
  bool skinny;
  int mt, nt, nw;    // skinny: 16-row and 16-column tiles per wave, waves per workgroup
  int grid_x;        // skinny: column groups; tile: output tiles
  int splits, kb_per_split;
};

// Skinny plan (measured on MI355X over the DeepSeek-V3 decode shapes, weights streamed from HBM):
// one 16-column tile per wave while the activations are a few rows (two once n >= 16384, which
// leaves >= 512 groups), two at m <= 16, four at m <= 32, and at m <= 64 four when K is long (>= 64
// blocks) else two, so activation re-reads from L2 stay a fraction of the weight bytes; waves per
// workgroup sized for ~2048 streaming waves chip-wide (4 or 8, each wave >= 2 K blocks); K split
// across two workgroups only when that still leaves fewer than 1024 waves, since the split's
// coherent hand-off costs about a kernel launch. Row tiles 1-2 keep two K blocks in flight per
// wave; four row tiles keep one (their registers would otherwise spill).
static Plan8 plan8(int64_t m, int64_t n, int64_t k) {
  Plan8 p;
  const int64_t KB = k / 128;
  int64_t s = 1;
  if (m <= kSkinnyMaxM) {
    p.skinny = true;
    p.mt = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    if (p.mt == 4)
      p.nt = KB >= 64 ? 4 : 2;
    else
      p.nt = m <= 8 ? (n >= 16384 ? 2 : 1) : (m <= 16 ? 2 : 4);
    const int64_t groups = (n + 16 * p.nt - 1) / (16 * p.nt);
    p.grid_x = (int)groups;
    p.nw = (2048 / groups >= 8 && KB >= 16 && !(p.mt == 4 && p.nt == 4)) ? 8 : 4;
    if (groups * p.nw < 1024 && KB >= 4 * p.nw) s = 2;
  } else {
    p.skinny = false;
    p.mt = p.nt = p.nw = 0;
    const int64_t tiles = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN);
    p.grid_x = (int)tiles;
    // Split K when the tiles alone leave CUs idle: aim at 2 workgroups per CU (512), keep at least 4
    // K blocks per split, and keep the fp32 partials within the weight's own bytes.
    if (tiles < 512) {
      s = (512 + tiles - 1) / tiles;
      int64_t s_max = KB / 4;
      const int64_t s_traffic = k / (8 * m);
      if (s_traffic < s_max) s_max = s_traffic;
      if (s > s_max) s = s_max;
    }
  }
  if (s < 1 || p.grid_x > kSplitkMaxTiles) s = 1;  // one counter per output tile must fit the region
  p.kb_per_split = (int)((KB + s - 1) / s);
  p.splits = (int)((KB + p.kb_per_split - 1) / p.kb_per_split);
  return p;
}

static size_t workspace8(const Plan8& p, int64_t m, int64_t n) {
  if (p.splits <= 1) return 0;
  return kSplitkCounterBytes + (size_t)p.splits * (size_t)round4(m) * (size_t)n * sizeof(float);
}

template <int MT, int NT, int NW, int FMT, bool PRE>
static void launch_skinny(const Gemm8Args& a, const Plan8& d, hipStream_t s) {
  constexpr int D = MT >= 4 ? 1 : 2;
  dim3 grid((unsigned)d.grid_x, (unsigned)d.splits);
  hipLaunchKernelGGL((gemm8_skinny_kernel<MT, NT, NW, D, FMT, PRE>), grid, dim3(NW * 64), 0, s, a);
}

template <int MT, int NT, int FMT, bool PRE>
static void dispatch_skinny_nw(const Gemm8Args& a, const Plan8& d, hipStream_t s) {
  if (d.nw == 8) launch_skinny<MT, NT, 8, FMT, PRE>(a, d, s);
  else launch_skinny<MT, NT, 4, FMT, PRE>(a, d, s);
}

template <int MT, int FMT, bool PRE>
static void dispatch_skinny_nt(const Gemm8Args& a, const Plan8& d, hipStream_t s) {
  if (d.nt == 4) dispatch_skinny_nw<MT, 4, FMT, PRE>(a, d, s);
  else if (d.nt == 2) dispatch_skinny_nw<MT, 2, FMT, PRE>(a, d, s);
  else dispatch_skinny_nw<MT, 1, FMT, PRE>(a, d, s);
}

template <int FMT, bool PRE>
static void dispatch_skinny(const Gemm8Args& a, const Plan8& d, hipStream_t s) {
  if (d.mt == 1) dispatch_skinny_nt<1, FMT, PRE>(a, d, s);
  else if (d.mt == 2) dispatch_skinny_nt<2, FMT, PRE>(a, d, s);
  else if (d.nt == 4) launch_skinny<4, 4, 4, FMT, PRE>(a, d, s);  // 4x4 tiles run with 4 waves only
  else if (d.nw == 8) launch_skinny<4, 2, 8, FMT, PRE>(a, d, s);
  else launch_skinny<4, 2, 4, FMT, PRE>(a, d, s);
}

template <int FMT, bool PRE>
static void launch_tile(const Gemm8Args& a, const Plan8& t, hipStream_t s) {
  hipLaunchKernelGGL((gemm8_tile_kernel<FMT, PRE>), dim3((unsigned)(t.grid_x * t.splits)), dim3(256), 0, s, a);
}

}  // namespace aklr

using namespace aklr;

extern "C" size_t aklr_gemm_a8w8_blockscale_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k < 128) return 0;
  return workspace8(plan8(m, n, k), m, n);
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
  g.counters = nullptr;
  g.partial = nullptr;
  const bool pre = b_layout == AKLR_B_PRESHUFFLE_16x16;
  const bool e5 = fp8_dtype == AKLR_FP8_E5M2;

  const Plan8 plan = plan8(m, n, k);
  g.splits = plan.splits;
  g.kb_per_split = plan.kb_per_split;
  if (plan.splits > 1) {
    const size_t need = workspace8(plan, m, n);
    if (!workspace || workspace_bytes < need || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
    g.counters = static_cast<unsigned*>(workspace);
    g.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kSplitkCounterBytes);
  }
  if (plan.skinny) {
    if (e5) pre ? dispatch_skinny<1, true>(g, plan, stream) : dispatch_skinny<1, false>(g, plan, stream);
    else pre ? dispatch_skinny<0, true>(g, plan, stream) : dispatch_skinny<0, false>(g, plan, stream);
  } else {
    if (e5) pre ? launch_tile<1, true>(g, plan, stream) : launch_tile<1, false>(g, plan, stream);
    else pre ? launch_tile<0, true>(g, plan, stream) : launch_tile<0, false>(g, plan, stream);
  }
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}
