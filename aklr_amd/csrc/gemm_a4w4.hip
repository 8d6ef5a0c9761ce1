// MXFP4 GEMM for gfx950: out = (a * 2^(a_scale-127)) @ (b * 2^(b_scale-127))^T + bias.
//
// Both operands are e2m1 (two per byte, low nibble first) with one e8m0 scale per 32 values along K.
// V_MFMA_SCALE_F32_16X16X128_F8F6F4 with FP4 on both sides takes exactly that: each lane carries 32
// values of one row (lane group g = lane/16 holds k = 32g..32g+31 of the 128-wide step) and the e8m0
// scale of that row and 32-block, and the atom applies the scales itself. No VALU fold: the MFMA
// accumulates straight into the fp32 result.
//
// * skinny (m <= 16, and 16 < m <= 32 with unaligned row-major scales): weight streaming -- a
//   workgroup owns 32 columns and a K range, each wave a contiguous K sub-range with a register ring;
//   fixed-order wave reduction in LDS, then (when K is also split across workgroups) fp32 partials
//   summed in split order by the last workgroup to arrive.
// * stream (16 < m <= 32): the FP8 stream kernel's design -- compute waves stream their own weight
//   columns into register rings while a loader wave stages A and its scales in LDS for all of them.
// * lds (m > 32, k % 256 == 0): the FP8 LDS kernel's tiles and direct-to-LDS ring, K steps of 256
//   values with the scale bytes staged beside the codes (see gemm4_lds_kernel).
// * tile (m > 32, other k): 128x128 tiles, 4 waves of 64x64, K steps of 256 (128 bytes per row)
//   double-buffered in LDS through registers with the scale bytes staged beside them.
// K % 64 == 0: a K step reaching past K reads zero codes and unit scales there.
#include "common.h"

AKLR_SCALAR_FP32_BEGIN

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
  int nt_out;   // lds kernel: output stores are non-temporal
  int64_t pc;  // padded scale columns (shuffled layout)
  float* partial;
  uint64_t* counters;  // split-K arrival words, one per output tile (launch-tagged)
  int splits;
  int ks_per_split;  // K steps per split: 128 values (decode), 256 values (lds)
  int pr_a, pr_b;    // padded scale rows (shuffled layout)
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
// skinny (m <= 32): weight streaming. A workgroup owns
// 16 * NT output columns and a K range (split across workgroups when the columns alone leave the chip
// idle); each of its NW waves streams its own contiguous sub-range of 128-value K steps straight from
// HBM into MFMA operand registers through raw buffer loads, a D-deep register ring, steps past the
// range (or lane groups past k) loading zeros through the out-of-range offset. The e8m0 scales ride
// the MFMA: shuffled scales come as the dword of the row's 2 x 2 (K step, 16-row half) bytes, shifted
// to the one needed; row-major ones as single bytes. Waves are summed in LDS in wave order; K splits
// go through fp32 partials and the arrival counters, the last workgroup summing in split order.
template <int MT, int NT>
struct Skinny4Frag {
  u32x4 a[MT];
  u32x4 b[NT];
  uint32_t sa[MT];
  uint32_t sb[NT];
};

__device__ __forceinline__ uint32_t buf_ld4(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_ld1(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}

template <int MT, int NT, int NW, int D, bool PRE, bool SSHUF>
__global__ __launch_bounds__(NW * 64) void gemm4_skinny_kernel(Gemm4Args p) {
  constexpr int T = MT * NT;
  __shared__ f32x4 red[T][64];
  __shared__ unsigned arrive_slot;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT;
  const int split = blockIdx.y;
  const int KS = (p.k + 127) >> 7;
  const int ks_base = split * p.ks_per_split;
  const int ks_len = min(p.ks_per_split, KS - ks_base);
  const int chunk = (ks_len + NW - 1) / NW;
  const int ks_begin = ks_base + min(w * chunk, ks_len);
  const int ks_end = ks_base + min((w + 1) * chunk, ks_len);
  const int64_t kbytes = p.k >> 1, kt32 = kbytes >> 5;
  const int kcols = p.k >> 5;  // scale columns
  const int64_t c8 = p.pc >> 3;
  // split-K: thread 0 arrives for the workgroup; its peek of the arrival word returns first
  uint64_t seen = 0;
  if (p.splits > 1 && w == 0) seen = splitk_peek(p.counters + blockIdx.x);

  rsrc_t brs[NT];
  int64_t bcol[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t c0 = (n0 + nt * 16) < p.n ? n0 + nt * 16 : 0;  // tiles past n read tile 0, never stored
    bcol[nt] = c0 + li;
    if (PRE)
      brs[nt] = make_rsrc(p.b + (c0 >> 4) * kt32 * 512, (uint32_t)(kt32 * 512));
    else
      brs[nt] = make_rsrc(p.b + c0 * p.ldb, (uint32_t)(15 * p.ldb + kbytes));
  }
  const uint32_t b_lane = PRE ? (uint32_t)((g >> 1) * 512 + (g & 1) * 256 + li * 16) : (uint32_t)(li * p.ldb + g * 16);
  const uint32_t b_step = PRE ? 1024u : 64u;
  const rsrc_t ars = make_rsrc(p.a, (uint32_t)((p.m - 1) * p.lda + kbytes));
  uint32_t a_lane[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 16 + li;
    a_lane[mt] = row < p.m ? (uint32_t)(row * p.lda + g * 16) : kOobOffset;
  }
  // scales
  const rsrc_t sars = SSHUF ? make_rsrc(p.sa, (uint32_t)((int64_t)p.pr_a * p.pc))
                            : make_rsrc(p.sa, (uint32_t)((p.m - 1) * p.lds_a + kcols));
  const rsrc_t sbrs = SSHUF ? make_rsrc(p.sb, (uint32_t)((int64_t)p.pr_b * p.pc))
                            : make_rsrc(p.sb, (uint32_t)((p.n - 1) * p.lds_b + kcols));
  uint32_t sa_base[MT], sb_base[NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 16 + li;
    sa_base[mt] = SSHUF ? (uint32_t)(((int64_t)(row >> 5) * c8) * 256 + (g * 16 + (row & 15)) * 4)
                        : (row < p.m ? (uint32_t)(row * p.lds_a + g) : kOobOffset);
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    sb_base[nt] = SSHUF ? (uint32_t)(((bcol[nt] >> 5) * c8) * 256 + (g * 16 + (bcol[nt] & 15)) * 4)
                        : (uint32_t)(bcol[nt] * p.lds_b + g);

  auto load = [&](int ks, Skinny4Frag<MT, NT>& f) {
    const bool on = ks < ks_end && (int64_t)ks * 64 + g * 16 < kbytes;  // this lane group's 32 values exist
    const uint32_t dk = on ? 0u : kOobOffset;
    const uint32_t so = SSHUF ? (uint32_t)(ks >> 1) * 256u : (uint32_t)ks * 4u;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f.b[nt] = buf_ld16<kNt>(brs[nt], on ? b_lane + (uint32_t)ks * b_step : kOobOffset);
      f.sb[nt] = SSHUF ? buf_ld4(sbrs, on ? sb_base[nt] + so : kOobOffset)
                       : buf_ld1(sbrs, on ? sb_base[nt] + so : kOobOffset);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f.a[mt] = buf_ld16(ars, (on && a_lane[mt] != kOobOffset) ? a_lane[mt] + (uint32_t)ks * 64u : kOobOffset);
      f.sa[mt] = SSHUF ? buf_ld4(sars, on ? sa_base[mt] + so : kOobOffset)
                       : buf_ld1(sars, (on && sa_base[mt] != kOobOffset) ? sa_base[mt] + so : kOobOffset);
    }
    (void)dk;
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  Skinny4Frag<MT, NT> f[D];
#pragma unroll
  for (int j = 0; j < D; ++j) load(ks_begin + j, f[j]);
  for (int ks0 = ks_begin; ks0 < ks_end; ks0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int ks = ks0 + j;
      // shuffled scales: byte (K step parity) * 2 + (16-row half) of the dword
      const int kshift = SSHUF ? 16 * (ks & 1) : 0;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int asc = (int)(f[j].sa[mt] >> (kshift + (SSHUF ? 8 * (mt & 1) : 0)));
        const i32x8 af = fp4_frag(f[j].a[mt]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int bsc = (int)(f[j].sb[nt] >> (kshift + (SSHUF ? 8 * (int)((bcol[nt] >> 4) & 1) : 0)));
          acc[mt][nt] = mfma16x128_scaled<kFp4, 0, 0>(af, fp4_frag(f[j].b[nt]), acc[mt][nt], asc, bsc);
        }
      }
      load(ks0 + j + D, f[j]);
      __builtin_amdgcn_sched_barrier(0);  // refill slot j before consuming slot j + 1
    }
  }

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

  const int64_t m4 = round4(p.m);
  const int64_t plane = (int64_t)p.n * m4;
  for (int t = w; t < T; t += NW) {
    const int mt = t / NT, nt = t % NT;
    const int c0 = n0 + nt * 16;
    if (c0 >= p.n) continue;
    const f32x4 sv = red[t][lane];
    const int col = c0 + li;
    const int row0 = mt * 16 + 4 * g;
    if (p.splits > 1) {
      if (row0 < p.m) store_partial4(partial_rsrc(p.partial, split, plane), (int64_t)col * m4 + row0, sv);
      continue;
    }
    const float bv = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (row0 + r < p.m) store_out(p.out, (int64_t)(row0 + r) * p.ldo + col, sv[r] + bv, p.out_dtype);
  }
  if (p.splits == 1) return;
  if (!splitk_arrive(p.counters + blockIdx.x, seen, p.splits, &arrive_slot)) return;
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
// stream (16 < m <= 32): the FP8 stream kernel's design (gemm_a8w8.hip) on e2m1. A workgroup owns
// NW * NT * 16 output columns and a K range of 256-value blocks (128 bytes of codes per row). Its NW
// compute waves stream their NT weight tiles from HBM straight into a D-deep register ring (codes and
// the tiles' e8m0 scales); one loader wave moves each K block of A -- the codes as whole 128-byte rows
// (row r of row tile mt at mt * 2048 + r * 128, its 16-byte chunk c at position c ^ (r & 7), so the
// fragment reads are conflict-free) and the rows' 8 scale bytes, 256 bytes per 32 rows in the
// caller's layout -- into an
// NS-stage LDS ring. One LDS-fenced barrier per block hands a stage over; the MFMA applies both
// scales, so there is no fold. Lane groups past k load zero codes and take scale 1.0, so padding scale
// bytes never reach the MFMA. Row-major scales need 4-byte-aligned rows (stream4_ok).
template <int NT>
struct Stream4Frag {
  u32x4 b[NT][2];
  uint32_t sb[NT];  // shuffled: the tile row's dword (both K steps, both 16-row halves); row-major: 2 bytes
};

template <int MT, int NT, int NW, int D, int NS, bool PRE, bool SSHUF>
__global__ __launch_bounds__((NW + 1) * 64) void gemm4_stream_kernel(Gemm4Args p) {
  static_assert(NS >= 2 && D >= 1 && MT >= 1 && MT <= 8 && 128 % (NT * 16) == 0, "stream shape");
  constexpr int kSGroups = MT >= 2 ? MT / 2 : 1;     // 32-row scale groups per stage
  constexpr int kLoadsA = 2 * MT + kSGroups;         // loader loads per stage
  constexpr int kCols = NW * NT * 16;
  static_assert((NS - 2) * kLoadsA <= 63, "the loader's wait count must fit vmcnt");
  __shared__ __attribute__((aligned(1024))) uint8_t sA[NS][MT * 2048];
  __shared__ __attribute__((aligned(16))) uint8_t sS[NS][kSGroups * 256];
  __shared__ unsigned arrive_slot;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * kCols;
  const int split = blockIdx.y;
  const int KB = (p.k + 255) >> 8;  // 256-value blocks
  const int kb_begin = split * p.ks_per_split;
  const int kb_end = min(KB, kb_begin + p.ks_per_split);
  const int64_t kbytes = p.k >> 1, kt32 = kbytes >> 5;
  const int kcols = p.k >> 5;  // scale columns
  const int64_t c8 = p.pc >> 3;

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int c0w = n0 + w * NT * 16;
  const int col_w = c0w + 4 * g;
  const int64_t plane = (int64_t)gridDim.x * NW * MT * NT * 256;  // split-K partials, accumulator order
  const int64_t part_base = ((int64_t)blockIdx.x * NW + w) * (MT * NT) * 256 + lane * 4;
  // the loader's lane 0 arrives for the workgroup (split-K); its peek of the arrival word goes out
  // before the stage loads, so it returns first
  constexpr unsigned kArriver = NW * 64;
  uint64_t seen = 0;

  if (w == NW) {
    // Loader. Rows past m and byte granules past k read the out-of-range offset (zeros).
    if (p.splits > 1) seen = splitk_peek(p.counters + blockIdx.x);
    const i32x4 ars = make_rsrc_words(p.a, rsrc_bytes((int64_t)(p.m - 1) * p.lda + kbytes));
    const i32x4 sars = SSHUF ? make_rsrc_words(p.sa, rsrc_bytes((int64_t)p.pr_a * p.pc))
                             : make_rsrc_words(p.sa, rsrc_bytes((int64_t)(p.m - 1) * p.lds_a + kcols));
    // Load h of row tile mt moves rows mt * 16 + 8h .. + 7 as whole 128-byte lines: lane l takes chunk
    // cl = (l % 8) ^ (l / 8) of row 8h + l / 8 into position l % 8 of that row (chunks XOR-swizzled by row).
    const int cl = (lane & 7) ^ (lane >> 3);
    uint32_t a_off[MT][2], s_off[kSGroups];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = mt * 16 + 8 * h + (lane >> 3);
        a_off[mt][h] = row < p.m ? (uint32_t)((int64_t)row * p.lda + cl * 16) : kOobOffset;
      }
#pragma unroll
    for (int r = 0; r < kSGroups; ++r) {
      if (SSHUF) {
        s_off[r] = (uint32_t)((int64_t)r * c8 * 256 + lane * 4);
      } else {
        const int row = r * 32 + (lane >> 1);
        s_off[r] = row < p.m ? (uint32_t)((int64_t)row * p.lds_a + (lane & 1) * 4) : kOobOffset;
      }
    }
    const uint32_t lds_a0 = lds_addr(&sA[0][0]), lds_s0 = lds_addr(&sS[0][0]);
    auto issue = [&](int kb, int st) {
      const bool on = kb < kb_end;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t byte = (int64_t)kb * 128 + cl * 16;  // this lane's granule along the row
          lds_dma16(ars, lds_a0 + st * (MT * 2048) + mt * 2048 + h * 1024,
                    on && byte < kbytes && a_off[mt][h] != kOobOffset ? a_off[mt][h] + (uint32_t)(kb * 128) : kOobOffset);
        }
#pragma unroll
      for (int r = 0; r < kSGroups; ++r)
        lds_dma4(sars, lds_s0 + st * (kSGroups * 256) + r * 256,
                 on && s_off[r] != kOobOffset ? s_off[r] + (uint32_t)kb * (SSHUF ? 256u : 8u) : kOobOffset);
    };
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(kb_begin + s, s);
    int st_fill = NS - 1;
    for (int kb = kb_begin; kb < kb_end; ++kb) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * kLoadsA) : "memory");
      stage_barrier();
      issue(kb + NS - 1, st_fill);
      st_fill = st_fill + 1 == NS ? 0 : st_fill + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    // Compute wave. Column tiles past n read tile 0 (never stored).
    rsrc_t brs[NT];
    int bcol[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int64_t c0 = (c0w + nt * 16) < p.n ? c0w + nt * 16 : 0;
      bcol[nt] = (int)c0 + li;
      if (PRE)
        brs[nt] = make_rsrc(p.b + (c0 >> 4) * kt32 * 512, (uint32_t)(kt32 * 512));
      else
        brs[nt] = make_rsrc(p.b + c0 * p.ldb, (uint32_t)(15 * p.ldb + kbytes));
    }
    const uint32_t b_lane = PRE ? (uint32_t)((g >> 1) * 512 + (g & 1) * 256 + li * 16) : (uint32_t)(li * p.ldb + g * 16);
    const rsrc_t sbrs = SSHUF ? make_rsrc(p.sb, (uint32_t)((int64_t)p.pr_b * p.pc))
                              : make_rsrc(p.sb, (uint32_t)((int64_t)(p.n - 1) * p.lds_b + kcols));
    uint32_t sb_base[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      sb_base[nt] = SSHUF ? (uint32_t)((((int64_t)bcol[nt] >> 5) * c8) * 256 + (g * 16 + (bcol[nt] & 15)) * 4)
                          : (uint32_t)((int64_t)bcol[nt] * p.lds_b + g);
    auto load = [&](int kb, Stream4Frag<NT>& f) {
      const bool on = kb < kb_end;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool gr = on && (int64_t)kb * 128 + 64 * h + g * 16 < kbytes;
        const uint32_t off = gr ? (uint32_t)(PRE ? kb * 2048 + 1024 * h : kb * 128 + 64 * h) : kOobOffset;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) f.b[nt][h] = buf_ld16<kNt>(brs[nt], off == kOobOffset ? kOobOffset : b_lane + off);
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if (SSHUF) {
          f.sb[nt] = buf_ld4(sbrs, on ? sb_base[nt] + (uint32_t)kb * 256u : kOobOffset);
        } else {
          const uint32_t o = on ? sb_base[nt] + (uint32_t)kb * 8u : kOobOffset;
          f.sb[nt] = buf_ld1(sbrs, o) | (buf_ld1(sbrs, on ? o + 4 : kOobOffset) << 8);
        }
      }
    };
    // The scale byte of K step h of this block for lane group g; 127 (1.0) past k.
    auto pick_b = [&](const Stream4Frag<NT>& f, int nt, int h, bool valid) {
      const uint32_t v = SSHUF ? f.sb[nt] >> (16 * h + 8 * ((bcol[nt] >> 4) & 1)) : f.sb[nt] >> (8 * h);
      return valid ? (int)(v & 0xFF) : 127;
    };

    int st = 0;
    auto step = [&](int kb, Stream4Frag<NT>& f) {
      stage_barrier();
      const uint8_t* A = sA[st];
      const uint8_t* S = sS[st];
      i32x8 af[MT][2];
      uint32_t sw[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int h = 0; h < 2; ++h)  // K step h: chunk 4h + g of row li
          af[mt][h] = fp4_frag(*reinterpret_cast<const u32x4*>(A + mt * 2048 + li * 128 + (((4 * h + g) ^ (li & 7)) << 4)));
        const int row = mt * 16 + li;
        if (SSHUF) {
          sw[mt] = *reinterpret_cast<const uint32_t*>(S + (row >> 5) * 256 + (g * 16 + (row & 15)) * 4);
        } else {
          const uint8_t* rs = S + (row >> 5) * 256 + (row & 31) * 8 + g;
          sw[mt] = (uint32_t)rs[0] | ((uint32_t)rs[4] << 8);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool valid = (kb * 2 + h) * 4 + g < kcols;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint32_t v = SSHUF ? sw[mt] >> (16 * h + 8 * (mt & 1)) : sw[mt] >> (8 * h);
          const int asc = valid ? (int)(v & 0xFF) : 127;
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = mfma16x128_scaled<kFp4, 0, 0>(fp4_frag(f.b[nt][h]), af[mt][h], acc[mt][nt],
                                                          pick_b(f, nt, h, valid), asc);
        }
      }
      load(kb + D, f);
      __builtin_amdgcn_sched_barrier(0);  // refill this slot before consuming the next
      st = st + 1 == NS ? 0 : st + 1;
    };

    Stream4Frag<NT> f[D];
#pragma unroll
    for (int j = 0; j < D; ++j) load(kb_begin + j, f[j]);
    const int len = kb_end - kb_begin, full = len / D * D;
    for (int kb0 = kb_begin; kb0 < kb_begin + full; kb0 += D) {
#pragma unroll
      for (int j = 0; j < D; ++j) step(kb0 + j, f[j]);
    }
#pragma unroll
    for (int j = 0; j < D - 1; ++j)
      if (full + j < len) step(kb_begin + full + j, f[j]);
    if (p.splits > 1) {
      const rsrc_t prs = partial_rsrc(p.partial, split, plane);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) store_partial4(prs, part_base + (mt * NT + nt) * 256, acc[mt][nt]);
    }
  }

  if (p.splits > 1) {
    if (!splitk_arrive(p.counters + blockIdx.x, seen, p.splits, &arrive_slot, kArriver)) return;
    if (w == NW) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < p.splits; ++sp) {
      const rsrc_t r = partial_rsrc(p.partial, sp, plane);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] += __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)((part_base + (mt * NT + nt) * 256) * 4), 0, kSc1));
    }
  }
  if (w == NW) return;

  // Output: a lane holds 4 consecutive columns of one row per tile; 8 bytes per tile and row.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int col = col_w + nt * 16;
    if (col >= p.n) continue;
    f32x4 bx = {0.f, 0.f, 0.f, 0.f};
    if (p.bias) {
#pragma unroll
      for (int r = 0; r < 4; ++r) bx[r] = p.bias[col + r];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = mt * 16 + li;
      if (row >= p.m) continue;
      const f32x4 x = acc[mt][nt] + bx;
      const u32x2 v = {pack_out2(x[0], x[1], p.out_dtype), pack_out2(x[2], x[3], p.out_dtype)};
      *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + (int64_t)row * p.ldo + col) = v;
    }
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
// lds (m > 32, k % 256 == 0): the FP8 LDS kernel's design (gemm_a8w8.hip) -- TM x TN tiles of 8
// waves in 2 (m) x 4 (n), an S-stage direct-to-LDS ring with the same count of loads per wave per
// stage, the weight as the first MFMA operand so a lane holds 4 columns of one row -- with K steps
// of 256 values (128 bytes per row, the same XOR-swizzled LDS tiles) feeding two MFMAs each. The
// e8m0 scales ride the MFMA; they are staged per step beside the codes: TM x 8 and TN x 8 bytes.
// In aiter's shuffled scale layout the 8 scale columns of a K step and a 32-row block are one
// contiguous 256-byte chunk, loaded as it is; lane (li, g) then finds its scales for both MFMAs of
// the step and both 16-row halves in the dword at (16g + li) * 4, byte 2 * mfma + half. Row-major
// scales are staged as 8 bytes per row (lane pairs load a row's two dwords).
template <int TM, int TN, int S, bool PRE, bool SSHUF>
__global__ __launch_bounds__(512) void gemm4_lds_kernel(Gemm4Args p) {
  static_assert(TM % 64 == 0 && TN % 128 == 0 && S >= 2, "tile shape");
  constexpr int MT = TM / 32, NT = TN / 64, AI = TM / 64, BI = TN / 64;
  constexpr int kLoads = AI + BI + 2;  // + one A-scale and one B-scale load
  constexpr int kStageA = TM * 128, kStageB = TN * 128, kScaleA = TM * 8, kScaleB = TN * 8;
  __shared__ __attribute__((aligned(1024))) uint8_t sA[S * kStageA];
  __shared__ __attribute__((aligned(1024))) uint8_t sB[S * kStageB];
  __shared__ __attribute__((aligned(16))) uint8_t sSA[S * kScaleA];
  __shared__ __attribute__((aligned(16))) uint8_t sSB[S * kScaleB];
  __shared__ __attribute__((aligned(16))) uint32_t sDummy[8 * 64];
  __shared__ unsigned arrive_slot;

  const int tiles_m = (p.m + TM - 1) / TM, tiles_n = (p.n + TN - 1) / TN;
  const int lid = (int)xcd_remap(blockIdx.x, gridDim.x);
  const int pid = lid / p.splits, split = lid % p.splits;
  constexpr int kGroup = 8;
  const int per_group = kGroup * tiles_n;
  const int first_m = (pid / per_group) * kGroup;
  const int gsize = min(tiles_m - first_m, kGroup);
  const int pm = first_m + (pid % per_group) % gsize;
  const int pn = (pid % per_group) / gsize;
  const int m0 = pm * TM, n0 = pn * TN;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int wm = w >> 2, wn = w & 3;
  const int KS = p.k >> 8;
  const int ks_begin = split * p.ks_per_split;
  const int ks_end = min(KS, ks_begin + p.ks_per_split);
  const int64_t kbytes = p.k >> 1, kt32 = kbytes >> 5;
  // split-K: thread 0 arrives for the workgroup; its peek of the arrival word goes out before the
  // stage loads, so it returns first
  uint64_t seen = 0;
  if (p.splits > 1 && w == 0) seen = splitk_peek(p.counters + pid);

  auto clamp_bytes = [](int64_t b) { return (uint32_t)(b > 0x7FFFFFFFll ? 0x7FFFFFFFll : (b < 0 ? 0 : b)); };
  const i32x4 ars = make_rsrc_words(p.a + (int64_t)m0 * p.lda, clamp_bytes((int64_t)(p.m - 1 - m0) * p.lda + kbytes));
  const int64_t b_base = PRE ? (int64_t)(n0 >> 4) * kt32 * 512 : (int64_t)n0 * p.ldb;
  const int64_t b_total = PRE ? (int64_t)p.n * kbytes : (int64_t)(p.n - 1) * p.ldb + kbytes;
  const i32x4 brs = make_rsrc_words(p.b + b_base, clamp_bytes(b_total - b_base));
  const int lr = lane >> 3, lp = lane & 7;
  const int c = lp ^ lr;
  uint32_t a_off[AI], b_off[BI];
#pragma unroll
  for (int j = 0; j < AI; ++j) {
    const int r = w * (TM / 8) + j * 8 + lr;
    a_off[j] = m0 + r < p.m ? (uint32_t)(r * p.lda + c * 16) : kOobOffset;
  }
#pragma unroll
  for (int j = 0; j < BI; ++j) {
    const int r = w * (TN / 8) + j * 8 + lr;
    if (PRE)
      b_off[j] = n0 + r < p.n ? (uint32_t)((((r >> 4) * kt32 + (c >> 1)) * 512) + (c & 1) * 256 + (r & 15) * 16)
                              : kOobOffset;
    else
      b_off[j] = n0 + r < p.n ? (uint32_t)(r * p.ldb + c * 16) : kOobOffset;
  }
  // scales: wave w < TM/32 (TN/32) moves 32 rows' 8 bytes of the step
  const bool sa_wave = w < TM / 32, sb_wave = w < TN / 32;
  i32x4 sars, sbrs;
  uint32_t sa_off, sb_off, sa_step, sb_step;
  if (SSHUF) {
    const int64_t c8 = (int64_t)(p.pc >> 3);
    sars = make_rsrc_words(p.sa, clamp_bytes((int64_t)p.pr_a * p.pc));
    sbrs = make_rsrc_words(p.sb, clamp_bytes((int64_t)p.pr_b * p.pc));
    sa_off = sa_wave ? (uint32_t)(((int64_t)(m0 / 32 + w) * c8) * 256 + lane * 4) : kOobOffset;
    sb_off = sb_wave ? (uint32_t)(((int64_t)(n0 / 32 + w) * c8) * 256 + lane * 4) : kOobOffset;
    sa_step = sb_step = 256;
  } else {
    sars = make_rsrc_words(p.sa, clamp_bytes((int64_t)(p.m - 1) * p.lds_a + (p.k >> 5)));
    sbrs = make_rsrc_words(p.sb, clamp_bytes((int64_t)(p.n - 1) * p.lds_b + (p.k >> 5)));
    const int ra = m0 + w * 32 + (lane >> 1), rb = n0 + w * 32 + (lane >> 1);
    sa_off = sa_wave && ra < p.m ? (uint32_t)((int64_t)ra * p.lds_a + (lane & 1) * 4) : kOobOffset;
    sb_off = sb_wave && rb < p.n ? (uint32_t)((int64_t)rb * p.lds_b + (lane & 1) * 4) : kOobOffset;
    sa_step = sb_step = 8;
  }
  const uint32_t lds_a = lds_addr(&sA[w * (TM / 8) * 128]), lds_b = lds_addr(&sB[w * (TN / 8) * 128]);
  const uint32_t lds_sa = sa_wave ? lds_addr(&sSA[w * 256]) : lds_addr(&sDummy[w * 64]);
  const uint32_t lds_sb = sb_wave ? lds_addr(&sSB[w * 256]) : lds_addr(&sDummy[w * 64]);
  const uint32_t lds_sa_step = sa_wave ? kScaleA : 0, lds_sb_step = sb_wave ? kScaleB : 0;
  auto issue = [&](int ks, int st) {
    const bool on = ks < ks_end;
    const uint32_t ak = (uint32_t)ks * 128u, bk = PRE ? (uint32_t)ks * 2048u : (uint32_t)ks * 128u;
#pragma unroll
    for (int j = 0; j < AI; ++j) lds_dma16(ars, lds_a + st * kStageA + j * 1024, on ? a_off[j] + ak : kOobOffset);
#pragma unroll
    for (int j = 0; j < BI; ++j) lds_dma16(brs, lds_b + st * kStageB + j * 1024, on ? b_off[j] + bk : kOobOffset);
    lds_dma4(sars, lds_sa + st * lds_sa_step, on && sa_off != kOobOffset ? sa_off + (uint32_t)ks * sa_step : kOobOffset);
    lds_dma4(sbrs, lds_sb + st * lds_sb_step, on && sb_off != kOobOffset ? sb_off + (uint32_t)ks * sb_step : kOobOffset);
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int a_row = (wm * (TM / 2) + li) * 128, b_row = (wn * (TN / 4) + li) * 128;
  // scale word addresses: shuffled -> the row block's chunk, dword (16g + li); row-major -> row * 8
  const int sa_word = SSHUF ? ((wm * (TM / 2)) / 32) * 256 + (16 * g + li) * 4 : (wm * (TM / 2) + li) * 8;
  const int sb_word = SSHUF ? ((wn * (TN / 4)) / 32) * 256 + (16 * g + li) * 4 : (wn * (TN / 4) + li) * 8;
  auto compute = [&](int st) {
    const uint8_t* A = sA + st * kStageA;
    const uint8_t* B = sB + st * kStageB;
    const uint8_t* SA = sSA + st * kScaleA + sa_word;
    const uint8_t* SB = sSB + st * kScaleB + sb_word;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int swz = ((4 * j + g) ^ (li & 7)) << 4;
      i32x8 bf[NT];
      int bsc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        bf[nt] = fp4_frag(*reinterpret_cast<const u32x4*>(B + b_row + swz + nt * 2048));
        if (SSHUF) {
          const uint32_t wd = *reinterpret_cast<const uint32_t*>(SB + (nt >> 1) * 256);
          bsc[nt] = (int)(wd >> (8 * (2 * j + (nt & 1))));
        } else {
          const uint32_t wd = *reinterpret_cast<const uint32_t*>(SB + nt * 128 + 4 * j);
          bsc[nt] = (int)(wd >> (8 * g));
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const i32x8 af = fp4_frag(*reinterpret_cast<const u32x4*>(A + a_row + swz + mt * 2048));
        int asc;
        if (SSHUF) {
          const uint32_t wd = *reinterpret_cast<const uint32_t*>(SA + (mt >> 1) * 256);
          asc = (int)(wd >> (8 * (2 * j + (mt & 1))));
        } else {
          const uint32_t wd = *reinterpret_cast<const uint32_t*>(SA + mt * 128 + 4 * j);
          asc = (int)(wd >> (8 * g));
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] = mfma16x128_scaled<kFp4, 0, 0>(bf[nt], af, acc[mt][nt], bsc[nt], asc);  // lane: row li, cols 4g..
      }
    }
  };

#pragma unroll
  for (int s = 0; s < S - 1; ++s) issue(ks_begin + s, s);
  int st = 0, st_fill = S - 1;
  for (int ks = ks_begin; ks < ks_end; ++ks) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((S - 2) * kLoads) : "memory");
    __syncthreads();
    issue(ks + S - 1, st_fill);
    compute(st);
    st = st + 1 == S ? 0 : st + 1;
    st_fill = st_fill + 1 == S ? 0 : st_fill + 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if (p.splits > 1) {
    // partials in accumulator order, [split][tile][wave][mt][nt][lane] x 4 fp32: the workgroup that
    // reduces them runs the same lanes over the same tiles, so every store and load is 1 KiB of
    // contiguous full lines
    const int64_t plane = (int64_t)tiles_m * tiles_n * TM * TN;
    const int64_t part_base = ((int64_t)pid * 8 + w) * (MT * NT) * 256 + lane * 4;
    const rsrc_t prs = partial_rsrc(p.partial, split, plane);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) store_partial4(prs, part_base + (mt * NT + nt) * 256, acc[mt][nt]);
    if (!splitk_arrive(p.counters + pid, seen, p.splits, &arrive_slot)) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < p.splits; ++sp) {
      const rsrc_t r = partial_rsrc(p.partial, sp, plane);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] += __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)((part_base + (mt * NT + nt) * 256) * 4), 0, kSc1));
    }
  }

  // Output: whole-line stores through the ring's LDS, rows [0, TM/2) staged in sA and the rest in sB.
  static_assert((TM / 2) * TN * 2 <= S * kStageA && (TM / 2) * TN * 2 <= S * kStageB, "output staging");
  store_tile_via_lds<TM, TN, 2, 4, MT, NT>(acc, sA, sB, wm, wn, m0, n0, p.m, p.n, p.out, p.ldo, p.bias, p.out_dtype,
                                           p.nt_out != 0);
}

// ---------------------------------------------------------------------------------------------
static constexpr int64_t kDecode4MaxM = 32;

// Skinny plan (m <= 32), measured on MI355X over the Llama-70B MXFP4 shapes at m = 1 and 32: one or
// two 16-row tiles, two 16-column tiles and 4 waves per workgroup, 2 K steps in flight per wave
// (best or within 3% of the best of 2-8 in flight, 4 or 8 waves, 1-4 column tiles and 1-4 K splits);
// K is split in two only when the columns give fewer than 512 waves (small n).
struct Skinny4Plan {
  int mt, nt, nw, d, groups, splits, ks_per_split;
};

static Skinny4Plan plan_skinny4(int64_t m, int64_t n, int64_t k) {
  Skinny4Plan p;
  p.mt = m <= 16 ? 1 : 2;
  const int64_t KS = (k + 127) / 128;
  // one column tile per workgroup (twice the workgroups) on long K at one row tile: measured on cold
  // weights at m = 1, 8192 x 28672 (224 K steps), 24.82 -> 22.83 us; on 8192-long K it was within 3% either
  // way (10240 x 8192 11.44 -> 11.12 us, 57344 x 8192 42.84 -> 45.23) and keeps two
  p.nt = (p.mt == 1 && KS >= 128) ? 1 : 2;
  p.groups = (int)((n + 16 * p.nt - 1) / (16 * p.nt));
  p.nw = 4;
  p.d = (p.mt == 1 && KS >= 128) ? 4 : 2;
  int64_t s = ((int64_t)p.groups * p.nw < 512 && KS >= 16) ? 2 : 1;
  if (p.groups > kSplitkMaxTiles) s = 1;
  p.ks_per_split = (int)((KS + s - 1) / s);
  p.splits = (int)((KS + p.ks_per_split - 1) / p.ks_per_split);
  return p;
}

template <int MT, int NT, int D, bool PRE, bool SSHUF>
static void launch_skinny4(const Gemm4Args& g, const Skinny4Plan& p, hipStream_t s) {
  hipLaunchKernelGGL((gemm4_skinny_kernel<MT, NT, 4, D, PRE, SSHUF>), dim3((unsigned)p.groups, (unsigned)p.splits),
                     dim3(256), 0, s, g);
}

template <bool PRE, bool SSHUF>
static void launch_skinny4(const Gemm4Args& g, const Skinny4Plan& p, hipStream_t s) {
  if (p.mt == 1 && p.d == 4) p.nt == 1 ? launch_skinny4<1, 1, 4, PRE, SSHUF>(g, p, s) : launch_skinny4<1, 2, 4, PRE, SSHUF>(g, p, s);
  else if (p.mt == 1) launch_skinny4<1, 2, 2, PRE, SSHUF>(g, p, s);
  else launch_skinny4<2, 2, 2, PRE, SSHUF>(g, p, s);
}

// Stream plan for 16 < m <= 32 (two row tiles; measured on MI355X over the Llama-70B MXFP4 shapes,
// where the stream kernel beats the skinny kernel by 18-20% at m = 32 but not at m = 1, and the LDS
// kernel from m = 64): 4 compute waves of one column tile each (8 A stages), or 8 waves of two once
// n >= 32768 (4 A stages); ring depth 2; K split in 2 or 4 (a power of two) until about 2048 compute
// waves run. Row-major scales need 4-byte-aligned rows (direct-to-LDS loads of whole dwords).
static constexpr int64_t kStream4MinM = 17;

struct Stream4Plan {
  int nt, nw, groups, splits, ks_per_split;
};

static Stream4Plan plan_stream4(int64_t n, int64_t k) {
  Stream4Plan p;
  p.nt = n >= 32768 ? 2 : 1;
  p.nw = p.nt == 2 ? 8 : 4;
  p.groups = (int)((n + 16 * p.nt * p.nw - 1) / (16 * p.nt * p.nw));
  const int64_t KB = (k + 255) / 256;
  int64_t s = 1;
  while (s < 4 && (int64_t)p.groups * p.nw * s * 2 <= 2048 && KB >= 8 * s) s *= 2;
  if (p.groups > kSplitkMaxTiles) s = 1;
  p.ks_per_split = (int)((KB + s - 1) / s);
  p.splits = (int)((KB + p.ks_per_split - 1) / p.ks_per_split);
  return p;
}

static size_t stream4_partial_bytes(const Stream4Plan& p) {
  return (size_t)p.splits * (size_t)p.groups * p.nw * 2 * p.nt * 1024;
}

static bool stream4_ok(int64_t m, int scale_layout, int64_t lds_a, const uint8_t* sa) {
  if (m < kStream4MinM || m > kDecode4MaxM) return false;
  return scale_layout == AKLR_SCALES_SHUFFLED || (lds_a % 4 == 0 && (reinterpret_cast<uintptr_t>(sa) & 3u) == 0);
}

template <bool PRE, bool SSHUF>
static void launch_stream4(const Gemm4Args& g, const Stream4Plan& p, hipStream_t s) {
  const dim3 grid((unsigned)p.groups, (unsigned)p.splits);
  if (p.nt == 2)
    hipLaunchKernelGGL((gemm4_stream_kernel<2, 2, 8, 2, 4, PRE, SSHUF>), grid, dim3(9 * 64), 0, s, g);
  else  // 8 A stages (interleaved medians, m = 32, us: 10240 x 8192 14.29 -> 13.98, 8192 x 28672 26.27 -> 26.17)
    hipLaunchKernelGGL((gemm4_stream_kernel<2, 1, 4, 2, 8, PRE, SSHUF>), grid, dim3(5 * 64), 0, s, g);
}

// LDS-kernel plan for m > 32 when k % 256 == 0 (and, for row-major scales, 4-byte aligned scale rows):
// tile and split count by the FP8 LDS kernel's cost model (per-K-step times per tile shape, rounds of
// 256 workgroups, only 128x128 tiles split K).
struct Lds4Plan {
  int tm, tn, tiles, splits, ks_per_split;
};

static Lds4Plan lds4_plan_for(int64_t m, int64_t n, int64_t k, int tm, int tn) {
  Lds4Plan p;
  p.tm = tm;
  p.tn = tn;
  const int64_t KS = k / 256;
  const int64_t tiles = ((m + tm - 1) / tm) * ((n + tn - 1) / tn);
  p.tiles = (int)tiles;
  int64_t s = tiles >= 256 || tm + tn > 256 ? 1 : 256 / tiles;
  if (s > 4) s = 4;
  if (s > KS / 4) s = KS / 4;
  if (s < 1 || tiles > kSplitkMaxTiles) s = 1;
  p.ks_per_split = (int)((KS + s - 1) / s);
  p.splits = (int)((KS + p.ks_per_split - 1) / p.ks_per_split);
  return p;
}

static Lds4Plan plan_lds4(int64_t m, int64_t n, int64_t k) {
  static const int kShapes[4][2] = {{256, 256}, {256, 128}, {128, 256}, {128, 128}};
  Lds4Plan best{};
  double best_t = 1e30;
  for (const auto& sh : kShapes) {
    if (sh[0] > 128 && m <= 128) continue;
    const Lds4Plan p = lds4_plan_for(m, n, k, sh[0], sh[1]);
    const double step = p.tm + p.tn == 512 ? 1.96 : (p.tm + p.tn == 384 ? 1.15 : 0.70);
    const int64_t wgs = (int64_t)p.tiles * p.splits;
    double t = (double)((wgs + 255) / 256) * (p.ks_per_split * step + 3.0);
    if (p.splits > 1) t += 3.0 + (double)p.splits * p.tm * p.tn * 4 / 100e3;
    if (t < best_t) {
      best = p;
      best_t = t;
    }
  }
  return best;
}

static bool lds4_ok(int64_t m, int64_t k, int scale_layout, int64_t lds_a, int64_t lds_b, const uint8_t* sa,
                    const uint8_t* sb) {
  if (m <= kDecode4MaxM || k % 256 != 0) return false;
  if (scale_layout == AKLR_SCALES_ROW_MAJOR &&
      (lds_a % 4 || lds_b % 4 || (reinterpret_cast<uintptr_t>(sa) & 3u) || (reinterpret_cast<uintptr_t>(sb) & 3u)))
    return false;
  return true;
}

template <int TM, int TN, bool PRE, bool SSHUF>
static void launch_lds4_t(const Gemm4Args& g, const Lds4Plan& p, hipStream_t s) {
  constexpr int S = TM + TN == 512 ? 2 : (TM + TN == 384 ? 3 : 4);
  hipLaunchKernelGGL((gemm4_lds_kernel<TM, TN, S, PRE, SSHUF>), dim3((unsigned)(p.tiles * p.splits)), dim3(512), 0, s, g);
}

template <bool PRE, bool SSHUF>
static void launch_lds4(const Gemm4Args& g, const Lds4Plan& p, hipStream_t s) {
  if (p.tm == 256 && p.tn == 256) launch_lds4_t<256, 256, PRE, SSHUF>(g, p, s);
  else if (p.tm == 256) launch_lds4_t<256, 128, PRE, SSHUF>(g, p, s);
  else if (p.tn == 256) launch_lds4_t<128, 256, PRE, SSHUF>(g, p, s);
  else launch_lds4_t<128, 128, PRE, SSHUF>(g, p, s);
}

}  // namespace aklr

using namespace aklr;

// Workspace: kSplitkCounterBytes of arrival words, then fp32 partials: [splits, n, round4(m)] for
// the skinny kernel, whole workgroup tiles for the LDS kernel. The LDS kernel may be declined at call
// time (row-major scales with unaligned rows); the tile kernel that runs instead does not split K.
static size_t lds4_partial_bytes(const Lds4Plan& p) {
  return (size_t)p.splits * (size_t)p.tiles * p.tm * p.tn * sizeof(float);
}

extern "C" size_t aklr_gemm_a4w4_mxfp4_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k < 64) return 0;
  if (m <= kDecode4MaxM) {  // the stream kernel may be declined at call time: cover the skinny kernel too
    const Skinny4Plan d = plan_skinny4(m, n, k);
    size_t need = d.splits > 1 ? (size_t)d.splits * (size_t)round4(m) * (size_t)n * sizeof(float) : 0;
    if (m >= kStream4MinM) {
      const Stream4Plan sp = plan_stream4(n, k);
      if (sp.splits > 1 && stream4_partial_bytes(sp) > need) need = stream4_partial_bytes(sp);
    }
    return need ? kSplitkCounterBytes + need : 0;
  }
  if (k % 256 != 0) return 0;
  const Lds4Plan lp = plan_lds4(m, n, k);
  return lp.splits > 1 ? kSplitkCounterBytes + lds4_partial_bytes(lp) : 0;
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
  g.nt_out = ldo * 2 != 8192 && ldo * 2 != 16384;
  g.pc = (k / 32 + 7) / 8 * 8;
  g.partial = nullptr;
  g.counters = nullptr;
  g.splits = 1;
  g.ks_per_split = (int)((k + 127) / 128);
  g.pr_a = (int)((m + 255) / 256 * 256);
  g.pr_b = (int)((n + 255) / 256 * 256);

  if (stream4_ok(m, scale_layout, lds_a, a_scale)) {
    const Stream4Plan sp = plan_stream4(n, k);
    g.splits = sp.splits;
    g.ks_per_split = sp.ks_per_split;
    if (sp.splits > 1) {
      const size_t need = kSplitkCounterBytes + stream4_partial_bytes(sp);
      if (!workspace || workspace_bytes < need || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
      g.counters = static_cast<uint64_t*>(workspace);
      g.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kSplitkCounterBytes);
    }
    const bool sshuf = scale_layout == AKLR_SCALES_SHUFFLED;
    if (g.b_pre) sshuf ? launch_stream4<true, true>(g, sp, stream) : launch_stream4<true, false>(g, sp, stream);
    else sshuf ? launch_stream4<false, true>(g, sp, stream) : launch_stream4<false, false>(g, sp, stream);
    AKLR_LAUNCH_CHECK();
    return AKLR_OK;
  }
  if (m <= kDecode4MaxM) {
    const Skinny4Plan d = plan_skinny4(m, n, k);
    g.splits = d.splits;
    g.ks_per_split = d.ks_per_split;
    if (d.splits > 1) {
      const size_t need = kSplitkCounterBytes + (size_t)d.splits * (size_t)round4(m) * (size_t)n * sizeof(float);
      if (!workspace || workspace_bytes < need || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
      g.counters = static_cast<uint64_t*>(workspace);
      g.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kSplitkCounterBytes);
    }
    const bool sshuf = scale_layout == AKLR_SCALES_SHUFFLED;
    if (g.b_pre) sshuf ? launch_skinny4<true, true>(g, d, stream) : launch_skinny4<true, false>(g, d, stream);
    else sshuf ? launch_skinny4<false, true>(g, d, stream) : launch_skinny4<false, false>(g, d, stream);
    AKLR_LAUNCH_CHECK();
    return AKLR_OK;
  }
  if (lds4_ok(m, k, scale_layout, lds_a, lds_b, a_scale, b_scale)) {
    const Lds4Plan lp = plan_lds4(m, n, k);
    g.splits = lp.splits;
    g.ks_per_split = lp.ks_per_split;
    if (lp.splits > 1) {
      const size_t need = kSplitkCounterBytes + lds4_partial_bytes(lp);
      if (!workspace || workspace_bytes < need || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
      g.counters = static_cast<uint64_t*>(workspace);
      g.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kSplitkCounterBytes);
    }
    const bool sshuf = scale_layout == AKLR_SCALES_SHUFFLED;
    if (g.b_pre) sshuf ? launch_lds4<true, true>(g, lp, stream) : launch_lds4<true, false>(g, lp, stream);
    else sshuf ? launch_lds4<false, true>(g, lp, stream) : launch_lds4<false, false>(g, lp, stream);
    AKLR_LAUNCH_CHECK();
    return AKLR_OK;
  }
  const int tiles = (int)(((m + kT4M - 1) / kT4M) * ((n + kT4N - 1) / kT4N));
  hipLaunchKernelGGL(gemm4_tile_kernel, dim3((unsigned)tiles), dim3(256), 0, stream, g);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

AKLR_SCALAR_FP32_END
