// 128x128-block-scaled FP8 GEMM for gfx950: out = (a * a_scale) @ (b * b_scale)^T + bias.
//
// Every kernel runs one V_MFMA_SCALE_F32_16X16X128_F8F6F4 atom (unit e8m0 scales) per 16x16 output
// tile per 128-wide K block, into a zero accumulator, and folds that partial into the fp32 result
// with one FMA per element: acc += partial * (a_scale[row, kb] * b_scale[n/128, kb]). The fp32 block
// scales are not powers of two, so they cannot ride the MFMA's e8m0 scale operands.
//
// * stream (m <= 128): weight streaming with the activations shared through LDS. Each compute wave
//   streams its own weight columns over the workgroup's K range from HBM straight into MFMA operand
//   registers (a register ring, no LDS), and a loader wave fills an LDS ring with each K block of A
//   (whole 128-byte rows, chunks XOR-swizzled by row).
// * lds (m > 128): 256x256, 256x224, 256x192, 192x192, 256x128, 128x256, 128x192 or 128x128 workgroup
//   tiles of 8 waves, K steps of 128
//   through a 2- to 4-stage LDS ring filled by direct-to-LDS loads (16-byte chunks XOR-swizzled by
//   row), a_scale staged in LDS, XCD-aware tile order, 16-byte output stores.
//
// When K is also split across workgroups, each stores an fp32 partial into the caller's workspace
// and the last workgroup of the output tile to arrive (a launch-tagged agent-scope counter, valid
// whatever the workspace held before) sums the partials in split order and writes the output: one
// launch, and every sum has a fixed order, so results are bitwise reproducible.
#include "common.h"

AKLR_SCALAR_FP32_BEGIN

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
  int nt_out;          // lds kernel: output stores are non-temporal
  uint64_t* counters;  // when splits > 1: one arrival word per output tile (launch-tagged)
  float* partial;      // when splits > 1: per 16x16 tile, in accumulator order
  int splits;
  int kb_per_split;
};

// ---------------------------------------------------------------------------------------------
// stream: weight streaming with the activations shared through LDS, for a few row tiles (MT <= 8).
// A workgroup owns NW * NT * 16 output columns and a K range. Its NW compute waves own NT 16-column
// tiles each and stream those weight columns from HBM straight into a D-deep register ring (loads
// past the K range use an out-of-range offset: zeros, no memory access); one more wave, the loader,
// moves each 128-wide K block of A (all MT row tiles) and its a_scale column into an NS-stage LDS ring
// with direct-to-LDS loads, so A crosses L2 once per workgroup instead of once per wave. A row tile
// of a stage is 16 rows of 128 bytes, each row fetched whole by 8 lanes of one load (one cache line a
// row; fragment-order loads took two half lines from two loads), its 16-byte chunks XOR-swizzled by row
// so that the compute waves' ds_read_b128 of their fragments are free of bank conflicts. (Measured in
// single runs on cold weights, us: m = 128 on 2112 x 7168 16.8 -> 15.4 and on 24576 x 1536 14.7 -> 13.8;
// m = 16 on 2112 x 7168 7.96 -> 7.56; outputs bitwise the same.)
// The loader issues only LDS-bound loads and the compute waves only register-bound ones, so both
// sides' wait counts are exact: the loader waits for its own stage with an immediate count, and the
// compiler tracks the weight ring. One barrier per K block, fenced for LDS only, hands a stage from
// the loader to the compute waves and the consumed slot back, without draining the weight ring.
template <int NT>
struct StreamFrag {
  i32x8 b[NT];
};

// Fused activation quantization (QA, one row tile): p.a is then bf16 x [m, lda elements], and the
// compute waves quantize each K block of it per 1 x 128 group with the arithmetic of
// quant_fp8_1x128_kernel (amax floored at 1e-10, s = amax * fl(1/448), codes e4m3(clamp(x * (1/s)))),
// writing the codes in fragment order and s into the stage: the LDS stage holds exactly the bytes the
// loader would have moved from per_group_quant_fp8's output. Compute wave w quantizes rows
// [4w, 4w + 4) of the 16: 16 lanes per row, 8 values (one 16-byte load) per lane. (The index
// arithmetic is written for MT row tiles, 16 / MT lanes per row; only MT = 1 is instantiated, being
// the only row count at which the fused kernel beats the two launches.)
template <int MT>
struct XStage {
  u32x4 v[MT];
};

// KW > 1 splits the workgroup's K range over its waves instead of its columns: the NW compute waves
// form KW groups of NW / KW, all groups on the same columns, and group kw takes the contiguous K blocks
// [kb_begin + kw * steps, + steps) (steps = the range over KW, rounded up), one per step. A stage then
// holds one K block per group and the groups' partial sums meet in LDS at the end, in group order, so
// a narrow workgroup covers its columns over the whole K range with no split-K partials in memory (the
// plan then runs one K split).
//
// Row blocks: with gridDim.z > 1, workgroup (x, y, z) computes rows [z * MT * 16, + MT * 16) -- its A
// rows, their a_scale and its output rows start there -- and its split-K arrival word and partials are
// those of tile z * gridDim.x + x. (Not with fused quantization.) With K splits, or where gridDim.x *
// gridDim.y is not a multiple of 8, (x, y, z) come from a logical id, z fastest and then y, that keeps the
// row blocks and K splits of a column group consecutive on one XCD, so they read its weight columns
// through one L2: in hardware order the blocks of a column group are gridDim.x * gridDim.y ids apart and,
// unless that is a multiple of 8, on different XCDs (M = 128, 2112 x 7168, 33 x 2 x 2 workgroups: 40.1 MB
// fetched past L2 against 16.6 MB of operands). Interleaved A/B, cold weights, us (hardware order ->
// logical): M = 128 on 2112 x 7168 15.21 -> 14.24, on 4096 x 8192 16.38 -> 15.99, M = 100 on 4096 x 8192
// 15.67 -> 15.35. One split where that multiple of 8 already puts a group on one XCD keeps the hardware
// order, which also spreads neighbouring groups over the 8 XCDs: the logical order measured 3-5% slower
// there (M = 128 on 7168 x 2048 7.99 -> 8.32, on 3072 x 1536 6.08 -> 6.39; M = 256 on 8192 x 1024 7.18 ->
// 7.54).
//
// KS (a K-major a_scale, K contiguous per row): a stage's a_scale load takes 16 rows x 4 consecutive K
// blocks (16 cache lines) instead of one K block of 64 rows (64 lines, one a row: as many line lookups
// as the stage's A codes, on the loader's critical path). Groups of 4 K blocks (all rows) then live in
// a 3-slot LDS ring: the 4 stages of group q each carry a quarter of group q + 1 (the first group is
// loaded with stage 0), so a group is whole one stage before its first block is consumed, and its slot
// is refilled 4 stages after its last block was read (NS <= 5 keeps that ordering under the stage
// barriers). The loads per stage stay kSRows / 64, as for a column-major a_scale.
template <int MT, int NT, int NW, int D, int NS, int FMT, bool PRE, bool QA = false, int KW = 1, bool ROT = false,
          bool KS = false>
__global__ __launch_bounds__((NW + 1) * 64) void gemm8_stream_kernel(Gemm8Args p) {
  static_assert(!QA || (MT == 1 && FMT == 0 && NW == 4 && KW == 1), "fused quantization: e4m3, one row tile, 4 waves");
  static_assert(!ROT || (KW == 1 && !QA), "rotated K order: one K group, no fused quantization");
  static_assert(!KS || (!QA && !ROT && NS <= 5), "K-major a_scale ring: no fused quantization or rotated K order");
  static_assert(NS >= 2 && D >= 1 && MT >= 1 && MT <= 8 && 128 % (NT * 16) == 0 && NW % KW == 0, "stream shape");
  constexpr int kSRows = (MT * 16 + 63) / 64 * 64;     // a_scale floats per K block: whole 64-lane loads
  constexpr int kLoadsA = KW * (2 * MT + kSRows / 64);  // loader loads per stage
  constexpr int kWC = NW / KW;                          // waves across the columns
  constexpr int kCols = kWC * NT * 16;
  // 128-column b_scale blocks under the workgroup: its columns start at a multiple of kCols, so a width
  // that neither divides nor is a multiple of 128 (96, 112) can straddle one more block
  constexpr int kNBlk = kCols % 128 == 0 ? kCols / 128 : (128 % kCols == 0 ? 1 : kCols / 128 + 2);
  static_assert((NS - 1) * kLoadsA <= 63, "the loader's wait counts must fit vmcnt");
  __shared__ __attribute__((aligned(1024))) uint8_t sA[NS][KW * MT * 2048];
  __shared__ __attribute__((aligned(16))) float sS[NS][KW * kSRows];
  __shared__ float sSB[kNBlk][512];
  __shared__ float sQSink[QA ? 64 : 1];  // fused quantization: landing place of the unused scale stores
  __shared__ f32x4 sRed[KW > 1 ? (NW - kWC) * MT * NT * 64 : 1];  // KW > 1: the groups' partial sums
  // KS: the a_scale ring, [slot][K group][kSRows][4 K blocks] floats (a fragment's 16 rows 4 floats apart)
  __shared__ __attribute__((aligned(16))) float sS4[KS ? 3 * KW * kSRows * 4 : 1];
  __shared__ unsigned arrive_slot;

  uint32_t bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  if (!QA && gridDim.z > 1 && (gridDim.y > 1 || (gridDim.x * gridDim.y) % 8 != 0)) {
    const uint32_t lid =
        xcd_remap_any(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), gridDim.x * gridDim.y * gridDim.z);
    bz = lid % gridDim.z;
    by = (lid / gridDim.z) % gridDim.y;
    bx = lid / (gridDim.z * gridDim.y);
  }
  if (!QA && bz > 0) {
    const int64_t m0 = (int64_t)bz * MT * 16;
    p.a += m0 * p.lda;
    p.sa += m0 * p.sa_sm;
    p.out = reinterpret_cast<uint16_t*>(p.out) + m0 * p.ldo;  // 16-bit outputs
    p.m -= (int)m0;
  }
  const int tile = (int)(bz * gridDim.x + bx);  // the split-K word and partials' tile
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int n0 = (int)bx * kCols;
  // the loader's lane 0 arrives for the workgroup (split-K): it has no accumulators to keep in registers
  constexpr unsigned kArriver = NW * 64;
  uint64_t seen = 0;
  const int split = (int)by;
  const int KB = p.k >> 7;
  const int kb_begin = split * p.kb_per_split;
  const int kb_end = min(KB, kb_begin + p.kb_per_split);
  const int steps = (kb_end - kb_begin + KW - 1) / KW;  // K steps (of KW blocks each)
  const int kw = w / kWC;                               // compute waves: K group
  // ROT: workgroup x walks its K range from block r0 on, wrapping, so that at any moment the workgroups
  // fetch different A blocks and weight offsets (r0 spreads evenly over the grid).
  const int len_k = kb_end - kb_begin;
  const int r0 = ROT ? (int)((int64_t)bx * len_k / gridDim.x) : 0;
  auto rotk = [&](int kb) {
    if constexpr (!ROT) return kb;
    const int t = kb - kb_begin + r0;
    return kb_begin + (t >= len_k ? t - len_k : t);
  };
  const int64_t kt32 = p.k >> 5;

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int c0w = n0 + (w % kWC) * NT * 16;  // compute wave's first column
  const int col_w = c0w + 4 * g;     // + nt * 16: the lane's first output column
  // split-K partials: one plane per split of gridDim.x * gridDim.z * NW * MT * NT 1 KiB tiles (fp32 elements)
  const int64_t stream_plane = (int64_t)gridDim.x * gridDim.z * NW * MT * NT * 256;
  const int64_t part_base = ((int64_t)tile * NW + w) * (MT * NT) * 256 + lane * 4;

  if (QA && w == NW) {
    // Fused quantization: the compute waves fill the A stages; the loader stages b_scale and keeps
    // the barrier count.
    if (p.splits > 1) seen = splitk_peek(p.counters + tile);
    const int len = kb_end - kb_begin;
    const int last_row = (p.n - 1) >> 7;
    for (int i = lane; i < kNBlk * len; i += 64) {
      const int r = i / len, kk = i - r * len;
      sSB[r][kk] = p.sb[(int64_t)min((n0 >> 7) + r, last_row) * p.ldbs + kb_begin + kk];
    }
    stage_barrier();
    for (int kb = kb_begin; kb < kb_end; ++kb) stage_barrier();
  } else if (w == NW) {
    // Loader. Rows past m read the out-of-range offset: zeros, no memory access. The arrival word's
    // peek goes out first, so it has returned by the first full wait below.
    if (p.splits > 1) seen = splitk_peek(p.counters + tile);
    const i32x4 ars = make_rsrc_words(p.a, rsrc_bytes((int64_t)(p.m - 1) * p.lda + p.k));
    const i32x4 sars =
        make_rsrc_words(p.sa, rsrc_bytes(((int64_t)(p.m - 1) * p.sa_sm + (int64_t)(KB - 1) * p.sa_sk + 1) * 4));
    // Load h of row tile mt moves rows mt * 16 + 8h .. + 7 as whole 128-byte lines: lane l takes chunk
    // (l % 8) ^ (l / 8) of row 8h + l / 8 into position l % 8 of that row (the layout kLineA describes).
    uint32_t a_off[MT][2], s_off[kSRows / 64];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = mt * 16 + 8 * h + (lane >> 3);
        a_off[mt][h] = row < p.m ? (uint32_t)((int64_t)row * p.lda + (((lane & 7) ^ (lane >> 3)) << 4)) : kOobOffset;
      }
#pragma unroll
    for (int i = 0; i < kSRows / 64; ++i) {
      const int row = i * 64 + lane;
      s_off[i] = row < p.m ? (uint32_t)((int64_t)row * p.sa_sm * 4) : kOobOffset;
    }
    const uint32_t lds_a0 = lds_addr(&sA[0][0]), lds_s0 = lds_addr(&sS[0][0]), lds_s4 = lds_addr(&sS4[0]);
    // KS: quarter u (rows 16 u .. + 15) of group q of K group j (step blocks 4 q .. + 3) into its slot
    auto ks_load = [&](int j, int q, int u) {
      const int row = u * 16 + (lane >> 2), tk = 4 * q + (lane & 3), kb = kb_begin + j * steps + tk;
      const bool on = row < p.m && tk < steps && kb < kb_end;
      lds_dma4(sars, lds_s4 + (((q % 3) * KW + j) * kSRows + u * 16) * 16,
               on ? (uint32_t)(((int64_t)row * p.sa_sm + (int64_t)kb * p.sa_sk) * 4) : kOobOffset);
    };
    auto issue = [&](int t, int st) {  // step t: group j's block t, j < KW
#pragma unroll
      for (int j = 0; j < KW; ++j) {
        const int kb0 = kb_begin + j * steps + t;  // group j's blocks are [kb_begin + j steps, + steps)
        const bool on = t < steps && kb0 < kb_end;
        const int kb = on ? rotk(kb0) : kb0;
        const uint32_t ak = (uint32_t)kb * 128u, sk = (uint32_t)kb * (uint32_t)(p.sa_sk * 4);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            lds_dma16(ars, lds_a0 + st * (KW * MT * 2048) + (j * MT + mt) * 2048 + h * 1024,
                      on && a_off[mt][h] != kOobOffset ? a_off[mt][h] + ak : kOobOffset);
        if constexpr (KS) {
#pragma unroll
          for (int i = 0; i < kSRows / 64; ++i) ks_load(j, t / 4 + 1, t % 4 + 4 * i);
        } else {
#pragma unroll
          for (int i = 0; i < kSRows / 64; ++i)
            lds_dma4(sars, lds_s0 + (st * KW + j) * (kSRows * 4) + i * 256,
                     on && s_off[i] != kOobOffset ? s_off[i] + sk : kOobOffset);
        }
      }
    };
    // Stage kb lives in slot (kb - kb_begin) % NS, and all NS slots start filled. A first barrier
    // publishes stage kb_begin; then barrier kb publishes stage kb + 1 (the loader's own loads of it
    // have landed, NS - 2 younger stages stay in flight), and by then every compute wave has read
    // stage kb -- fragments are read one K block ahead -- so its slot takes stage kb + NS. Issues past
    // the K range load zeros, which keeps the count exact.
    issue(0, 0);
    // b_scale of the workgroup's column blocks over its K range (kb_per_split <= 512), staged once by
    // direct-to-LDS loads behind the first A stage and ahead of the others, so stage 0 and b_scale
    // take one round trip together with every stage in flight; the first stage barrier publishes them.
    {
      const int len = kb_end - kb_begin;
      const int last_row = (p.n - 1) >> 7;
      const i32x4 sbrs = make_rsrc_words(p.sb, rsrc_bytes(((int64_t)last_row * p.ldbs + KB) * 4));
      for (int r = 0; r < kNBlk; ++r) {
        const int64_t row0 = (int64_t)min((n0 >> 7) + r, last_row) * p.ldbs + kb_begin;
        for (int j0 = 0; j0 < len; j0 += 64)
          lds_dma4(sbrs, lds_addr(&sSB[r][j0]), j0 + lane < len ? (uint32_t)((row0 + j0 + lane) * 4) : kOobOffset);
      }
    }
    if constexpr (KS) {  // the first a_scale group, whole, with stage 0
#pragma unroll
      for (int j = 0; j < KW; ++j)
#pragma unroll
        for (int u = 0; u < kSRows / 16; ++u) ks_load(j, 0, u);
    }
#pragma unroll
    for (int s = 1; s < NS; ++s) issue(s, s);  // only stage loads from here: the counts are exact
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 1) * kLoadsA) : "memory");  // stage 0 and b_scale
    stage_barrier();
    int st_fill = 0;
    for (int t = 0; t < steps; ++t) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * kLoadsA) : "memory");
      stage_barrier();
      issue(t + NS, st_fill);
      st_fill = st_fill + 1 == NS ? 0 : st_fill + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    // Compute wave. Column tiles past n read tile 0: they feed only outputs that are never stored.
    rsrc_t brs[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int64_t c0 = (c0w + nt * 16) < p.n ? c0w + nt * 16 : 0;
      if (PRE)
        brs[nt] = make_rsrc(p.b + (c0 >> 4) * kt32 * 512, (uint32_t)(kt32 * 512));
      else
        brs[nt] = make_rsrc(p.b + c0 * p.ldb, (uint32_t)(15 * p.ldb + p.k));
    }
    const uint32_t b_lane = PRE ? (uint32_t)((g >> 1) * 512 + (g & 1) * 256 + li * 16)
                                : (uint32_t)(li * p.ldb + g * 16);
    // Step counter kb runs kb_begin, kb_begin + 1, ...; this wave's K block at step kb is kbw(kb).
    auto kbw = [&](int kb) { return KW == 1 ? kb : kb_begin + kw * steps + (kb - kb_begin); };
    auto load = [&](int kb, StreamFrag<NT>& f) {
      const bool on = kbw(kb) < kb_end && (KW == 1 || kb - kb_begin < steps);
      const int kb_w = on ? rotk(kbw(kb)) : 0;
      const uint32_t boff = on ? (uint32_t)(PRE ? kb_w * 2048 : kb_w * 128) : kOobOffset;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        f.b[nt] = cat(buf_ld16<kNt>(brs[nt], b_lane + boff), buf_ld16<kNt>(brs[nt], b_lane + boff + (PRE ? 1024 : 64)));
    };
    const float* sbw = sSB[(c0w >> 7) - (n0 >> 7)];

    // Fused quantization: this wave's rows of each stage (see XStage), from an x register ring that runs
    // beside the weight ring.
    constexpr int kLpr = 16 / MT;  // lanes per row
    const int qrow = w * 4 * MT + lane / kLpr, qp = lane % kLpr;
    const rsrc_t xrs = make_rsrc(p.a, QA ? rsrc_bytes(((int64_t)(p.m - 1) * p.lda + p.k) * 2) : 0u);
    const uint32_t x_off = QA && qrow < p.m ? (uint32_t)(((int64_t)qrow * p.lda + qp * 8 * MT) * 2) : kOobOffset;
    auto xload = [&](int kb, XStage<MT>& xs) {
      const bool on = kb < kb_end && x_off != kOobOffset;
#pragma unroll
      for (int i = 0; i < MT; ++i) xs.v[i] = buf_ld16(xrs, on ? x_off + (uint32_t)kb * 256u + 16u * i : kOobOffset);
    };
    auto qwrite = [&](const XStage<MT>& xs, int slot) {
      float f[8 * MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const uint32_t wv[4] = {xs.v[i].x, xs.v[i].y, xs.v[i].z, xs.v[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f[8 * i + 2 * j] = bf16_lo(wv[j]);
          f[8 * i + 2 * j + 1] = bf16_hi(wv[j]);
        }
      }
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8 * MT; ++i) amax = fmaxf(amax, fabsf(f[i]));
      // a row's lanes are one quad, half row or row of 16 lanes: reduce with DPP moves, not LDS permutes
      amax = fmaxf(amax, dpp_f32<0xB1>(amax));                   // quad_perm [1,0,3,2]
      amax = fmaxf(amax, dpp_f32<0x4E>(amax));                   // quad_perm [2,3,0,1]
      if constexpr (kLpr >= 8) amax = fmaxf(amax, dpp_f32<0x141>(amax));  // row_half_mirror
      if constexpr (kLpr >= 16) amax = fmaxf(amax, dpp_f32<0x140>(amax));  // row_mirror
      amax = fmaxf(amax, kAmaxFloor);
      const float sc = amax * kInv448;  // rounds once to fp32
      const float inv = 1.0f / sc;      // IEEE division, as the quantizer
      uint32_t o[2 * MT];
#pragma unroll
      for (int i = 0; i < 2 * MT; ++i) {
        const float a = fminf(fmaxf(f[4 * i + 0] * inv, -448.0f), 448.0f);
        const float b = fminf(fmaxf(f[4 * i + 1] * inv, -448.0f), 448.0f);
        const float c = fminf(fmaxf(f[4 * i + 2] * inv, -448.0f), 448.0f);
        const float d = fminf(fmaxf(f[4 * i + 3] * inv, -448.0f), 448.0f);
        o[i] = pack4_e4m3(a, b, c, d);
      }
      // byte b0 of the row lands in chunk (row tile, b0 / 64), lane group (b0 % 64) / 16
      const int b0 = qp * 8 * MT;
      uint8_t* dst = &sA[slot][(qrow >> 4) * 2048 + (b0 >> 6) * 1024 + ((((b0 & 63) >> 4) * 16) + (qrow & 15)) * 16 +
                               (b0 & 15)];
      if constexpr (MT == 1) {
        *reinterpret_cast<u32x2*>(dst) = u32x2{o[0], o[1]};
      } else {
        *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
        if constexpr (MT == 4) *reinterpret_cast<u32x4*>(dst + 256) = u32x4{o[4], o[5], o[6], o[7]};
      }
      // one lane per row stores the scale, the others store into sQSink: a branch here would split the
      // step into blocks and let the compiler sink the step's MFMAs past the following barriers
      *(qp == 0 ? &sS[slot][qrow] : &sQSink[lane]) = sc;
    };
    // D-deep ring: block kb_begin + i lives in slot i % D. Its first D blocks go out at once, before
    // the first stage barrier, so the weight stream starts with the kernel rather than one round trip
    // (the loader's first stage) later. The x ring's loads go out just ahead of the weight loads of the
    // same slot, in the order the steps issue them, so that the loop head sees one order of outstanding
    // loads and waits for no more than the slot it consumes.
    StreamFrag<NT> f[D];
    XStage<MT> xr[QA ? D : 1];
    XStage<MT> pro[QA ? NS : 1];
    if constexpr (QA) {
      // every slot starts filled: stages kb_begin .. kb_begin + NS - 1, loaded first
#pragma unroll
      for (int s0 = 0; s0 < NS; ++s0) xload(kb_begin + s0, pro[s0]);
    }
#pragma unroll
    for (int j = 0; j < D; ++j) {
      if constexpr (QA) xload(kb_begin + NS + j, xr[j]);
      load(kb_begin + j, f[j]);
    }
    if constexpr (QA) {
#pragma unroll
      for (int s0 = 0; s0 < NS; ++s0) qwrite(pro[s0], s0);
    }
    int qs = 0;  // QA: slot of stage kb during block kb, which takes stage kb + NS

    // Fragments are read one K block ahead: the MFMAs of block kb run on registers read during block
    // kb - 1, and each row tile's registers take block kb + 1's fragment as soon as its MFMAs have
    // issued, so the LDS latency hides behind the MFMAs instead of stalling them. Then the weight slot
    // is refilled with block kb + D.
    i32x8 af[MT];
    float s[MT];
    // kLineA: a stage's row tile is 16 rows of 128 bytes, chunk c of row r at position c ^ (r & 7) (the
    // loader's whole-line loads); lane (li, g) reads chunks g and 4 + g of row li, conflict-free. The fused
    // quantization writes the fragment order instead: lane l's 32 bytes at l * 16 and 1024 + l * 16.
    constexpr bool kLineA = !QA;
    const int fa_lo = kLineA ? li * 128 + ((g ^ (li & 7)) << 4) : lane * 16;
    const int fa_hi = kLineA ? li * 128 + (((4 + g) ^ (li & 7)) << 4) : 1024 + lane * 16;
    auto read_frags = [&](int mt, int slot, int t) {  // t: the block's step (KS: its a_scale group and place)
      af[mt] = cat(*reinterpret_cast<const u32x4*>(&sA[slot][(kw * MT + mt) * 2048 + fa_lo]),
                   *reinterpret_cast<const u32x4*>(&sA[slot][(kw * MT + mt) * 2048 + fa_hi]));
      if constexpr (KS)
        s[mt] = sS4[((((t >> 2) % 3) * KW + kw) * kSRows + mt * 16 + li) * 4 + (t & 3)];
      else
        s[mt] = sS[slot][kw * kSRows + mt * 16 + li];
    };
    stage_barrier();  // publishes stage kb_begin
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) read_frags(mt, 0, 0);
    int st = 0;  // slot of stage kb + 1 during block kb
    auto step = [&](int kb, StreamFrag<NT>& f, XStage<MT>& xq) {
      stage_barrier();  // publishes stage kb + 1; every wave is done reading stage kb
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (QA) {
        // Stage kb + NS into the slot stage kb leaves. Its x arrived before this block's weights (the x
        // loads of a block are issued ahead of its weight loads), so this work fills the wait for them.
        qwrite(xq, qs);
        xload(kb + NS + D, xq);
        qs = qs + 1 == NS ? 0 : qs + 1;
        __builtin_amdgcn_sched_barrier(0);
      }
      st = st + 1 == NS ? 0 : st + 1;
      // a group's blocks past the K range hold zeros; their b_scale slot was never staged
      const float sb = KW == 1 ? sbw[rotk(kb) - kb_begin] : (kbw(kb) < kb_end ? sbw[kbw(kb) - kb_begin] : 0.0f);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float sc = s[mt] * sb;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          const f32x4 part = mfma16x128<FMT>(f.b[nt], af[mt], z);  // lane: row li, columns 4g..4g+3
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(part[r], sc, acc[mt][nt][r]);
        }
        read_frags(mt, st, kb + 1 - kb_begin);  // block kb + 1 (past the K range: the zeros of an empty stage)
      }
      // Interleave: every MFMA after the first is followed by five VALU slots, which take the scale
      // products and the fold FMAs of earlier MFMAs, so the fold runs while the matrix core works.
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
      for (int i = 1; i < MT * NT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
      }
      load(kb + D, f);
      __builtin_amdgcn_sched_barrier(0);  // refill this slot before consuming the next
    };

    // Whole groups of D blocks run in a loop with no exit inside (its head then has one ring state, and
    // the compiler waits for exactly the slot it consumes); the remaining < D blocks follow, one guarded
    // step each.
    const int len = steps, full = len / D * D;
    for (int kb0 = kb_begin; kb0 < kb_begin + full; kb0 += D) {
#pragma unroll
      for (int j = 0; j < D; ++j) step(kb0 + j, f[j], xr[QA ? j : 0]);
    }
#pragma unroll
    for (int j = 0; j < D - 1; ++j)
      if (full + j < len) step(kb_begin + full + j, f[j], xr[QA ? j : 0]);
  }

  if constexpr (KW > 1) {
    // The K groups' sums meet in LDS and the waves of group 0 add them in group order. Every wave stays
    // until past the split-K arrival's barriers, then only group 0's waves go on.
    if (w < NW && kw > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) sRed[(((w - kWC) * MT + mt) * NT + nt) * 64 + lane] = acc[mt][nt];
    }
    __syncthreads();
    if (w < kWC) {
#pragma unroll
      for (int j = 1; j < KW; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] += sRed[((((j - 1) * kWC + w) * MT + mt) * NT + nt) * 64 + lane];
    }
  }

  if (p.splits > 1) {
    if (w < kWC) {
      // partials in accumulator order, [split][group][wave][tile][lane] x 4 fp32 (the waves of K group 0,
      // which hold the workgroup's sums): the workgroup that reduces them runs the same lanes over the
      // same tiles, so every store and load is 1 KiB of contiguous full lines
      const rsrc_t prs = partial_rsrc(p.partial, split, stream_plane);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) store_partial4(prs, part_base + (mt * NT + nt) * 256, acc[mt][nt]);
    }
    if (!splitk_arrive(p.counters + tile, seen, p.splits, &arrive_slot, kArriver)) return;
    if (w >= kWC) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Each coherent load is a trip to the memory side, so loads go in rounds of up to 32 per lane
    // (the weight ring and fragment registers are free by now): chunks of up to 8 tiles times batches
    // of 4 splits, slots past the last split loading zeros. Per tile the sum runs in split order.
    constexpr int T = MT * NT, kBatch = 4, kChunk = T < 8 ? T : 8;
    for (int sp0 = 0; sp0 < p.splits; sp0 += kBatch) {
      rsrc_t r[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
        r[b] = partial_rsrc(p.partial, sp0 + b < p.splits ? sp0 + b : 0, stream_plane);
#pragma unroll
      for (int t0 = 0; t0 < T; t0 += kChunk) {
        f32x4 v[kChunk][kBatch];
#pragma unroll
        for (int c = 0; c < kChunk; ++c)
#pragma unroll
          for (int b = 0; b < kBatch; ++b)
            v[c][b] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           r[b], sp0 + b < p.splits ? (int)((part_base + (t0 + c) * 256) * 4) : (int)kOobOffset, 0,
                           kSc1));
#pragma unroll
        for (int c = 0; c < kChunk; ++c)
#pragma unroll
          for (int b = 0; b < kBatch; ++b) acc[(t0 + c) / NT][(t0 + c) % NT] += v[c][b];
        __builtin_amdgcn_sched_barrier(0);  // one round at a time
      }
    }
  }
  if (w >= kWC) return;  // the loader, and the K groups past the first

  // Output. Even NT: for each pair of column tiles a lane packs its 4 columns of each into two words
  // and permlane16_swap exchanges the odd lane groups of the first with the even lane groups of the
  // second, so lane group g stores columns 8 * (g / 2) .. + 7 of tile nt + (g & 1) as 16 bytes.
  // NT = 1: each lane stores its 4 columns as 8 bytes.
  if constexpr (NT % 2 == 0) {
    const int col_s = c0w + (g & 1) * 16 + (g >> 1) * 8;  // + nt * 16 (nt even)
#pragma unroll
    for (int nt = 0; nt < NT; nt += 2) {
      f32x4 bx = {0.f, 0.f, 0.f, 0.f}, by = {0.f, 0.f, 0.f, 0.f};
      if (p.bias) {
        const int cx = min(col_w + nt * 16, p.n - 4), cy = min(col_w + nt * 16 + 16, p.n - 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          bx[r] = p.bias[cx + r];
          by[r] = p.bias[cy + r];
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const f32x4 x = acc[mt][nt] + bx, y = acc[mt][nt + 1] + by;
        const uint32_t x0 = pack_out2(x[0], x[1], p.out_dtype), x1 = pack_out2(x[2], x[3], p.out_dtype);
        const uint32_t y0 = pack_out2(y[0], y[1], p.out_dtype), y1 = pack_out2(y[2], y[3], p.out_dtype);
        const auto s0 = __builtin_amdgcn_permlane16_swap(x0, y0, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(x1, y1, false, false);
        const u32x4 v = {s0[0], s1[0], s0[1], s1[1]};
        const int row = mt * 16 + li, col = col_s + nt * 16;
        if (row < p.m && col < p.n)
          *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p.out) + (int64_t)row * p.ldo + col) = v;
      }
    }
  } else {
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
}

// ---------------------------------------------------------------------------------------------
// lds (m > 128; row-major weights from m = 65): TM x TN workgroup tiles (TM = 64 with TN = 64 or 128), 8
// waves in 2 (m) x 4 (n) -- 4 x 2 for TN = 224 -- each wave (TM/WM) x (TN/WN), K steps of 128 through LDS
// rings of SA stages of A (with the step's a_scale column and b_scale row) and SB stages of B, filled by
// direct-to-LDS buffer loads (no register staging): A runs
// SA - 1 stages ahead of the compute and B SB - 1. With SA = SB + 1, A -- the operand whose lines miss
// L2 more often in the XCD tile order below (each A row block serves 4 resident tiles of an XCD, each B
// column block 8) -- gets one stage more latency to hide than B in the same LDS. Every wave issues the
// same number of loads per stage, so one immediate wait count per step leaves exactly the younger stages
// in flight.
// Each LDS operand tile is rows of 128 bytes with the 16-byte chunks XOR-swizzled by row (chunk c of
// row r at position c ^ (r & 7)): lane i of a load writes position i % 8 of row i / 8 of its 8-row
// slab and so fetches chunk (i % 8) ^ (r & 7) of that row; the MFMA fragment reads (row li, chunks
// g and 4 + g, lanes in groups of 8 rows) are then bank-conflict free.
// The MFMA runs with the weight as its first operand, so a lane's accumulator holds 4 consecutive
// output columns of one row: the block-scale fold takes one a_scale per row tile, fp32 partials go
// out as 16-byte stores, and a lane pair (lane, lane +- 16) swaps halves so that every lane stores
// 8 consecutive 16-bit outputs.
// Buffer descriptors start at the workgroup's own tile, so 32-bit offsets cover any matrix size.
constexpr int kLdsGroup = 8;  // tile rows per raster group

// LDS bytes of an A stage (codes, a_scale column, b_scale row) and of a B stage of a TM x TN tile.
__host__ __device__ constexpr int lds8_stage_a(int tm) { return tm * 128 + (tm + 64) * 4; }
__host__ __device__ constexpr int lds8_stage_b(int tn) { return tn * 128; }

// KS (a K-major a_scale, row pitch >= K / 128): the a_scale ring of the stream kernel. An a_scale wave's
// per-stage load takes 16 of its 64 rows x 4 consecutive K blocks (16 cache lines, not 64) into a 3-slot
// LDS ring of 4-block groups; stage t carries quarter t % 4 of group t / 4 + 1, the first group goes out
// before stage 0. A slot is refilled SA stages after the step that read its last block began (SA <= 5),
// and a group is whole when the first stage of its blocks has landed. Rows past m fall outside the
// descriptor (the pitch is at least K / 128) and read zeros.
template <int TM, int TN, int SA, int SB, int FMT, bool PRE, bool KS = false>
__global__ __launch_bounds__(512) void gemm8_lds_kernel(Gemm8Args p) {
  static_assert(TM % 64 == 0 && TM <= 256 && (TN == 64 || TN == 128 || TN == 192 || TN == 224 || TN == 256),
                "tile shape");
  static_assert(SB >= 2 && (SA == SB || SA == SB + 1), "stage counts");
  static_assert(!KS || SA <= 5, "a_scale ring: a slot's refill must follow the reads of its last block");
  constexpr int WN = TN == 224 ? 2 : 4, WM = 8 / WN;  // waves along n and m
  constexpr int MT = TM / (16 * WM), NT = TN / (16 * WN);  // 16x16 tiles per wave along m and n
  // TN = 192 (N = 2112 = 11 x 192) and 224 (N = 7168 = 32 x 224): tiles start at multiples of 64 or
  // 32 columns, so a wave's columns can straddle two 128-column b_scale blocks.
  constexpr bool kBlkPerTile = TN % 128 != 0;
  constexpr int kNBlk = TN == 224 ? 3 : (TN + 127) / 128;  // 128-column b_scale blocks a tile spans
  // B moves in slabs of 8 rows, BI per wave. When the slabs do not divide evenly (TN = 224: 28 slabs),
  // wave w takes slabs w, w + 8, ... and the slots past TN issue an empty load into a shared landing
  // area, so every wave's count stays the same.
  constexpr int kSlabsB = TN / 8;
  constexpr int BI = (kSlabsB + 7) / 8;
  constexpr bool kEvenB = kSlabsB % 8 == 0;
  constexpr int AI = TM / 64;                // 1 KiB A loads per wave per stage
  constexpr int kLoadsA = AI + 1;            // + one scale load (a_scale rows, b_scale row, or empty)
  constexpr int kLoads = kLoadsA + BI;
  constexpr int kStageA = TM * 128, kStageB = lds8_stage_b(TN);
  constexpr int kScaleWaves = TM / 64;       // waves whose scale load carries a_scale rows
  constexpr int kSStride = TM + 64;          // floats per stage: a_scale rows, then b_scale blocks
  // Loads still in flight at a step's wait: the younger stages. With SA = SB + 1 each step issues B of
  // stage kb + SB - 1 and then A of stage kb + SA - 1 = kb + SB, so when step kb needs A(kb) and B(kb),
  // what was issued after B(kb) is A(kb + 1) and the SB - 2 whole steps after that.
  constexpr int kInFlight = SA == SB ? (SB - 2) * kLoads : (SB - 2) * kLoads + kLoadsA;
  // Each MFMA's fold runs kLag MFMAs after it (the last kLag of a step at the start of the next), so
  // its FMAs read a result that is already complete and issue while the matrix core works on later
  // tiles; folding the newest result instead stalls every step on the MFMA latency (measured 8-10%
  // slower on 256x224 tiles, bitwise the same output).
  constexpr int kT = MT * NT;
  constexpr int kLag = kT > 3 ? 3 : kT - 1;  // (64x64 tiles: 2 MFMA tiles a wave)
  static_assert(kT > kLag, "fold lag");
  static_assert(kScaleWaves < 8, "a wave left for the b_scale row");
  __shared__ __attribute__((aligned(1024))) uint8_t sA[SA * kStageA];
  __shared__ __attribute__((aligned(1024))) uint8_t sB[SB * kStageB];
  __shared__ __attribute__((aligned(16))) float sS[SA * kSStride];
  __shared__ __attribute__((aligned(16))) uint8_t sDummy[1024];  // landing area of the empty loads
  __shared__ unsigned arrive_slot;
  __shared__ __attribute__((aligned(16))) float sS4[KS ? 3 * TM * 4 : 1];  // KS: [slot][row][4 K blocks]

  const int tiles_m = (p.m + TM - 1) / TM;
  const int tiles_n = (p.n + TN - 1) / TN;
  // XCD-aware order (the K splits of one tile are consecutive, so they share an XCD and its L2),
  // then groups of kLdsGroup tile rows so neighbouring tiles share A rows and B columns. Workgroup
  // counts that are not a multiple of 8 (the 192x192 tiles on N = 2112) get the same order (cold
  // operands, us, hardware order -> this: 2112 x 7168 at m = 2048 50.3 -> 48.3, m = 4096 74.5 -> 73.5,
  // m = 8192 144.1 -> 139.5).
  const int lid = (int)xcd_remap_any(blockIdx.x, gridDim.x);
  const int pid = lid / p.splits, split = lid % p.splits;
  const int per_group = kLdsGroup * tiles_n;
  const int first_m = (pid / per_group) * kLdsGroup;
  const int gsize = min(tiles_m - first_m, kLdsGroup);
  const int pm = first_m + (pid % per_group) % gsize;
  const int pn = (pid % per_group) / gsize;
  const int m0 = pm * TM, n0 = pn * TN;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int wm = w / WN, wn = w % WN;
  const int KB = p.k >> 7;
  const int kb_begin = split * p.kb_per_split;
  const int kb_end = min(KB, kb_begin + p.kb_per_split);
  const int64_t kt32 = p.k >> 5;
  // split-K: thread 0 arrives for the workgroup; its peek of the arrival word goes out before the
  // stage loads, so it returns first
  uint64_t seen = 0;
  if (p.splits > 1 && w == 0) seen = splitk_peek(p.counters + pid);

  // Wave w moves rows [w*TM/8, (w+1)*TM/8) of the A tile and its BI slabs of the B tile, in slabs of 8
  // rows. Its scale load: waves below kScaleWaves move a_scale rows [64w, 64w + 64); wave kScaleWaves
  // moves the b_scale of the tile's kNBlk column blocks (lane r: block n0 / 128 + r, clamped to the last
  // row of b_scale); the others issue an empty load. Every wave's count per stage is kLoads.
  const i32x4 ars = make_rsrc_words(p.a + (int64_t)m0 * p.lda, rsrc_bytes((int64_t)(p.m - 1 - m0) * p.lda + p.k));
  const int64_t b_base = PRE ? (int64_t)(n0 >> 4) * kt32 * 512 : (int64_t)n0 * p.ldb;
  const int64_t b_total = PRE ? (int64_t)p.n * p.k : (int64_t)(p.n - 1) * p.ldb + p.k;
  const i32x4 brs = make_rsrc_words(p.b + b_base, rsrc_bytes(b_total - b_base));
  const int last_row = (p.n - 1) >> 7;
  const bool a_scale_wave = w < kScaleWaves, b_scale_wave = w == kScaleWaves;
  const i32x4 srs =
      a_scale_wave ? make_rsrc_words(p.sa + (int64_t)m0 * p.sa_sm,
                                     rsrc_bytes(((int64_t)(p.m - 1 - m0) * p.sa_sm + (int64_t)(KB - 1) * p.sa_sk + 1) * 4))
                   : make_rsrc_words(p.sb, rsrc_bytes(((int64_t)last_row * p.ldbs + KB) * 4));
  const int lr = lane >> 3, lp = lane & 7;  // row within the slab, LDS chunk position
  const int c = lp ^ lr;                     // every slab starts at a multiple of 8 rows
  uint32_t a_off[AI], b_off[BI], b_lds[BI], b_lds_step[BI];
#pragma unroll
  for (int j = 0; j < AI; ++j) {
    const int r = w * (TM / 8) + j * 8 + lr;
    a_off[j] = m0 + r < p.m ? (uint32_t)(r * p.lda + c * 16) : kOobOffset;
  }
#pragma unroll
  for (int j = 0; j < BI; ++j) {
    const int slab = kEvenB ? w * BI + j : w + 8 * j;  // wave-uniform
    const int r = slab * 8 + lr;
    // the LDS targets go to m0 through an SGPR: readfirstlane makes their uniformity explicit
    b_lds[j] = __builtin_amdgcn_readfirstlane(slab < kSlabsB ? lds_addr(&sB[slab * 1024]) : lds_addr(sDummy));
    b_lds_step[j] = slab < kSlabsB ? kStageB : 0;
    if (slab >= kSlabsB)
      b_off[j] = kOobOffset;
    else if (PRE)
      b_off[j] = n0 + r < p.n ? (uint32_t)((((r >> 4) * kt32 + (c >> 1)) * 512) + (c & 1) * 256 + (r & 15) * 16)
                              : kOobOffset;
    else
      b_off[j] = n0 + r < p.n ? (uint32_t)(r * p.ldb + c * 16) : kOobOffset;
  }
  uint32_t s_off = kOobOffset, s_kstep = 0, lds_s = lds_addr(sDummy), lds_s_step = 0;
  if (KS && a_scale_wave) {
    s_off = (uint32_t)(((w * 64 + (lane >> 2)) * p.sa_sm + (lane & 3)) * 4);  // quarter 0 of group 0
    lds_s = lds_addr(&sS4[w * 64 * 4]);
  } else if (a_scale_wave) {
    if (m0 + w * 64 + lane < p.m) s_off = (uint32_t)((w * 64 + lane) * p.sa_sm * 4);
    s_kstep = (uint32_t)(p.sa_sk * 4);
    lds_s = lds_addr(&sS[w * 64]);
    lds_s_step = kSStride * 4;
  } else if (b_scale_wave) {
    if (lane < kNBlk) s_off = (uint32_t)((int64_t)min((n0 >> 7) + lane, last_row) * p.ldbs * 4);
    s_kstep = 4;
    lds_s = lds_addr(&sS[TM]);
    lds_s_step = kSStride * 4;
  }
  lds_s = __builtin_amdgcn_readfirstlane(lds_s);
  lds_s_step = __builtin_amdgcn_readfirstlane(lds_s_step);
  const uint32_t lds_a = lds_addr(&sA[w * (TM / 8) * 128]);
  // The lane offsets stay fixed; a stage's K offset rides soffset, so an issue is scalar work only.
  // A stage past the K range loads through a descriptor of no bytes: zeros, no memory traffic, and
  // the same load count.
  // KS: quarter u (rows 16 u .. + 15 of this wave's 64) of group q into slot q % 3. The whole offset rides
  // voffset (the descriptor's range check does not cover soffset): blocks past the K range read zeros.
  auto ks_load = [&](const i32x4& r, int q, int u) {
    const bool in = 4 * q + (lane & 3) < kb_end - kb_begin;
    lds_dma4_so(r, lds_s + ((q % 3) * TM + 16 * u) * 16,
                in ? s_off + (uint32_t)((16 * u * p.sa_sm + kb_begin + 4 * q) * 4) : kOobOffset, 0u);
  };
  auto issue_a = [&](int kb, int st) {
    const bool on = kb < kb_end;
    i32x4 ra = ars, rs = srs;
    ra[2] = on ? ars[2] : 0;
    rs[2] = on ? srs[2] : 0;
#pragma unroll
    for (int j = 0; j < AI; ++j) lds_dma16_so(ra, lds_a + st * kStageA + j * 1024, a_off[j], (uint32_t)kb * 128u);
    if (KS && a_scale_wave) {
      const int t = kb - kb_begin, q = t / 4 + 1, u = t % 4;  // quarter u of group q
      ks_load(rs, q, u);
    } else {
      lds_dma4_so(rs, lds_s + st * lds_s_step, s_off, (uint32_t)kb * s_kstep);
    }
  };
  auto issue_b = [&](int kb, int st) {
    const bool on = kb < kb_end;
    i32x4 rb = brs;
    rb[2] = on ? brs[2] : 0;
    const uint32_t bk = PRE ? (uint32_t)kb * 2048u : (uint32_t)kb * 128u;
#pragma unroll
    for (int j = 0; j < BI; ++j) lds_dma16_so(rb, b_lds[j] + st * b_lds_step[j], b_off[j], bk);
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // A wave's columns (at most 112) lie in at most two 128-column blocks: block blk0 and, from column
  // tile split_nt on, blk0 + 1. The K loop is instantiated per split_nt, so a step computes 2 * MT
  // scale products (a_scale x each block's b_scale) instead of one per MFMA.
  const int wcol = n0 + wn * (TN / WN);
  const int blk0 = (wcol >> 7) - (n0 >> 7);
  const int split_nt = min(NT, (128 - (wcol & 127)) >> 4);
  const int sb_lo_i = TM + blk0, sb_hi_i = TM + min(blk0 + 1, kNBlk - 1);

  // Fragment addresses: every row a lane reads is congruent to li mod 8, so the swizzle term is the
  // same for all its row tiles and each read is one base plus an immediate (stage and tile offsets).
  const int swz_lo = (g ^ (li & 7)) << 4, swz_hi = ((4 + g) ^ (li & 7)) << 4;
  const int a_row = (wm * (TM / WM) + li) * 128, b_row = (wn * (TN / WN) + li) * 128;
  const int s_row = wm * (TM / WM) + li;
  // A step holds the smaller set of fragments (A's MT or B's NT) in registers for all its MFMAs and
  // streams the other, one tile ahead; tile t is (mt, nt) with the streamed index outer.
  constexpr bool kHoldA = MT <= NT;
  constexpr int kHeld = kHoldA ? MT : NT, kStreamed = kHoldA ? NT : MT;
  auto tmt = [](int t) { return kHoldA ? t % MT : t / NT; };
  auto tnt = [](int t) { return kHoldA ? t / MT : t % NT; };
  f32x4 pend[kLag];  // the previous step's last kLag partials and their scales
  float pend_s[kLag];
#pragma unroll
  for (int j = 0; j < kLag; ++j) {
    pend[j] = f32x4{0.f, 0.f, 0.f, 0.f};  // folds of zero into the zero accumulators
    pend_s[j] = 0.f;
  }

  auto kloop = [&](auto split_c) {
    constexpr int SPLIT = decltype(split_c)::value;  // first column tile in block blk0 + 1 (NT: none)
    auto compute = [&](auto sa_c, auto sb_c, int kb) {
      constexpr int STA = decltype(sa_c)::value, STB = decltype(sb_c)::value;
      const uint8_t* A = sA + STA * kStageA;
      const uint8_t* B = sB + STB * kStageB;
      const float* SS = sS + STA * kSStride;
      const int t4 = kb - kb_begin;  // KS: the block's group t4 / 4 and place t4 % 4
      const float* SA_ = KS ? sS4 + ((t4 >> 2) % 3) * TM * 4 + s_row * 4 + (t4 & 3) : SS + s_row;
      auto read_a = [&](int mt) {
        return cat(*reinterpret_cast<const u32x4*>(A + a_row + swz_lo + mt * 2048),
                   *reinterpret_cast<const u32x4*>(A + a_row + swz_hi + mt * 2048));
      };
      auto read_b = [&](int nt) {
        return cat(*reinterpret_cast<const u32x4*>(B + b_row + swz_lo + nt * 2048),
                   *reinterpret_cast<const u32x4*>(B + b_row + swz_hi + nt * 2048));
      };
      i32x8 held[kHeld];
#pragma unroll
      for (int i = 0; i < kHeld; ++i) held[i] = kHoldA ? read_a(i) : read_b(i);
      const float sb_lo = SS[sb_lo_i];
      const float sb_hi = SPLIT < NT ? SS[sb_hi_i] : 0.f;
      float sc_lo[MT], sc_hi[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float sa_row = SA_[mt * 16 * (KS ? 4 : 1)];
        sc_lo[mt] = sa_row * sb_lo;
        sc_hi[mt] = SPLIT < NT ? sa_row * sb_hi : 0.f;
      }
      i32x8 cur, nxt = kHoldA ? read_b(0) : read_a(0);
      f32x4 part[kT];
      float sc[kT];
#pragma unroll
      for (int t = 0; t < kT; ++t) {
        const int mt = tmt(t), nt = tnt(t);
        const int si = t / kHeld, hi = t % kHeld;
        // The two waves of a SIMD share its matrix core; the older one wins it when both are ready,
        // runs ahead and then waits at the next barrier while the other finishes alone (measured:
        // 38% of the K loop at the barrier against 4%). Priority falling with the step's progress
        // hands the matrix core to the wave that is behind (the older wave's barrier share fell to
        // 30%; 7168 x 16384 at m = 4096: 447 -> 439 us, bitwise the same output).
        if (t == 0) __builtin_amdgcn_s_setprio(3);
        else if (t == kT / 4) __builtin_amdgcn_s_setprio(2);
        else if (t == kT / 2) __builtin_amdgcn_s_setprio(1);
        else if (t == 3 * kT / 4) __builtin_amdgcn_s_setprio(0);
        if (hi == 0) {
          cur = nxt;
          if (si + 1 < kStreamed) nxt = kHoldA ? read_b(si + 1) : read_a(si + 1);
        }
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        // lane: row li, columns 4g..4g+3 (the weight is the first operand)
        part[t] = kHoldA ? mfma16x128<FMT>(cur, held[hi], z) : mfma16x128<FMT>(held[hi], cur, z);
        sc[t] = nt < SPLIT ? sc_lo[mt] : sc_hi[mt];
        // The empty asm makes the fold of tile t - kLag (or the previous step's pending tile) come
        // after MFMA t in the schedule; it emits nothing.
        if (t >= kLag) {
          const int u = t - kLag;
          asm volatile("" : "+v"(part[u]) : "v"(part[t]));
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[tmt(u)][tnt(u)][r] = fmaf(part[u][r], sc[u], acc[tmt(u)][tnt(u)][r]);
        } else {
          const int u = kT - kLag + t;
          asm volatile("" : "+v"(pend[t]) : "v"(part[t]));
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[tmt(u)][tnt(u)][r] = fmaf(pend[t][r], pend_s[t], acc[tmt(u)][tnt(u)][r]);
        }
      }
#pragma unroll
      for (int j = 0; j < kLag; ++j) {
        pend[j] = part[kT - kLag + j];
        pend_s[j] = sc[kT - kLag + j];
      }
    };
    // Stage kb lives in A slot (kb - kb_begin) % SA and B slot (kb - kb_begin) % SB. At each step this
    // wave's loads of the stage about to be computed are waited for (the younger stages stay in
    // flight), then the barrier makes every wave's loads visible and guarantees that no wave still reads
    // the slots the issues refill (those of the stage computed one step earlier). The loop runs whole
    // rounds of SA * SB / gcd steps, so every slot index is a constant.
    auto step = [&](int kb, auto j_c) {
      constexpr int J = decltype(j_c)::value;
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kInFlight) : "memory");
      __syncthreads();
      issue_b(kb + SB - 1, (J + SB - 1) % SB);
      issue_a(kb + SA - 1, (J + SA - 1) % SA);
      compute(IC<J % SA>{}, IC<J % SB>{}, kb);
    };
    constexpr int kRound = SA == SB ? SA : SA * SB;  // SA = SB + 1: coprime
    int kb = kb_begin;
    for (; kb + kRound <= kb_end; kb += kRound) {
      auto ring = [&](auto j) { step(kb + decltype(j)::value, j); };
      SFor<0, kRound>::run(ring);
    }
    auto tail = [&](auto j) {
      if (kb + decltype(j)::value < kb_end) step(kb + decltype(j)::value, j);
    };
    SFor<0, kRound - 1>::run(tail);
  };

  // Prologue, in the steady state's issue order: with SA = SB + 1, A(0) and then (B(j), A(j + 1)) for
  // j < SB - 1; with SA = SB, (B(j), A(j)) for j < SB - 1. KS: the a_scale waves' first group goes first.
  if (KS && a_scale_wave) {
#pragma unroll
    for (int u = 0; u < 4; ++u) ks_load(srs, 0, u);
  }
  if constexpr (SA == SB + 1) issue_a(kb_begin, 0);
#pragma unroll
  for (int j = 0; j < SB - 1; ++j) {
    issue_b(kb_begin + j, j);
    issue_a(kb_begin + j + SA - SB, j + SA - SB);
  }
  if constexpr (!kBlkPerTile) {
    kloop(IC<NT>{});
  } else {
    auto pick = [&](auto v) {
      if (split_nt == decltype(v)::value + 1) kloop(IC<decltype(v)::value + 1>{});
    };
    SFor<0, NT>::run(pick);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int j = 0; j < kLag; ++j) {
    const int u = kT - kLag + j;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[tmt(u)][tnt(u)][r] = fmaf(pend[j][r], pend_s[j], acc[tmt(u)][tnt(u)][r]);
  }

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
    // Sum in split order, with all MT * NT loads of a batch of splits in flight together.
    uint32_t poff[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        poff[mt][nt] = (uint32_t)((part_base + (mt * NT + nt) * 256) * 4);
        acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    // Splits go in batches of up to kBatch whose loads are all issued before any is added (each
    // coherent load costs a trip to the memory side); slots past the last split load zeros.
    // The split tiles are 128x128 (MT * NT = 8: 4 splits in flight, 128 VGPRs of loads), 128x192 and
    // 192x192 (12 and 18: one split at a time; a batch of 2 would hold 96 or 144 more VGPRs beside the
    // accumulators, past the 256 a wave of this 512-thread kernel has).
    constexpr int kBatch = MT * NT <= 8 ? 4 : 1;
    for (int sp0 = 0; sp0 < p.splits; sp0 += kBatch) {
      f32x4 v[kBatch][MT][NT];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const bool on = sp0 + b < p.splits;
        const rsrc_t r = partial_rsrc(p.partial, on ? sp0 + b : 0, plane);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            v[b][mt][nt] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, on ? (int)poff[mt][nt] : (int)kOobOffset, 0, kSc1));
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[mt][nt] += v[b][mt][nt];
    }
  }

  // Output: whole-line stores through the rings' LDS, rows [0, TM/2) staged in sA and the rest in sB.
  static_assert((TM / 2) * TN * 2 <= SA * kStageA && (TM / 2) * TN * 2 <= SB * kStageB, "output staging");
  store_tile_via_lds<TM, TN, WM, WN, MT, NT>(acc, sA, sB, wm, wn, m0, n0, p.m, p.n, p.out, p.ldo, p.bias,
                                             p.out_dtype, p.nt_out != 0);
}

// ---------------------------------------------------------------------------------------------
// host-side planning

// m <= kStreamMaxM streams the weight through the stream kernel (activations shared in LDS); larger m
// runs the LDS kernel, but for the row-block stream plans (plan8_rowblocks), which also take m = 129..256.
static constexpr int64_t kStreamMaxM = 128;

enum class Kernel8 { kStream, kLds };

struct Plan8 {
  Kernel8 kind;
  int mt, nt, nw;    // stream: 16-row and 16-column tiles per wave, compute waves per workgroup
  int kw;            // stream: K groups among the compute waves (1: the waves split the columns)
  int tm, tn;        // lds: workgroup tile
  int grid_x;        // stream: column groups; lds: output tiles
  int splits, kb_per_split;
  bool rot = false;  // stream: the long-K plan (each workgroup walks its K range from its own block)
  int dd = 0;        // stream: weight-ring depth when not the default (4 at 1-2 row tiles, 2 beyond)
  int rt = 1;        // stream: row blocks of mt * 16 rows (grid z)
};

static void finish_splits(Plan8& p, int64_t KB, int64_t s) {
  // one arrival word per output tile must fit the region, and the count field the splits
  if (s < 1 || (int64_t)p.grid_x * p.rt > kSplitkMaxTiles) s = 1;
  if (s > kSplitkMaxSplits) s = kSplitkMaxSplits;
  p.kb_per_split = (int)((KB + s - 1) / s);
  p.splits = (int)((KB + p.kb_per_split - 1) / p.kb_per_split);
}

// LDS plan for a given tile and split count. s = 0 picks it: 128x128, 128x192 and 192x192 tiles split K
// into as many parts as fill one 512-thread workgroup per CU (at most 4, >= 4 K blocks each); the larger
// tiles do not split (measured: their partials, 2-4x larger, cost more than the parallelism gains;
// 192x192 at m = 2048 on 2112 x 7168: 2 splits 48.9 us, none 63.0).
static Plan8 plan8_lds(int64_t m, int64_t n, int64_t k, int tm, int tn, int64_t s = 0) {
  Plan8 p;
  p.kind = Kernel8::kLds;
  p.mt = p.nt = p.nw = 0;
  p.kw = 1;
  p.tm = tm;
  p.tn = tn;
  const int64_t KB = k / 128;
  const int64_t tiles = ((m + tm - 1) / tm) * ((n + tn - 1) / tn);
  p.grid_x = (int)tiles;
  if (s <= 0) {
    s = tiles >= 256 || (tm + tn > 320 && tm != 192) ? 1 : 256 / tiles;
    if (s > 4) s = 4;
    if (s > KB / 4) s = KB / 4;
  }
  finish_splits(p, KB, s);
  return p;
}

// Estimated time (us) of an LDS plan, fitted to MI355X measurements over the DeepSeek-V3 shapes at
// m = 128..8192 (it picks the fastest measured plan, or one within 2% of it, on all of them; and the
// fastest, or within 4%, of sweeps with the 192- and 224-column tiles at m = 1024..8192): per K block
// of one tile (256x256: 1.96, 256x224: 1.76, 256x192: 1.55, 192x192: 1.25, 256x128 and 128x256: 1.15,
// 128x192: 0.90, 128x128: 0.70, 64x128: 0.58, 64x64: 0.35), rounds of 256 workgroups, a fixed 3 us per
// round, and for a K split the partial traffic (s * tile * 4 bytes, stored and then summed by one
// workgroup at ~100 GB/s) plus 3 us. (The 64-row figures are fits to sweeps of 64x64 and 64x128 tiles at
// 1-4 K splits over 13 shapes with m = 256..2048, n = 512..8192 and K = 256..7168.)
// The 192x192 tile serves N = 2112 = 11 x 192, where 22 x 11 = 242 tiles fill the chip at m = 4096 and
// 256-row tiles leave 80 CUs idle (cold operands, us, 256x192 -> 192x192: m = 4096 93.5 -> 72.3,
// m = 8192 158.0 -> 137.8; 128x192 -> 192x192 at m = 2048: 52.5 -> 48.9). On ten other reference and
// DeepSeek-V3 prefill shapes it measured slower than the planned tile or within 2% of it.
static double lds_cost(const Plan8& p, int64_t k) {
  const int area = p.tm * p.tn;
  const double step = area == 65536   ? 1.96
                      : area == 57344 ? 1.76
                      : area == 49152 ? 1.55
                      : area == 36864 ? 1.25
                      : area == 32768 ? 1.15
                      : area == 24576 ? 0.90
                      : area == 16384 ? 0.70
                      : area == 8192  ? 0.58
                                      : 0.35;
  const int64_t wgs = (int64_t)p.grid_x * p.splits;
  const double rounds = (double)((wgs + 255) / 256);
  double t = rounds * (p.kb_per_split * step + 3.0);
  if (p.splits > 1) t += 3.0 + (double)p.splits * p.tm * p.tn * 4 / 100e3;
  (void)k;
  return t;
}

// The cost model picks among the tiles below, each at the split count plan8_lds gives it and unsplit.
// The 64-row tiles win where the output is small (at most 256 64x64 tiles, or 256 64x128 ones): there
// the 128-row tiles, split to fill the chip, lost; their split costs more than the model priced. Cold
// preshuffled operands, us, the earlier pick (128-row tiles) -> this: 256 x 512 x 4096 14.1 -> 8.9 (64x64,
// 4 splits), 512 x 1024 x 4096 15.0 -> 11.3 (64x64, 2), 1024 x 512 x 4096 14.9 -> 11.2, 256 x 4096 x 4096
// 16.9 -> 14.5 (64x64, none), 512 x 2048 x 4096 16.6 -> 14.2, 512 x 4096 x 1024 13.7 -> 9.0 (64x128, none),
// 512 x 4096 x 2048 16.6 -> 13.0, 512 x 4096 x 256 6.7 -> 5.8. On short K (<= 16 K blocks) at m = 129..256
// it gives 64x128 tiles on wide N (7168 x 2048 at m = 256 15.8 -> 13.0 and at m = 192 15.3 -> 12.9 against
// the 128-row tiles it picked before) and unsplit 64x64 ones up to N = 4096 (row-major 3072 x 1536 at
// m = 256 9.9 -> 7.4 and at m = 192 9.0 -> 7.4 against split 64x128 ones). Preshuffled weights take the
// row-block stream plans first where those fit. The DeepSeek-V3 prefill shapes and the reference's other
// recorded shapes keep their tiles.
static Plan8 plan8_lds_best(int64_t m, int64_t n, int64_t k) {
  static const int kShapes[10][2] = {{256, 256}, {256, 224}, {256, 192}, {192, 192}, {256, 128},
                                     {128, 256}, {128, 192}, {128, 128}, {64, 128},  {64, 64}};
  Plan8 best = plan8_lds(m, n, k, 128, 128);
  double best_t = lds_cost(best, k);
  for (const auto& sh : kShapes) {
    if (sh[0] > 128 && m <= 128) continue;  // half of every A tile would be padding
    if ((sh[1] == 192 || sh[1] == 224) && n % sh[1] != 0) continue;  // only where they fit N exactly
    for (const int64_t s : {int64_t{0}, int64_t{1}}) {  // plan8_lds's split count, then none
      const Plan8 p = plan8_lds(m, n, k, sh[0], sh[1], s);
      const double t = lds_cost(p, k);
      if (t < best_t) {
        best = p;
        best_t = t;
      }
    }
  }
  return best;
}

// Stream plan (m <= 128; measured on MI355X over the DeepSeek-V3 shapes at m = 1, 16, 32, 64, 128,
// where it is the fastest or within 4% of the fastest of 1-4 column tiles, 2, 4 or 8 waves, ring
// depths 2-8, 3-8 A stages and 1-8 K splits): 1, 2, 4 or 8 row tiles, 4 compute waves, two 16-column
// tiles per wave once n >= 4096 (one below; one also at m <= 16 while that leaves at most 256
// workgroups of columns: the narrower workgroups then need fewer K splits, so less partial traffic,
// for the same workgroup count), and K split in up to 4 parts until about 256 workgroups run (each
// split >= 4 K blocks).
static Plan8 plan8_stream(int64_t m, int64_t n, int64_t k, bool fill = true) {
  Plan8 p;
  p.kind = Kernel8::kStream;
  p.tm = p.tn = 0;
  const int64_t KB = k / 128;
  p.mt = m <= 16 ? 1 : (m <= 32 ? 2 : (m <= 64 ? 4 : 8));
  p.nt = n >= 4096 && (m > 16 || (n + 63) / 64 > 256) ? 2 : 1;
  // At 4 and 8 row tiles and K <= 64 blocks, one column tile per wave while that leaves <= 256 column
  // groups: twice the workgroups or half the K splits (measured, us, two tiles -> one: 7168 x 2048
  // 11.5 -> 9.4 at m = 64 and 15.7 -> 13.4 at m = 128; 4096 x 8192 16.6 -> 14.2 and 22.0 -> 19.0). Longer
  // K keeps two (7168 x 16384 at m = 128: 38 vs 47 us, the narrower groups re-reading A from L2).
  if (p.mt >= 4 && KB <= 64 && (n + 63) / 64 <= 256) p.nt = 1;
  p.nw = 4;
  p.kw = 1;
  const int64_t groups = (n + 64 * p.nt - 1) / (64 * p.nt);
  p.grid_x = (int)groups;
  int64_t s = 256 / groups;
  if (s > 4) s = 4;
  if (s > KB / 4) s = KB / 4;
  finish_splits(p, KB, s);
  // Where that plan splits K over workgroups and K is short, the waves split K instead: 2 or 4 K
  // groups of one 16-column tile each, the smaller count that still makes >= 200 workgroups, one K
  // split, no partials in memory. Measured at m = 1, 16 and 32 (16-row tiles: 1, 1, 2): N x K =
  // 4096 x 8192 10.9 -> 9.1 us (m = 1), 4096 x 4096 7.4 -> 6.3, 7168 x 2048 6.9 -> 5.6, 8192 x 1024
  // 5.6 -> 4.4 (m = 32: 7.4 -> 5.4). Longer K (7168 x 16384: 128 K blocks) amortizes the split-K
  // epilogue and keeps the split plan; at 2 row tiles the wave split loses beyond 32 K blocks.
  if (p.mt <= 2 && p.splits > 1 && KB <= (p.mt == 1 ? 64 : 32)) {
    for (int kw = 2; kw <= 4; kw *= 2) {
      const int64_t wgs = (n + 64 / kw - 1) / (64 / kw);
      if (wgs >= 200) {
        p.kw = kw;
        p.nt = 1;
        p.grid_x = (int)wgs;
        finish_splits(p, KB, 1);
        break;
      }
    }
  }
  // One row tile on fewer than 240 workgroups leaves CUs idle. Then workgroups of 32, 96 or 112 columns
  // (1, 3 or 7 compute waves) that make 240-264 workgroups with the same K splits take over: two
  // column tiles per wave first, then the count nearest 256. The same splits keep every output's
  // arithmetic that of the 4-wave plan (only the K split changes the order of the sums), so results
  // stay bitwise the same and the fused-quantization kernel, which keeps the 4-wave plan, agrees with
  // the two ops. Measured against the 4-wave plan at m = 1 / 16, us: 2112 x 7168 7.76 -> 7.13 / 8.03 ->
  // 7.84 (32 columns), 2048 x 7168 7.72 -> 6.82 / 7.97 -> 6.95, 24576 x 1536 9.45 -> 8.96 / 9.27 -> 9.18
  // (96 columns). More splits to fill the chip lost where the 4-wave plan splits K over its waves
  // (7168 x 2048..4096: +11-16%) and on short K (1024 x 4096: +12-14%).
  if (fill && p.mt == 1 && p.kw == 1 && (int64_t)p.grid_x * p.splits < 240) {
    struct Cand { int nw, nt; };
    constexpr Cand kCands[] = {{1, 2}, {3, 2}, {7, 1}};
    int64_t best_knt = 2, best_d = 0, best_groups = 0;
    int best_nw = 0, best_nt = 0;
    for (const Cand& c : kCands) {
      const int64_t groups = (n + c.nw * c.nt * 16 - 1) / (c.nw * c.nt * 16), wgs = groups * p.splits;
      if (wgs < 240 || wgs > 264) continue;
      const int64_t knt = c.nt == 2 ? 0 : 1, d = wgs > 256 ? wgs - 256 : 256 - wgs;
      if (knt < best_knt || (knt == best_knt && d < best_d)) {
        best_knt = knt;
        best_d = d;
        best_groups = groups;
        best_nw = c.nw;
        best_nt = c.nt;
      }
    }
    if (best_nw > 0) {
      p.nw = best_nw;
      p.nt = best_nt;
      p.grid_x = (int)best_groups;
      // (one compute wave runs 8 A stages; with the loader's overlapped prologue, measured against the 4-stage
      // kernel before it at m = 1 / 16, us, 2112 x 7168: 7.11 -> 6.90 / 7.92 -> 7.71)
    }
  }
  // Long K at one row tile (>= 96 K blocks, e.g. 7168 x 16384): one K split, 32-column workgroups of
  // two compute waves, an 8-deep weight ring behind an 8-stage A ring, and each workgroup starting its
  // K walk at its own block (r0 = its index x K blocks / workgroups, wrapping), when that makes
  // 192-256 workgroups. No partials, no split-K epilogue; the spread start keeps the workgroups from
  // fetching the same A block at once. Measured on cold weights, 7168 x 16384, m = 1 / 16 (us): the
  // split plan 24.0 / 23.1, this plan 20.8 / 21.9 (21.2 / 22.6 without the rotation; 29.9 / 30.9 with
  // the 4-stage A ring, whose one round trip per 2-3 K blocks then paces the workgroup).
  if (fill && p.mt == 1 && p.kw == 1 && KB >= 96) {
    const int64_t groups = (n + 31) / 32;
    if (groups >= 192 && groups <= 256) {
      p.nw = 2;
      p.nt = 1;
      p.grid_x = (int)groups;
      finish_splits(p, KB, 1);
      p.rot = true;
    }
  }
  // The same at 4 and 8 row tiles, where a workgroup's work is long: 240-256 workgroups (a second
  // workgroup on a CU doubles that CU's time), one column tile per wave, 2, 6 or 7 compute waves, the
  // count nearest 256 and then the most waves. Measured against the 4-wave plan at m = 64 / 128, us:
  // 24576 x 1536 12.64 -> 10.96 / 15.94 -> 15.31 (6 waves), 7168 x 16384 30.02 -> 27.02 / 39.13 -> 38.30
  // (7 waves), 2048 x 7168 11.06 -> 10.45 / 16.14 -> 14.94 (2 waves); 264 workgroups of 2112 x 7168 lost
  // 20-30%.
  if (fill && (p.mt == 4 || p.mt == 8) && p.kw == 1 && (int64_t)p.grid_x * p.splits < 240) {
    constexpr int kWaves[] = {7, 6, 2};
    int best_nw = 0;
    int64_t best_d = 0, best_groups = 0;
    for (const int nw : kWaves) {
      const int64_t groups = (n + nw * 16 - 1) / (nw * 16), wgs = groups * p.splits;
      if (wgs < 240 || wgs > 256) continue;
      if (best_nw == 0 || 256 - wgs < best_d) {
        best_nw = nw;
        best_d = 256 - wgs;
        best_groups = groups;
      }
    }
    if (best_nw > 0) {
      p.nw = best_nw;
      p.nt = 1;
      p.grid_x = (int)best_groups;
    }
  }
  // Short K (<= 16 K blocks) at 4 or 8 row tiles, where 32-column workgroups make 192-256 of them: two
  // compute waves, one K split, a 4-deep weight ring. No partials and no split-K epilogue; each
  // workgroup re-reads A from L2, which costs less here than the partials. Measured on cold weights,
  // 7168 x 2048, medians of interleaved runs (us, the plan above -> this one): m = 128 12.32 -> 10.76,
  // m = 64 9.46 -> 7.57 (the same two waves with a 2-deep ring: 11.60 and 8.62; one split over 16- or
  // 64-column workgroups: 12.11 / 7.88 and 12.01 / 8.62). On longer K (56-128 K blocks) every no-split
  // plan lost by 35-80% (2112 x 7168 and 7168 x 16384 need the split to fill the chip).
  if (fill && (p.mt == 4 || p.mt == 8) && KB <= 16) {
    const int64_t groups = (n + 31) / 32;
    if (groups >= 192 && groups <= 256) {
      p.nw = 2;
      p.nt = 1;
      p.grid_x = (int)groups;
      finish_splits(p, KB, 1);
      p.dd = 4;
      return p;
    }
  }
  // Long K at 7 waves of 4 or 8 row tiles: a deeper weight ring, 4 or 3 blocks (measured on cold weights,
  // 7168 x 16384, medians of interleaved runs, us: m = 64 26.26 -> 25.94, m = 128 33.50 -> 33.26; on
  // K <= 56 blocks the deeper rings were even or slower).
  if (fill && (p.mt == 4 || p.mt == 8) && p.nw == 7 && KB >= 96) p.dd = p.mt == 4 ? 4 : 3;
  return p;
}

// fill = false keeps the one-row-tile plans at 4 compute waves (the fused-quantization kernel's shape).
// Row-block stream plans: 64-row blocks (4 row tiles) over the grid's z, so that a
// workgroup reads 64 rows of A and its own columns of the weight where the 8-row-tile plans read all
// 128 rows of A for 32-112 columns and the LDS tiles split K; 32-row blocks (2 row tiles) at m = 33..64,
// where the 4-row-tile plan reads all 64 rows. At m = 33..128 on K <= 64 blocks with 2
// (K <= 16 blocks) or 4 compute waves, at m = 129..256 on K <= 16 blocks with 4 or 8: the narrowest
// workgroup (32, 64 or 128 columns) that makes at most 256 of them, and K
// split into as many parts as keep them <= 256 with >= 8 K blocks each. A 4-deep weight ring.
// Measured on cold preshuffled weights (us, the plan before -> this one): m = 128: 7168 x 2048
// 10.60 -> 7.98 (4 waves), 4096 x 8192 18.55 -> 16.13 (2 splits), 4096 x 4096 13.67 -> 10.83, 8192 x 1024
// 7.71 -> 5.93, 3072 x 1536 10.95 -> 6.07 (2 waves), 2112 x 7168 16.28 -> 12.25 (3 splits, 198 workgroups;
// 2 splits 14.28), 576 x 7168 10.28 -> 9.71 (7 splits), 1536 x 7168 10.75 -> 10.87 (5 splits);
// m = 96 on 512 x 7168 9.84 -> 9.53 (7 splits), on 7168 x 2048
// 9.95 -> 7.78; m = 256 (the LDS 64x128 tile before): 7168 x 2048 12.92 -> 10.13 (8 waves), 3072 x 1536
// 10.35 -> 6.68, 8192 x 1024 8.96 -> 7.17; m = 192 on 7168 x 2048 12.82 -> 9.88. Row-major weights (each
// 128-byte weight line read by two loads) take only the 2-wave plan (K <= 16 blocks, n <= 4096 at two
// blocks): 3072 x 1536 8.27 -> 5.79 at m = 64 (the 4-row-tile plan before) and 7.73 -> 7.03 at m = 128 (the
// 64x64 LDS tile before). With 4 or 8 waves they lost: at m = 128 on 7168 x 2048 9.34 (64x64 LDS tile)
// -> 11.04, 4096 x 8192 21.55 -> 24.51, at m = 256 on 7168 x 2048 12.00 -> 15.58, at m = 64 on 7168 x 2048
// 8.72 -> 9.24 and on 2112 x 7168 14.36 -> 14.57 (128 x 2112 x 7168 gained, 19.45 -> 17.85, and is left
// to the 8-row-tile plan with the others). At m = 64 (32-row blocks; the 4-row-tile plan before): 3072 x 1536 7.60 -> 4.93 (2 waves; 4
// waves and 2 splits 6.89), 2112 x 7168 11.33 -> 10.24 (3 splits), 4096 x 4096 10.18 -> 9.21 (2 splits; 8
// waves 9.86), 7168 x 2048 7.37 -> 6.79 (8 waves 9.30), 8192 x 1024 5.49 -> 5.07, 4096 x 8192 14.20 ->
// 13.45; m = 48 on 7168 x 2048 7.04 -> 6.64. Longer K at m > 128 (2112 x 7168:
// 19.13 -> 21.45), more than 256 workgroups (24576 x 1536 at m = 64 and 128; 8 waves there: 10.76 ->
// 15.37 at m = 64) and K > 64 blocks (7168 x 16384 at m = 128: 34.0 -> 40.7) keep the other plans.
static bool plan8_rowblocks(int64_t m, int64_t n, int64_t k, bool pre, Plan8& p) {
  const int64_t KB = k / 128;
  if (m <= 32 || m > 1024) return false;
  // m = 257..1024 (preshuffled, 16..32 K blocks): 64-row blocks, the narrowest of 2, 4 and 8 waves that
  // makes <= 256 workgroups, where the LDS tiles run 16-64 row blocks' worth of 128- or 64-row tiles.
  // Measured on cold weights, us (the LDS plan -> this): 1024 x 1536 x 4096 21.06 -> 16.32 (8 waves),
  // 1024 x 2048 x 4096 21.30 -> 16.25, 512 x 4096 x 4096 21.32 -> 16.56, 512 x 2048 x 4096 14.06 -> 11.46
  // (4 waves), 1024 x 1024 x 4096 13.73 -> 11.52, 512 x 1024 x 4096 11.08 -> 10.16 (2 waves), 1024 x 512 x
  // 4096 10.92 -> 10.16, 512 x 512 x 4096 9.09 -> 8.73 (2 splits), 768 x 1536 x 4096 16.86 -> 16.09, 384 x
  // 1536 x 4096 12.76 -> 11.19, 512 x 4096 x 2048 13.02 -> 9.85, 640 x 2048 x 2048 13.98 -> 9.20, 1024 x
  // 1536 x 2048 12.53 -> 9.81. More than 256 workgroups lost (1024 x 2112 x 4096 24.3 -> 30.5, 1024 x 4096
  // x 2048 15.9 -> 17.5, 2048 x 1536 x 4096 26.4 -> 32.1), and K = 8192 gained 4% (512 x 1536 x 8192).
  // Their K splits keep >= 16 K blocks each: 300 x 512 x 2048 on 2 splits 7.01, on one 6.53 (80
  // workgroups); 512 x 512 x 4096 on 2 splits 8.73, on one 9.96 (128); 1024 x 256 x 4096 9.11 and 9.92.
  // (The K-group blocks below come first where they fit, from 8 K blocks: several of these shapes now
  // take them.)
  if (m > 256 && (!pre || KB < 8 || KB > 32)) return false;
  // m = 33..128 on 16..32 K blocks (preshuffled weights): 32-row blocks whose 4 waves split K among
  // themselves (4 groups of one wave, 16 columns, while that makes <= 256 workgroups; else 2 groups of
  // two, 32 columns, from 24 K blocks), no K split across workgroups, so no partials. Measured on cold
  // weights, us (the row-block plan with K splits before -> this): m = 128: 512 x 4096 8.25 -> 6.35,
  // 1024 x 4096 8.76 -> 6.56, 1024 x 2048 7.04 -> 5.23, 2048 x 4096 9.15 -> 7.42 (2 groups); m = 96: 512 x
  // 4096 8.22 -> 6.42, 1536 x 4096 9.01 -> 7.27 (2); m = 64: 512 / 1024 / 1536 x 4096 6.80 / 7.36 / 7.61 ->
  // 6.34 / 6.41 / 6.69, 4096 x 4096 9.19 -> 7.90 (2), 2048 x 2048 5.97 -> 5.21; m = 48: 2048 x 4096 7.65 ->
  // 6.72. Even at 2 groups on <= 16 K blocks (4096 x 2048 at m = 64: 5.64 -> 5.71, 3072 x 1536 4.96 ->
  // 4.89) and slower on 56 K blocks (2112 x 7168 at m = 64: 10.21 -> 11.85 with 2 groups, 1536 x 7168 9.02
  // -> 9.09 with 4), where the K splits make more workgroups. The same up to m = 1024 while the blocks make
  // <= 256 workgroups (small N), against the 64x64 LDS tiles with K splits or the 64-row blocks: 256 x 512
  // x 4096 8.79 -> 6.45 (4 groups), 192 x 512 x 4096 8.46 -> 6.46, 256 x 256 x 4096 8.26 -> 6.36, 256 x 512
  // x 3072 8.18 -> 5.83, 256 x 1024 x 4096 8.96 -> 7.34 (2 groups), 192 x 1024 x 4096 8.79 -> 7.32, 160 x
  // 1024 x 4096 8.74 -> 7.23, 200 x 768 x 4096 8.77 -> 7.13, 512 x 512 x 4096 8.78 -> 7.23; more than 256
  // workgroups lost (256 x 1536 x 4096 11.06 -> 12.82 on 384, 256 x 1024 x 4096 with 4 groups 11.35).
  // Past m = 128 the 2 groups also take 16..23 K blocks (against the 64-row blocks of 2 waves, us: 512 x
  // 512 x 2048 6.64 -> 5.32, 1024 x 256 x 2048 6.61 -> 5.25, 300 x 768 x 2048 6.65 -> 5.29, 384 x 512 x 2048
  // 6.60 -> 5.22, 700 x 256 x 2048 6.53 -> 5.20, 512 x 512 x 2560 7.60 -> 5.82; against the 64-row K-group
  // blocks: 200 x 1024 x 2048 6.89 -> 5.26, 160 x 1536 x 2048 6.95 -> 5.41), and 8..15 K blocks with 2
  // groups only (against the LDS tiles or 64-row blocks, us: 512 x 512 x 1024 6.34 -> 4.31, 1024 x 256 x
  // 1024 6.13 -> 4.31, 256 x 1024 x 1024 5.32 -> 4.28, 256 x 512 x 1024 5.24 -> 4.21 where 4 groups of 2
  // blocks gave 4.46, 300 x 768 x 1536 7.59 -> 4.63); the same 2 groups at m = 65..128 on 8..15 K
  // blocks (against the 4- and 8-row-tile plans: 128 x 512 x 1024 4.91 -> 4.16, 128 x 1024 x 1536 5.91 ->
  // 4.56, 96 x 768 x 1536 5.84 -> 4.56; at m = 64 those stay faster, 64 x 512 x 1024 3.86 against 4.12).
  if (pre && m <= 1024 && KB <= 32 && KB >= (m > 64 ? 8 : 16)) {
    const int64_t rt = (m + 31) / 32;
    for (const int kw : {4, 2}) {
      if (kw == 4 && KB < 16) continue;
      if (kw == 2 && m <= 128 && KB >= 16 && KB < 24) break;
      const int64_t wgs = (n + 64 / kw - 1) / (64 / kw);
      if (wgs * rt > 256) continue;
      p = Plan8{};
      p.kind = Kernel8::kStream;
      p.mt = 2;
      p.nt = 1;
      p.nw = 4;
      p.kw = kw;
      p.rt = (int)rt;
      p.grid_x = (int)wgs;
      finish_splits(p, KB, 1);
      return true;
    }
  }
  // m = 129..1024 on 24..32 K blocks, and m = 129..256 on 16..23 (preshuffled), where the 32-row blocks
  // above make too many workgroups: 64-row blocks whose 4 waves form 2 K groups of 2 (32 columns), while
  // those make <= 256 workgroups. Cold weights, us (the plan before -> this): 256 x 2048 x 4096 11.15 ->
  // 9.98 (LDS 64x64 before), 256 x 1536 x 4096 10.93 -> 9.84, 1024 x 512 x 4096 10.10 -> 9.80 (64-row
  // blocks of 2 waves before), 512 x 1024 x 4096 10.14 -> 9.86, 768 x 512 x 4096 9.99 -> 9.80, 384 x 1024 x
  // 4096 10.05 -> 9.77; 256 x 1536 x 2048 8.42 -> 7.03 (64-row blocks, 2 K splits), 256 x 2048 x 2048 8.59
  // -> 7.11. On 16 K blocks past m = 256 the unsplit 64-row blocks of 2
  // waves are faster (512 x 1024 x 2048 6.84 against 7.14, 1024 x 512 x 2048 6.77 against 7.12), and where
  // the 32-row blocks fit they are (512 x 512 x 4096 7.23 against 9.65).
  // On 12..15 K blocks too, at any m here (512 x 1024 x 1536 7.77 -> 6.44 and 1024 x 512 x 1536 7.53 ->
  // 6.48 against the LDS tiles, 256 x 2048 x 1536 6.52 -> 6.44 against the 64-row blocks), and on 8..11
  // past m = 256 (against the LDS tiles: 512 x 1024 x 1024 6.44 -> 5.79, 1024 x 512 x 1024 6.23 -> 5.77,
  // 768 x 640 x 1024 6.32 -> 6.02; at m = 256 the 64-row blocks of 4 waves stay faster, 256 x 1024 x 1024
  // 5.32 against 5.58, and past 256 workgroups it lost: 600 x 1024 x 1280 6.94 -> 9.70 on 320).
  if (pre && m > 128 && m <= 1024 && KB >= (m > 256 ? 8 : 12) && KB <= 32 && !(m > 256 && KB >= 16 && KB < 24)) {
    const int64_t rt = (m + 63) / 64, wgs = (n + 31) / 32;
    if (wgs * rt <= 256) {
      p = Plan8{};
      p.kind = Kernel8::kStream;
      p.mt = 4;
      p.nt = 1;
      p.nw = 4;
      p.kw = 2;
      p.rt = (int)rt;
      p.grid_x = (int)wgs;
      finish_splits(p, KB, 1);
      return true;
    }
  }
  if (m > 256 && KB < 16) return false;  // the 64-row blocks below: 16..32 K blocks past m = 256
  if (m <= 256 && KB > (m > 128 ? 16 : 64)) return false;
  const int mt = m <= 64 ? 2 : 4;  // 32-row blocks at m = 33..64, 64-row blocks above
  const int64_t rt = (m + mt * 16 - 1) / (mt * 16);
  static const int kWaves[3][3] = {{2, 4, 0}, {4, 8, 0}, {2, 4, 8}};
  for (const int nw : kWaves[m > 256 ? 2 : (m > 128 ? 1 : 0)]) {
    if (nw == 0) break;
    if (nw == 2 && KB > 16 && m <= 256) continue;
    if (!pre && nw != 2) continue;  // row-major weights: the 2-wave plan only
    const int64_t groups = (n + nw * 16 - 1) / (nw * 16);
    if (groups * rt > 256) continue;
    int64_t s = 256 / (groups * rt);
    if (s > KB / (m > 256 ? 16 : 8)) s = KB / (m > 256 ? 16 : 8);  // m > 256: 16 K blocks a split at least
    if (s < 1) s = 1;
    p = Plan8{};
    p.kind = Kernel8::kStream;
    p.mt = mt;
    p.nt = 1;
    p.nw = nw;
    p.kw = 1;
    p.rt = (int)rt;
    p.grid_x = (int)groups;
    p.dd = 4;
    finish_splits(p, KB, s);
    return true;
  }
  return false;
}

// Row-major weights at m = 65..128 on K <= 16 blocks run 64x64 LDS tiles (4 stages; the K split of
// plan8_lds): A and B both through whole-line loads into LDS, where the stream kernel reads each 128-byte
// weight line with two loads. Measured on cold operands (us, the row-block stream plan -> 64x64):
// 7168 x 2048 at m = 128 10.97 -> 9.37 (3, 6 and 8 stages: 10.03, 9.59, 9.84) and at m = 96 10.40 ->
// 8.72. Preshuffled weights lost there (7.96 -> 9.44), and at m = 256 both layouts (row-major 12.05 ->
// 14.00 against the 64x128 tile).
// pre: the weight is preshuffled.
static Plan8 plan8(int64_t m, int64_t n, int64_t k, bool pre, bool fill = true) {
  Plan8 p;
  if (fill && plan8_rowblocks(m, n, k, pre, p)) return p;
  if (!pre && m > 64 && m <= 128 && k <= 16 * 128) return plan8_lds(m, n, k, 64, 64);
  if (m <= kStreamMaxM) return plan8_stream(m, n, k, fill);
  return plan8_lds_best(m, n, k);
}

// The LDS kernel's output stores are non-temporal unless the output's row pitch is 16 KiB, or 8 KiB on
// K > 4 blocks.
// Measured on cold b_shuffled operands (us, cached -> non-temporal stores, both whole lines): 64 KiB
// pitch (n = 32768, k = 1024) 250 -> 190 at m = 4096 and 107 -> 100 at m = 2048; 48 KiB (24576 x 1536)
// 195 -> 176-183; 32 KiB at m = 8192 (k = 1024) 229 -> 181; 14 KiB (7168 x 2048) 70.9 -> 68.8; 6 KiB
// (3072 x 1536, m = 8192) 52.3 -> 49.5. At 16 KiB they lost: 91.7 -> 99.7 (8192 x 8192 x 1024) and
// 48.0 -> 51.3 (4096 x 8192 x 1024); at 8 KiB 48.8 -> 51.9 (8192 x 4096 x 1024). On K <= 4 blocks, where
// the output write is most of the kernel, they won at 8 KiB: 2048 x 4096 x 256 10.5 -> 9.3, x 512 12.7 ->
// 11.6, 1024 x 4096 x 256 / 512 7.4 / 8.7 -> 7.1 / 8.3, 4096 x 4096 x 256 15.0 -> 14.5 (at 16 KiB mixed:
// 4096 x 8192 x 512 35.0 -> 37.7, 1024 x 8192 x 512 12.8 -> 11.8).
static bool lds_nt_out(int64_t ldo_bytes, int64_t k) {
  return ldo_bytes != 16384 && (ldo_bytes != 8192 || k <= 4 * 128);
}

static size_t workspace8(const Plan8& p) {
  if (p.splits <= 1) return 0;
  if (p.kind == Kernel8::kStream)  // whole 16x16 tiles of every wave of every column group
    return kSplitkCounterBytes + (size_t)p.splits * (size_t)p.grid_x * p.rt * p.nw * p.mt * p.nt * 1024;
  // lds: whole workgroup tiles
  return kSplitkCounterBytes + (size_t)p.splits * (size_t)p.grid_x * p.tm * p.tn * sizeof(float);
}
// The workspace a call of either weight layout needs (the workspace queries take no layout).
static size_t workspace8_any(int64_t m, int64_t n, int64_t k) {
  const size_t a = workspace8(plan8(m, n, k, false)), b = workspace8(plan8(m, n, k, true));
  return a > b ? a : b;
}

// Stream kernel: NW compute waves (4 but for the fill and long-K plans) and 4 A stages (8 for the
// one-wave fill plans and the long-K plan); ring depth 4 at 1-2 row tiles, else 2, and 8 for the long-K
// plan, 4 and 3 for 7-wave plans of 4 and 8 row tiles at >= 96 K blocks (measured).
template <int MT, int NT, int FMT, bool PRE, bool QA = false, int KW = 1, int NW = 4, int NS = 4, int DD = 0,
          bool ROT = false, bool KS = false>
static void launch_stream(const Gemm8Args& a, const Plan8& d, hipStream_t s) {
  constexpr int D = DD ? DD : (MT <= 2 ? 4 : 2);
  hipLaunchKernelGGL((gemm8_stream_kernel<MT, NT, NW, D, NS, FMT, PRE, QA, KW, ROT, KS>),
                     dim3((unsigned)d.grid_x, (unsigned)d.splits, (unsigned)d.rt), dim3((NW + 1) * 64), 0, s, a);
}

// A K-major a_scale (the row-major a_scale variant: e4m3, preshuffled weights) on the 64-row-block plans
// of >= 24 K blocks a split takes the ring of a_scale quarters (KS). Cold weights, us (column-major
// a_scale; K-major with per-stage loads -> the ring): 1024 x 1536 x 4096 16.35; 19.05 -> 17.32, 1024 x
// 1024 x 4096 11.40; 12.63 -> 11.95, 512 x 1024 x 4096 10.18; 10.73 -> 10.56, 1024 x 512 x 4096 10.19;
// 10.75 -> 10.58. Not taken: 16 K blocks a split (512 x 512 x 4096 on 2 splits 8.95 -> 9.13), 8 (256 x
// 4096 x 1024 5.77 -> 5.91) and the wave-split 32-row blocks, where the ring measured 2.2-2.4 us slower
// (64 x 512 x 4096 6.66 -> 8.91, 128 x 1024 x 4096 6.91 -> 8.96, 64 x 4096 x 4096 8.31 -> 9.03) and the
// per-stage loads cost 2-5% over a column-major a_scale.
template <int FMT, bool PRE>
static void dispatch_stream(const Gemm8Args& a, const Plan8& d, hipStream_t s) {
  if constexpr (FMT == 0 && PRE) {
    if (a.sa_sk == 1 && a.sa_sm > 1 && !d.rot && d.kb_per_split >= 24) {
      if (d.kw == 1 && d.mt == 4 && d.dd && (d.nw == 4 || d.nw == 8)) {  // (2 waves: the K-group plan first)
        d.nw == 4 ? launch_stream<4, 1, 0, true, false, 1, 4, 4, 4, false, true>(a, d, s)
                  : launch_stream<4, 1, 0, true, false, 1, 8, 4, 4, false, true>(a, d, s);
        return;
      }
    }
  }
  if (d.kw > 1) {  // one column tile per wave, 1, 2 or 4 row tiles (4: 2 K groups only)
    if (d.mt == 1) d.kw == 2 ? launch_stream<1, 1, FMT, PRE, false, 2>(a, d, s) : launch_stream<1, 1, FMT, PRE, false, 4>(a, d, s);
    else if (d.mt == 4) launch_stream<4, 1, FMT, PRE, false, 2>(a, d, s);
    else d.kw == 2 ? launch_stream<2, 1, FMT, PRE, false, 2>(a, d, s) : launch_stream<2, 1, FMT, PRE, false, 4>(a, d, s);
  } else if (d.rot) {
    launch_stream<1, 1, FMT, PRE, false, 1, 2, 8, 8, true>(a, d, s);
  } else if (d.mt == 1 && d.nw == 1) {
    launch_stream<1, 2, FMT, PRE, false, 1, 1, 8>(a, d, s);
  } else if (d.mt == 1 && d.nw == 3) {
    launch_stream<1, 2, FMT, PRE, false, 1, 3>(a, d, s);
  } else if (d.mt == 1 && d.nw == 7) {
    launch_stream<1, 1, FMT, PRE, false, 1, 7>(a, d, s);
  } else if (d.mt == 1) d.nt == 2 ? launch_stream<1, 2, FMT, PRE>(a, d, s) : launch_stream<1, 1, FMT, PRE>(a, d, s);
  else if (d.mt == 2) {
    if (d.nw == 2) launch_stream<2, 1, FMT, PRE, false, 1, 2, 4, 4>(a, d, s);  // row blocks
    else if (d.dd) launch_stream<2, 1, FMT, PRE, false, 1, 4, 4, 4>(a, d, s);  // row blocks
    else d.nt == 2 ? launch_stream<2, 2, FMT, PRE>(a, d, s) : launch_stream<2, 1, FMT, PRE>(a, d, s);
  }
  else if (d.mt == 4) {
    if (d.nw == 2) d.dd ? launch_stream<4, 1, FMT, PRE, false, 1, 2, 4, 4>(a, d, s) : launch_stream<4, 1, FMT, PRE, false, 1, 2>(a, d, s);
    else if (d.nw == 6) launch_stream<4, 1, FMT, PRE, false, 1, 6>(a, d, s);
    else if (d.nw == 7) d.dd ? launch_stream<4, 1, FMT, PRE, false, 1, 7, 4, 4>(a, d, s) : launch_stream<4, 1, FMT, PRE, false, 1, 7>(a, d, s);
    else if (d.nw == 8) launch_stream<4, 1, FMT, PRE, false, 1, 8, 4, 4>(a, d, s);
    else if (d.nt == 2) launch_stream<4, 2, FMT, PRE>(a, d, s);
    else d.dd ? launch_stream<4, 1, FMT, PRE, false, 1, 4, 4, 4>(a, d, s) : launch_stream<4, 1, FMT, PRE>(a, d, s);
  } else {
    if (d.nw == 2) d.dd ? launch_stream<8, 1, FMT, PRE, false, 1, 2, 4, 4>(a, d, s) : launch_stream<8, 1, FMT, PRE, false, 1, 2>(a, d, s);
    else if (d.nw == 6) launch_stream<8, 1, FMT, PRE, false, 1, 6>(a, d, s);
    else if (d.nw == 7) d.dd ? launch_stream<8, 1, FMT, PRE, false, 1, 7, 4, 3>(a, d, s) : launch_stream<8, 1, FMT, PRE, false, 1, 7>(a, d, s);
    else d.nt == 2 ? launch_stream<8, 2, FMT, PRE>(a, d, s) : launch_stream<8, 1, FMT, PRE>(a, d, s);
  }
}

// The fused-quantization stream kernel serves plans of one row tile (m <= 16); larger m quantizes into
// the workspace and runs the GEMM. Measured on the DeepSeek-V3 shapes: one row tile saves 1-1.5 us a
// call over the two launches; at 2 row tiles (8 values a lane) the two are even, at 4 (32 values a
// lane) the quantization outgrows the wait for the weights and the fused call is 15-25% slower.
// The fused kernel runs the 4-wave plan (fill = false); it serves a call only where the GEMM's own plan
// sums every output in the same order (the same K splits, no rotated K walk), so the fused call equals
// the two ops bit for bit. Elsewhere the entry point runs the two kernels.
// (At one row tile the plans do not depend on the weight layout.)
static bool fused_quant_ok(int64_t m, int64_t n, int64_t k) {
  const Plan8 f = plan8(m, n, k, true, false);
  if (!(f.kind == Kernel8::kStream && f.mt == 1 && f.kw == 1 && f.nw == 4)) return false;
  const Plan8 t = plan8(m, n, k, true);
  return !t.rot && t.splits == f.splits;
}

template <bool PRE>
static void dispatch_stream_qa(const Gemm8Args& a, const Plan8& d, hipStream_t s) {
  d.nt == 2 ? launch_stream<1, 2, 0, PRE, true>(a, d, s) : launch_stream<1, 1, 0, PRE, true>(a, d, s);
}

// Workspace of the fused entry point: the GEMM's split-K workspace, then (unfused plans) the codes
// [m, k] and group-major scales [k/128, m] of the quantized activations, each 256-byte aligned. The
// codes start past the arrival-word region even when the GEMM runs unsplit, so the region's place is
// the same in every workspace.
static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }
static size_t quant_codes_offset(int64_t m, int64_t n, int64_t k) {  // past the GEMM's own workspace
  const size_t gemm = up256(workspace8_any(m, n, k));
  return gemm > kSplitkCounterBytes ? gemm : kSplitkCounterBytes;
}
static size_t quant_gemm_workspace(int64_t m, int64_t n, int64_t k) {
  if (fused_quant_ok(m, n, k)) return workspace8(plan8(m, n, k, true, false));
  return quant_codes_offset(m, n, k) + up256((size_t)m * k) + up256((size_t)(k / 128) * m * 4);
}

// Ring depths per tile shape: as many stages (at most 4) of both operands as 150 KiB of LDS holds. The
// 256x224 and 256x192 tiles run A one stage deeper (3 A, 2 B: 156.8 and 148.8 KiB), which fits only
// because b_scale rides the A stages. Measured on cold operands, medians of interleaved runs (us, 2 -> 3
// A stages, bitwise the same output): 256x224 at m = 4096 on 7168 x 16384 441.8 -> 432.7, at m = 8192
// 865.6 -> 856.1; 256x192 at m = 4096 on 24576 x 1536 210.5 -> 205.6 and at m = 1024 53.2 -> 52.3. The
// other tiles have no room for it; 128x192 with 4 A stages against 3 measured 35.9 against 35.4 us at
// m = 1024 on 2112 x 7168.
__host__ __device__ constexpr int lds8_stages(int tm, int tn) {
  return 150 * 1024 / (lds8_stage_a(tm) + lds8_stage_b(tn)) < 4 ? 150 * 1024 / (lds8_stage_a(tm) + lds8_stage_b(tn))
                                                                 : 4;
}
__host__ __device__ constexpr bool lds8_fits(int tm, int tn, int sa, int sb) {
  return sa * lds8_stage_a(tm) + sb * lds8_stage_b(tn) + 1024 + 16 <= 160 * 1024;
}
template <int TM, int TN, int FMT, bool PRE, int SA = lds8_stages(TM, TN), int SB = lds8_stages(TM, TN),
          bool KS = false>
static void launch_lds_t(const Gemm8Args& a, const Plan8& t, hipStream_t s) {
  static_assert(lds8_fits(TM, TN, SA, SB), "LDS budget");
  static_assert(!KS || SA * lds8_stage_a(TM) + SB * lds8_stage_b(TN) + 1024 + 16 + 48 * TM <= 160 * 1024,
                "LDS budget with the a_scale ring");
  hipLaunchKernelGGL((gemm8_lds_kernel<TM, TN, SA, SB, FMT, PRE, KS>), dim3((unsigned)(t.grid_x * t.splits)),
                     dim3(512), 0, s, a);
}

template <int FMT, bool PRE>
static void launch_lds(const Gemm8Args& a, const Plan8& t, hipStream_t s) {
  if constexpr (FMT == 0 && PRE) {
    // K-major a_scale (pitch >= K / 128) on the 64x64 .. 128x192 tiles: the a_scale ring. Cold operands,
    // us (column-major a_scale; K-major with per-stage loads -> the ring): 4096 x 1024 x 4096 (128x128, 2
    // splits) 25.10; 31.47 -> 27.31, 4096 x 512 x 4096 20.83; 23.37 -> 21.62, 2048 x 1024 x 4096 21.11;
    // 23.26 -> 21.53, 2048 x 512 x 4096 13.77; 15.65 -> 14.48, 2048 x 1536 x 4096 (128x192) 26.70; 29.51 ->
    // 27.50, 256 x 512 x 4096 (64x64, 4 splits) 8.74; 9.09 -> 9.00, 1500 x 512 x 3584 (64x64) 12.09; 12.46
    // -> 12.57. On the 128x256 and 192x192 tiles (16 and 18 MFMA tiles a wave) it ran 1.6-2.2x slower
    // (1100 x 7168 x 2048 26.12 -> 41.69, 2048 x 2112 x 7168 53.04 -> 117.83); the 256-row tiles were not
    // tried (256x224 and 256x192 have no LDS left for it): those keep the per-stage loads.
    if (a.sa_sk == 1 && a.sa_sm >= (a.k >> 7)) {
      if (t.tm == 64 && t.tn == 64) return launch_lds_t<64, 64, 0, true, lds8_stages(64, 64), lds8_stages(64, 64), true>(a, t, s);
      if (t.tm == 64 && t.tn == 128) return launch_lds_t<64, 128, 0, true, lds8_stages(64, 128), lds8_stages(64, 128), true>(a, t, s);
      if (t.tm == 128 && t.tn == 128) return launch_lds_t<128, 128, 0, true, lds8_stages(128, 128), lds8_stages(128, 128), true>(a, t, s);
      if (t.tm == 128 && t.tn == 192) return launch_lds_t<128, 192, 0, true, lds8_stages(128, 192), lds8_stages(128, 192), true>(a, t, s);
    }
  }
  if (t.tm == 192) {
    launch_lds_t<192, 192, FMT, PRE>(a, t, s);
  } else if (t.tm == 256) {
    if (t.tn == 256) launch_lds_t<256, 256, FMT, PRE>(a, t, s);
    else if (t.tn == 224) launch_lds_t<256, 224, FMT, PRE, 3, 2>(a, t, s);
    else if (t.tn == 192) launch_lds_t<256, 192, FMT, PRE, 3, 2>(a, t, s);
    else launch_lds_t<256, 128, FMT, PRE>(a, t, s);
  } else if (t.tm == 64) {
    t.tn == 64 ? launch_lds_t<64, 64, FMT, PRE>(a, t, s) : launch_lds_t<64, 128, FMT, PRE>(a, t, s);
  } else {
    if (t.tn == 256) launch_lds_t<128, 256, FMT, PRE>(a, t, s);
    else if (t.tn == 192) launch_lds_t<128, 192, FMT, PRE>(a, t, s);
    else launch_lds_t<128, 128, FMT, PRE>(a, t, s);
  }
}

}  // namespace aklr

using namespace aklr;

extern "C" size_t aklr_gemm_a8w8_blockscale_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k < 128) return 0;
  return workspace8_any(m, n, k);
}

// The FP8 GEMM with the scratch it needs taken from `workspace` (the caller's buffer of
// workspace_bytes), or, when scratch_cap is nonzero, from the device buffer `scratch` of scratch_cap
// bytes (a plan needing more returns AKLR_ERR_SCRATCH_LIMIT).
int aklr::gemm8_entry(const void* a, int64_t lda, const void* b, int64_t ldb, const float* a_scale,
                       int64_t sa_stride_m, int64_t sa_stride_k, const float* b_scale, int64_t ldbs,
                       const float* bias, void* out, int64_t ldo, int64_t m, int64_t n, int64_t k, int fp8_dtype,
                       int b_layout, int out_dtype, void* workspace, size_t workspace_bytes, void* scratch,
                       size_t scratch_cap, hipStream_t stream) {
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
  // Kernels address a tile's rows with 32-bit offsets from the tile's first row.
  if (lda >= (1 << 23) || (b_layout == AKLR_B_ROW_MAJOR && ldb >= (1 << 23))) return AKLR_ERR_INVALID_ARGUMENT;
  if (((m - 1) * sa_stride_m + (k / 128 - 1) * sa_stride_k + 1) * 4 > 0x7FFFFFFFll) return AKLR_ERR_INVALID_ARGUMENT;
  if (b_layout == AKLR_B_ROW_MAJOR && (ldb < k || ldb % 16 != 0)) return AKLR_ERR_INVALID_ARGUMENT;
  if (ldbs < k / 128 || sa_stride_m < 0 || sa_stride_k < 0) return AKLR_ERR_INVALID_ARGUMENT;
  // The stream kernel stages b_scale with 32-bit offsets from its start.
  if (((n - 1) / 128 * ldbs + k / 128) * 4 > 0x7FFFFFFFll) return AKLR_ERR_INVALID_ARGUMENT;
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
  g.nt_out = lds_nt_out(ldo * 2, k) ? 1 : 0;
  g.counters = nullptr;
  g.partial = nullptr;
  const bool pre = b_layout == AKLR_B_PRESHUFFLE_16x16;
  const bool e5 = fp8_dtype == AKLR_FP8_E5M2;

  const Plan8 plan = plan8(m, n, k, pre);
  g.splits = plan.splits;
  g.kb_per_split = plan.kb_per_split;
  if (plan.splits > 1) {
    const size_t need = workspace8(plan);
    if (scratch_cap) {
      if (need > scratch_cap) return AKLR_ERR_SCRATCH_LIMIT;
      workspace = scratch;
    } else if (!workspace || workspace_bytes < need || !aklr_aligned16(workspace)) {
      return AKLR_ERR_WORKSPACE;
    }
    g.counters = static_cast<uint64_t*>(workspace);
    g.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kSplitkCounterBytes);
  }
  if (plan.kind == Kernel8::kStream) {
    if (e5) pre ? dispatch_stream<1, true>(g, plan, stream) : dispatch_stream<1, false>(g, plan, stream);
    else pre ? dispatch_stream<0, true>(g, plan, stream) : dispatch_stream<0, false>(g, plan, stream);
  } else {
    if (e5) pre ? launch_lds<1, true>(g, plan, stream) : launch_lds<1, false>(g, plan, stream);
    else pre ? launch_lds<0, true>(g, plan, stream) : launch_lds<0, false>(g, plan, stream);
  }
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

extern "C" int aklr_gemm_a8w8_blockscale(const void* a, int64_t lda, const void* b, int64_t ldb,
                                         const float* a_scale, int64_t sa_stride_m, int64_t sa_stride_k,
                                         const float* b_scale, int64_t ldbs, const float* bias, void* out,
                                         int64_t ldo, int64_t m, int64_t n, int64_t k, int fp8_dtype, int b_layout,
                                         int out_dtype, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
  return gemm8_entry(a, lda, b, ldb, a_scale, sa_stride_m, sa_stride_k, b_scale, ldbs, bias, out, ldo, m, n, k,
                     fp8_dtype, b_layout, out_dtype, workspace, workspace_bytes, nullptr, 0, stream);
}

extern "C" size_t aklr_quant_gemm_a8w8_blockscale_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k < 128) return 0;
  return quant_gemm_workspace(m, n, k);
}

extern "C" int aklr_gemm_a8w8_blockscale_kernel(int64_t m, int64_t n, int64_t k, int b_layout) {
  if (m <= 0 || n <= 0 || k < 128 || k % 128 != 0) return -1;
  if (b_layout != AKLR_B_ROW_MAJOR && b_layout != AKLR_B_PRESHUFFLE_16x16) return -1;
  return plan8(m, n, k, b_layout == AKLR_B_PRESHUFFLE_16x16).kind == Kernel8::kStream ? 0 : 1;
}

extern "C" int aklr_quant_gemm_a8w8_blockscale_fused(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k < 128) return 0;
  return fused_quant_ok(m, n, k) ? 1 : 0;
}

extern "C" int aklr_quant_gemm_a8w8_blockscale(const void* x, int64_t ldx, const void* b, int64_t ldb,
                                               const float* b_scale, int64_t ldbs, const float* bias, void* out,
                                               int64_t ldo, int64_t m, int64_t n, int64_t k, int b_layout,
                                               int out_dtype, void* workspace, size_t workspace_bytes,
                                               hipStream_t stream) {
  if (!x || !b || !b_scale || !out) return AKLR_ERR_INVALID_ARGUMENT;
  if (m < 0 || n <= 0 || k <= 0 || k % 128 != 0 || n % 16 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (m > (1 << 20) || n > 262144 || k > 65536) return AKLR_ERR_INVALID_ARGUMENT;
  if (b_layout != AKLR_B_ROW_MAJOR && b_layout != AKLR_B_PRESHUFFLE_16x16) return AKLR_ERR_UNSUPPORTED;
  if (out_dtype != AKLR_OUT_BF16 && out_dtype != AKLR_OUT_F16) return AKLR_ERR_UNSUPPORTED;
  if (!aklr_aligned16(x) || !aklr_aligned16(b) || !aklr_aligned16(out)) return AKLR_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(b_scale) & 3u) || (bias && (reinterpret_cast<uintptr_t>(bias) & 3u)))
    return AKLR_ERR_INVALID_ARGUMENT;
  if (ldx < k || ldx % 8 != 0 || ldo < n || ldo % 8 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (b_layout == AKLR_B_ROW_MAJOR && (ldb < k || ldb % 16 != 0 || ldb >= (1 << 23))) return AKLR_ERR_INVALID_ARGUMENT;
  if (ldbs < k / 128) return AKLR_ERR_INVALID_ARGUMENT;
  if (m == 0) return AKLR_OK;
  const Plan8 plan = plan8(m, n, k, true, false);  // the fused kernel's plan (one row tile)
  const size_t need = quant_gemm_workspace(m, n, k);
  if (need > 0 && (!workspace || workspace_bytes < need || !aklr_aligned16(workspace))) return AKLR_ERR_WORKSPACE;
  uint8_t* ws = static_cast<uint8_t*>(workspace);

  if (!fused_quant_ok(m, n, k)) {
    // quantize into the workspace (past the GEMM's part), then the GEMM reads it
    uint8_t* q = ws + quant_codes_offset(m, n, k);
    float* sc = reinterpret_cast<float*>(q + up256((size_t)m * k));
    int st = aklr_per_group_quant_fp8(x, ldx, q, sc, m, k, stream);
    if (st != AKLR_OK) return st;
    const size_t gemm_ws = workspace8_any(m, n, k);
    return aklr_gemm_a8w8_blockscale(q, k, b, ldb, sc, 1, m, b_scale, ldbs, bias, out, ldo, m, n, k,
                                     AKLR_FP8_E4M3FN, b_layout, out_dtype, gemm_ws ? ws : nullptr, gemm_ws, stream);
  }
  // the loader addresses x with 32-bit byte offsets from its first row
  if (((m - 1) * ldx + k) * 2 > 0x7FFFFFFFll) return AKLR_ERR_INVALID_ARGUMENT;
  Gemm8Args g;
  g.a = static_cast<const uint8_t*>(x);
  g.lda = ldx;
  g.b = static_cast<const uint8_t*>(b);
  g.ldb = ldb;
  g.sa = nullptr;  // the loader computes the scales
  g.sa_sm = g.sa_sk = 0;
  g.sb = b_scale;
  g.ldbs = ldbs;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.m = (int)m;
  g.n = (int)n;
  g.k = (int)k;
  g.out_dtype = out_dtype;
  g.nt_out = 0;  // the stream kernel's stores are plain
  g.counters = nullptr;
  g.partial = nullptr;
  g.splits = plan.splits;
  g.kb_per_split = plan.kb_per_split;
  if (plan.splits > 1) {
    g.counters = reinterpret_cast<uint64_t*>(ws);
    g.partial = reinterpret_cast<float*>(ws + kSplitkCounterBytes);
  }
  if (b_layout == AKLR_B_PRESHUFFLE_16x16) dispatch_stream_qa<true>(g, plan, stream);
  else dispatch_stream_qa<false>(g, plan, stream);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

// ---------------------------------------------------------------------------------------------
// b given as (k, n) (trans_b = false): dst[c][r] = src[r][c] over bytes, so the GEMM entries read it
// as (n, k). A 256-thread workgroup moves a 64 x 64 byte tile through LDS: lane t loads 16 bytes of
// source row t / 4, then gathers the 16 bytes of destination row t / 4 from the tile's column and
// stores them as one 16-byte write. Rows of the LDS tile are 68 bytes apart (4-byte aligned, and the
// column gather spreads over banks).
namespace aklr {
__global__ __launch_bounds__(256) void transpose_b8_kernel(const uint8_t* __restrict__ src, int64_t rows,
                                                           int64_t cols, int64_t src_ld, uint8_t* __restrict__ dst,
                                                           int64_t dst_ld) {
  constexpr int kPitch = 68;
  __shared__ uint8_t tile[64 * kPitch];
  const int64_t tiles_c = (cols + 63) / 64;
  const int64_t r0 = (int64_t)(blockIdx.x / tiles_c) * 64, c0 = (int64_t)(blockIdx.x % tiles_c) * 64;
  const int t = threadIdx.x, tr = t >> 2, tc = (t & 3) * 16;
  u32x4 v = {0, 0, 0, 0};
  if (r0 + tr < rows && c0 + tc < cols) v = *reinterpret_cast<const u32x4*>(src + (r0 + tr) * src_ld + c0 + tc);
  uint32_t* row = reinterpret_cast<uint32_t*>(&tile[tr * kPitch + tc]);
  row[0] = v.x;
  row[1] = v.y;
  row[2] = v.z;
  row[3] = v.w;
  __syncthreads();
  // destination row c0 + tr (a source column), bytes from source rows r0 + tc .. + 15
  if (c0 + tr >= cols || r0 + tc >= rows) return;
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t x = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) x |= (uint32_t)tile[(tc + 4 * i + b) * kPitch + tr] << (8 * b);
    w[i] = x;
  }
  *reinterpret_cast<u32x4*>(dst + (c0 + tr) * dst_ld + r0 + tc) = u32x4{w[0], w[1], w[2], w[3]};
}
}  // namespace aklr

extern "C" int aklr_transpose_b8(const void* src, int64_t rows, int64_t cols, int64_t src_ld, void* dst,
                                 int64_t dst_ld, hipStream_t stream) {
  if (!src || !dst) return AKLR_ERR_INVALID_ARGUMENT;
  if (rows <= 0 || cols <= 0 || rows % 16 != 0 || cols % 16 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (src_ld < cols || dst_ld < rows || src_ld % 16 != 0 || dst_ld % 16 != 0) return AKLR_ERR_INVALID_ARGUMENT;
  if (!aklr_aligned16(src) || !aklr_aligned16(dst)) return AKLR_ERR_INVALID_ARGUMENT;
  const int64_t blocks = ((rows + 63) / 64) * ((cols + 63) / 64);
  if (blocks > 0x7FFFFFFF) return AKLR_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(aklr::transpose_b8_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(src), rows, cols, src_ld, static_cast<uint8_t*>(dst), dst_ld);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

AKLR_SCALAR_FP32_END
