// Grouped DeepSeek-V3 FP8 MoE for gfx950 (deepseek_v2_fp8_moe): router, grouped top-k, expert sort,
// per-token input quantization, two grouped 128x128-block-scaled FP8 GEMMs and a deterministic
// weighted combine, all on the caller's stream, scratch from the caller's workspace.
//
// Data flow for T tokens, S slots per token (topk routed + the shared expert), R = T * S rows:
//   router_kernel    logits[T, Er] = bf16(x @ router^T)                          (bf16 MFMA)
//   route_kernel     ids[T, S], weights[T, S]: sigmoid, grouped top-k, shared slot last
//   align_kernel     one workgroup: per-expert counts, the rows sorted by expert (stable only per
//                    expert, which nothing depends on), each row's position, and the tables of
//                    256-, 128- and 64-row blocks (expert, first row, rows) the GEMMs walk
//   quant_div_kernel x -> e4m3 per 1 x 128 at scale max(amax / 448, tiny) (a true division, as the
//                    checkpoint's FP8 scheme quantizes the linears' inputs), scales [D/128, T]
//   moe_gemm<GATEUP> per block class, per (block, 128 columns of the intermediate): rows gathered by token, gate and up
//                    weight rows interleaved per 16 so each lane holds both for the same columns;
//                    epilogue silu(gate) * up -> bf16 -> e4m3 per 1 x 128 (same division) into h
//   moe_gemm<DOWN>   per (block, 256 output columns): h rows in sorted order -> y (bf16, sorted)
//   combine_kernel   out[t] = bf16(sum over slots, in slot order, of weight * y[row of (t, slot)])
// The GEMMs are persistent (one 512-thread workgroup per CU walks the work items) and read the block
// count from device memory, so the whole pipeline runs without a host synchronization.
#include "common.h"

AKLR_SCALAR_FP32_BEGIN

namespace aklr {
namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Row-block classes: an expert's rows split into full 256-row blocks and one last block for the
// remainder, of the smallest class that holds it (64, 128 or 256 rows). Every block streams the
// expert's weight tile once, so an expert costs ceil(rows / 256) weight reads -- the fewest for tiles
// of at most 256 rows -- at the price of some padded MFMA rows in the last block.
constexpr int kClasses = 3;
constexpr int kMinTM = 64;
__host__ __device__ constexpr int class_rows(int k) { return k == 0 ? 256 : (k == 1 ? 128 : 64); }
constexpr int kTN = 256;   // weight rows per GEMM tile
constexpr int kMaxExperts = 2048;  // expert slots the align kernel's LDS holds
constexpr float kFp32Tiny = 1.17549435e-38f;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// ---------------------------------------------------------------------------------------------
// router: one wave computes 16 tokens x 16 * NT experts with V_MFMA_F32_16X16X32_BF16, operands
// straight from global memory: lane (li, g) loads the 8 bf16 at k0 + 8g of its row. The MFMA pairs
// A's and B's lane groups the same way, so this assignment of k only has to match between them.
template <int NT>
__global__ __launch_bounds__(256) void router_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
                                                     uint16_t* __restrict__ logits, int T, int E, int D) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int tiles_e = (E + 16 * NT - 1) / (16 * NT);
  const int tt = wave / tiles_e, te = wave % tiles_e;
  if (tt * 16 >= T) return;
  const int li = lane & 15, g = lane >> 4;
  const rsrc_t xr = make_rsrc(x + (int64_t)tt * 16 * D, (uint32_t)((int64_t)min(16, T - tt * 16) * D * 2));
  const uint32_t x_off = li < T - tt * 16 ? (uint32_t)((li * D + 8 * g) * 2) : kOobOffset;
  rsrc_t br[NT];
  uint32_t b_off[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int e0 = te * 16 * NT + nt * 16;
    br[nt] = make_rsrc(wr + (int64_t)min(e0, E - 1) * D, (uint32_t)((int64_t)max(0, min(16, E - e0)) * D * 2));
    b_off[nt] = e0 + li < E ? (uint32_t)((li * D + 8 * g) * 2) : kOobOffset;
  }
  f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < D; k0 += 32) {
    const uint32_t kb = (uint32_t)k0 * 2;
    const bf16x8 a = __builtin_bit_cast(bf16x8, buf_ld16(xr, x_off + kb));
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const bf16x8 b = __builtin_bit_cast(bf16x8, buf_ld16(br[nt], b_off[nt] + kb));
      acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[nt], 0, 0, 0);
    }
  }
  // lane holds tokens 4g + r, expert li of each tile
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int e = te * 16 * NT + nt * 16 + li;
    if (e >= E) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tt * 16 + 4 * g + r;
      if (t < T) logits[(int64_t)t * E + e] = (uint16_t)f32_to_bf16_bits(acc[nt][r]);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// route: one wave per token. (value, index) pairs compare by value, then the lower index first.
__device__ __forceinline__ bool better(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float w = __shfl_xor(v, off);
    const int j = __shfl_xor(i, off);
    if (better(w, j, v, i)) {
      v = w;
      i = j;
    }
  }
}

constexpr int kRouteMaxPerLane = 16;  // routed experts <= 1024

__global__ __launch_bounds__(64) void route_kernel(const uint16_t* __restrict__ logits, const uint16_t* __restrict__ bias,
                                                   int T, int E, int G, int topk, int topk_group, int renormalize,
                                                   float scale, int shared, int32_t* __restrict__ ids,
                                                   float* __restrict__ weights) {
  __shared__ float sv[1024];  // unbiased scores
  __shared__ float sb[1024];  // biased scores
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const int per = E / G;
  float b[kRouteMaxPerLane];
#pragma unroll
  for (int j = 0; j < kRouteMaxPerLane; ++j) {
    const int i = lane + 64 * j;
    b[j] = -INFINITY;
    if (i < E) {
      const float x = bf16_to_f32(logits[(int64_t)t * E + i]);
      const float v = 1.0f / (1.0f + expf(-x));
      b[j] = v + bf16_to_f32(bias[i]);
      sv[i] = v;
      sb[i] = b[j];
    }
  }
  __syncthreads();
  // group score: the sum of its two best biased scores
  float gs = -INFINITY;
  if (lane < G) {
    float m1 = -INFINITY, m2 = -INFINITY;
    for (int i = lane * per; i < lane * per + per; ++i) {
      const float x = sb[i];
      if (x > m1) {
        m2 = m1;
        m1 = x;
      } else if (x > m2) {
        m2 = x;
      }
    }
    gs = m1 + m2;
  }
  // keep the topk_group best groups (G <= 64)
  uint64_t kept = 0;
  bool mine = false;
  for (int r = 0; r < topk_group; ++r) {
    float v = (lane < G && !mine) ? gs : -INFINITY;
    int i = lane < G && !mine ? lane : 1 << 30;
    wave_argmax(v, i);
    if (i == lane) mine = true;
    kept |= 1ull << (i & 63);
  }
  // the topk best biased scores among the kept groups' experts
  uint32_t taken = 0;
  float wsum = 0.0f;
  int my_id = 0;
  float my_v = 0.0f;
  for (int r = 0; r < topk; ++r) {
    float v = -INFINITY;
    int i = 1 << 30;
#pragma unroll
    for (int j = 0; j < kRouteMaxPerLane; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !(taken >> j & 1u) && (kept >> (e / per) & 1ull) && better(b[j], e, v, i)) {
        v = b[j];
        i = e;
      }
    }
    wave_argmax(v, i);
    if ((i & 63) == lane) taken |= 1u << (i >> 6);
    const float sc = sv[i];
    wsum += sc;
    if (lane == r) {
      my_id = i;
      my_v = sc;
    }
  }
  const int S = topk + (shared ? 1 : 0);
  if (lane < topk) {
    const float w = renormalize ? my_v / wsum : my_v;
    ids[(int64_t)t * S + lane] = my_id;
    weights[(int64_t)t * S + lane] = w * scale;
  }
  if (shared && lane == 0) {
    ids[(int64_t)t * S + topk] = E;
    weights[(int64_t)t * S + topk] = 1.0f;
  }
}

// ---------------------------------------------------------------------------------------------
// align: one 1024-thread workgroup. Entries whose expert is out of [0, E) get row -1 (ignored).
__device__ int block_exclusive_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int i = 0; i < 16; ++i) {
      const int s = wsum[i];
      wsum[i] = acc;
      acc += s;
    }
    *total = acc;
  }
  __syncthreads();
  const int r = wsum[w] + incl - v;
  __syncthreads();
  return r;
}

// Block table: for each class k, expert[k][i], first row[k][i] and rows[k][i] of its blocks, cap
// entries per class, and count[k].
struct BlockTable {
  int32_t* expert;
  int32_t* row;
  int32_t* rows;
  int32_t* count;
  int cap;
};

__device__ __forceinline__ int class_blocks(int c, int k) {
  const int full = c / 256, rem = c - 256 * full;
  const int last = rem == 0 ? -1 : (rem > 128 ? 0 : (rem > 64 ? 1 : 2));  // class of the remainder block
  return (k == 0 ? full : 0) + (k == last ? 1 : 0);
}

__global__ __launch_bounds__(1024) void align_kernel(const int32_t* __restrict__ ids, int R, int S, int E,
                                                     int32_t* __restrict__ row_of, int32_t* __restrict__ sorted_tok,
                                                     BlockTable bt, int* __restrict__ tickets) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int off[kMaxExperts];
  __shared__ int boff[kClasses][kMaxExperts];
  __shared__ int wsum[16];
  __shared__ int total;
  const int tid = threadIdx.x;
  if (tid < 2) tickets[tid] = 0;  // the grouped GEMMs' work-item counters (gate-up, down)
  for (int e = tid; e < kMaxExperts; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < R; i += 1024) {
    const int e = ids[i];
    row_of[i] = (e >= 0 && e < E) ? atomicAdd(&cnt[e], 1) : -1;
  }
  __syncthreads();
  // two experts per thread: exclusive prefix of rows, then of each class's blocks
  const int e0 = 2 * tid, e1 = 2 * tid + 1;
  const int c0 = e0 < E ? cnt[e0] : 0, c1 = e1 < E ? cnt[e1] : 0;
  const int o = block_exclusive_scan(c0 + c1, wsum, &total);
  if (e0 < kMaxExperts) off[e0] = o;
  if (e1 < kMaxExperts) off[e1] = o + c0;
#pragma unroll
  for (int k = 0; k < kClasses; ++k) {
    const int b0 = class_blocks(c0, k), b1 = class_blocks(c1, k);
    const int bo = block_exclusive_scan(b0 + b1, wsum, &total);
    if (e0 < kMaxExperts) boff[k][e0] = bo;
    if (e1 < kMaxExperts) boff[k][e1] = bo + b0;
    if (tid == 0) bt.count[k] = total;
  }
  __syncthreads();
  for (int i = tid; i < R; i += 1024) {
    const int e = ids[i];
    if (e < 0 || e >= E) continue;
    const int pos = off[e] + row_of[i];
    row_of[i] = pos;
    sorted_tok[pos] = i / S;
  }
  for (int e = tid; e < E; e += 1024) {
    const int c = cnt[e];
    int row = off[e], left = c;
#pragma unroll
    for (int k = 0; k < kClasses; ++k) {
      const int nb = class_blocks(c, k);
      for (int j = 0; j < nb; ++j) {
        const int idx = k * bt.cap + boff[k][e] + j;
        const int n = min(class_rows(k), left);
        bt.expert[idx] = e;
        bt.row[idx] = row;
        bt.rows[idx] = n;
        row += n;
        left -= n;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// quant: 16 lanes per 1 x 128 group, 8 values each. scale = max(amax / 448, tiny); code =
// e4m3(x / scale), both true IEEE divisions.
__global__ __launch_bounds__(256) void quant_div_kernel(const uint16_t* __restrict__ x, int T, int D,
                                                        uint8_t* __restrict__ q, float* __restrict__ s) {
  const int groups = D / 128;
  const int gid = blockIdx.x * 16 + (threadIdx.x >> 4);
  if (gid >= T * groups) return;
  const int t = gid / groups, grp = gid - t * groups;
  const int sub = threadIdx.x & 15;
  const int64_t base = (int64_t)t * D + grp * 128 + sub * 8;
  const u32x4 v = ld16(x + base);
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float sc = fmaxf(__fdiv_rn(amax, 448.0f), kFp32Tiny);
  float c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = fminf(fmaxf(__fdiv_rn(f[i], sc), -448.0f), 448.0f);
  u32x2 out;
  out[0] = pack4_e4m3(c[0], c[1], c[2], c[3]);
  out[1] = pack4_e4m3(c[4], c[5], c[6], c[7]);
  *reinterpret_cast<u32x2*>(q + base) = out;
  if (sub == 0) s[(int64_t)grp * T + t] = sc;
}

// ---------------------------------------------------------------------------------------------
// grouped GEMM
enum { kGateUp = 0, kDown = 1 };

struct MoeGemmArgs {
  const uint8_t* a;          // GATEUP: x codes [T, K]; DOWN: h codes [R, K]
  const float* sa;           // a scales, [K/128, sa_ld]
  int64_t sa_ld;             // T (GATEUP) or R (DOWN)
  const int32_t* sorted_tok; // GATEUP: sorted row -> token
  const uint8_t* b;          // expert weights, [experts, N, K] row-major or 16x16-preshuffled per expert
  int64_t b_stride;          // bytes per expert
  const float* sb;           // [experts, ceil(N/128), K/128]
  int64_t sb_stride;         // floats per expert
  const int32_t* blk_expert;  // block table of class 0; class k at + k * blk_cap
  const int32_t* blk_row;
  const int32_t* blk_rows;
  const int32_t* nblk;        // blocks per class
  int blk_cap;
  int* tickets;               // work-item counter, zero at launch (align_kernel clears it)
  int K, N, I;               // reduction length, weight rows, intermediate size
  int tiles_n;               // GATEUP: I / 128; DOWN: ceil(N / 256)
  uint8_t* hq;               // GATEUP out: [R, I] codes
  float* hs;                 // GATEUP out: [I/128, R] scales
  int64_t R;
  uint16_t* y;               // DOWN out: [R, N] bf16
};

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float round_bf16(float v) { return __uint_as_float(f32_to_bf16_bits(v) << 16); }

// One work item: a TM-row block (class TM of the block table) x 256 weight rows; 8 waves in 2 (m) x 4
// (n), each TM/2 rows x 64 weight rows (MT = TM/32, NT = 4 tiles of 16x16); K steps of 128 through a
// direct-to-LDS ring of as many stages as LDS holds (3 for TM <= 128, 2 for 256), with the swizzled
// LDS tiles, load schedule and fold of the dense LDS kernel. GATEUP orders the tile's 256 weight rows
// as (gate 16, up 16) pairs over 128 intermediate columns, so tiles nt = 2q and 2q + 1 of a wave are
// the gate and the up of the same 16 columns. LDS comes from the caller's buffer (moe_smem_bytes).
template <int TM>
struct MoeSmem {
  static constexpr int S = TM == 256 ? 2 : 3, MT = TM / 32;
  static constexpr int kStageA = TM * 128, kStageB = kTN * 128;
  static constexpr int kA = 0, kB = kA + S * kStageA, kS = kB + S * kStageB, kDummy = kS + S * TM * 4,
                       kSB = kDummy + 8 * 64 * 4, kAmax = kSB + 2 * 512 * 4, kBytes = kAmax + 2 * MT * 16 * 4 * 4;
};
constexpr int kMoeSmemBytes =
    MoeSmem<256>::kBytes > MoeSmem<128>::kBytes
        ? (MoeSmem<256>::kBytes > MoeSmem<64>::kBytes ? MoeSmem<256>::kBytes : MoeSmem<64>::kBytes)
        : (MoeSmem<128>::kBytes > MoeSmem<64>::kBytes ? MoeSmem<128>::kBytes : MoeSmem<64>::kBytes);
static_assert(kMoeSmemBytes <= 160 * 1024, "LDS");

template <int MODE, bool PRE, int TM>
__device__ __forceinline__ void moe_item(const MoeGemmArgs& p, uint8_t* smem, int cls, int blk, int pn) {
  using L = MoeSmem<TM>;
  constexpr int TN = kTN, S = L::S;
  constexpr int MT = TM / 32, NT = TN / 64;
  constexpr int AI = TM / 64, BI = TN / 64;
  constexpr int kLoads = AI + BI + 1;
  constexpr int kScaleWaves = TM / 64;
  constexpr int kStageA = L::kStageA, kStageB = L::kStageB;
  uint8_t* sA = smem + L::kA;
  uint8_t* sB = smem + L::kB;
  float* sS = reinterpret_cast<float*>(smem + L::kS);
  float* sDummy = reinterpret_cast<float*>(smem + L::kDummy);
  float (*sSB)[512] = reinterpret_cast<float (*)[512]>(smem + L::kSB);
  float (*sAmax)[MT][16][4] = reinterpret_cast<float (*)[MT][16][4]>(smem + L::kAmax);

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int wm = w >> 2, wn = w & 3;
  const int lr = lane >> 3, lp = lane & 7;
  const int c = lp ^ lr;
  const int KB = p.K >> 7;
  const int64_t kt32 = p.K >> 5;
  {
    const int bi = cls * p.blk_cap + blk;
    const int e = p.blk_expert[bi], row0 = p.blk_row[bi], rows = p.blk_rows[bi];

    // A: wave w moves tile rows [w*TM/8, (w+1)*TM/8) in slabs of 8; waves below kScaleWaves also move
    // a_scale rows [64w, 64w + 64), the others an empty load (same count per wave).
    const i32x4 ars = make_rsrc_words(p.a, (uint32_t)(p.sa_ld * p.K));  // A has sa_ld rows of K codes
    uint32_t a_off[AI];
#pragma unroll
    for (int j = 0; j < AI; ++j) {
      const int ar = w * (TM / 8) + j * 8 + lr;
      int64_t arow = 0;
      if (ar < rows) arow = MODE == kGateUp ? p.sorted_tok[row0 + ar] : row0 + ar;
      a_off[j] = ar < rows ? (uint32_t)(arow * p.K + c * 16) : kOobOffset;
    }
    const bool scale_wave = w < kScaleWaves;
    const int sr = w * 64 + lane;
    int64_t srow = 0;
    if (scale_wave && sr < rows) srow = MODE == kGateUp ? p.sorted_tok[row0 + sr] : row0 + sr;
    const i32x4 sars = make_rsrc_words(p.sa, (uint32_t)((int64_t)KB * p.sa_ld * 4));
    const uint32_t sa_off = (scale_wave && sr < rows) ? (uint32_t)(srow * 4) : kOobOffset;
    const uint32_t sa_kstep = (uint32_t)(p.sa_ld * 4);
    // B: this expert's weight; wave w moves tile rows [32w, 32w + 32) in 4 slabs of 8.
    const i32x4 brs = make_rsrc_words(p.b + (int64_t)e * p.b_stride, (uint32_t)p.b_stride);
    uint32_t b_off[BI];
#pragma unroll
    for (int j = 0; j < BI; ++j) {
      const int rr = w * 32 + j * 8 + lr;
      int wrow;
      if (MODE == kGateUp) {
        const int blk16 = rr >> 4;
        wrow = ((blk16 & 1) ? p.I : 0) + pn * 128 + (blk16 >> 1) * 16 + (rr & 15);
      } else {
        wrow = pn * TN + rr;
      }
      if (wrow >= p.N)
        b_off[j] = kOobOffset;
      else if (PRE)
        b_off[j] = (uint32_t)(((int64_t)(wrow >> 4) * kt32 + (c >> 1)) * 512 + (c & 1) * 256 + (wrow & 15) * 16);
      else
        b_off[j] = (uint32_t)((int64_t)wrow * p.K + c * 16);
    }
    const uint32_t lds_a = lds_addr(&sA[w * (TM / 8) * 128]), lds_b = lds_addr(&sB[w * 32 * 128]);
    const uint32_t lds_s = scale_wave ? lds_addr(&sS[w * 64]) : lds_addr(&sDummy[w * 64]);
    const uint32_t lds_s_step = scale_wave ? TM * 4 : 0;
    auto issue = [&](int kb, int st) {
      const bool on = kb < KB;
      const uint32_t ak = (uint32_t)kb * 128u, bk = PRE ? (uint32_t)kb * 2048u : (uint32_t)kb * 128u;
#pragma unroll
      for (int j = 0; j < AI; ++j)
        lds_dma16(ars, lds_a + st * kStageA + j * 1024, on && a_off[j] != kOobOffset ? a_off[j] + ak : kOobOffset);
#pragma unroll
      for (int j = 0; j < BI; ++j)
        lds_dma16(brs, lds_b + st * kStageB + j * 1024, on && b_off[j] != kOobOffset ? b_off[j] + bk : kOobOffset);
      lds_dma4(sars, lds_s + st * lds_s_step, on && sa_off != kOobOffset ? sa_off + (uint32_t)kb * sa_kstep : kOobOffset);
    };

    // b_scale rows of the tile over K: GATEUP gate block pn and up block I/128 + pn; DOWN the
    // tile's two 128-row blocks.
    {
      const float* sbe = p.sb + (int64_t)e * p.sb_stride;
      const int last = (p.N - 1) >> 7;
      const int r0 = MODE == kGateUp ? pn : min(2 * pn, last);
      const int r1 = MODE == kGateUp ? (p.I >> 7) + pn : min(2 * pn + 1, last);
      for (int i = threadIdx.x; i < 2 * KB; i += 512) {
        const int r = i >= KB ? 1 : 0, kk = i - r * KB;
        sSB[r][kk] = sbe[(int64_t)(r ? r1 : r0) * KB + kk];
      }
    }

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int swz_lo = (g ^ (li & 7)) << 4, swz_hi = ((4 + g) ^ (li & 7)) << 4;
    const int a_row = (wm * (TM / 2) + li) * 128, b_row = (wn * 64 + li) * 128;
    // The dense LDS kernel's step (gemm_a8w8.hip): the smaller fragment set held, the other streamed
    // one tile ahead, and each MFMA's fold kLag MFMAs after it (bitwise the same sums).
    constexpr int kLag = 3, kT = MT * NT;
    constexpr bool kHoldA = MT <= NT;
    constexpr int kHeld = kHoldA ? MT : NT, kStreamed = kHoldA ? NT : MT;
    auto tmt = [](int t) { return kHoldA ? t % MT : t / NT; };
    auto tnt = [](int t) { return kHoldA ? t / MT : t % NT; };
    f32x4 pend[kLag];
    float pend_s[kLag];
#pragma unroll
    for (int j = 0; j < kLag; ++j) {
      pend[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      pend_s[j] = 0.f;
    }
    auto compute = [&](int kb, int st) {
      const uint8_t* A = sA + st * kStageA;
      const uint8_t* B = sB + st * kStageB;
      const float* SA = sS + st * TM + wm * (TM / 2) + li;
      float sbv[2];
      if (MODE == kGateUp) {
        sbv[0] = sSB[0][kb];
        sbv[1] = sSB[1][kb];
      } else {
        sbv[0] = sbv[1] = sSB[wn >> 1][kb];
      }
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
      float s0[MT], s1[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float sa = SA[mt * 16];
        s0[mt] = sa * sbv[0];
        s1[mt] = sa * sbv[1];
      }
      i32x8 cur, nxt = kHoldA ? read_b(0) : read_a(0);
      f32x4 part[kT];
      float sc[kT];
#pragma unroll
      for (int t = 0; t < kT; ++t) {
        const int mt = tmt(t), nt = tnt(t);
        const int si = t / kHeld, hi = t % kHeld;
        if (hi == 0) {
          cur = nxt;
          if (si + 1 < kStreamed) nxt = kHoldA ? read_b(si + 1) : read_a(si + 1);
        }
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        // lane: row li, columns 4g..4g+3 (the weight is the first operand)
        part[t] = kHoldA ? mfma16x128<0>(cur, held[hi], z) : mfma16x128<0>(held[hi], cur, z);
        sc[t] = (nt & 1) ? s1[mt] : s0[mt];
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

#pragma unroll
    for (int s = 0; s < S - 1; ++s) issue(s, s);
    int st = 0, st_fill = S - 1;
    for (int kb = 0; kb < KB; ++kb) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((S - 2) * kLoads) : "memory");
      __syncthreads();
      issue(kb + S - 1, st_fill);
      compute(kb, st);
      st = st + 1 == S ? 0 : st + 1;
      st_fill = st_fill + 1 == S ? 0 : st_fill + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < kLag; ++j) {
      const int u = kT - kLag + j;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[tmt(u)][tnt(u)][r] = fmaf(pend[j][r], pend_s[j], acc[tmt(u)][tnt(u)][r]);
    }

    if (MODE == kGateUp) {
      // h = bf16(silu(gate) * up), kept in the gate tiles' registers; per row, e4m3 at scale
      // max(amax / 448, tiny) over the tile's 128 columns (the wave's 32 here, the other 3 waves'
      // through LDS).
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float m = 0.0f;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = round_bf16(silu(acc[mt][2 * q][r]) * acc[mt][2 * q + 1][r]);
            acc[mt][2 * q][r] = v;
            m = fmaxf(m, fabsf(v));
          }
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        if (g == 0) sAmax[wm][mt][li][wn] = m;
      }
      __syncthreads();
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float m = fmaxf(fmaxf(sAmax[wm][mt][li][0], sAmax[wm][mt][li][1]),
                              fmaxf(sAmax[wm][mt][li][2], sAmax[wm][mt][li][3]));
        const float sc = fmaxf(__fdiv_rn(m, 448.0f), kFp32Tiny);
        const int tr = wm * (TM / 2) + mt * 16 + li;
        if (tr < rows) {
          const int64_t row = row0 + tr;
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            float cv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) cv[r] = fminf(fmaxf(__fdiv_rn(acc[mt][2 * q][r], sc), -448.0f), 448.0f);
            const int col = pn * 128 + wn * 32 + q * 16 + 4 * g;
            *reinterpret_cast<uint32_t*>(p.hq + row * p.I + col) = pack4_e4m3(cv[0], cv[1], cv[2], cv[3]);
          }
          if (wn == 0 && g == 0) p.hs[(int64_t)pn * p.R + row] = sc;
        }
      }
    } else {
      // y rows in sorted order, bf16; lane pairs swap halves for 16-byte stores (see the dense kernel)
      const int col_s = pn * TN + wn * 64 + (g & 1) * 16 + (g >> 1) * 8;
#pragma unroll
      for (int nt = 0; nt < NT; nt += 2)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4 xv = acc[mt][nt], yv = acc[mt][nt + 1];
          const uint32_t x0 = pack_bf16x2(xv[0], xv[1]), x1 = pack_bf16x2(xv[2], xv[3]);
          const uint32_t y0 = pack_bf16x2(yv[0], yv[1]), y1 = pack_bf16x2(yv[2], yv[3]);
          const auto s0 = __builtin_amdgcn_permlane16_swap(x0, y0, false, false);
          const auto s1 = __builtin_amdgcn_permlane16_swap(x1, y1, false, false);
          const u32x4 v = {s0[0], s1[0], s0[1], s1[1]};
          const int tr = wm * (TM / 2) + mt * 16 + li, col = col_s + nt * 16;
          if (tr < rows && col < p.N) *reinterpret_cast<u32x4*>(p.y + (int64_t)(row0 + tr) * p.N + col) = v;
        }
    }
  }
}

// Grouped GEMM over all three block classes in one persistent launch. Workgroups claim work items from
// a ticket counter; the claim order spreads the 256-row items (large experts, MFMA-bound) evenly
// among the 128- and 64-row items (small experts, bound by their weight stream), so at any time some
// CUs run each kind and the two overlap instead of running one after the other. Within a class the
// items run block by block (a block's weight tiles on consecutive tickets), so the re-reads of a
// block's A rows, and of a weight tile by the next block of the same expert, follow within a few
// microseconds, while the memory-side cache still holds them (the tile-major order put a block's
// tiles a whole class apart: T=4096 on Zipf(1.1) routing 3.226 -> 3.110 ms, T=1024 2.207 -> 2.146,
// T=64 1.125 -> 1.106, bitwise the same outputs; one queue per XCD measured 3.370 ms at T=4096). A
// workgroup leaves once its ticket is past the last item.
template <int MODE, bool PRE>
__global__ __launch_bounds__(512) void moe_gemm_kernel(MoeGemmArgs p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kMoeSmemBytes];
  __shared__ int ticket;
  const int tn = p.tiles_n;
  const int n0 = p.nblk[0], n1 = p.nblk[1], n2 = p.nblk[2];
  const int heavy = n0 * tn, c1 = n1 * tn, items = heavy + c1 + n2 * tn;
  for (;;) {
    __syncthreads();  // every wave is done with the previous item's LDS and has read the ticket
    if (threadIdx.x == 0) ticket = atomicAdd(p.tickets, 1);
    __syncthreads();
    const int t = ticket;
    if (t >= items) break;
    const int hk = (int)((int64_t)t * heavy / items);  // 256-row items before ticket t
    if ((int64_t)(t + 1) * heavy / items > hk) {
      moe_item<MODE, PRE, 256>(p, smem, 0, hk / tn, hk % tn);
    } else {
      const int i = t - hk;
      if (i < c1)
        moe_item<MODE, PRE, 128>(p, smem, 1, i / tn, i % tn);
      else
        moe_item<MODE, PRE, 64>(p, smem, 2, (i - c1) / tn, (i - c1) % tn);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// combine: out[t] = bf16(sum over slots in slot order of weight * y[row]); 8 columns per thread.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y, const int32_t* __restrict__ row_of,
                                                      const float* __restrict__ weights, int S, int D,
                                                      uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  for (int c0 = threadIdx.x * 8; c0 < D; c0 += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < S; ++s) {
      const int row = row_of[(int64_t)t * S + s];
      if (row < 0) continue;
      const float wt = weights[(int64_t)t * S + s];
      const u32x4 v = ld16(y + (int64_t)row * D + c0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = fmaf(wt, bf16_lo(v[i]), acc[2 * i]);
        acc[2 * i + 1] = fmaf(wt, bf16_hi(v[i]), acc[2 * i + 1]);
      }
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(acc[2 * i], acc[2 * i + 1]);
    *reinterpret_cast<u32x4*>(out + (int64_t)t * D + c0) = o;
  }
}

// ---------------------------------------------------------------------------------------------
// host side
struct Workspace {
  size_t logits, ids, weights, row_of, sorted_tok, blk_expert, blk_row, blk_rows, nblk, tickets, xq, xs, hq, hs, y,
      total;
  int blk_cap;  // block-table entries per class
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Scratch layout for T tokens, S slots, model dim D, intermediate I, E expert slots, Er router rows
// (0: no router scratch).
static Workspace layout(int64_t T, int64_t S, int64_t D, int64_t I, int64_t E, int64_t Er) {
  Workspace w{};
  const int64_t R = T * S;
  const int64_t cap = R / kMinTM + E + 1;
  const int64_t maxblk = cap * kClasses;
  w.blk_cap = (int)cap;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  w.logits = take((size_t)(T * Er * 2));
  w.ids = take((size_t)(Er ? R * 4 : 0));
  w.weights = take((size_t)(Er ? R * 4 : 0));
  w.row_of = take((size_t)R * 4);
  w.sorted_tok = take((size_t)R * 4);
  w.blk_expert = take((size_t)maxblk * 4);
  w.blk_row = take((size_t)maxblk * 4);
  w.blk_rows = take((size_t)maxblk * 4);
  w.nblk = take(4 * kClasses);
  w.tickets = take(4 * 2);
  w.xq = take((size_t)(T * D));
  w.xs = take((size_t)(D / 128 * T * 4));
  w.hq = take((size_t)(R * I));
  w.hs = take((size_t)(I / 128 * R * 4));
  w.y = take((size_t)(R * D * 2));
  w.total = o;
  return w;
}

// The persistent grid: one workgroup per CU of the current device (the runtime answers from its
// device table; nothing is kept between calls).
static int num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

static bool dims_ok(int64_t T, int64_t D, int64_t I, int64_t E, int64_t S) {
  if (T <= 0 || T > 65536 || D < 128 || D > 16384 || D % 128 || I < 128 || I > 16384 || I % 128) return false;
  if (E < 1 || E > kMaxExperts || S < 1 || S > 64) return false;
  const int64_t R = T * S;
  // 32-bit offsets: activations, h, y and a row's scales stay below 2 GiB
  return R * D * 2 < 0x7FFFFFFFll && R * I < 0x7FFFFFFFll && T * D < 0x7FFFFFFFll;
}

template <bool PRE>
static void launch_gemms(const MoeGemmArgs& gu, const MoeGemmArgs& dn, hipStream_t stream) {
  const dim3 grid((unsigned)num_cus());
  hipLaunchKernelGGL((moe_gemm_kernel<kGateUp, PRE>), grid, dim3(512), 0, stream, gu);
  hipLaunchKernelGGL((moe_gemm_kernel<kDown, PRE>), grid, dim3(512), 0, stream, dn);
}

// Experts on a routing already in ids/weights ([T, S], slots in [0, E); others are skipped).
static int run_experts(const uint16_t* hidden, int64_t T, int64_t D, int64_t I, int64_t E, const int32_t* ids,
                       const float* weights, int64_t S, const uint8_t* w1, const float* w1s, const uint8_t* w2,
                       const float* w2s, int w_layout, uint16_t* out, uint8_t* ws, const Workspace& L,
                       hipStream_t stream) {
  const int64_t R = T * S;
  int32_t* row_of = reinterpret_cast<int32_t*>(ws + L.row_of);
  int32_t* sorted_tok = reinterpret_cast<int32_t*>(ws + L.sorted_tok);
  BlockTable bt;
  bt.expert = reinterpret_cast<int32_t*>(ws + L.blk_expert);
  bt.row = reinterpret_cast<int32_t*>(ws + L.blk_row);
  bt.rows = reinterpret_cast<int32_t*>(ws + L.blk_rows);
  bt.count = reinterpret_cast<int32_t*>(ws + L.nblk);
  bt.cap = L.blk_cap;
  uint8_t* xq = ws + L.xq;
  float* xs = reinterpret_cast<float*>(ws + L.xs);
  uint8_t* hq = ws + L.hq;
  float* hs = reinterpret_cast<float*>(ws + L.hs);
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + L.y);
  int* tickets = reinterpret_cast<int*>(ws + L.tickets);

  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(1024), 0, stream, ids, (int)R, (int)S, (int)E, row_of, sorted_tok, bt,
                     tickets);
  const int64_t qgroups = T * (D / 128);
  hipLaunchKernelGGL(quant_div_kernel, dim3((unsigned)((qgroups + 15) / 16)), dim3(256), 0, stream, hidden, (int)T,
                     (int)D, xq, xs);
  MoeGemmArgs gu{};
  gu.a = xq;
  gu.sa = xs;
  gu.sa_ld = T;
  gu.sorted_tok = sorted_tok;
  gu.b = w1;
  gu.b_stride = 2 * I * D;
  gu.sb = w1s;
  gu.sb_stride = (2 * I / 128) * (D / 128);
  gu.K = (int)D;
  gu.N = (int)(2 * I);
  gu.I = (int)I;
  gu.tiles_n = (int)(I / 128);
  gu.hq = hq;
  gu.hs = hs;
  gu.R = R;
  gu.blk_expert = bt.expert;
  gu.blk_row = bt.row;
  gu.blk_rows = bt.rows;
  gu.nblk = bt.count;
  gu.blk_cap = bt.cap;
  gu.tickets = tickets;
  MoeGemmArgs dn = gu;
  dn.a = hq;
  dn.sa = hs;
  dn.sa_ld = R;
  dn.sorted_tok = nullptr;
  dn.b = w2;
  dn.b_stride = D * I;
  dn.sb = w2s;
  dn.sb_stride = ((D + 127) / 128) * (I / 128);
  dn.K = (int)I;
  dn.N = (int)D;
  dn.tiles_n = (int)((D + kTN - 1) / kTN);
  dn.y = y;
  dn.tickets = tickets + 1;
  if (w_layout == AKLR_B_PRESHUFFLE_16x16)
    launch_gemms<true>(gu, dn, stream);
  else
    launch_gemms<false>(gu, dn, stream);
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)T), dim3(256), 0, stream, y, row_of, weights, (int)S, (int)D, out);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

}  // namespace moe
}  // namespace aklr

using namespace aklr;
using namespace aklr::moe;

extern "C" size_t aklr_moe_fp8_workspace_bytes(int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t n_experts,
                                               int64_t slots, int64_t n_router_rows) {
  if (!dims_ok(tokens, model_dim, inter_dim, n_experts, slots) || n_router_rows < 0) return 0;
  return layout(tokens, slots, model_dim, inter_dim, n_experts, n_router_rows).total;
}

extern "C" int aklr_moe_fp8_route(const void* logits, const void* bias, int64_t tokens, int64_t n_routed, int topk,
                                  int num_expert_group, int topk_group, int renormalize, float routed_scaling_factor,
                                  int append_shared, int32_t* ids, float* weights, hipStream_t stream) {
  if (!logits || !bias || !ids || !weights) return AKLR_ERR_INVALID_ARGUMENT;
  if (tokens <= 0 || tokens > 65536 || n_routed < 2 || n_routed > 1024) return AKLR_ERR_INVALID_ARGUMENT;
  if (num_expert_group < 1 || num_expert_group > 64 || n_routed % num_expert_group) return AKLR_ERR_INVALID_ARGUMENT;
  if (n_routed / num_expert_group < 2 || topk_group < 1 || topk_group > num_expert_group) return AKLR_ERR_INVALID_ARGUMENT;
  if (topk < 1 || topk > 63 || topk > topk_group * (n_routed / num_expert_group)) return AKLR_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(route_kernel, dim3((unsigned)tokens), dim3(64), 0, stream, static_cast<const uint16_t*>(logits),
                     static_cast<const uint16_t*>(bias), (int)tokens, (int)n_routed, num_expert_group, topk, topk_group,
                     renormalize ? 1 : 0, routed_scaling_factor, append_shared ? 1 : 0, ids, weights);
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

extern "C" int aklr_moe_fp8_experts(const void* hidden, int64_t tokens, int64_t model_dim, int64_t inter_dim,
                                    int64_t n_experts, const int32_t* ids, const float* weights, int64_t slots,
                                    const void* w1, const float* w1_scale, const void* w2, const float* w2_scale,
                                    int w_layout, void* out, void* workspace, size_t workspace_bytes,
                                    hipStream_t stream) {
  if (!hidden || !ids || !weights || !w1 || !w1_scale || !w2 || !w2_scale || !out) return AKLR_ERR_INVALID_ARGUMENT;
  if (!dims_ok(tokens, model_dim, inter_dim, n_experts, slots)) return AKLR_ERR_INVALID_ARGUMENT;
  if (w_layout != AKLR_B_ROW_MAJOR && w_layout != AKLR_B_PRESHUFFLE_16x16) return AKLR_ERR_UNSUPPORTED;
  if (!aklr_aligned16(hidden) || !aklr_aligned16(w1) || !aklr_aligned16(w2) || !aklr_aligned16(out))
    return AKLR_ERR_INVALID_ARGUMENT;
  const Workspace L = layout(tokens, slots, model_dim, inter_dim, n_experts, 0);
  if (!workspace || workspace_bytes < L.total || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
  return run_experts(static_cast<const uint16_t*>(hidden), tokens, model_dim, inter_dim, n_experts, ids, weights, slots,
                     static_cast<const uint8_t*>(w1), w1_scale, static_cast<const uint8_t*>(w2), w2_scale, w_layout,
                     static_cast<uint16_t*>(out), static_cast<uint8_t*>(workspace), L, stream);
}

extern "C" int aklr_deepseek_v2_fp8_moe(const void* hidden, const void* router_weight, const void* correction_bias,
                                        const void* w1, const float* w1_scale, const void* w2, const float* w2_scale,
                                        int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t n_routed,
                                        int topk, int num_expert_group, int topk_group, int renormalize,
                                        float routed_scaling_factor, int w_layout, void* out, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream) {
  if (!hidden || !router_weight || !correction_bias || !w1 || !w1_scale || !w2 || !w2_scale || !out)
    return AKLR_ERR_INVALID_ARGUMENT;
  if (n_routed < 2 || n_routed > 1024 || topk < 1 || topk > 63) return AKLR_ERR_INVALID_ARGUMENT;
  const int64_t S = topk + 1, E = n_routed + 1;
  if (!dims_ok(tokens, model_dim, inter_dim, E, S)) return AKLR_ERR_INVALID_ARGUMENT;
  if (w_layout != AKLR_B_ROW_MAJOR && w_layout != AKLR_B_PRESHUFFLE_16x16) return AKLR_ERR_UNSUPPORTED;
  if (!aklr_aligned16(hidden) || !aklr_aligned16(router_weight) || !aklr_aligned16(w1) || !aklr_aligned16(w2) ||
      !aklr_aligned16(out))
    return AKLR_ERR_INVALID_ARGUMENT;
  const Workspace L = layout(tokens, S, model_dim, inter_dim, E, n_routed);
  if (!workspace || workspace_bytes < L.total || !aklr_aligned16(workspace)) return AKLR_ERR_WORKSPACE;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* logits = reinterpret_cast<uint16_t*>(ws + L.logits);
  int32_t* ids = reinterpret_cast<int32_t*>(ws + L.ids);
  float* weights = reinterpret_cast<float*>(ws + L.weights);
  const int nt = tokens >= 1024 ? 4 : 1;
  const int64_t waves = ((tokens + 15) / 16) * ((n_routed + 16 * nt - 1) / (16 * nt));
  if (nt == 4)
    hipLaunchKernelGGL((router_kernel<4>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(router_weight), logits,
                       (int)tokens, (int)n_routed, (int)model_dim);
  else
    hipLaunchKernelGGL((router_kernel<1>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(router_weight), logits,
                       (int)tokens, (int)n_routed, (int)model_dim);
  const int st = aklr_moe_fp8_route(logits, correction_bias, tokens, n_routed, topk, num_expert_group, topk_group,
                                    renormalize, routed_scaling_factor, 1, ids, weights, stream);
  if (st != AKLR_OK) return st;
  return run_experts(static_cast<const uint16_t*>(hidden), tokens, model_dim, inter_dim, E, ids, weights, S,
                     static_cast<const uint8_t*>(w1), w1_scale, static_cast<const uint8_t*>(w2), w2_scale, w_layout,
                     static_cast<uint16_t*>(out), ws, L, stream);
}

AKLR_SCALAR_FP32_END
