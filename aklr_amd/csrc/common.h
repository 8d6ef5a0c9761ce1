// Device helpers shared by the gfx950 kernels of this library: element conversions, MFMA atoms,
// workgroup-id remapping. gfx950 (CDNA4) only; 64-wide wavefronts.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/aklr_amd.h"

// Packed fp32 VALU instructions (v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32) are switched off for all
// device code of this library, in the source, so that every build of these files -- this library's
// own, and an AKLR schema package built with AKLR's plain -O3 -- keeps the fp32 arithmetic scalar per
// lane. Each kernel source opens AKLR_SCALAR_FP32_BEGIN after its includes and closes
// AKLR_SCALAR_FP32_END at its end (a clang attribute push must be popped in the same file).
#if defined(__HIP_DEVICE_COMPILE__)
#define AKLR_SCALAR_FP32_BEGIN \
  _Pragma("clang attribute push (__attribute__((target(\"no-packed-fp32-ops\"))), apply_to = function)")
#define AKLR_SCALAR_FP32_END _Pragma("clang attribute pop")
#else
#define AKLR_SCALAR_FP32_BEGIN
#define AKLR_SCALAR_FP32_END
#endif

AKLR_SCALAR_FP32_BEGIN

namespace aklr {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16-byte loads: plain (cached) and non-temporal (streamed once, kept out of the caches' way).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Raw buffer loads. A descriptor covers `bytes` from `base`; a load whose 32-bit offset is at or past
// `bytes` returns zeros and touches no memory, so an offset of kOobOffset switches a load off without
// a branch. kNt marks a stream that is read once (non-temporal).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOobOffset = 0x80000000u;
constexpr int kNt = 2;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
template <int AUX = 0>
__device__ __forceinline__ u32x4 buf_ld16(rsrc_t r, uint32_t voffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, 0, AUX));
}

// Direct-to-LDS buffer loads: lane i of the wave writes its 16 (or 4) bytes at lds + i * 16 (i * 4), so
// the LDS placement is fixed by the lane and the global address each lane picks sets the layout.
// An out-of-range offset (kOobOffset) reads zeros.
typedef __attribute__((address_space(3))) void lds_void;
// The same 16-byte direct-to-LDS load issued from inline assembly, with a descriptor built by
// make_rsrc_words. The compiler's wait-count pass does not see it, so it adds no conservative wait
// before later LDS reads of other buffers; the caller waits (s_waitcnt vmcnt) and synchronises
// itself before reading what it loaded. `lds` must be wave-uniform. The statement declares no memory
// clobber, so loads of read-only kernel inputs after it can still go through the scalar unit;
// callers order it against LDS reads with barriers.
__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xFFFFu);
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void lds_dma16(const i32x4& rsrc, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(voffset), "s"(rsrc)
               : "m0");
}
__device__ __forceinline__ void lds_dma4(const i32x4& rsrc, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(lds), "v"(voffset), "s"(rsrc)
               : "m0");
}

// The same loads with the K advance in soffset: the per-lane voffset stays fixed across a loop, so
// issuing a stage costs no vector instructions. A descriptor whose byte count is 0 reads zeros.
__device__ __forceinline__ void lds_dma16_so(const i32x4& rsrc, uint32_t lds, uint32_t voffset, uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voffset), "s"(rsrc),
               "s"(soffset)
               : "m0");
}
__device__ __forceinline__ void lds_dma4_so(const i32x4& rsrc, uint32_t lds, uint32_t voffset, uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(lds), "v"(voffset), "s"(rsrc),
               "s"(soffset)
               : "m0");
}

// Compile-time loop: SFor<0, N>::run(f) calls f(IC<0>{}), ..., f(IC<N - 1>{}), so a generic lambda
// sees its index as a constant (decltype(i)::value).
template <int V>
struct IC {
  static constexpr int value = V;
};
template <int I, int N>
struct SFor {
  template <typename F>
  __device__ __forceinline__ static void run(F& f) {
    f(IC<I>{});
    SFor<I + 1, N>::run(f);
  }
};
template <int N>
struct SFor<N, N> {
  template <typename F>
  __device__ __forceinline__ static void run(F&) {}
};

__device__ __forceinline__ void buf_ld_lds16(rsrc_t r, void* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, (int)voffset, 0, 0, 0);
}
__device__ __forceinline__ void buf_ld_lds4(rsrc_t r, void* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 4, (int)voffset, 0, 0, 0);
}

// Byte extent for a buffer descriptor, clamped to the 31-bit range raw buffer offsets address.
__device__ __forceinline__ uint32_t rsrc_bytes(int64_t bytes) {
  return (uint32_t)(bytes > 0x7FFFFFFFll ? 0x7FFFFFFFll : (bytes < 0 ? 0 : bytes));
}

// Workgroup barrier fenced for LDS only (s_waitcnt lgkmcnt(0) + s_barrier): global loads in flight,
// such as a register ring of weight tiles, stay in flight across it.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// fl32(1/448) = 0x3B124925 (0x1.24924ap-9): the e4m3fn quantizer multiplies amax by this constant
// (it does not divide by 448).
constexpr float kInv448 = 0x1.24924ap-9f;
constexpr float kAmaxFloor = 1e-10f;

// v read from another lane of the same 16-lane row through a DPP control (quad_perm, row_mirror, ...).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// fp32 -> bf16, round to nearest even, with gfx950's V_CVT_PK_BF16_F32 (one instruction for two
// values). On every finite fp32 input, denormals and overflow to infinity included, it gives the
// bits of the integer rule u + 0x7FFF + ((u >> 16) & 1) >> 16 (checked over all 2^32 patterns on an
// MI355X); a NaN stays a NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));  // a in the low half
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack_bf16x2(f, 0.0f) & 0xFFFFu; }

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Four floats -> four e4m3fn bytes (OCP fp8 on gfx950), round to nearest even, byte 0 = a.
// Callers clamp to +-448 first, so the conversion's overflow rule never applies.
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// Workgroup-id remap: the hardware hands consecutive workgroup ids round-robin to the 8 XCDs, so
// id -> (id % 8) * per_xcd + id / 8 makes consecutive *logical* ids land on one XCD (one L2).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t id, uint32_t total) {
  constexpr uint32_t kXcd = 8;
  if (total < kXcd || (total % kXcd) != 0) return id;
  return (id % kXcd) * (total / kXcd) + id / kXcd;
}
// The same for any total: XCD x receives ids x, x + 8, ..., one more of them for x < total % 8, and its
// logical ids are one consecutive range.
__device__ __forceinline__ uint32_t xcd_remap_any(uint32_t id, uint32_t total) {
  constexpr uint32_t kXcd = 8;
  const uint32_t q = total / kXcd, r = total % kXcd, x = id % kXcd;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + id / kXcd;
}

// Two 16-byte halves -> one 32-byte MFMA operand (lo = bytes 0-15).
__device__ __forceinline__ i32x8 cat(const u32x4& lo, const u32x4& hi) {
  i32x8 r;
  r[0] = (int)lo[0]; r[1] = (int)lo[1]; r[2] = (int)lo[2]; r[3] = (int)lo[3];
  r[4] = (int)hi[0]; r[5] = (int)hi[1]; r[6] = (int)hi[2]; r[7] = (int)hi[3];
  return r;
}

// 16x16x128 F8F6F4 MFMA. FMT: 0 e4m3, 1 e5m2, 4 e2m1 (both operands). Scale bytes are e8m0;
// 127 is 1.0. D[i][j] for i = 4*(lane/16) + r, j = lane % 16.
template <int FMT>
__device__ __forceinline__ f32x4 mfma16x128(const i32x8& a, const i32x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT, FMT, 0, 127, 0, 127);
}

template <int FMT, int OPSEL_A, int OPSEL_B>
__device__ __forceinline__ f32x4 mfma16x128_scaled(const i32x8& a, const i32x8& b, const f32x4& c, int sa,
                                                    int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT, FMT, OPSEL_A, sa, OPSEL_B, sb);
}

__device__ __forceinline__ void store_out(void* out, int64_t idx, float v, int out_dtype) {
  if (out_dtype == AKLR_OUT_BF16)
    reinterpret_cast<uint16_t*>(out)[idx] = (uint16_t)f32_to_bf16_bits(v);
  else
    reinterpret_cast<uint16_t*>(out)[idx] = (uint16_t)f32_to_f16_bits(v);
}

// Two outputs -> one word of two bf16 / fp16 values (a in the low half).
__device__ __forceinline__ uint32_t pack_out2(float a, float b, int out_dtype) {
  return out_dtype == AKLR_OUT_BF16 ? pack_bf16x2(a, b) : (f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16));
}

// Output tile store through LDS, for a 512-thread workgroup whose LDS operand ring is free. The
// TM x TN tile is held as 16x16 fp32 accumulators by a WM x WN grid of waves: wave (wm, wn), fragment
// (mt, nt), lane (li = lane & 15, g = lane >> 4) holds row wm * (TM / WM) + mt * 16 + li, columns
// wn * (TN / WN) + nt * 16 + 4g .. + 3. Rows [0, TM/2) are packed (bias added) into `lo` and rows
// [TM/2, TM) into `hi`, as rows of TN * 2 bytes; then each thread moves 16-byte chunks to memory, so
// that a wave stores 1 KiB of whole tile rows (full 128-byte lines) per instruction, where a lane's
// own fragments would store two 64-byte halves of each line from two instructions. nt_store selects
// non-temporal stores. n % 16 == 0.
//
// LDS banks: a 16-byte access serves 8 lanes per 128 bytes of banks. For the writes, permlane16_swap
// pairs column tiles (nt, nt + 1) so that lane group g holds 8 columns of tile nt + (g & 1); 8 lanes
// then write one chunk column of 8 consecutive rows. Chunk c of row r sits at c ^ swz(r): with a row
// pitch of 0 mod 8 chunks (TN = 128, 192, 256) swz(r) = r & 7, with 4 mod 8 (TN = 224: 28 chunks)
// swz(r) = (r >> 1) & 3, which puts 8 consecutive rows of one chunk column on 8 different 16-byte
// bank groups, and keeps the 8 chunks a read phase takes from one row on 8 different ones.
template <int TM, int TN, int WM, int WN, int MT, int NT>
__device__ __forceinline__ void store_tile_via_lds(const f32x4 (&acc)[MT][NT], uint8_t* lo, uint8_t* hi, int wm,
                                                   int wn, int m0, int n0, int m, int n, void* out, int64_t ldo,
                                                   const float* bias, int out_dtype, bool nt_store) {
  constexpr int kCpr = TN / 8;  // 16-byte chunks per tile row
  constexpr int kHalfRows = TM / 2;
  static_assert(MT * 16 * WM == TM && NT * 16 * WN == TN && WM % 2 == 0, "wave grid");
  static_assert(kCpr % 8 == 0 || kCpr % 8 == 4, "row pitch in chunks");
  auto at = [](int r, int c) {  // byte offset of chunk c of row r within a half
    return r * (TN * 2) + (c ^ (kCpr % 8 == 0 ? (r & 7) : ((r >> 1) & 3))) * 16;
  };
  const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  __syncthreads();  // every wave's last operand reads are done
  {
    uint8_t* const half = wm < WM / 2 ? lo : hi;
    const int r0 = (wm % (WM / 2)) * (TM / WM) + li;  // + mt * 16: the lane's row within its half
    const int c0 = wn * (TN / WN) / 8;               // the wave's first chunk column
    const int col_w = n0 + wn * (TN / WN) + 4 * g;   // + nt * 16: the lane's first output column
    auto load_bias = [&](int nt) {
      f32x4 b = {0.f, 0.f, 0.f, 0.f};
      if (bias) {
        const int cx = min(col_w + nt * 16, n - 4);  // columns past n are computed, never stored
#pragma unroll
        for (int r = 0; r < 4; ++r) b[r] = bias[cx + r];
      }
      return b;
    };
#pragma unroll
    for (int nt = 0; nt + 1 < NT; nt += 2) {
      const f32x4 bx = load_bias(nt), by = load_bias(nt + 1);
      const int c = c0 + (nt + (g & 1)) * 2 + (g >> 1);  // lane group g: 8 columns of tile nt + (g & 1)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const f32x4 x = acc[mt][nt] + bx, y = acc[mt][nt + 1] + by;
        const uint32_t x0 = pack_out2(x[0], x[1], out_dtype), x1 = pack_out2(x[2], x[3], out_dtype);
        const uint32_t y0 = pack_out2(y[0], y[1], out_dtype), y1 = pack_out2(y[2], y[3], out_dtype);
        const auto s0 = __builtin_amdgcn_permlane16_swap(x0, y0, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(x1, y1, false, false);
        *reinterpret_cast<u32x4*>(half + at(r0 + mt * 16, c)) = u32x4{s0[0], s1[0], s0[1], s1[1]};
      }
    }
    if constexpr (NT % 2 == 1) {  // the odd last column tile: 8 bytes per lane
      constexpr int nt = NT - 1;
      const f32x4 bx = load_bias(nt);
      const int c = c0 + nt * 2 + (g >> 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const f32x4 x = acc[mt][nt] + bx;
        const u32x2 v = {pack_out2(x[0], x[1], out_dtype), pack_out2(x[2], x[3], out_dtype)};
        *reinterpret_cast<u32x2*>(half + at(r0 + mt * 16, c) + (g & 1) * 8) = v;
      }
    }
  }
  __syncthreads();
  // passes of 512 threads over each half; the last one partial when the half is not a whole number of
  // them (192-row tiles)
  constexpr int kHalfChunks = kHalfRows * kCpr, kHalfIters = (kHalfChunks + 511) / 512;
  auto store_rows = [&](auto nt_c) {
#pragma unroll
    for (int it = 0; it < 2 * kHalfIters; ++it) {
      const int idx = (it % kHalfIters) * 512 + (int)threadIdx.x;
      if (kHalfChunks % 512 != 0 && idx >= kHalfChunks) continue;
      const int r = idx / kCpr, ch = idx % kCpr;
      const uint8_t* const half = it < kHalfIters ? lo : hi;
      const u32x4 v = *reinterpret_cast<const u32x4*>(half + at(r, ch));
      const int row = m0 + (it < kHalfIters ? 0 : kHalfRows) + r, col = n0 + ch * 8;
      if (row < m && col < n) {  // n % 16 == 0: a chunk is wholly inside or past n
        u32x4* const dst = reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(out) + (int64_t)row * ldo + col);
        if constexpr (decltype(nt_c)::value)
          __builtin_nontemporal_store(v, dst);
        else
          *dst = v;
      }
    }
  };
  if (nt_store)
    store_rows(IC<1>{});
  else
    store_rows(IC<0>{});
}

// Split-K partials: layout [split][col][m4] fp32 with m4 = m rounded up to 4, so a lane's 4 rows of
// one column (an MFMA 16x16 accumulator's rows 4g..4g+3) are one 16-byte access and a wave's
// accesses are contiguous runs. They travel through device-coherent (sc1) buffer accesses, which go
// past the XCD-local caches to the memory-side coherence point without the whole-L2 write-back /
// invalidate that an agent-scope fence costs. One descriptor per split (a split's plane is < 4 GiB).
constexpr int kSc1 = 16;
__device__ __forceinline__ rsrc_t partial_rsrc(float* partial, int split, int64_t plane) {
  return make_rsrc(partial + (int64_t)split * plane, (uint32_t)(plane * 4));
}
__device__ __forceinline__ void store_partial4(rsrc_t r, int64_t elem, const f32x4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, (int)(elem * 4), 0, kSc1);
}
__device__ __forceinline__ f32x4 load_partial4(rsrc_t r, int64_t elem) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(elem * 4), 0, kSc1));
}
__host__ __device__ inline int64_t round4(int64_t m) { return (m + 3) / 4 * 4; }

// Split-K arrival words. One 64-bit word per output tile: bits 63..8 hold a tag of the launch, bits
// 7..0 how many of the launch's workgroups of that tile have arrived. The tag is the dispatch packet's
// id (its index in the HSA queue, new for every launch, graph replays included) xor a hash of the
// queue's address (ids of two queues count from the same start), with bit 63 set, so a word whose tag
// is not this launch's is a leftover of an earlier call, or garbage, and counts as zero arrivals. The
// workgroup that completes a tile's count writes the reserved word kWordIdle (0: bit 63 clear, so no
// launch's tag), so a word that a finished launch used never holds a tag that a later launch could
// produce again (a queue made again at the same address restarts its dispatch ids); only words of a
// launch that did not finish, or never-used memory, rely on the tag. No call depends on what the
// workspace held before it; calls that may run at the same time need their own workspace.
extern "C" __device__ uint64_t aklr_dispatch_id() __asm("llvm.amdgcn.dispatch.id");
constexpr uint64_t kTagMask = ~(uint64_t)0xFF;
constexpr uint64_t kWordIdle = 0;
__device__ __forceinline__ uint64_t launch_tag() {
  const uint64_t q = (uint64_t)(uintptr_t)__builtin_amdgcn_queue_ptr();
  return ((aklr_dispatch_id() ^ ((q * 0x9E3779B97F4A7C15ull) >> 8)) << 8) | (1ull << 63);
}

// The tile's word as the kernel starts, read by the thread that will arrive for its workgroup (before
// that wave's other global loads, so it returns first). It is only a guess of the word's content:
// splitk_arrive claims the word with a compare-and-swap against it, issued beside the partial
// stores, and falls back to the value the swap returns.
__device__ __forceinline__ uint64_t splitk_peek(const uint64_t* word) {
  return __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K arrival. Each workgroup of an output tile stores its fp32 partial with store_partial4,
// then calls this (every thread of the workgroup). Thread `arriver` first claims the tile's word
// for this launch -- a stale word becomes (tag, 0) by a compare-and-swap, which fails harmlessly
// when another workgroup of the launch got there first -- in flight together with the partial
// stores; once those are acknowledged it adds one arrival, and the workgroup that brings the count
// to `splits` returns true. That one owns the reduction, which it reads with load_partial4 and sums
// in split order, so the result does not depend on the arrival order. The arrival that completes the
// count stores kWordIdle (no workgroup of the launch touches the word after it). `seen` is
// splitk_peek's value (meaningful in the arriver only); `slot` is the workgroup's LDS word for the
// broadcast.
__device__ __forceinline__ bool splitk_arrive(uint64_t* word, uint64_t seen, int splits, unsigned* slot,
                                              unsigned arriver = 0) {
  const uint64_t tag = launch_tag();
  uint64_t cur = seen;
  bool claimed = (seen & kTagMask) == tag;
  if (threadIdx.x == arriver && !claimed)
    claimed = __hip_atomic_compare_exchange_strong(word, &cur, tag, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores (and the claim) are acknowledged
  __syncthreads();                // ... and every other wave's
  if (threadIdx.x == arriver) {
    // a failed swap returned the word: tagged by this launch, unless the peek was older than a value
    // no workgroup of this launch wrote (then claim again from what the swap returned). Every failed
    // swap means another workgroup's swap or add succeeded, and there are finitely many of those;
    // the bound only keeps a misuse (two launches sharing a workspace at once) from spinning.
    for (int i = 0; i < 64 && !claimed && (cur & kTagMask) != tag; ++i)
      claimed = __hip_atomic_compare_exchange_strong(word, &cur, tag, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t old = __hip_atomic_fetch_add(word, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *slot = (unsigned)(old & 0xFF);
    if ((old & 0xFF) == (uint64_t)(splits - 1))
      __hip_atomic_store(word, kWordIdle, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return *slot == (unsigned)(splits - 1);
}

// Workspace layout of the split-K GEMMs: a fixed 128 KiB region of arrival words, one per output tile
// (at most 16384: n / 16 column groups for n <= 262144, or <= 512 tiles; no initial content needed),
// then fp32 partials, each written by this call before any workgroup reads it. The region's size is
// the same for every call, so one call's partials never land on another's words.
constexpr size_t kSplitkCounterBytes = 131072;
constexpr int64_t kSplitkMaxTiles = (int64_t)(kSplitkCounterBytes / 8);
constexpr int kSplitkMaxSplits = 255;  // the count field's range

// The FP8 GEMM entry (gemm_a8w8.hip) behind aklr_gemm_a8w8_blockscale: the caller's workspace of
// workspace_bytes, or, when scratch_cap is nonzero, the device buffer `scratch` of scratch_cap bytes
// (a plan that needs more returns AKLR_ERR_SCRATCH_LIMIT and launches nothing).
int gemm8_entry(const void* a, int64_t lda, const void* b, int64_t ldb, const float* a_scale, int64_t sa_stride_m,
                int64_t sa_stride_k, const float* b_scale, int64_t ldbs, const float* bias, void* out, int64_t ldo,
                int64_t m, int64_t n, int64_t k, int fp8_dtype, int b_layout, int out_dtype, void* workspace,
                size_t workspace_bytes, void* scratch, size_t scratch_cap, hipStream_t stream);

}  // namespace aklr

AKLR_SCALAR_FP32_END

#define AKLR_LAUNCH_CHECK()                          \
  do {                                               \
    if (hipGetLastError() != hipSuccess) return AKLR_ERR_LAUNCH; \
  } while (0)

static inline bool aklr_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
