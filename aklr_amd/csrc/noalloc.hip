// No-allocation entry point of the block-scaled FP8 GEMM, for callers that cannot allocate device memory
// (code under HIP graph capture that must not call hipMalloc, tight serving loops, harnesses that forbid
// allocation). It runs exactly the kernels and plans of aklr_gemm_a8w8_blockscale; the split-K scratch
// those need (launch-tagged arrival words, then fp32 partials) lives in `scratch`, a file-scope device
// array of AKLR_NOALLOC_SCRATCH_BYTES, one copy per GPU, held until the process ends.
//
// In host code `scratch` names a host-side handle, not a device address: passing it to a kernel would
// fault. Its address on the current device comes from hipGetSymbolAddress, once per device with that
// device current, and only that pointer is handed to the kernels. The arrival words carry a tag of
// the launch, so nothing in the array needs clearing between calls (it keeps the last call's
// contents); calls that overlap in time on one GPU share the array and race.
#include "common.h"

#include <mutex>

AKLR_SCALAR_FP32_BEGIN

namespace aklr {

static __device__ __align__(256) uint8_t scratch[AKLR_NOALLOC_SCRATCH_BYTES];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_lock;
static void* g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`, looked up on its first call there.
static int scratch_on_current_device(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return AKLR_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return AKLR_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return AKLR_OK;
}

}  // namespace aklr

extern "C" int aklr_gemm_a8w8_blockscale_noalloc(const void* a, int64_t lda, const void* b, int64_t ldb,
                                                 const float* a_scale, int64_t sa_stride_m, int64_t sa_stride_k,
                                                 const float* b_scale, int64_t ldbs, const float* bias, void* out,
                                                 int64_t ldo, int64_t m, int64_t n, int64_t k, int fp8_dtype,
                                                 int b_layout, int out_dtype, hipStream_t stream) {
  void* ptr = nullptr;
  const int st = aklr::scratch_on_current_device(&ptr);
  if (st != AKLR_OK) return st;
  return aklr::gemm8_entry(a, lda, b, ldb, a_scale, sa_stride_m, sa_stride_k, b_scale, ldbs, bias, out, ldo, m, n,
                           k, fp8_dtype, b_layout, out_dtype, nullptr, 0, ptr, AKLR_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int aklr_noalloc_scratch(void** ptr, size_t* bytes) {
  if (!ptr || !bytes) return AKLR_ERR_INVALID_ARGUMENT;
  const int st = aklr::scratch_on_current_device(ptr);
  *bytes = st == AKLR_OK ? (size_t)AKLR_NOALLOC_SCRATCH_BYTES : 0;
  return st;
}

AKLR_SCALAR_FP32_END
