// Calibration kernel for the decode roofline: a pure HBM stream read with the decode GEMM's access
// pattern (16-byte non-temporal loads, several per lane in flight), and nothing else. Timed back to
// back like the GEMMs, it gives the floor a kernel that reads N bytes cannot beat on this GPU: launch,
// first-load latency and the stream itself. The loads are folded into one word per lane that is
// compared against a constant, so nothing is written unless the data happen to match it.
#include "common.h"

AKLR_SCALAR_FP32_BEGIN

namespace aklr {

template <int U>
__global__ __launch_bounds__(256) void probe_read_kernel(const uint8_t* src, int64_t bytes, uint32_t* sink) {
  // each workgroup one contiguous chunk; loads past the chunk (or past the buffer) are out of the
  // descriptor's range: they return zeros and touch no memory
  const int64_t per_wg = ((bytes + gridDim.x - 1) / gridDim.x + 15) & ~(int64_t)15;
  const int64_t start = (int64_t)blockIdx.x * per_wg;
  const int64_t mine = start < bytes ? (bytes - start < per_wg ? bytes - start : per_wg) : 0;
  const uint8_t* base = src + (start < bytes ? start : 0);
  const rsrc_t r = make_rsrc(base, rsrc_bytes(mine));
  uint32_t acc = 0;
  for (int64_t off = 0; off < mine; off += 256 * 16 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = buf_ld16<kNt>(r, (uint32_t)(off + (u * 256 + threadIdx.x) * 16));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x * 256 + threadIdx.x] = acc;
}

}  // namespace aklr

extern "C" int aklr_probe_hbm_read(const void* src, int64_t bytes, uint32_t* sink, int workgroups, int unroll,
                                   hipStream_t stream) {
  using namespace aklr;
  if (!src || !sink || bytes < 0 || workgroups < 1 || workgroups > 65536) return AKLR_ERR_INVALID_ARGUMENT;
  if (!aklr_aligned16(src) || bytes / workgroups + 16 > 0x7FFFFFFFll - 256 * 16 * 8) return AKLR_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)workgroups), block(256);
  if (unroll == 4) hipLaunchKernelGGL(probe_read_kernel<4>, grid, block, 0, stream, static_cast<const uint8_t*>(src), bytes, sink);
  else if (unroll == 8) hipLaunchKernelGGL(probe_read_kernel<8>, grid, block, 0, stream, static_cast<const uint8_t*>(src), bytes, sink);
  else return AKLR_ERR_UNSUPPORTED;
  AKLR_LAUNCH_CHECK();
  return AKLR_OK;
}

AKLR_SCALAR_FP32_END
