// moe_probe.hip - the sustainable HBM read rate of this device.
//
// Decode streams weights and writes almost nothing, so a device copy (read +
// write) is not its roof.  This kernel only reads: each lane keeps UNROLL
// independent 16-byte loads in flight per step of a grid-stride walk over the
// buffer, folds them with xor, and stores the fold only when all 128 bits of
// it are ones (2^-128 per lane for random data), so the loads cannot be
// dropped and in practice nothing is written.  The caller fills the buffer
// with random bytes: a uniform fill could be served faster than real data.
#include "moe_common.h"
#include "moe_internal.h"

namespace {

template <int UNROLL>
__global__ __launch_bounds__(256) void k_read_probe(const uint4 *__restrict__ buf, uint64_t n16,
                                                    uint4 *__restrict__ sink) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  uint4 acc = make_uint4(0, 0, 0, 0);
  for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
    uint4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = buf[i + u * stride];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      acc.x ^= v[u].x; acc.y ^= v[u].y; acc.z ^= v[u].z; acc.w ^= v[u].w;
    }
  }
  for (; i < n16; i += stride) {
    const uint4 v = buf[i];
    acc.x ^= v.x; acc.y ^= v.y; acc.z ^= v.z; acc.w ^= v.w;
  }
  if ((acc.x & acc.y & acc.z & acc.w) == 0xFFFFFFFFu)
    sink[0] = acc;
}

}  // namespace

extern "C" int ainfer_moe_read_probe(const void *buf, uint64_t bytes, int32_t unroll,
                                     int32_t blocks_per_cu, int32_t iters, void *stream,
                                     float *gbs) {
  if (!buf || !gbs || bytes < 16 || (bytes & 15) || ((uintptr_t)buf & 15) || iters <= 0 ||
      iters > 1000 || blocks_per_cu < 1 || blocks_per_cu > 64)
    return AINFER_ERR_ARG;
  if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8 && unroll != 16) return AINFER_ERR_ARG;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return AINFER_ERR_HIP;
  const hipStream_t s = (hipStream_t)stream;
  const uint4 *p = (const uint4 *)buf;
  const uint64_t n16 = bytes / 16;
  const dim3 grid((unsigned)(cus * blocks_per_cu)), block(256);
  // the sink is the probe buffer's own first 16 bytes
  uint4 *sink = (uint4 *)buf;
  auto launch = [&]() {
    switch (unroll) {
      case 1: k_read_probe<1><<<grid, block, 0, s>>>(p, n16, sink); break;
      case 2: k_read_probe<2><<<grid, block, 0, s>>>(p, n16, sink); break;
      case 4: k_read_probe<4><<<grid, block, 0, s>>>(p, n16, sink); break;
      case 8: k_read_probe<8><<<grid, block, 0, s>>>(p, n16, sink); break;
      default: k_read_probe<16><<<grid, block, 0, s>>>(p, n16, sink); break;
    }
  };
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return AINFER_ERR_HIP;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return AINFER_ERR_HIP;
  }
  int rc = AINFER_OK;
  float ms = 0.f;
  launch();
  if (hipEventRecord(e0, s) != hipSuccess) rc = AINFER_ERR_HIP;
  for (int it = 0; rc == AINFER_OK && it < iters; ++it) launch();
  if (rc != AINFER_OK || hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
      hipEventElapsedTime(&ms, e0, e1) != hipSuccess || hipGetLastError() != hipSuccess)
    rc = AINFER_ERR_HIP;
  else
    *gbs = (float)((double)bytes * iters / (ms * 1e-3) / 1e9);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}
