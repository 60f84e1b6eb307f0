// Streaming-read probe (measurement only, not part of the W4A8 path): one launch of a plain read
// kernel over `bytes` bytes, the floor the decode GEMV's per-call times are read against
// (bench.py --read-floor). Each thread reads U 16-byte pieces with the weight stream's non-temporal
// buffer loads and folds them into one word; a store that the data never triggers keeps the loads
// alive. One-shot grids cover the buffer once (U pieces per thread); persistent grids of `grid`
// workgroups stride over it.
#include "w4a8_common.h"
#include "../../include/w4a8_probe.h"

namespace w4a8 {

template <int U>
__global__ void __launch_bounds__(1024) probe_oneshot_kernel(const void* buf, uint32_t n16, uint32_t* sink) {
  const BufRsrc src = make_rsrc(buf, n16 * 16u);
  const uint32_t base = (uint32_t)blockIdx.x * blockDim.x * U + threadIdx.x;
  uint4 v[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint32_t idx = base + (uint32_t)i * blockDim.x;
    idx = idx < n16 ? idx : n16 - 1;
    v[i] = bload128_nt(src, idx * 16u, 0u);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < U; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

template <int U>
__global__ void __launch_bounds__(1024) probe_persist_kernel(const void* buf, uint32_t n16, uint32_t* sink) {
  const BufRsrc src = make_rsrc(buf, n16 * 16u);
  const uint32_t chunk = blockDim.x * U;
  uint32_t acc = 0;
  for (uint32_t c = blockIdx.x * chunk; c < n16; c += gridDim.x * chunk) {
    uint4 v[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      uint32_t idx = c + threadIdx.x + (uint32_t)i * blockDim.x;
      idx = idx < n16 ? idx : n16 - 1;
      v[i] = bload128_nt(src, idx * 16u, 0u);
    }
#pragma unroll
    for (int i = 0; i < U; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace w4a8

using namespace w4a8;

extern "C" int w4a8_probe_read(const void* buf, int64_t bytes, int loads_per_thread, int threads, int grid,
                               uint32_t* sink, void* stream) {
  if (!buf || !sink || bytes < 16 || bytes % 16 || bytes >= (1ll << 32)) return kErrInvalid;
  if (threads != 64 && threads != 256 && threads != 512 && threads != 1024) return kErrInvalid;
  if (grid < 0) return kErrInvalid;
  const uint32_t n16 = (uint32_t)(bytes / 16);
  const int64_t per = (int64_t)threads * loads_per_thread;
  const dim3 g(grid > 0 ? (unsigned)grid : (unsigned)((n16 + per - 1) / per)), b((unsigned)threads);
  const hipStream_t st = (hipStream_t)stream;
#define W4A8_PROBE(U)                                                                                              \
  do {                                                                                                             \
    if (grid > 0)                                                                                                  \
      hipLaunchKernelGGL(probe_persist_kernel<U>, g, b, 0, st, buf, n16, sink);            \
    else                                                                                                           \
      hipLaunchKernelGGL(probe_oneshot_kernel<U>, g, b, 0, st, buf, n16, sink);            \
  } while (0)
  switch (loads_per_thread) {
    case 1: W4A8_PROBE(1); break;
    case 4: W4A8_PROBE(4); break;
    case 8: W4A8_PROBE(8); break;
    case 16: W4A8_PROBE(16); break;
    default: return kErrInvalid;
  }
#undef W4A8_PROBE
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}
