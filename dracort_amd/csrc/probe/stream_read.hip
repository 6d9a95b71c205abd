// Streaming-read probe: the per-launch ceiling of a kernel that does nothing
// but read a buffer once (16-byte loads, 4 / 8 / 16 in flight per thread,
// one contiguous span per workgroup), for comparison with the decode GEMV
// launches of the same size.
// Measurement only: bench.py loads this library for its --stream-probe mode;
// the GGUF operators never use it.
#include <hip/hip_runtime.h>
#include <stdint.h>

// U 16-byte loads in flight per thread; each workgroup walks its own
// contiguous span of the buffer (U x 4 KB per step).
template <int U>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, int64_t n16,
                                                          uint32_t* __restrict__ sink, uint32_t key) {
  const int64_t per_block = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t begin = (int64_t)blockIdx.x * per_block;
  const int64_t end = begin + per_block < n16 ? begin + per_block : n16;
  uint32_t acc = 0;
  int64_t i = begin + threadIdx.x;
  for (; i + (U - 1) * 256 < end; i += U * 256) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = p[i + u * 256];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < end; i += 256) {
    const uint4 a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  // a store only when the xor of everything read equals the key: keeps the loads live
  if (acc == key) sink[blockIdx.x & 255] = acc;
}

extern "C" int draco_probe_stream_read(const void* p, int64_t bytes, int blocks, int loads, void* sink,
                                       void* stream) {
  if (!p || !sink || bytes < 16 || (bytes & 15) || blocks < 1 || (reinterpret_cast<uintptr_t>(p) & 15)) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint4* q = static_cast<const uint4*>(p);
  uint32_t* k = static_cast<uint32_t*>(sink);
  switch (loads) {
    case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, q, bytes / 16, k, 0x9E3779B9u); break;
    case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, s, q, bytes / 16, k, 0x9E3779B9u); break;
    case 16: hipLaunchKernelGGL(stream_read_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, s, q, bytes / 16, k, 0x9E3779B9u); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
