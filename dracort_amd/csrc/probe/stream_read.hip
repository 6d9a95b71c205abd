// Streaming-read probe: the per-launch ceiling of a kernel that does nothing
// but read a buffer once (16-byte loads, grid-stride, four loads in flight
// per thread), for comparison with the decode GEMV launches of the same size.
// Measurement only: bench.py loads this library for its --stream-probe mode;
// the GGUF operators never use it.
#include <hip/hip_runtime.h>
#include <stdint.h>

__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, int64_t n16,
                                                          uint32_t* __restrict__ sink, uint32_t key) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  // a store only when the xor of everything read equals the key: keeps the loads live
  if (acc == key) sink[blockIdx.x & 255] = acc;
}

extern "C" int draco_probe_stream_read(const void* p, int64_t bytes, int blocks, void* sink, void* stream) {
  if (!p || !sink || bytes < 16 || (bytes & 15) || blocks < 1 || (reinterpret_cast<uintptr_t>(p) & 15)) return -1;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(p), bytes / 16, static_cast<uint32_t*>(sink), 0x9E3779B9u);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
