// Plain streaming read: the bandwidth floor that the GEMM's weight stream is
// measured against (same bytes, nothing but 16-byte loads).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moat {

// Workgroup b reads chunks b, b + grid, ... of 4 x 16 bytes per thread (the
// four loads of a thread are 4 KB apart, all issued before any is used).
// The XOR of everything read is stored only if it equals a value the caller
// chose never to occur, so the loads are kept and nothing is written.
__global__ void __launch_bounds__(256) stream_read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink, uint32_t never) {
  const int64_t per_block = 4 * 256;
  uint32_t acc = 0;
  for (int64_t base = (int64_t)blockIdx.x * per_block; base < n16; base += (int64_t)gridDim.x * per_block) {
    uint4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t e = base + i * 256 + threadIdx.x;
      v[i] = e < n16 ? src[e] : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  }
  if (acc == never) sink[0] = acc;
}

hipError_t launch_stream_read(const void* src, int64_t bytes, uint32_t* sink, int blocks, hipStream_t st) {
  const int64_t n16 = bytes / 16;
  if (n16 == 0) return hipSuccess;
  const int64_t need = (n16 + 1023) / 1024;
  if (blocks <= 0) blocks = 2048;
  if (blocks > need) blocks = (int)need;
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, st, static_cast<const uint4*>(src), n16, sink,
                     0x9E3779B9u);
  return hipGetLastError();
}

}  // namespace moat
