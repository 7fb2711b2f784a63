// Quantizers and the superblock writer for gfx950.
//
// quantize: per group, alpha = max|w| (float32), s = alpha == 0 ? 1 : alpha/7
// (correctly rounded float32 division), q = clip(rint_half_even(w / d), -8, 7)
// with d = s (surface A, src/dequant.py:47-53) or d = fp16(s) widened back to
// float32 (surface B, antigravity-engine/src/dequant.py:56-58); the stored
// scale is fp16(s).  NaN anywhere in a group makes alpha NaN (numpy's max
// propagates NaN), and a NaN quotient is stored as q = 0.
#include "superblock_device.h"

namespace moat {

__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  if (dtype == 0) return static_cast<const float*>(p)[i];
  if (dtype == 1) return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p)[i]);
  return (float)static_cast<const double*>(p)[i];  // float64: one round-to-nearest-even
}

__device__ __forceinline__ float group_scale(float amax, bool has_nan) {
  if (has_nan) return __builtin_nanf("");
  return amax == 0.0f ? 1.0f : __fdiv_rn(amax, 7.0f);
}

__device__ __forceinline__ int quantize_one(float w, float d) {
  const float r = rintf(__fdiv_rn(w, d));
  if (r != r) return 0;
  return (int)fminf(fmaxf(r, -8.0f), 7.0f);
}

__global__ void __launch_bounds__(256) quantize_kernel(const void* __restrict__ w, int dtype, int64_t n_groups,
                                                       int gsize, int scale_mode, int8_t* __restrict__ q,
                                                       uint16_t* __restrict__ scales) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < n_groups; g += stride) {
    const int64_t base = g * gsize;
    float amax = 0.0f;
    bool nan = false;
    for (int i = 0; i < gsize; ++i) {
      const float a = fabsf(load_as_f32(w, dtype, base + i));
      nan |= (a != a);
      amax = fmaxf(amax, a);
    }
    const float s = group_scale(amax, nan);
    const _Float16 s16 = (_Float16)s;
    const float d = scale_mode ? (float)s16 : s;
    for (int i = 0; i < gsize; ++i) q[base + i] = (int8_t)quantize_one(load_as_f32(w, dtype, base + i), d);
    scales[g] = __builtin_bit_cast(uint16_t, s16);
  }
}

// 8 codes (int8 values, taken mod 16 after +8) -> one payload dword.
__device__ __forceinline__ uint32_t pack8(uint32_t lo4, uint32_t hi4) {
  // lo4/hi4 hold 4 int8 values each; u = ((q & 15) + 8) & 15 per byte (no carries between bytes)
  const uint32_t u0 = ((lo4 & 0x0F0F0F0Fu) + 0x08080808u) & 0x0F0F0F0Fu;
  const uint32_t u1 = ((hi4 & 0x0F0F0F0Fu) + 0x08080808u) & 0x0F0F0F0Fu;
  const uint32_t p0 = u0 | (u0 >> 4);  // byte0 = e0 | e1<<4, byte2 = e2 | e3<<4
  const uint32_t p1 = u1 | (u1 >> 4);
  const uint32_t h0 = (p0 & 0xFFu) | ((p0 >> 8) & 0xFF00u);
  const uint32_t h1 = (p1 & 0xFFu) | ((p1 >> 8) & 0xFF00u);
  return h0 | (h1 << 16);
}

// One thread per group: 32 codes + one fp16 scale -> 16 payload bytes and
// the scale slot of the record.
template <bool kAligned>
__global__ void __launch_bounds__(256) pack_superblocks_kernel(const int8_t* __restrict__ q,
                                                               const uint16_t* __restrict__ scales,
                                                               int64_t n_groups, uint8_t* __restrict__ sb) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < n_groups; g += stride) {
    uint32_t d[8];
    if (kAligned) {
      const uint4 a = reinterpret_cast<const uint4*>(q + g * kGroup)[0];
      const uint4 b = reinterpret_cast<const uint4*>(q + g * kGroup)[1];
      d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w; d[4] = b.x; d[5] = b.y; d[6] = b.z; d[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(q + g * kGroup + 4 * i);
        d[i] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
      }
    }
    uint4 out;
    out.x = pack8(d[0], d[1]);
    out.y = pack8(d[2], d[3]);
    out.z = pack8(d[4], d[5]);
    out.w = pack8(d[6], d[7]);
    *reinterpret_cast<uint4*>(sb + group_payload_offset((uint64_t)g)) = out;
    *reinterpret_cast<uint16_t*>(sb + group_scale_offset((uint64_t)g)) = scales[g];
  }
}

// Quantize + serialize, group size 32.
__global__ void __launch_bounds__(256) quantize_pack_kernel(const void* __restrict__ w, int dtype, int64_t n_groups,
                                                            int scale_mode, uint8_t* __restrict__ sb) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < n_groups; g += stride) {
    const int64_t base = g * kGroup;
    float v[kGroup];
    float amax = 0.0f;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      v[i] = load_as_f32(w, dtype, base + i);
      const float a = fabsf(v[i]);
      nan |= (a != a);
      amax = fmaxf(amax, a);
    }
    const float s = group_scale(amax, nan);
    const _Float16 s16 = (_Float16)s;
    const float d = scale_mode ? (float)s16 : s;
    uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const uint32_t code = (uint32_t)(quantize_one(v[i], d) + 8) & 0xFu;
      words[i >> 3] |= code << (4 * (i & 7));
    }
    *reinterpret_cast<uint4*>(sb + group_payload_offset((uint64_t)g)) = uint4{words[0], words[1], words[2], words[3]};
    *reinterpret_cast<uint16_t*>(sb + group_scale_offset((uint64_t)g)) = __builtin_bit_cast(uint16_t, s16);
  }
}

// The same, four lanes per group: lane p of a group loads elements 8p..8p+7
// with 16-byte loads (a wave covers 16 groups' contiguous bytes), the group's
// max|w| and NaN flag are combined across the four lanes, and lane p writes
// payload dword p of the group (lane 0 the scale).  The bits are those of
// quantize_pack_kernel.  w must be 16-byte aligned.
__device__ __forceinline__ void load8_f32(const void* w, int dtype, int64_t e0, float (&v)[8]) {
  if (dtype == 1) {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + e0);
    const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] & 0xFFFFu));
      v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] >> 16));
    }
  } else if (dtype == 0) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(w) + e0);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const double2* p = reinterpret_cast<const double2*>(static_cast<const double*>(w) + e0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const double2 d = p[i];
      v[2 * i] = (float)d.x;
      v[2 * i + 1] = (float)d.y;
    }
  }
}

__global__ void __launch_bounds__(256) quantize_pack4_kernel(const void* __restrict__ w, int dtype, int64_t n_groups,
                                                             int scale_mode, uint8_t* __restrict__ sb) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t total = n_groups * 4;
  // every lane of the wave runs the same number of iterations (the shuffles
  // need all four lanes of a group); lanes past the end load group 0 and store nothing
  const int64_t iters = (total + stride - 1) / stride;
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t it = 0; it < iters; ++it, t += stride) {
    const bool live = t < total;
    const int64_t g = live ? (t >> 2) : 0;
    const int part = (int)(t & 3);
    float v[8];
    load8_f32(w, dtype, g * kGroup + 8 * part, v);
    float amax = 0.0f;
    int nan = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = fabsf(v[i]);
      nan |= (a != a);
      amax = fmaxf(amax, a);
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    nan |= __shfl_xor(nan, 1);
    nan |= __shfl_xor(nan, 2);
    const float s = group_scale(amax, nan != 0);
    const _Float16 s16 = (_Float16)s;
    const float d = scale_mode ? (float)s16 : s;
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) word |= ((uint32_t)(quantize_one(v[i], d) + 8) & 0xFu) << (4 * i);
    if (live) {
      *reinterpret_cast<uint32_t*>(sb + group_payload_offset((uint64_t)g) + 4 * part) = word;
      if (part == 0) *reinterpret_cast<uint16_t*>(sb + group_scale_offset((uint64_t)g)) = __builtin_bit_cast(uint16_t, s16);
    }
  }
}

static unsigned qgrid(int64_t items) {
  int64_t b = (items + 255) / 256;
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return (unsigned)b;
}

hipError_t launch_quantize(const void* w, int dtype, int64_t n, int gsize, int scale_mode, int8_t* q,
                           uint16_t* scales, hipStream_t st) {
  const int64_t n_groups = n / gsize;
  hipLaunchKernelGGL(quantize_kernel, dim3(qgrid(n_groups)), dim3(256), 0, st, w, dtype, n_groups, gsize, scale_mode,
                     q, scales);
  return hipGetLastError();
}

hipError_t launch_pack_superblocks(const int8_t* q, const uint16_t* scales, int64_t n_sb, uint8_t* sb,
                                   hipStream_t st) {
  const int64_t n_groups = n_sb * kGroupsPerSb;
  if ((reinterpret_cast<uintptr_t>(q) & 15) == 0) {
    hipLaunchKernelGGL(pack_superblocks_kernel<true>, dim3(qgrid(n_groups)), dim3(256), 0, st, q, scales, n_groups, sb);
  } else {
    hipLaunchKernelGGL(pack_superblocks_kernel<false>, dim3(qgrid(n_groups)), dim3(256), 0, st, q, scales, n_groups,
                       sb);
  }
  return hipGetLastError();
}

hipError_t launch_quantize_pack(const void* w, int dtype, int64_t n, int scale_mode, uint8_t* sb, hipStream_t st) {
  const int64_t n_groups = n / kGroup;
  if ((reinterpret_cast<uintptr_t>(w) & 15) == 0) {
    hipLaunchKernelGGL(quantize_pack4_kernel, dim3(qgrid(n_groups * 4)), dim3(256), 0, st, w, dtype, n_groups,
                       scale_mode, sb);
  } else {
    hipLaunchKernelGGL(quantize_pack_kernel, dim3(qgrid(n_groups)), dim3(256), 0, st, w, dtype, n_groups,
                       scale_mode, sb);
  }
  return hipGetLastError();
}

}  // namespace moat
