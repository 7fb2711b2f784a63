// Element-wise kernels of the superblock format for gfx950: stream decode,
// nibble pack/unpack, per-group dequant, table gather and fp16 rounding.
//
// Every kernel is a grid-stride loop over independent items, so any grid
// size is correct; the host side picks one that fills the 256 CUs.
#include "superblock_device.h"

namespace moat {

// One thread per 32-element group: a 16-byte payload load, one scale load,
// 64 bytes of fp16 out.  Bit-exact with src/dequant.py:116-147 and
// antigravity-engine/src/shaders/batched_gemm.metal:41-66.
__global__ void __launch_bounds__(256) dequant_stream_kernel(const uint8_t* __restrict__ sb, int64_t n_groups,
                                                             uint16_t* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < n_groups; g += stride) {
    const uint4 pl = *reinterpret_cast<const uint4*>(sb + group_payload_offset((uint64_t)g));
    const uint32_t s = *reinterpret_cast<const uint16_t*>(sb + group_scale_offset((uint64_t)g));
    const half2_t sc = bitcast<half2_t>(s | (s << 16));
    const uint32_t words[4] = {pl.x, pl.y, pl.z, pl.w};
    uint4* dst = reinterpret_cast<uint4*>(out + g * kGroup);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      half2_t h[4];
      dequant_dword_in_order(words[w], sc, h);
      dst[w] = uint4{bits(h[0]), bits(h[1]), bits(h[2]), bits(h[3])};
    }
  }
}

// packed[j] = ((q[2j] + 8) & 15) | (((q[2j+1] + 8) & 15) << 4); 4 bytes per thread.
__global__ void __launch_bounds__(256) pack_nibbles_kernel(const int8_t* __restrict__ q, int64_t n_bytes,
                                                           uint8_t* __restrict__ packed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < n_bytes; b += stride) {
    const uint32_t lo = (uint32_t)(q[2 * b] + 8) & 0xF;
    const uint32_t hi = (uint32_t)(q[2 * b + 1] + 8) & 0xF;
    packed[b] = (uint8_t)(lo | (hi << 4));
  }
}

__global__ void __launch_bounds__(256) unpack_nibbles_kernel(const uint8_t* __restrict__ packed, int64_t n_bytes,
                                                             int8_t* __restrict__ q) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < n_bytes; b += stride) {
    const int v = packed[b];
    q[2 * b] = (int8_t)((v & 0xF) - 8);
    q[2 * b + 1] = (int8_t)(((v >> 4) & 0xF) - 8);
  }
}

// fp16(f32(q) * scale) in float32 then one rounding to fp16: for an fp16
// scale the product is exact; for a float32 scale this is the reference's
// float32 product followed by astype(float16).
template <typename QT>
__device__ __forceinline__ float q_as_f32(const QT* q, int64_t i) {
  return (float)q[i];
}

__device__ __forceinline__ float scale_as_f32(const void* scales, int dtype, int64_t g) {
  if (dtype == 1) return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(scales)[g]);
  if (dtype == 3) return (float)static_cast<const double*>(scales)[g];
  return static_cast<const float*>(scales)[g];
}

template <typename QT>
__global__ void __launch_bounds__(256) group_dequant_kernel(const QT* __restrict__ q, const void* __restrict__ scales,
                                                            int scale_dtype, int64_t n_elems, int group_size,
                                                            int table_mode, uint16_t* __restrict__ out,
                                                            int32_t* err_flag) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_elems; i += stride) {
    const float s = scale_as_f32(scales, scale_dtype, i / group_size);
    float v = q_as_f32(q, i);
    if (table_mode) {
      // lut[q + 8] of a 16-entry table with Python's negative-index wrap;
      // the index is the int16 value of q (the wrapper hands over q already
      // reduced to int16 range).
      const int64_t idx = (int64_t)v + 8;
      if (idx >= 16 || idx < -16) {
        out[i] = 0;
        if (err_flag) *err_flag = 1;
        continue;
      }
      v = (float)((idx < 0 ? idx + 16 : idx) - 8);
    }
    float prod = v * s;
    // Materialise the float32 product: without this the compiler folds the
    // multiply and the fp16 conversion into one v_fma_mixlo_f16, which rounds
    // once instead of twice and differs from the reference for float32 scales.
    asm volatile("" : "+v"(prod));
    const _Float16 h = (_Float16)prod;
    out[i] = __builtin_bit_cast(uint16_t, h);
  }
}

// Clipped table gather of src/dequant.py:79-112.
__global__ void __launch_bounds__(256) lut_gather_kernel(const int64_t* __restrict__ q, int64_t n, int index_mode,
                                                         const uint16_t* __restrict__ lut, int64_t per_row,
                                                         int lut_len, uint16_t* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t v = q[i];
    int64_t idx;
    if (index_mode == 0) {
      idx = v + 8;
    } else {
      const int32_t v32 = (int32_t)(uint32_t)(uint64_t)v;  // astype(int32): keep the low 32 bits
      idx = (index_mode == 1) ? (int64_t)(int32_t)((uint32_t)v32 + 8u) : (int64_t)v32;
    }
    idx = idx < 0 ? 0 : (idx > lut_len - 1 ? lut_len - 1 : idx);
    out[i] = lut[(i / per_row) * lut_len + idx];
  }
}

__global__ void any_negative_kernel(const int64_t* __restrict__ q, int64_t n, int32_t* flag) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int neg = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) neg |= (q[i] < 0);
  if (__any(neg) && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

__global__ void fill_u8_kernel(uint8_t* p, int64_t n, uint8_t v) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// float64 -> binary16, round to nearest even in ONE step (a float64 -> float32
// -> float16 chain can round twice).  Written from the IEEE 754 encoding.
__device__ __forceinline__ uint16_t f64_to_f16_rne(double d) {
  const uint64_t b = __builtin_bit_cast(uint64_t, d);
  const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  const int exp = (int)((b >> 52) & 0x7FF);
  uint64_t mant = b & 0xFFFFFFFFFFFFFull;
  if (exp == 0x7FF) {  // inf / nan (keep the top payload bits, stay a NaN)
    if (mant == 0) return sign | 0x7C00u;
    uint16_t pl = (uint16_t)(mant >> 42);
    return sign | 0x7C00u | (pl ? pl : 1u);
  }
  if (exp == 0 && mant == 0) return sign;
  // value = 1.mant * 2^(exp-1023) (normal) or 0.mant * 2^-1022 (subnormal double)
  int e = exp - 1023;
  uint64_t sig = exp ? (mant | (1ull << 52)) : mant;  // 53-bit significand
  if (!exp) e = -1022;
  // target: half exponent range [-14, 15], 10 fraction bits; subnormal quantum 2^-24
  int shift;  // number of low bits of sig to drop
  if (e >= -14) shift = 52 - 10;
  else shift = 52 - 10 + (-14 - e);
  if (shift > 63) return sign;  // far below half the smallest subnormal
  uint64_t kept = sig >> shift;
  const uint64_t rem = sig & ((1ull << shift) - 1);
  const uint64_t halfway = 1ull << (shift - 1);
  if (rem > halfway || (rem == halfway && (kept & 1))) kept += 1;
  if (e >= -14) {
    // kept has 11 significant bits (may carry to 12)
    if (kept >> 11) { kept >>= 1; e += 1; }
    if (e > 15) return sign | 0x7C00u;
    return sign | (uint16_t)(((e + 15) << 10) | (kept & 0x3FF));
  }
  // subnormal: kept counts quanta of 2^-24; 1024 quanta is the smallest normal
  return sign | (uint16_t)kept;
}

__global__ void __launch_bounds__(256) to_f16_kernel(const void* __restrict__ src, int src_dtype, int64_t n,
                                                     uint16_t* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    if (src_dtype == 3) {
      out[i] = f64_to_f16_rne(static_cast<const double*>(src)[i]);
    } else {
      const _Float16 h = (_Float16)static_cast<const float*>(src)[i];
      out[i] = __builtin_bit_cast(uint16_t, h);
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers.

static unsigned grid_for(int64_t items, int per_block = 256) {
  int64_t b = (items + per_block - 1) / per_block;
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return (unsigned)b;
}

hipError_t launch_dequant_stream(const uint8_t* sb, int64_t n_sb, uint16_t* out, hipStream_t st) {
  const int64_t n_groups = n_sb * kGroupsPerSb;
  hipLaunchKernelGGL(dequant_stream_kernel, dim3(grid_for(n_groups)), dim3(256), 0, st, sb, n_groups, out);
  return hipGetLastError();
}

hipError_t launch_pack_nibbles(const int8_t* q, int64_t n, uint8_t* packed, hipStream_t st) {
  hipLaunchKernelGGL(pack_nibbles_kernel, dim3(grid_for(n / 2)), dim3(256), 0, st, q, n / 2, packed);
  return hipGetLastError();
}

hipError_t launch_unpack_nibbles(const uint8_t* packed, int64_t n_bytes, int8_t* q, hipStream_t st) {
  hipLaunchKernelGGL(unpack_nibbles_kernel, dim3(grid_for(n_bytes)), dim3(256), 0, st, packed, n_bytes, q);
  return hipGetLastError();
}

hipError_t launch_group_dequant(const void* q, int q_dtype, const void* scales, int scale_dtype, int64_t n_groups,
                                int group_size, int table_mode, uint16_t* out, int32_t* err_flag, hipStream_t st) {
  const int64_t n = n_groups * group_size;
  const dim3 g(grid_for(n)), b(256);
  if (q_dtype == 2) {
    hipLaunchKernelGGL(group_dequant_kernel<int8_t>, g, b, 0, st, static_cast<const int8_t*>(q), scales, scale_dtype,
                       n, group_size, table_mode, out, err_flag);
  } else if (q_dtype == 4) {
    hipLaunchKernelGGL(group_dequant_kernel<int64_t>, g, b, 0, st, static_cast<const int64_t*>(q), scales,
                       scale_dtype, n, group_size, table_mode, out, err_flag);
  } else {
    hipLaunchKernelGGL(group_dequant_kernel<float>, g, b, 0, st, static_cast<const float*>(q), scales, scale_dtype, n,
                       group_size, table_mode, out, err_flag);
  }
  return hipGetLastError();
}

hipError_t launch_lut_gather(const int64_t* q, int64_t n, int index_mode, const uint16_t* lut, int64_t lut_rows,
                             int lut_len, uint16_t* out, hipStream_t st) {
  const int64_t per_row = n / lut_rows;
  hipLaunchKernelGGL(lut_gather_kernel, dim3(grid_for(n)), dim3(256), 0, st, q, n, index_mode, lut, per_row, lut_len,
                     out);
  return hipGetLastError();
}

hipError_t launch_any_negative(const int64_t* q, int64_t n, int32_t* flag, hipStream_t st) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, st, reinterpret_cast<uint32_t*>(flag), (int64_t)1, 0u);
  hipLaunchKernelGGL(any_negative_kernel, dim3(grid_for(n)), dim3(256), 0, st, q, n, flag);
  return hipGetLastError();
}

// fp16(f32(q) / divisor): numpy's float16 division of an int8 tensor cast to
// float16 (exact) by a float16 scalar, which divides in float32 (correctly
// rounded) and rounds the quotient to float16.
__global__ void __launch_bounds__(256) i8_div_to_f16_kernel(const int8_t* __restrict__ q, int64_t n, float divisor,
                                                            uint16_t* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const _Float16 h = (_Float16)((float)q[i] / divisor);
    out[i] = __builtin_bit_cast(uint16_t, h);
  }
}

hipError_t launch_i8_div_to_f16(const int8_t* q, int64_t n, float divisor, uint16_t* out, hipStream_t st) {
  hipLaunchKernelGGL(i8_div_to_f16_kernel, dim3(grid_for(n)), dim3(256), 0, st, q, n, divisor, out);
  return hipGetLastError();
}

hipError_t launch_to_f16(const void* src, int src_dtype, int64_t n, uint16_t* out, hipStream_t st) {
  hipLaunchKernelGGL(to_f16_kernel, dim3(grid_for(n)), dim3(256), 0, st, src, src_dtype, n, out);
  return hipGetLastError();
}

hipError_t launch_clear(void* p, int64_t bytes, hipStream_t st) {
  if (bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(p) & 3) == 0) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(bytes / 4)), dim3(256), 0, st, static_cast<uint32_t*>(p),
                       bytes / 4, 0u);
  } else {
    hipLaunchKernelGGL(fill_u8_kernel, dim3(grid_for(bytes)), dim3(256), 0, st, static_cast<uint8_t*>(p), bytes,
                       (uint8_t)0);
  }
  return hipGetLastError();
}

}  // namespace moat
