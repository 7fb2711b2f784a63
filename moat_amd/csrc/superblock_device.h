// Device-side helpers shared by the gfx950 kernels of libmoat_int4.so.
//
// Superblock record (antigravity-engine/src/shaders/batched_gemm.metal:16-20):
// 144 bytes = 8 fp16 scales + 128 payload bytes; group g of the flat stream
// (elements 32g..32g+31) has its scale at byte 144*(g/8) + 2*(g%8) and its
// 16 payload bytes at 144*(g/8) + 16 + 16*(g%8).  Every group payload is one
// 16-byte aligned chunk, so a lane can fetch a whole group with one dwordx4.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moat {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kGroup = 32;
constexpr int kGroupsPerSb = 8;
constexpr int kSbElems = 256;
constexpr int kSbBytes = 144;
constexpr int kSbHeader = 16;

__device__ __forceinline__ uint64_t group_payload_offset(uint64_t g) {
  return (g >> 3) * kSbBytes + kSbHeader + ((g & 7) << 4);
}
__device__ __forceinline__ uint64_t group_scale_offset(uint64_t g) {
  return (g >> 3) * kSbBytes + ((g & 7) << 1);
}

template <typename T>
__device__ __forceinline__ T bitcast(uint32_t v) {
  return __builtin_bit_cast(T, v);
}
__device__ __forceinline__ uint32_t bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Nibble -> fp16 without a conversion instruction.  A nibble n placed in
// mantissa bits [0,4) under exponent 10 (0x6400) reads as 1024 + n; placed in
// bits [4,8) under exponent 6 (0x5400) it reads as 64 + n.  Both are exact,
// and subtracting 1032 (resp. 72) leaves exactly n - 8.  The final fp16
// multiply by the scale is one IEEE round-to-nearest-even of the exact
// product, i.e. the same bits as fp16(f32(n - 8) * f32(scale)).
constexpr uint32_t kMagicLo = 0x64006400u;  // 1024 in both halves
constexpr uint32_t kMagicHi = 0x54005400u;  // 64 in both halves

// The magic words can be passed in from VGPRs: with one mask constant in an
// SGPR and the magic in a VGPR, (p & mask) | magic is a single v_and_or_b32
// (GFX9 VOP3 takes no literal and one scalar operand).
__device__ __forceinline__ half2_t nib_lo_pair(uint32_t p, uint32_t magic = kMagicLo) {  // bits 0-3 and 16-19
  const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
  return bitcast<half2_t>((p & 0x000F000Fu) | magic) - off;
}
__device__ __forceinline__ half2_t nib_hi_pair(uint32_t p, uint32_t magic = kMagicHi) {  // bits 4-7 and 20-23
  const half2_t off = {(_Float16)72.0f, (_Float16)72.0f};
  return bitcast<half2_t>((p & 0x00F000F0u) | magic) - off;
}

// The two magic words as opaque VGPR values (see nib_lo_pair).
struct MagicWords {
  uint32_t lo, hi;
};
__device__ __forceinline__ MagicWords magic_words() {
  MagicWords m{kMagicLo, kMagicHi};
  asm volatile("" : "+v"(m.lo), "+v"(m.hi));
  return m;
}

// v_perm_b32: result byte i = byte sel_i of the 8-byte value {hi: s0, lo: s1};
// selector 0x0c yields 0x00.  byte_pair(a, b, i) = [a.byte_i, 0, b.byte_i, 0].
template <int I>
__device__ __forceinline__ uint32_t byte_pair(uint32_t a, uint32_t b) {
  constexpr uint32_t sel = (0x0Cu << 24) | (uint32_t(I) << 16) | (0x0Cu << 8) | uint32_t(4 + I);
  return __builtin_amdgcn_perm(a, b, sel);
}

// One dword (8 consecutive elements of one row) -> 4 half2 in element order:
// out[i] = (e_{2i}, e_{2i+1}) * scale.
__device__ __forceinline__ void dequant_dword_in_order(uint32_t v, half2_t sc, half2_t out[4]) {
  // [v.byte_i, 0, v.byte_i, 0]: low half keeps e_{2i} in bits 0-3, high half keeps e_{2i+1} in bits 20-23
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t sel = (0x0Cu << 24) | (uint32_t(i) << 16) | (0x0Cu << 8) | uint32_t(i);
    const uint32_t p = __builtin_amdgcn_perm(0u, v, sel);
    const uint32_t m = (p & 0x00F0000Fu) | 0x54006400u;  // (1024 + e_{2i}, 64 + e_{2i+1})
    const half2_t off = {(_Float16)1032.0f, (_Float16)72.0f};
    out[i] = (bitcast<half2_t>(m) - off) * sc;
  }
}

// Two dwords of the same 8 columns in consecutive rows (a = row t, b = row
// t+1) -> 8 half2, out[c] = (W[t][c], W[t+1][c]) for column c = 0..7.
__device__ __forceinline__ void dequant_row_pair(uint32_t a, uint32_t b, half2_t sc, half2_t out[8],
                                                 MagicWords mw = MagicWords{kMagicLo, kMagicHi}) {
  const uint32_t p0 = byte_pair<0>(a, b), p1 = byte_pair<1>(a, b);
  const uint32_t p2 = byte_pair<2>(a, b), p3 = byte_pair<3>(a, b);
  out[0] = nib_lo_pair(p0, mw.lo) * sc;
  out[1] = nib_hi_pair(p0, mw.hi) * sc;
  out[2] = nib_lo_pair(p1, mw.lo) * sc;
  out[3] = nib_hi_pair(p1, mw.hi) * sc;
  out[4] = nib_lo_pair(p2, mw.lo) * sc;
  out[5] = nib_hi_pair(p2, mw.hi) * sc;
  out[6] = nib_lo_pair(p3, mw.lo) * sc;
  out[7] = nib_hi_pair(p3, mw.hi) * sc;
}

// SwiGLU of the two projections: silu(g) * u = g / (1 + e^-g) * u in fp32
// (as the reference's silu_elementwise_mul_kernel), then fp16.  The empty asm
// keeps the fp32 product a value of its own: without it the compiler fuses
// the multiply into the fp16 conversion (v_fma_mix), one rounding where the
// reference has two.
__device__ __forceinline__ uint2 swiglu4(float4_t g, float4_t u) {
  uint32_t o[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float a = g[2 * i] / (1.0f + expf(-g[2 * i])) * u[2 * i];
    float b = g[2 * i + 1] / (1.0f + expf(-g[2 * i + 1])) * u[2 * i + 1];
    asm volatile("" : "+v"(a), "+v"(b));
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    o[i] = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
  }
  return uint2{o[0], o[1]};
}

}  // namespace moat
