// Inline-assembly memory helpers shared by the record-stream and strip GEMM
// kernels (gfx950): LDS-DMA copies with explicit vmcnt waits, and the
// device-coherent 16-byte accesses of the split-K hand-off (handoff.h).
#pragma once

#include "handoff.h"
#include "superblock_device.h"

namespace moat {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt left unconstrained),
// then a compiler barrier so that no LDS read of the stage moves above it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}

// Inline assembly that reads scalar registers in a vector memory instruction
// starts with kSgprVmemNops: on gfx9 a VMEM instruction needs 5 wait states
// after a VALU instruction (v_readlane, v_readfirstlane, v_cmp ...) writes an
// SGPR it reads, and the compiler, which inserts those wait states between
// its own instructions, does not look inside inline assembly -- it may reload
// a spilled base address with v_readlane right before the block.
#define MOAT_SGPR_VMEM_NOPS "s_nop 4\n\t"

// One global_load_lds_dwordx4: lane l's 16 bytes at base + off (base in
// scalar registers, a 32-bit per-lane offset) land at LDS byte lds_base +
// 16*l.  Written as inline assembly so that the compiler, which cannot tell
// the ring's stages apart, does not guard every later LDS read with a wait for
// all of these copies; the explicit vmcnt waits above are the only ordering
// the ring needs.  (s_nop 0: one wait state between writing M0 and the
// instruction that reads it.)
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile(MOAT_SGPR_VMEM_NOPS "s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off),
               "s"(base), "s"(lds_base) : "memory", "m0");
}

// Device-coherent (agent scope) vector accesses for the in-kernel hand-off:
// sc1 stores write through and sc1 loads read past the per-XCD L2s, the
// same cache policy as relaxed agent-scope atomics, 16 bytes at a time.
__device__ __forceinline__ void store_sc1(float* p, float4_t v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// Partials of the in-kernel hand-off travel encoded (handoff.h): each word is
// the bitwise complement of the value, NaN first made the canonical
// 0x7FC00000, so a word of zero means "not written yet".  The owner of a tile
// group clears the chunks it consumed, which leaves every slot at zero for
// the next call.
__device__ __forceinline__ float4_t enc_partial(float4_t v) {
  float4_t e;
#pragma unroll
  for (int i = 0; i < 4; ++i) e[i] = __uint_as_float(handoff_encode(__float_as_uint(v[i])));
  return e;
}

__device__ __forceinline__ bool partial_ready(float4_t w) {
  return handoff_chunk_written(__float_as_uint(w[0]), __float_as_uint(w[1]), __float_as_uint(w[2]),
                               __float_as_uint(w[3]));
}

__device__ __forceinline__ float4_t dec_partial(float4_t w) {
  float4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(handoff_decode(__float_as_uint(w[i])));
  return v;
}

// The workspace's sticky status word, copied into LDS at the start of a call
// (global_load_lds_dword: every lane of the wave copies the same word, 64
// copies in 256 bytes) without waiting for it: the copy is the wave's oldest
// memory operation, so the copy ring's first explicit vmcnt wait covers it,
// and it is read from LDS only after such a wait.  (A compiler-visible load
// would get a wait at its first use, which the compiler may place before the
// first weight copy is issued -- a memory round trip at the start of every
// workgroup; a register loaded by inline assembly can be copied by the
// compiler before the wait that covers it.)  Without a workspace the LDS
// word is simply set to 0.
__device__ __forceinline__ void status_to_lds(const uint32_t* status, uint32_t* lds_word) {
  if (status) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_ptr_t)lds_word;
    asm volatile(MOAT_SGPR_VMEM_NOPS "s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" : :
                 "v"(0u), "s"(status), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
  } else if ((threadIdx.x & 63) == 0) {
    *lds_word = 0u;
  }
}

// The status word copied by status_to_lds, after a vmcnt wait that covers the
// copy.
constexpr int kStatusLdsBytes = 256;

// (An LDS read, ds_read_b32: through a generic pointer the volatile read
// would be a flat load, which also waits for vmcnt, i.e. for every copy in
// flight.)
typedef __attribute__((address_space(3))) const volatile uint32_t lds_cv_u32;
__device__ __forceinline__ uint32_t status_from_lds(const uint32_t* lds_word) {
  return *(lds_cv_u32*)lds_word;
}

// A value to add to every result: 0 when the status word read at the start
// of the call is clear, NaN when it is set (adding 0 leaves a result
// unchanged, -0 aside).
__device__ __forceinline__ float status_poison(uint32_t st) { return st ? __uint_as_float(0x7FC00000u) : 0.0f; }

__device__ __forceinline__ float4_t poisoned(float4_t v, float poison) {
  return v + float4_t{poison, poison, poison, poison};
}

// Workgroup barrier for LDS hand-over between waves that keep vector memory
// copies in flight: waits for this wave's LDS accesses only (lgkmcnt 0;
// vmcnt and expcnt unconstrained), unlike __syncthreads, whose fence would
// also wait for every outstanding copy.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Repeated batch loads a thread of the owner may spend on chunks not yet
// written before it stops waiting and adds them as they read (NaN): about a
// second, a bound on the wait that contributors, which store their partials
// before they wait for anything, never let it reach.
constexpr int kMaxPolls = 1 << 19;

// Sixteen independent sc1 loads in flight, then one wait: base (scalar) +
// per-lane 32-bit byte offsets.
__device__ __forceinline__ void load16_sc1(float4_t (&t)[16], const float* base, const uint32_t (&o)[16]) {
  asm volatile(
      MOAT_SGPR_VMEM_NOPS
      "global_load_dwordx4 %0, %16, %32 sc1\n\t"
      "global_load_dwordx4 %1, %17, %32 sc1\n\t"
      "global_load_dwordx4 %2, %18, %32 sc1\n\t"
      "global_load_dwordx4 %3, %19, %32 sc1\n\t"
      "global_load_dwordx4 %4, %20, %32 sc1\n\t"
      "global_load_dwordx4 %5, %21, %32 sc1\n\t"
      "global_load_dwordx4 %6, %22, %32 sc1\n\t"
      "global_load_dwordx4 %7, %23, %32 sc1\n\t"
      "global_load_dwordx4 %8, %24, %32 sc1\n\t"
      "global_load_dwordx4 %9, %25, %32 sc1\n\t"
      "global_load_dwordx4 %10, %26, %32 sc1\n\t"
      "global_load_dwordx4 %11, %27, %32 sc1\n\t"
      "global_load_dwordx4 %12, %28, %32 sc1\n\t"
      "global_load_dwordx4 %13, %29, %32 sc1\n\t"
      "global_load_dwordx4 %14, %30, %32 sc1\n\t"
      "global_load_dwordx4 %15, %31, %32 sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7]),
        "=&v"(t[8]), "=&v"(t[9]), "=&v"(t[10]), "=&v"(t[11]), "=&v"(t[12]), "=&v"(t[13]), "=&v"(t[14]),
        "=&v"(t[15])
      : "v"(o[0]), "v"(o[1]), "v"(o[2]), "v"(o[3]), "v"(o[4]), "v"(o[5]), "v"(o[6]), "v"(o[7]), "v"(o[8]),
        "v"(o[9]), "v"(o[10]), "v"(o[11]), "v"(o[12]), "v"(o[13]), "v"(o[14]), "v"(o[15]), "s"(base)
      : "memory");
}

__device__ __forceinline__ void store_sc1_at(float* base, uint32_t o, float4_t v) {
  asm volatile(MOAT_SGPR_VMEM_NOPS "global_store_dwordx4 %0, %1, %2 sc1" : : "v"(o), "v"(v), "s"(base) : "memory");
}

}  // namespace moat
