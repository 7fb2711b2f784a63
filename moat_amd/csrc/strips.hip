// Strip order and its GEMM kernel (gfx950).
//
// Strip order is a storage order for the 144-byte records of W[K][M] that a
// loader chooses once (no counterpart in the reference, whose stream is the
// row order of src/dequant.py:116-147).  The quantized values and scales are
// the reference's, bit for bit; only the grouping of elements into records
// changes:
//  * strip g is the 32 columns 32g .. 32g+31 of W (one quantization group per
//    row), and the strips follow each other in column order;
//  * inside strip g, record b (144 bytes) holds rows 8b .. 8b+7: bytes
//    [0,16) are the 8 fp16 scales of those rows' group g; byte 16 + 8j +
//    strip_row_pos(i) is byte j of row 8b+i's 16 payload bytes of group g
//    (column 32g + 2j in the low nibble, 32g + 2j + 1 in the high nibble,
//    each stored as q + 8): the payload bytes column pair by column pair, so
//    that the 8 rows of one column pair are 8 consecutive bytes, rows in the
//    order 0 2 1 3 4 6 5 7.
// A strip is one contiguous run of K x 18 bytes, and 32 rows of it (a "unit",
// one matrix-core K step) are 576 contiguous bytes.
//
// GEMM over strip order (int4_gemm_strips_kernel), for 1 <= N <= 8:
//  * the units of all strips form one stream (strip-major); workgroup p takes
//    an equal contiguous range of it (stream-K), which is one contiguous byte
//    range of the records.  When M/32 is between 128 and 256 the plan gives
//    every workgroup exactly one whole strip, and nothing is shared;
//  * the W waves of a workgroup (4, 8 or 12) walk its range in rounds of
//    64, 64 or 48 consecutive units, wave w taking the w-th run of 16, 8 or 4
//    of them (one contiguous run of records); each keeps a private LDS ring
//    of `depth` such stages (576 bytes a unit, copied by
//    global_load_lds_dwordx4) with the X rows
//    those units need, issues every stage whole `depth` - 1 stages ahead, and
//    keeps copying across strip boundaries: the ring never drains until the
//    range ends;
//  * per unit a lane (q, j) reads the 8 bytes of column pair j of rows
//    8q .. 8q+7 (record q, one 8-byte read) and the record's 8 row scales,
//    forms the two fp16 B operands of v_mfma_f32_16x16x32_f16 for columns 2j
//    and 2j+1 (magic-exponent nibble decode straight from the loaded words
//    and from the words shifted right by 8, one v_pk_mul by the row-pair
//    scales: fp16(f32(q - 8) * f32(s)) exactly), and the A operand is
//    X[row j][32u + 8q .. +7] from the stage;
//  * where the range crosses a strip boundary the waves put their fp32
//    accumulators in a small LDS area apart from the ring, meet at one
//    barrier, and one wave adds the W sums in wave order and writes the part:
//    a whole strip goes to Y; the first part of a range (a strip that began
//    in an earlier workgroup's range) is stored encoded for that workgroup; the
//    last part of a range (a strip whose first unit it holds) is the
//    workgroup's own and, after its stream ends, it adds the later
//    workgroups' parts in workgroup order (polling, bounded, as the
//    record-stream kernel's hand-off does; the parts of up to two later
//    workgroups are loaded during the last stage) and writes Y.  Results are
//    deterministic.
#include "stream_device.h"

namespace moat {

constexpr int kStripCols = 32;
constexpr int kUnitRows = 32;
constexpr int kUnitBytes = 576;  // 32 rows x 18 bytes: 4 records
constexpr int kStripMaxN = 8;

// Position of row 8b+i's byte among the 8 bytes of one column pair of
// record b: rows 0, 2, 1, 3, 4, 6, 5, 7 (bits 0 and 1 of i swapped), so that
// bytes 0 and 2 of a 32-bit word, and of the word shifted right by 8, hold two
// consecutive rows.  Its own inverse.
__host__ __device__ constexpr int strip_row_pos(int i) { return (i & 4) | ((i & 1) << 1) | ((i >> 1) & 1); }

struct StripParams {
  const uint16_t* x;   // [n][k] fp16, 16-byte aligned
  const uint8_t* w;    // strip-order records
  float* y;            // [n][m] fp32
  float* slots;        // per workgroup n x 32 fp32 (encoded contributions); null when nothing is shared
  uint32_t* status;    // workspace status word (null when nothing is shared)
  int n, k, m;
  int units;           // units per strip, k / 32
  int base, rem;       // workgroup p covers units [p*base + min(p, rem), +base + (p < rem)), cut at the last unit
  int y_vec;           // y 16-byte aligned
  uint16_t* h;         // wide kernel's SwiGLU epilogue: fp16 [n][m / 2] (else unused)
};

// Geometry of a workgroup of W waves (4, 8 or 12) staging NX rows of X.
// One stage of a wave holds 16, 8 or 4 consecutive units of its workgroup's
// range (wave w the w-th run of the workgroup's 64, 64 or 48 consecutive
// units per stage round), 576 bytes each, copied by global_load_lds_dwordx4
// (64 lanes x 16 bytes; the last copy of a stage has only as many lanes as
// chunks remain).
// X: one copy per row of the units' 64-byte slices, rows 64 bytes apart
// beyond their slices (a row's slices start 64 bytes further along the LDS
// banks than the previous row's) and the 16-byte quarters of rows 4r..4r+3
// XOR-permuted by r, so that one quarter of 16 rows falls on 16 different
// 16-byte bank groups.
template <int NX, int W>
struct StripGeom {
  static_assert(W == 4 || W == 8 || W == 12, "4, 8 or 12 waves");
  static constexpr int kStageUnits = W == 12 ? 4 : 64 / W;            // 16, 8, 4
  static constexpr int kWChunks = 36 * kStageUnits;                   // 16-byte chunks of a stage
  static constexpr int kWLoads = (kWChunks + 63) / 64;                // 9, 5, 3
  static constexpr int kWTail = kWChunks - 64 * (kWLoads - 1);        // lanes of the last copy: 64, 32, 16
  static constexpr int kWStage = 16 * kWChunks;                       // 9216, 4608, 2304
  static constexpr int kXLanes = 4 * kStageUnits;                     // lanes of a row's copy
  static constexpr int kXRowBytes = 64 * kStageUnits + 64;
  static constexpr int kXStage = NX * kXRowBytes;
  template <int kDepth>
  static constexpr int wave_bytes() { return kDepth * (kWStage + kXStage); }
  static constexpr int kSlotBytes = NX * kStripCols * 4;  // one wave's part of a strip
  template <int kDepth>
  static constexpr size_t lds_bytes() {  // rings, slots, the status word's copies
    return (size_t)W * wave_bytes<kDepth>() + (size_t)2 * W * kSlotBytes + kStatusLdsBytes;
  }
};

__device__ __forceinline__ int strip_owner(const StripParams& P, int u) {
  const int big = P.rem * (P.base + 1);
  return u < big ? u / (P.base + 1) : P.rem + (u - big) / P.base;
}

// Eight independent device-coherent loads, then one wait.
__device__ __forceinline__ void load8_sc1(float4_t (&t)[8], const float* base, const uint32_t (&o)[8]) {
  asm volatile(
      MOAT_SGPR_VMEM_NOPS
      "global_load_dwordx4 %0, %8, %16 sc1\n\t"
      "global_load_dwordx4 %1, %9, %16 sc1\n\t"
      "global_load_dwordx4 %2, %10, %16 sc1\n\t"
      "global_load_dwordx4 %3, %11, %16 sc1\n\t"
      "global_load_dwordx4 %4, %12, %16 sc1\n\t"
      "global_load_dwordx4 %5, %13, %16 sc1\n\t"
      "global_load_dwordx4 %6, %14, %16 sc1\n\t"
      "global_load_dwordx4 %7, %15, %16 sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7])
      : "v"(o[0]), "v"(o[1]), "v"(o[2]), "v"(o[3]), "v"(o[4]), "v"(o[5]), "v"(o[6]), "v"(o[7]), "s"(base)
      : "memory");
}

// 16-byte device-coherent (sc1) buffer accesses through the compiler, which
// schedules them, waits for the loads and keeps the matrix-core hazards of
// their operands (inline assembly would hide an accumulator's pending write
// from it); one 16-byte access a lane writes whole cache lines a wave.
typedef unsigned int u32x4_t __attribute__((__vector_size__(16)));
constexpr int kCpolSc1 = 16;  // cache-policy bit SC1 of a buffer access
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ void store16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, (int)off, 0, kCpolSc1);
}
__device__ __forceinline__ float4_t load16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCpolSc1));
}
// A 16-byte device-coherent load as two agent-scope 8-byte atomics (sc1).
__device__ __forceinline__ float4_t load16_coherent(const float* base, uint32_t byte_off) {
  const unsigned long long* q = reinterpret_cast<const unsigned long long*>(reinterpret_cast<const uint8_t*>(base) + byte_off);
  const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return float4_t{__builtin_bit_cast(float, (uint32_t)a), __builtin_bit_cast(float, (uint32_t)(a >> 32)),
                  __builtin_bit_cast(float, (uint32_t)b), __builtin_bit_cast(float, (uint32_t)(b >> 32))};
}

// Contributions an owner may have loaded before its output (the slots of
// workgroups p+1 .. p+kStripPrefetch).
constexpr int kStripPrefetch = 2;

// Output of rows row0 .. row0+7 of one part of a strip by one wave (the
// part's sums of the W waves are in `sl`, wave-major, NX rows each): lane l
// holds four columns of row row0 + l / 8 (rows past N idle).  `pre` holds
// the contributions of the first `npre` later workgroups when the caller
// loaded them ahead (npre = 0: none).
template <int NX, int W>
__device__ __forceinline__ void strip_part_out(const StripParams& P, const float* sl, int p, int strip, bool whole,
                                               bool owner, int last_unit, float poison,
                                               const float4_t (&pre)[kStripPrefetch], int npre, int row0 = 0) {
  const int lane = threadIdx.x & 63;
  const int r = row0 + (lane >> 3), c4 = 4 * (lane & 7);
  const bool active = r < P.n;
  float4_t v = {0.f, 0.f, 0.f, 0.f};
  if (active) {
#pragma unroll
    for (int w = 0; w < W; ++w)  // in wave order
      v += *reinterpret_cast<const float4_t*>(sl + w * NX * kStripCols + r * kStripCols + c4);
  }
  const uint32_t chunk = (uint32_t)(4 * (r * kStripCols + c4));  // bytes inside a slot
  const uint32_t slot_bytes = (uint32_t)(4 * P.n * kStripCols);
  if (!whole && !owner) {  // the first part of the range: another workgroup's strip
    if (active) store_sc1_at(P.slots, (uint32_t)p * slot_bytes + chunk, enc_partial(v));
    return;
  }
  if (owner) {
    // add the parts of the later workgroups that hold units of this strip,
    // in workgroup order
    const int q_last = strip_owner(P, last_unit);
    const float4_t zero = {0.f, 0.f, 0.f, 0.f};
    bool done = false;
    if (q_last - p <= npre) {  // all of them loaded ahead: use them if every one was written
      bool ready = true;
#pragma unroll
      for (int i = 0; i < kStripPrefetch; ++i)
        if (active && i < q_last - p) ready = ready && partial_ready(pre[i]);
      if (ready) {
#pragma unroll
        for (int i = 0; i < kStripPrefetch; ++i)
          if (active && i < q_last - p) v += dec_partial(pre[i]);
#pragma unroll
        for (int i = 0; i < kStripPrefetch; ++i)
          if (active && i < q_last - p) store_sc1_at(P.slots, (uint32_t)(p + 1 + i) * slot_bytes + chunk, zero);
        done = true;
      }
    }
    if (!done) {
      int polls = kMaxPolls;
      for (int c0 = p + 1; c0 <= q_last; c0 += 8) {
        uint32_t a[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = (uint32_t)min(c0 + i, q_last) * slot_bytes + (active ? chunk : 0u);
        float4_t t[8];
        load8_sc1(t, P.slots, a);
        bool ready;
        for (;;) {
          ready = true;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (active && c0 + i <= q_last) ready = ready && partial_ready(t[i]);
          if (handoff_stop(ready, polls)) break;
          --polls;
          __builtin_amdgcn_s_sleep(1);
          load8_sc1(t, P.slots, a);
        }
        if (handoff_gave_up(ready, polls))
          __hip_atomic_fetch_or(P.status, kWsStatusHandoffTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (active && c0 + i <= q_last) v += dec_partial(t[i]);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (active && c0 + i <= q_last) store_sc1_at(P.slots, a[i], zero);
      }
    }
  }
  if (!active) return;
  v = poisoned(v, poison);
  float* yp = P.y + (int64_t)r * P.m + kStripCols * strip + c4;
  if (P.y_vec) {
    *reinterpret_cast<float4_t*>(yp) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) yp[e] = v[e];
  }
}

// acc + sum of x[i] * w[i] over 8 fp16 pairs, four v_dot2_f32_f16.
__device__ __forceinline__ float dot8_f16(half8_t x, half8_t w, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc = __builtin_amdgcn_fdot2(half2_t{x[2 * i], x[2 * i + 1]}, half2_t{w[2 * i], w[2 * i + 1]}, acc, false);
  return acc;
}

// kDot: the same walk with the products on the vector ALUs instead of the
// matrix cores (v_dot2_f32_f16; lane (q, j) keeps the sums of columns 2j,
// 2j+1 over rows 8q..8q+7 of each unit for every row of X, reduced across
// the four q lanes at a part's end) -- the wavefront-reduction GEMV, kept
// to measure against the matrix-core path for N <= 4.
template <int NX, int kDepth, int W, bool kDot = false>
__global__ void __launch_bounds__(W * 64) int4_gemm_strips_kernel(StripParams P) {
  static_assert(!kDot || NX <= 4, "the dot2 variant stages at most 4 rows");
  using G = StripGeom<NX, W>;
  constexpr int kSU = G::kStageUnits;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, j = lane & 15;
  const int p = blockIdx.x;
  const int U = P.units;
  const int lo = p * P.base + min(p, P.rem);
  const int hi = lo + P.base + (p < P.rem ? 1 : 0);
  const MagicWords mw = magic_words();

  // Weight copies: a wave's stage is kSU consecutive units, one contiguous
  // run of 576 kSU bytes; slot s = 64 i + lane carries its 16-byte chunk s
  // (unit s / 36); units past the range re-load the stage's first unit.
  uint32_t woff[G::kWLoads], wfirst[G::kWLoads];
  int wunit[G::kWLoads];
#pragma unroll
  for (int i = 0; i < G::kWLoads; ++i) {
    const int s = min(64 * i + lane, G::kWChunks - 1);  // lanes past the last chunk copy nothing
    wunit[i] = s / 36;
    wfirst[i] = (uint32_t)(16 * (s % 36));
    woff[i] = (uint32_t)(16 * s);
  }
  // X copies, one per row n (rows past N repeat row N - 1): lane l < 4 *
  // kSU carries unit l / 4, quarter (l & 3) ^ ((n >> 2) & 3).
  const int xk = lane >> 2;
  uint32_t xoff[NX], xflat[NX];
#pragma unroll
  for (int n = 0; n < NX; ++n) {
    const int row = min(n, P.n - 1);
    const int quarter = (lane & 3) ^ ((n >> 2) & 3);
    xoff[n] = (uint32_t)(2 * (row * P.k + 8 * quarter));
    xflat[n] = xoff[n] + 64u * (uint32_t)xk;  // from the stage's first unit when no unit wraps
  }
  // LDS reads of a unit k: record q's 8 row scales, the 8 bytes of column
  // pair j of its rows, and X row j's quarter q (rows past N read row N - 1,
  // whose products are never stored)
  const uint32_t rsc = 144 * q, rpay = 144 * q + 16 + 8 * j;
  const int xrow = min(j, P.n - 1);
  const uint32_t rx = (uint32_t)(G::kXRowBytes * xrow + 16 * (q ^ ((xrow >> 2) & 3)));
  uint32_t rxd[NX];  // kDot: quarter q of every staged row
#pragma unroll
  for (int n = 0; n < NX; ++n) rxd[n] = (uint32_t)(G::kXRowBytes * n + 16 * (q ^ ((n >> 2) & 3)));

  uint8_t* wring = smem + wave * G::template wave_bytes<kDepth>();
  uint8_t* xring = wring + kDepth * G::kWStage;
  const uint32_t wring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)wring;
  const uint32_t xring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)xring;
  float* slots = reinterpret_cast<float*>(smem + W * G::template wave_bytes<kDepth>());
  uint32_t* lds_status =
      reinterpret_cast<uint32_t*>(smem + W * G::template wave_bytes<kDepth>() + 2 * W * G::kSlotBytes);
  status_to_lds(P.status, lds_status);  // the wave's oldest copy: the first ring wait covers it

  // Stage s of wave w: units first + W kSU s .. + kSU - 1 (first = lo +
  // kSU w), so that the workgroup walks W kSU consecutive units a round.
  const int first = lo + kSU * wave;
  const int nst = first < hi ? (hi - first + W * kSU - 1) / (W * kSU) : 0;
  // strip-relative unit of the first unit of the next stage to issue
  // (scalar, kept up to date stage by stage)
  int ub_issue = first % U;

  // A stage's copies take per-lane offsets fixed for the whole call (a
  // scalar base moves) unless the stage runs past the range (its weights) or
  // a unit wraps into the next strip (its X): those stages, uniform
  // branches, select per lane.
  auto issue_w = [&](int s) {
    const int u0 = first + W * kSU * s;
    const uint8_t* base = P.w + (uint64_t)u0 * kUnitBytes;
    const uint32_t st = __builtin_amdgcn_readfirstlane(wring_lds + (s % kDepth) * G::kWStage);
    if (u0 + kSU <= hi) {
#pragma unroll
      for (int i = 0; i < G::kWLoads; ++i)
        if (i < G::kWLoads - 1 || lane < G::kWTail) lds_dma16(base, woff[i], st + 1024 * i);
    } else {
#pragma unroll
      for (int i = 0; i < G::kWLoads; ++i) {
        const uint32_t off = u0 + wunit[i] < hi ? woff[i] : wfirst[i];
        if (i < G::kWLoads - 1 || lane < G::kWTail) lds_dma16(base, off, st + 1024 * i);
      }
    }
  };
  auto issue_x = [&](int s, int ub) {  // ub: strip-relative unit of the stage's first unit
    const uint32_t st = __builtin_amdgcn_readfirstlane(xring_lds + (s % kDepth) * G::kXStage);
    if (ub + kSU <= U) {
      const uint8_t* xb = reinterpret_cast<const uint8_t*>(P.x) + 64 * ub;
#pragma unroll
      for (int n = 0; n < NX; ++n)
        if (lane < G::kXLanes) lds_dma16(xb, xflat[n], st + G::kXRowBytes * n);
    } else {
      int t = ub + xk;
      if (t >= U) t -= U;  // U >= 64 > xk
#pragma unroll
      for (int n = 0; n < NX; ++n)
        if (lane < G::kXLanes) lds_dma16(P.x, xoff[n] + 64u * (uint32_t)t, st + G::kXRowBytes * n);
    }
  };

  // Stages go out whole (weights, then X), kDepth - 1 ahead of the one in
  // use: copies complete in issue order, so the wait for stage s leaves
  // exactly the later stages in flight.
  auto issue = [&](int s) {
    issue_w(s);
    issue_x(s, ub_issue);
    ub_issue += W * kSU;
    while (ub_issue >= U) ub_issue -= U;
  };
#pragma unroll
  for (int s = 0; s < kDepth - 1; ++s)
    if (s < nst) issue(s);
  if (nst == 0) wait_vmcnt<0>();  // no ring wait will cover the status copy

  // parts of the range: one per strip it touches, in order
  const int strip0 = lo / U;
  const int nparts = hi > lo ? (hi - 1) / U - strip0 + 1 : 0;
  int part = 0;
  int part_end = min(hi, (strip0 + 1) * U);

  // The wave that writes the range's last part, when that part begins a
  // strip that later workgroups finish, loads their contributions during
  // its last stage (they stored them at the start of their ranges), so that
  // the loads' latency overlaps arithmetic instead of following it.
  float4_t pre[kStripPrefetch] = {};
  int npre = 0, pre_cnt = 0;
  uint32_t pre_chunk = 0, pre_slot_bytes = 0;
  if (nparts > 0 && wave == (nparts - 1) % W) {
    const int strip = strip0 + nparts - 1;
    const bool starts = max(lo, strip * U) == strip * U, ends = min(hi, (strip + 1) * U) == (strip + 1) * U;
    if (starts && !ends) {
      pre_cnt = strip_owner(P, (strip + 1) * U - 1) - p;
      const int r = lane >> 3;
      pre_chunk = r < P.n ? (uint32_t)(4 * (r * kStripCols + 4 * (lane & 7))) : 0u;
      pre_slot_bytes = (uint32_t)(4 * P.n * kStripCols);
    }
  }
  auto prefetch = [&]() {
    if (pre_cnt < 1 || pre_cnt > kStripPrefetch) return;
#pragma unroll
    for (int i = 0; i < kStripPrefetch; ++i)
      if (i < pre_cnt) pre[i] = load16_coherent(P.slots, (uint32_t)(p + 1 + i) * pre_slot_bytes + pre_chunk);
    npre = pre_cnt;
  };

  float4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  float dacc[NX][2] = {};  // kDot: row n, columns 2j and 2j+1, rows 8q..8q+7 of the units

  auto flush = [&](int pi) {
    float* sl = slots + ((pi & 1) * W + wave) * NX * kStripCols;
    if constexpr (kDot) {
#pragma unroll
      for (int n = 0; n < NX; ++n)
#pragma unroll
        for (int c = 0; c < 2; ++c) {  // the four q lanes of column pair j, in q order
          const float v0 = dacc[n][c], v1 = __shfl_xor(v0, 16), v2 = __shfl_xor(v0, 32), v3 = __shfl_xor(v0, 48);
          dacc[n][c] = q == 0 ? (v0 + v1) + (v2 + v3) : 0.f;
        }
      if (q == 0) {
#pragma unroll
        for (int n = 0; n < NX; ++n) *reinterpret_cast<float2*>(sl + n * kStripCols + 2 * j) = float2{dacc[n][0], dacc[n][1]};
      }
#pragma unroll
      for (int n = 0; n < NX; ++n) dacc[n][0] = dacc[n][1] = 0.f;
    } else if (q < 2) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = 4 * q + v;
        if (r < NX) *reinterpret_cast<float2*>(sl + r * kStripCols + 2 * j) = float2{acc0[v], acc1[v]};
      }
    }
    acc0 = float4_t{0.f, 0.f, 0.f, 0.f};
    acc1 = float4_t{0.f, 0.f, 0.f, 0.f};
    lds_barrier();
    if (wave == pi % W) {
      const int strip = strip0 + pi;
      const int a = max(lo, strip * U), b = min(hi, (strip + 1) * U);
      const bool whole = a == strip * U && b == (strip + 1) * U;
      const bool owner = !whole && a == strip * U;
      strip_part_out<NX, W>(P, slots + (pi & 1) * W * NX * kStripCols, p, strip, whole, owner,
                            (strip + 1) * U - 1, status_poison(status_from_lds(lds_status)), pre,
                            pi == nparts - 1 ? npre : 0);
    }
  };

  // One unit's LDS reads (X slice, the 8 row scales, the 8 bytes of column
  // pair j), then its arithmetic: the reads of a batch of units go out before
  // the first unit's arithmetic.
  struct UnitRegs {
    half8_t a[kDot ? NX : 1];
    uint4 sc;
    uint2 b;
  };
  auto load_unit = [&](UnitRegs& r, const uint8_t* wu, const uint8_t* xu) {
    if constexpr (kDot) {
#pragma unroll
      for (int n = 0; n < NX; ++n) r.a[n] = *reinterpret_cast<const half8_t*>(xu + rxd[n]);
    } else {
      r.a[0] = *reinterpret_cast<const half8_t*>(xu + rx);
    }
    r.sc = *reinterpret_cast<const uint4*>(wu + rsc);
    r.b = *reinterpret_cast<const uint2*>(wu + rpay);
  };
  auto math_unit = [&](const UnitRegs& r) {
    // r.b.x holds rows 0, 2, 1, 3 of column pair j (low nibble: column 2j,
    // high: 2j+1), r.b.y rows 4, 6, 5, 7: bytes 0 and 2 of a word and of the
    // word shifted right by 8 are the row pairs (0,1), (2,3), (4,5), (6,7)
    const uint32_t words[4] = {r.b.x, r.b.x >> 8, r.b.y, r.b.y >> 8};
    const uint32_t scp[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};  // (s_{2p}, s_{2p+1}) per row pair
    half2_t lo2[4], hi2[4];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const half2_t s2 = bitcast<half2_t>(scp[pp]);
      lo2[pp] = nib_lo_pair(words[pp], mw.lo) * s2;
      hi2[pp] = nib_hi_pair(words[pp], mw.hi) * s2;
    }
    half8_t b0, b1;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      b0[2 * pp] = lo2[pp][0];
      b0[2 * pp + 1] = lo2[pp][1];
      b1[2 * pp] = hi2[pp][0];
      b1[2 * pp + 1] = hi2[pp][1];
    }
    if constexpr (kDot) {
#pragma unroll
      for (int n = 0; n < NX; ++n) {
        dacc[n][0] = dot8_f16(r.a[n], b0, dacc[n][0]);
        dacc[n][1] = dot8_f16(r.a[n], b1, dacc[n][1]);
      }
    } else {
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a[0], b0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a[0], b1, acc1, 0, 0, 0);
    }
  };
  auto compute = [&](const uint8_t* wu, const uint8_t* xu) {
    UnitRegs r;
    load_unit(r, wu, xu);
    math_unit(r);
  };

  constexpr int kLS = G::kWLoads + NX;  // copies per stage
  // Issue the stage kDepth - 1 ahead, then wait for stage s (the later
  // stages stay in flight).
  auto next_stage = [&](int s) {
    if (s + kDepth - 1 < nst) issue(s + kDepth - 1);
    const int ahead = min(kDepth - 1, nst - 1 - s);  // stages issued after this one
    if (ahead >= 3) wait_vmcnt<3 * kLS>();
    else if (ahead == 2) wait_vmcnt<2 * kLS>();
    else if (ahead == 1) wait_vmcnt<kLS>();
    else wait_vmcnt<0>();
  };
  int s = 0;
  while (s < nst) {
    // Stages whose units all lie in range and in the current part (u0 + kSU
    // <= part_end <= hi), the last one aside, run in a loop of one path:
    // batches of 4 units, every read of a batch before its arithmetic, the
    // accumulators carried in the same registers from stage to stage.
    const int room = part_end - kSU - first;
    const int s_clean = room < 0 ? s : min(nst - 1, max(s, room / (W * kSU) + 1));
    for (; s < s_clean; ++s) {
      next_stage(s);
      const uint8_t* wst = wring + (s % kDepth) * G::kWStage;
      const uint8_t* xst = xring + (s % kDepth) * G::kXStage;
#pragma unroll
      for (int k0 = 0; k0 < kSU; k0 += 4) {
        UnitRegs r[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) load_unit(r[u], wst + kUnitBytes * (k0 + u), xst + 64 * (k0 + u));
#pragma unroll
        for (int u = 0; u < 4; ++u) math_unit(r[u]);
      }
    }
    if (s >= nst) break;
    // a stage that meets the part's end or the range's end, or the last one
    next_stage(s);
    if (s == nst - 1) prefetch();  // no ring wait follows
    const uint8_t* wst = wring + (s % kDepth) * G::kWStage;
    const uint8_t* xst = xring + (s % kDepth) * G::kXStage;
    const int u0 = first + W * kSU * s;
    const int kmax = min(kSU, hi - u0);
    // units k < kb of this stage belong to the current part; a stage (at
    // most 16 consecutive units, U >= 64) meets at most one part boundary
    const int kb = max(0, min(kmax, part_end - u0));
    // units [k_begin, k_end) of the stage: batches of 4 units, every read
    // of a batch issued before its arithmetic, where a whole batch is in
    // range; single units at the edges
    auto run_units = [&](int k_begin, int k_end) {
      constexpr int kBatch = 4;
#pragma unroll
      for (int k0 = 0; k0 < kSU; k0 += kBatch) {
        if (k0 >= k_begin && k0 + kBatch <= k_end) {
          UnitRegs r[kBatch];
#pragma unroll
          for (int u = 0; u < kBatch; ++u) load_unit(r[u], wst + kUnitBytes * (k0 + u), xst + 64 * (k0 + u));
#pragma unroll
          for (int u = 0; u < kBatch; ++u) math_unit(r[u]);
        } else {
#pragma unroll
          for (int u = 0; u < kBatch; ++u)
            if (k0 + u >= k_begin && k0 + u < k_end) compute(wst + kUnitBytes * (k0 + u), xst + 64 * (k0 + u));
        }
      }
    };
    run_units(0, kb);
    if (kb < kmax) {
      flush(part);
      ++part;
      part_end = min(hi, part_end + U);
      run_units(kb, kmax);
    }
    ++s;
  }
  // the parts this wave has not flushed yet (always the last; also any it
  // holds no unit of)
  for (; part < nparts; ++part) flush(part);
}

// ---------------------------------------------------------------------------
// Host side.

constexpr size_t kStripMaxLds = 156 * 1024;

template <int NX, int kDepth, int W, bool kDot = false>
static hipError_t launch_strips_one(const StripParams& P, int wgs, hipStream_t stream) {
  const size_t lds = StripGeom<NX, W>::template lds_bytes<kDepth>();
  if (lds > kStripMaxLds) return hipErrorInvalidValue;  // never launch past the LDS
  hipLaunchKernelGGL((int4_gemm_strips_kernel<NX, kDepth, W, kDot>), dim3(wgs), dim3(W * 64), lds, stream, P);
  return hipGetLastError();
}

// X rows staged: N rounded up to 1, 2, 4 or 8.  Waves: 4, 8 or 12 (8 rows:
// 4 or 12, the LDS holds no 8-wave ring of them).  A single wave issues a
// vector instruction at most every other cycle slot, so that two or three
// waves a SIMD hide each other's LDS and matrix-core latencies; the plan
// picks 12 for short ranges (their 4-unit stages ramp up sooner), 8 for
// longer ones, and 4 for 8 rows (12 waves copy 8 rows as 8 narrow copies a
// stage, measured slower).  Ring depth 2 unless the caller asks for more (one
// stage in flight a wave keeps the HBM busy; deeper rings measured slower).
int strips_rows_staged(int n) { return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : 8; }
int strips_waves(int n, int waves) {
  if (strips_rows_staged(n) == 8) return waves == 12 ? 12 : 4;
  return waves == 4 || waves == 12 ? waves : 8;
}
template <int NX, int W>
static int strips_max_depth() {
  static_assert(StripGeom<NX, W>::template lds_bytes<2>() <= kStripMaxLds, "a two-stage ring must fit");
  return StripGeom<NX, W>::template lds_bytes<4>() <= kStripMaxLds   ? 4
         : StripGeom<NX, W>::template lds_bytes<3>() <= kStripMaxLds ? 3
                                                                      : 2;
}
int strips_depth(int n, int waves, int depth) {
  const int nx = strips_rows_staged(n);
  const int w = strips_waves(n, waves);
  int max_depth = 2;
  if (w == 12) max_depth = nx == 1 ? strips_max_depth<1, 12>() : nx == 2 ? strips_max_depth<2, 12>()
                          : nx == 4 ? strips_max_depth<4, 12>() : strips_max_depth<8, 12>();
  else if (w == 8) max_depth = nx == 1 ? strips_max_depth<1, 8>() : nx == 2 ? strips_max_depth<2, 8>() : strips_max_depth<4, 8>();
  else max_depth = nx == 1 ? strips_max_depth<1, 4>() : nx == 2 ? strips_max_depth<2, 4>()
                   : nx == 4 ? strips_max_depth<4, 4>() : strips_max_depth<8, 4>();
  return depth <= 2 ? 2 : depth > max_depth ? max_depth : depth;
}

template <int NX, int W>
static hipError_t launch_strips_w(const StripParams& P, int wgs, int depth, hipStream_t stream) {
  if constexpr (StripGeom<NX, W>::template lds_bytes<4>() <= kStripMaxLds)
    if (depth >= 4) return launch_strips_one<NX, 4, W>(P, wgs, stream);
  if constexpr (StripGeom<NX, W>::template lds_bytes<3>() <= kStripMaxLds)
    if (depth >= 3) return launch_strips_one<NX, 3, W>(P, wgs, stream);
  return launch_strips_one<NX, 2, W>(P, wgs, stream);
}

// dot: the v_dot2 variant (n <= 4, ring depth 2).
hipError_t launch_gemm_strips(const uint16_t* x, const uint8_t* w, float* y, int n, int k, int m, int wgs, int depth,
                              int waves, bool dot, float* slots, uint32_t* status, hipStream_t stream) {
  StripParams P = {};
  P.x = x; P.w = w; P.y = y; P.slots = slots; P.status = status;
  P.n = n; P.k = k; P.m = m;
  P.units = k / kUnitRows;
  const int total = (m / kStripCols) * P.units;
  P.base = total / wgs;
  P.rem = total % wgs;
  P.y_vec = (reinterpret_cast<uintptr_t>(y) & 15) == 0 ? 1 : 0;
  const int nx = strips_rows_staged(n);
  waves = strips_waves(n, waves);
  depth = strips_depth(n, waves, depth);
  if (dot) {
    if (nx > 4) return hipErrorInvalidValue;
    if (waves == 12)
      return nx == 1 ? launch_strips_one<1, 2, 12, true>(P, wgs, stream)
             : nx == 2 ? launch_strips_one<2, 2, 12, true>(P, wgs, stream) : launch_strips_one<4, 2, 12, true>(P, wgs, stream);
    if (waves == 8)
      return nx == 1 ? launch_strips_one<1, 2, 8, true>(P, wgs, stream)
             : nx == 2 ? launch_strips_one<2, 2, 8, true>(P, wgs, stream) : launch_strips_one<4, 2, 8, true>(P, wgs, stream);
    return nx == 1 ? launch_strips_one<1, 2, 4, true>(P, wgs, stream)
           : nx == 2 ? launch_strips_one<2, 2, 4, true>(P, wgs, stream) : launch_strips_one<4, 2, 4, true>(P, wgs, stream);
  }
  if (waves == 12) {
    if (nx == 1) return launch_strips_w<1, 12>(P, wgs, depth, stream);
    if (nx == 2) return launch_strips_w<2, 12>(P, wgs, depth, stream);
    if (nx == 4) return launch_strips_w<4, 12>(P, wgs, depth, stream);
    return launch_strips_w<8, 12>(P, wgs, depth, stream);
  }
  if (waves == 8) {
    if (nx == 1) return launch_strips_w<1, 8>(P, wgs, depth, stream);
    if (nx == 2) return launch_strips_w<2, 8>(P, wgs, depth, stream);
    return launch_strips_w<4, 8>(P, wgs, depth, stream);
  }
  if (nx == 1) return launch_strips_w<1, 4>(P, wgs, depth, stream);
  if (nx == 2) return launch_strips_w<2, 4>(P, wgs, depth, stream);
  if (nx == 4) return launch_strips_w<4, 4>(P, wgs, depth, stream);
  return launch_strips_w<8, 4>(P, wgs, depth, stream);
}

// ---------------------------------------------------------------------------
// Wide strips: the strip kernel's walk for up to 32 rows of X in one launch.
//  * the same unit ranges, ring and hand-off as the strip kernel, with 8
//    waves and R = 8, 16 or 32 rows of X (one or two 16-row MFMA tiles on the
//    same decoded weights; with 8 rows, lanes of tile rows 8..15 read row 7
//    and their products are never stored), so that a strip's weights are read
//    once for all N rows and, where the plan gives each workgroup whole
//    strips, nothing is handed between workgroups;
//  * a wave's stage is SU = 1, 2, 4 or (8 rows) 8 consecutive units (one
//    contiguous run of 576 SU bytes of records, and 64 SU contiguous bytes
//    of each X row); the 8 waves' stages are 8 SU consecutive units a round;
//  * its X is R x SU x 64 bytes, rows kRowChunks = 4 SU 16-byte chunks apart,
//    copied as 1 KB copies that each cover 64 / kRowChunks whole rows; chunk
//    c of row r sits at position c ^ wide_swz(r) of its row, so that one
//    quarter of 16 rows falls on 16 different 16-byte bank groups;
//  * at a strip boundary every wave leaves its sums in LDS, and 2 or 4 waves
//    each reduce and write (or hand off) 8 rows of the part.
constexpr int kWideWaves = 8;

template <int R, int SU>
struct WideGeom {
  static_assert(SU == 1 || SU == 2 || SU == 4 || SU == 8, "1, 2, 4 or 8 units a stage");
  static_assert(R == 8 || R == 16 || R == 32, "8, 16 or 32 rows");
  static constexpr int kRows = R;                                // X rows staged (rows past N repeat row N - 1)
  static constexpr int kTiles = (R + 15) / 16;                   // 16-row MFMA tiles
  static constexpr int kStageUnits = SU;                         // a wave's units a stage
  static constexpr int kWChunks = 36 * kStageUnits;              // 288, 144, 72, 36
  static constexpr int kWLoads = (kWChunks + 63) / 64;           // 5, 3, 2, 1
  static constexpr int kWTail = kWChunks - 64 * (kWLoads - 1);   // lanes of the last weight copy: 32, 16, 8, 36
  static constexpr int kWStage = 16 * kWChunks;                  // 4608, 2304, 1152, 576
  static constexpr int kRowChunks = 4 * kStageUnits;             // 16-byte chunks of a row's stage: 32, 16, 8, 4
  static constexpr int kXStage = kRows * 16 * kRowChunks;
  static constexpr int kXLoads = kXStage / 1024;
  static_assert(kXStage % 1024 == 0, "whole 1 KB copies");
  static constexpr int kLS = kWLoads + kXLoads;                  // copies a stage
  static constexpr int kSlotBytes = kRows * kStripCols * 4;      // one wave's sums of a part
  static constexpr int kPasses = kRows / 8;                      // output waves of a part
  template <int kDepth>
  static constexpr int wave_bytes() { return kDepth * (kWStage + kXStage); }
  static constexpr int kGateBytes = kRows * kStripCols * 4;      // SwiGLU epilogue: a gate strip's sums
  template <int kDepth, bool kSwiglu = false>
  static constexpr size_t lds_bytes() {
    return (size_t)kWideWaves * wave_bytes<kDepth>() + (size_t)2 * kWideWaves * kSlotBytes + kStatusLdsBytes +
           (kSwiglu ? kGateBytes : 0);
  }
};

// Position swizzle of a row's chunks: rows r and r + 16 / kRowChunks apart
// get different XOR patterns, so the 16 rows of a quarter spread over 16
// bank groups (kRowChunks = 32 or 16, 8, 4: r & 15, (r >> 1) & 7, (r >> 2) &
// 3; a row of 32 chunks is two whole turns of the 16 bank groups).
template <int SU>
__device__ __forceinline__ int wide_swz(int r) {
  return SU >= 4 ? (r & 15) : SU == 2 ? ((r >> 1) & 7) : ((r >> 2) & 3);
}

// kSwiglu: the matrix is [W_gate | W_up] with their strips interleaved (strip
// 2c gate strip c, 2c + 1 up strip c) and every workgroup holds whole pairs;
// at a gate part the output waves keep its sums in LDS, at the up part that
// follows they write h[r][32c + j] = fp16(silu(g) * u) instead of Y.
template <int R, int SU, int kDepth, bool kSwiglu = false>
__global__ void __launch_bounds__(kWideWaves * 64) int4_gemm_strips_wide_kernel(StripParams P) {
  using G = WideGeom<R, SU>;
  constexpr int NT = G::kTiles;
  constexpr int W = kWideWaves;
  constexpr int kSU = G::kStageUnits;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, j = lane & 15;
  const int p = blockIdx.x;
  const int U = P.units;
  const int lo = p * P.base + min(p, P.rem);
  const int hi = min(lo + P.base + (p < P.rem ? 1 : 0), (P.m / kStripCols) * U);

  // Stage s of wave w: units first + W SU s .. + SU - 1 (first = lo + SU w),
  // so that the workgroup walks W SU consecutive units a round.
  const int first = lo + kSU * wave;
  const int nst = first < hi ? (hi - first + W * kSU - 1) / (W * kSU) : 0;
  uint8_t* wring = smem + wave * G::template wave_bytes<kDepth>();
  uint8_t* xring = wring + kDepth * G::kWStage;
  const uint32_t wring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)wring;
  const uint32_t xring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)xring;
  float* slots = reinterpret_cast<float*>(smem + W * G::template wave_bytes<kDepth>());
  uint32_t* lds_status =
      reinterpret_cast<uint32_t*>(smem + W * G::template wave_bytes<kDepth>() + 2 * W * G::kSlotBytes);
  float* gate_lds = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(lds_status) + kStatusLdsBytes);

  // Weight copies: a wave's stage is SU consecutive units, one contiguous
  // run of 576 SU bytes; slot s = 64 i + lane carries its 16-byte chunk s
  // (unit s / 36); units past the range re-load the stage's first unit.
  uint32_t woff[G::kWLoads], wfirst[G::kWLoads];
  int wunit[G::kWLoads];
#pragma unroll
  for (int i = 0; i < G::kWLoads; ++i) {
    const int s = min(64 * i + lane, G::kWChunks - 1);  // lanes past the last chunk copy nothing
    wunit[i] = s / 36;
    wfirst[i] = (uint32_t)(16 * (s % 36));
    woff[i] = (uint32_t)(16 * s);
  }
  // A stage's copies take per-lane offsets fixed for the whole call (a
  // scalar base moves) unless the stage runs past the range (its weights) or
  // a unit wraps into the next strip (its X): those stages, uniform
  // branches, select per lane.
  auto issue_w = [&](int s) {
    const int u0 = first + W * kSU * s;
    const uint8_t* base = P.w + (uint64_t)u0 * kUnitBytes;
    const uint32_t wst = __builtin_amdgcn_readfirstlane(wring_lds + (s % kDepth) * G::kWStage);
    if (u0 + kSU <= hi) {
#pragma unroll
      for (int i = 0; i < G::kWLoads; ++i)
        if (i < G::kWLoads - 1 || lane < G::kWTail) lds_dma16(base, woff[i], wst + 1024 * i);
    } else {
#pragma unroll
      for (int i = 0; i < G::kWLoads; ++i) {
        const uint32_t off = u0 + wunit[i] < hi ? woff[i] : wfirst[i];
        if (i < G::kWLoads - 1 || lane < G::kWTail) lds_dma16(base, off, wst + 1024 * i);
      }
    }
  };
  // The first stage's weights go out before the rest of the set-up (its
  // X, the status word's copy and the read offsets follow; a stage's copies
  // stay in the order weights, X, and the first ring wait covers all of
  // them).
  if (nst > 0) issue_w(0);
  status_to_lds(P.status, lds_status);

  // X copies: copy i, lane l fills position 64 i + l of the stage: row
  // r = position / kRowChunks, chunk c = (position % kRowChunks) ^
  // wide_swz(r), i.e. quarter c % 4 of the stage's unit c / 4 (rows past N
  // read row N - 1)
  uint32_t xoff[G::kXLoads], xflat[G::kXLoads];
  int xk[G::kXLoads];
#pragma unroll
  for (int i = 0; i < G::kXLoads; ++i) {
    const int pos = 64 * i + lane;
    const int r = pos / G::kRowChunks;
    const int c = (pos % G::kRowChunks) ^ wide_swz<SU>(r);
    xk[i] = c >> 2;
    xoff[i] = (uint32_t)(2 * (min(r, P.n - 1) * P.k + 8 * (c & 3)));
    xflat[i] = xoff[i] + 64u * (uint32_t)xk[i];  // from the stage's first unit when no unit wraps
  }
  int ub_issue = first % U;  // strip-relative unit of the next X stage's first unit
  auto issue_x = [&](int s) {  // stages in order
    const uint32_t xst = __builtin_amdgcn_readfirstlane(xring_lds + (s % kDepth) * G::kXStage);
    if (ub_issue + kSU <= U) {
      const uint8_t* xb = reinterpret_cast<const uint8_t*>(P.x) + 64 * ub_issue;
#pragma unroll
      for (int i = 0; i < G::kXLoads; ++i) lds_dma16(xb, xflat[i], xst + 1024 * i);
    } else {
#pragma unroll
      for (int i = 0; i < G::kXLoads; ++i) {
        int t = ub_issue + xk[i];
        if (t >= U) t -= U;  // U >= 64 > xk
        lds_dma16(P.x, xoff[i] + 64u * (uint32_t)t, xst + 1024 * i);
      }
    }
    ub_issue += W * kSU;
    while (ub_issue >= U) ub_issue -= U;
  };
  auto issue = [&](int s) {
    issue_w(s);
    issue_x(s);
  };
  if (nst > 0) issue_x(0);
#pragma unroll
  for (int s = 1; s < kDepth - 1; ++s)
    if (s < nst) issue(s);
  if (nst == 0) wait_vmcnt<0>();  // no ring wait will cover the status copy

  const MagicWords mw = magic_words();
  // LDS reads of unit k of a stage: record q's 8 row scales, the 8 bytes of
  // column pair j, and quarter q of X row 16 tt + j (past the staged rows:
  // the last one)
  const uint32_t rsc = 144 * q, rpay = 144 * q + 16 + 8 * j;
  uint32_t rx[NT][kSU];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int r = min(16 * tt + j, R - 1);
#pragma unroll
    for (int k = 0; k < kSU; ++k) rx[tt][k] = (uint32_t)(16 * (G::kRowChunks * r + ((4 * k + q) ^ wide_swz<SU>(r))));
  }

  const int strip0 = lo / U;
  const int nparts = hi > lo ? (hi - 1) / U - strip0 + 1 : 0;
  int part = 0;
  int part_end = min(hi, (strip0 + 1) * U);

  float4_t acc[NT][2];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) acc[tt][0] = acc[tt][1] = float4_t{0.f, 0.f, 0.f, 0.f};

  const float4_t no_pre[kStripPrefetch] = {};
  auto flush = [&](int pi) {
    float* sl = slots + ((pi & 1) * W + wave) * G::kRows * kStripCols;
    // tile tt, lane (q, j): rows 16 tt + 4 q + v, columns 2 j and 2 j + 1
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (16 * tt + 4 * q + v < R)
          *reinterpret_cast<float2*>(sl + (16 * tt + 4 * q + v) * kStripCols + 2 * j) = float2{acc[tt][0][v], acc[tt][1][v]};
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) acc[tt][0] = acc[tt][1] = float4_t{0.f, 0.f, 0.f, 0.f};
    lds_barrier();
    // rows 8 rp .. 8 rp + 7 of the part: wave (kPasses pi + rp) % W
    const int rp = (wave - (G::kPasses * pi) % W + W) % W;
    if (rp < G::kPasses && 8 * rp < P.n) {
      const int strip = strip0 + pi;
      if constexpr (kSwiglu) {  // whole strips: the plan gives every workgroup whole gate/up pairs
        const float* sl = slots + (pi & 1) * W * G::kRows * kStripCols;
        const int r = 8 * rp + (lane >> 3), c4 = 4 * (lane & 7);
        if (r < P.n) {
          float4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int w = 0; w < W; ++w)  // in wave order
            v += *reinterpret_cast<const float4_t*>(sl + w * G::kRows * kStripCols + r * kStripCols + c4);
          float4_t* g = reinterpret_cast<float4_t*>(gate_lds + r * kStripCols + c4);
          if ((strip & 1) == 0) {
            *g = v;
          } else {
            const float poison = status_poison(status_from_lds(lds_status));
            *reinterpret_cast<uint2*>(P.h + (int64_t)r * (P.m / 2) + kStripCols * (strip >> 1) + c4) =
                swiglu4(poisoned(*g, poison), v);
          }
        }
      } else {
        const int a = max(lo, strip * U), b = min(hi, (strip + 1) * U);
        const bool whole = a == strip * U && b == (strip + 1) * U;
        const bool owner = !whole && a == strip * U;
        strip_part_out<G::kRows, W>(P, slots + (pi & 1) * W * G::kRows * kStripCols, p, strip, whole, owner,
                                    (strip + 1) * U - 1, status_poison(status_from_lds(lds_status)), no_pre, 0,
                                    8 * rp);
      }
    }
  };

  struct UnitRegs {
    half8_t a[NT];
    uint4 sc;
    uint2 b;
  };
  auto load_unit = [&](UnitRegs& r, const uint8_t* wst, const uint8_t* xst, int k) {
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) r.a[tt] = *reinterpret_cast<const half8_t*>(xst + rx[tt][k]);
    r.sc = *reinterpret_cast<const uint4*>(wst + kUnitBytes * k + rsc);
    r.b = *reinterpret_cast<const uint2*>(wst + kUnitBytes * k + rpay);
  };
  auto math_unit = [&](const UnitRegs& r) {
    // r.b.x holds rows 0, 2, 1, 3 of column pair j, r.b.y rows 4, 6, 5, 7
    const uint32_t words[4] = {r.b.x, r.b.x >> 8, r.b.y, r.b.y >> 8};
    const uint32_t scp[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
    half8_t b0, b1;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const half2_t s2 = bitcast<half2_t>(scp[pp]);
      const half2_t lo2 = nib_lo_pair(words[pp], mw.lo) * s2;
      const half2_t hi2 = nib_hi_pair(words[pp], mw.hi) * s2;
      b0[2 * pp] = lo2[0];
      b0[2 * pp + 1] = lo2[1];
      b1[2 * pp] = hi2[0];
      b1[2 * pp + 1] = hi2[1];
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      acc[tt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a[tt], b0, acc[tt][0], 0, 0, 0);
      acc[tt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a[tt], b1, acc[tt][1], 0, 0, 0);
    }
  };

  // Issue the stage kDepth - 1 ahead, then wait for stage s (the later
  // stages stay in flight).
  auto next_stage = [&](int s) {
    if (s + kDepth - 1 < nst) issue(s + kDepth - 1);
    const int ahead = min(kDepth - 1, nst - 1 - s);  // stages issued after this one
    if (ahead >= 3) wait_vmcnt<3 * G::kLS>();
    else if (ahead == 2) wait_vmcnt<2 * G::kLS>();
    else if (ahead == 1) wait_vmcnt<G::kLS>();
    else wait_vmcnt<0>();
  };
  int s = 0;
  while (s < nst) {
    // Stages whose units all lie in range and in the current part (u0 + SU
    // <= part_end <= hi) run in a loop of one path: every read of the stage,
    // then its arithmetic, the accumulators carried in the same registers
    // from stage to stage.
    const int room = part_end - kSU - first;
    const int s_clean = room < 0 ? s : min(nst, max(s, room / (W * kSU) + 1));
    for (; s < s_clean; ++s) {
      next_stage(s);
      const uint8_t* wst = wring + (s % kDepth) * G::kWStage;
      const uint8_t* xst = xring + (s % kDepth) * G::kXStage;
      UnitRegs r[kSU];
#pragma unroll
      for (int k = 0; k < kSU; ++k) load_unit(r[k], wst, xst, k);
#pragma unroll
      for (int k = 0; k < kSU; ++k) math_unit(r[k]);
    }
    if (s >= nst) break;
    // a stage that meets the part's end or the range's end
    next_stage(s);
    const uint8_t* wst = wring + (s % kDepth) * G::kWStage;
    const uint8_t* xst = xring + (s % kDepth) * G::kXStage;
    const int u0 = first + W * kSU * s;
    const int kmax = min(kSU, hi - u0);
    // units k < kb of this stage belong to the current part; a stage (SU
    // consecutive units, U >= 64) meets at most one part boundary
    const int kb = max(0, min(kmax, part_end - u0));
    // units [k_begin, k_end) of the stage, every read of the stage issued
    // before its arithmetic where the whole stage is in range
    auto run_units = [&](int k_begin, int k_end) {
      if (k_begin == 0 && k_end == kSU) {
        UnitRegs r[kSU];
#pragma unroll
        for (int k = 0; k < kSU; ++k) load_unit(r[k], wst, xst, k);
#pragma unroll
        for (int k = 0; k < kSU; ++k) math_unit(r[k]);
      } else {
#pragma unroll
        for (int k = 0; k < kSU; ++k)
          if (k >= k_begin && k < k_end) {
            UnitRegs r;
            load_unit(r, wst, xst, k);
            math_unit(r);
          }
      }
    };
    run_units(0, kb);
    if (kb < kmax) {
      flush(part);
      ++part;
      part_end = min(hi, part_end + U);
      run_units(kb, kmax);
    }
    ++s;
  }
  for (; part < nparts; ++part) flush(part);
}

constexpr size_t kWideMaxLds = 156 * 1024;

template <int R, int SU, int kDepth, bool kSwiglu = false>
static hipError_t launch_wide_one(const StripParams& P, int wgs, hipStream_t stream) {
  const size_t lds = WideGeom<R, SU>::template lds_bytes<kDepth, kSwiglu>();
  if (lds > kWideMaxLds) return hipErrorInvalidValue;  // never launch past the LDS
  hipLaunchKernelGGL((int4_gemm_strips_wide_kernel<R, SU, kDepth, kSwiglu>), dim3(wgs), dim3(kWideWaves * 64), lds,
                     stream, P);
  return hipGetLastError();
}

// The deepest ring up to `depth` (2..4) that the LDS holds for SU units a
// stage; hipErrorInvalidValue when not even two stages fit.
template <int R, int SU>
static hipError_t launch_wide_su(const StripParams& P, int wgs, int depth, hipStream_t stream) {
  using G = WideGeom<R, SU>;
  if constexpr (G::template lds_bytes<4>() <= kWideMaxLds)
    if (depth >= 4) return launch_wide_one<R, SU, 4>(P, wgs, stream);
  if constexpr (G::template lds_bytes<3>() <= kWideMaxLds)
    if (depth >= 3) return launch_wide_one<R, SU, 3>(P, wgs, stream);
  if constexpr (G::template lds_bytes<2>() <= kWideMaxLds) return launch_wide_one<R, SU, 2>(P, wgs, stream);
  return hipErrorInvalidValue;
}

// Rows staged: N rounded up to 8, 16 or 32.  su: units a stage (0: 4 up to
// 16 rows, 2 for 32 rows, whose 4-unit ring the LDS does not hold --
// measured fastest; 8 rows take 2, 4 or 8); depth: ring stages (0: 2,
// measured fastest).
hipError_t launch_gemm_strips_wide(const uint16_t* x, const uint8_t* w, float* y, int n, int k, int m, int wgs,
                                   int su, int depth, float* slots, uint32_t* status, hipStream_t stream) {
  StripParams P = {};
  P.x = x; P.w = w; P.y = y; P.slots = slots; P.status = status;
  P.n = n; P.k = k; P.m = m;
  P.units = k / kUnitRows;
  const int total = (m / kStripCols) * P.units;
  P.base = total / wgs;
  P.rem = total % wgs;
  P.y_vec = (reinterpret_cast<uintptr_t>(y) & 15) == 0 ? 1 : 0;
  if (depth <= 0) depth = 2;
  if (su <= 0) su = n <= 16 ? 4 : 2;
  if (n <= 8) {
    if (su == 2) return launch_wide_su<8, 2>(P, wgs, depth, stream);
    if (su == 8) return launch_wide_su<8, 8>(P, wgs, depth, stream);
    return launch_wide_su<8, 4>(P, wgs, depth, stream);
  }
  if (n <= 16) {
    if (su == 1) return launch_wide_su<16, 1>(P, wgs, depth, stream);
    if (su == 2) return launch_wide_su<16, 2>(P, wgs, depth, stream);
    return launch_wide_su<16, 4>(P, wgs, depth, stream);
  }
  if (su == 1) return launch_wide_su<32, 1>(P, wgs, depth, stream);
  return launch_wide_su<32, 2>(P, wgs, depth, stream);
}

// The wide strip kernel with its SwiGLU epilogue over the interleaved
// [W_gate | W_up] stream of 2m columns (m gate and m up columns): wgs
// workgroups of `per` gate/up pairs each (the last one the rest), each
// writing h[.][32c ..) for its pairs c; rows staged and stage size as the
// automatic plan's.
hipError_t launch_gemm_strips_swiglu(const uint16_t* x, const uint8_t* w, uint16_t* h, int n, int k, int m, int wgs,
                                     int per, hipStream_t stream) {
  StripParams P = {};
  P.x = x; P.w = w; P.h = h;
  P.n = n; P.k = k; P.m = 2 * m;
  P.units = k / kUnitRows;
  P.base = 2 * per * P.units;  // whole pairs; the kernel cuts the last range at the last unit
  P.rem = 0;
  if (n <= 8) return launch_wide_one<8, 4, 2, true>(P, wgs, stream);
  if (n <= 16) return launch_wide_one<16, 4, 2, true>(P, wgs, stream);
  return launch_wide_one<32, 2, 2, true>(P, wgs, stream);
}

// ---------------------------------------------------------------------------
// Strip groups: the GEMM over strip order for 9 <= N <= 32 in one pass.
//  * strips are taken 8 at a time (a group, 256 columns); the (group, unit)
//    items form one stream (group-major), and workgroup p takes an equal
//    contiguous range of it, as the strip kernel does with units;
//  * the 8 waves of a workgroup walk the range's units together, wave w on
//    strip 8g + w of the unit's group g: each keeps a private ring of
//    `depth` stages of 4 units (2304 bytes), and the X rows of a stage's 4
//    units (N rounded up to 16 or 32, 256 bytes a row) are staged once for
//    all 8 waves (one 1 KB copy per wave), behind one barrier a stage;
//  * per unit a wave decodes its strip's 32 x 32 block exactly as the strip
//    kernel does and multiplies it by one or two 16-row tiles of X
//    (v_mfma_f32_16x16x32_f16, the decoded operands reused by both tiles);
//  * a wave owns its strip's sums: at a group boundary it writes them to Y
//    (whole), or stores them (device-coherent) for the workgroup that began
//    the group -- the workgroup's waves meet at a barrier and wave 0 raises
//    the workgroup's flag with an agent-scope release -- or, owning the
//    group's start, waits for every later workgroup's flag (wave 0, bounded
//    polling as in the strip kernel's hand-off), acquires once (the L2 may
//    hold stale copies of their slots), shares the outcome through LDS, and
//    every wave loads and adds their sums in workgroup order, zeroes their
//    slots and writes Y.  No cross-wave sums.  (The sums travel as
//    plain fp32 behind a flag rather than complement-encoded like the strip
//    kernel's: encoding the accumulators in place gave wrong words in a few
//    lanes on the GPU, a schedule-dependent failure traced to the encode and
//    not further; the flag protocol has no such step.)
constexpr int kGroupWaves = 8;       // strips of a group, one a wave
constexpr int kGroupStageUnits = 4;  // units of a stage
constexpr int kGroupWStage = kGroupStageUnits * kUnitBytes;       // 2304: 2 full copies + 16 lanes
constexpr int kGroupWLoads = (36 * kGroupStageUnits + 63) / 64;   // 3
constexpr int kGroupWTail = 36 * kGroupStageUnits - 64 * (kGroupWLoads - 1);  // 16

struct GroupParams {
  const uint16_t* x;   // [n][k] fp16, 16-byte aligned
  const uint8_t* w;    // strip-order records (fewer than 2^32 bytes)
  float* y;            // [n][m] fp32
  float* slots;        // per (workgroup, wave) NT x 2 KB of fp32 sums; null when nothing is shared
  uint32_t* status;    // workspace status word, followed after 256 bytes by one flag word per
                       // workgroup; null when nothing is shared
  int n, k, m;
  int units;           // units per strip, k / 32
  int strips;          // m / 32
  int base, rem;       // workgroup p covers items [p*base + min(p, rem), +base + (p < rem))
  int y_vec8;          // y 8-byte aligned
};

template <bool B>
struct FlushTag {
  static constexpr bool value = B;
};

template <int NT>
struct GroupGeom {
  static constexpr int kRows = 16 * NT;      // X rows staged (rows past N repeat row N - 1)
  static constexpr int kXLoads = kRows / 4;  // 1 KB copies: 4 rows x 4 units x 64 bytes
  static constexpr int kXStage = kRows * 256;
  static constexpr int kSlotBytes = NT * 2 * 64 * 16;  // one wave's sums: (tile, column half, lane) x 16 bytes
  template <int kDepth>
  static constexpr size_t lds_bytes() {
    return kStatusLdsBytes + (size_t)kDepth * (kXStage + kGroupWaves * kGroupWStage);
  }
};

// Workgroup holding item t of the group stream.
__device__ __forceinline__ int group_owner(const GroupParams& P, int t) {
  const int big = P.rem * (P.base + 1);
  return t < big ? t / (P.base + 1) : P.rem + (t - big) / P.base;
}

template <int NT, int kDepth>
__global__ void __launch_bounds__(kGroupWaves * 64) int4_gemm_strip_groups_kernel(GroupParams P) {
  using G = GroupGeom<NT>;
  constexpr int kSU = kGroupStageUnits;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, j = lane & 15;
  const int p = blockIdx.x;
  const int U = P.units;
  const int lo = p * P.base + min(p, P.rem);
  const int hi = lo + P.base + (p < P.rem ? 1 : 0);
  const MagicWords mw = magic_words();

  uint32_t* lds_status = reinterpret_cast<uint32_t*>(smem);
  uint8_t* xring = smem + kStatusLdsBytes;
  uint8_t* wring = xring + kDepth * G::kXStage + wave * kDepth * kGroupWStage;
  const uint32_t xring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)xring;
  const uint32_t wring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)wring;
  status_to_lds(P.status, lds_status);  // the oldest copy: the first ring wait covers it

  // Weight copies: slot c = 64 i + lane carries chunk c % 36 of the stage's
  // unit c / 36 (lanes past the 144 chunks copy nothing).
  int wunit[kGroupWLoads];
  uint32_t wchunk[kGroupWLoads];
#pragma unroll
  for (int i = 0; i < kGroupWLoads; ++i) {
    const int c = min(64 * i + lane, 36 * kSU - 1);
    wunit[i] = c / 36;
    wchunk[i] = (uint32_t)(16 * (c % 36));
  }
  // X copy of this wave: rows 4xc .. 4xc+3 (waves past the copies repeat
  // them: the same bytes to the same place).  Lane l: row 4xc + l / 16,
  // physical unit ((l >> 2) & 3) holds unit (physical - row) & 3 of the
  // stage, physical quarter (l & 3) holds quarter (l & 3) ^ ((row >> 2) & 3):
  // a quarter of 16 rows falls on 16 different 16-byte bank groups.
  const int xc = wave % G::kXLoads;
  const int xr = 4 * xc + (lane >> 4);
  const int xk = (((lane >> 2) & 3) - xr) & 3;
  const uint32_t xrow_off = (uint32_t)(2 * (min(xr, P.n - 1) * P.k + 8 * ((lane & 3) ^ ((xr >> 2) & 3))));
  // LDS reads: record q's scales and column pair j's 8 bytes of a unit; X
  // row 16 tt + j (rows past N read row N - 1), quarter q, of unit k
  const uint32_t rsc = 144 * q, rpay = 144 * q + 16 + 8 * j;
  uint32_t rx[NT][kSU];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int rr = min(16 * tt + j, P.n - 1);
#pragma unroll
    for (int k = 0; k < kSU; ++k) rx[tt][k] = (uint32_t)(256 * rr + 64 * ((k + rr) & 3) + 16 * (q ^ ((rr >> 2) & 3)));
  }

  const int nst = (hi - lo + kSU - 1) / kSU;  // the same for every wave
  // group and strip-relative unit of the next stage to issue (scalars)
  int g_issue = lo / U, u_issue = lo - g_issue * U;
  // A stage's copies: the wave's own weights (its private ring) and its
  // share of the workgroup's X stage; g_issue / u_issue advance after the X.
  auto issue_w = [&](int s) {
    const int t0 = lo + kSU * s;
    const uint32_t wst = __builtin_amdgcn_readfirstlane(wring_lds + (s % kDepth) * kGroupWStage);
#pragma unroll
    for (int i = 0; i < kGroupWLoads; ++i) {
      int g = g_issue, u = u_issue + wunit[i];
      if (u >= U) { u -= U; ++g; }
      if (t0 + wunit[i] >= hi) { g = g_issue; u = u_issue; }  // past the range: the stage's first unit
      const int strip = min(kGroupWaves * g + wave, P.strips - 1);  // waves past the last strip copy a real one
      const uint32_t off = (uint32_t)(strip * U + u) * (uint32_t)kUnitBytes + wchunk[i];
      if (i < kGroupWLoads - 1 || lane < kGroupWTail) lds_dma16(P.w, off, wst + 1024 * i);
    }
  };
  auto issue_x = [&](int s) {
    const int t0 = lo + kSU * s;
    int ux = u_issue + xk;
    if (ux >= U) ux -= U;
    if (t0 + xk >= hi) ux = u_issue;
    lds_dma16(P.x, xrow_off + 64u * (uint32_t)ux,
              __builtin_amdgcn_readfirstlane(xring_lds + (s % kDepth) * G::kXStage + 1024 * xc));
    u_issue += kSU;
    if (u_issue >= U) { u_issue -= U; ++g_issue; }
  };
  auto issue = [&](int s) {
    issue_w(s);
    issue_x(s);
  };
#pragma unroll
  for (int s = 0; s < kDepth - 1; ++s)
    if (s < nst) issue(s);
  if (nst == 0) wait_vmcnt<0>();

  // parts: one per group the range touches
  int gcur = lo / U;
  int part_end = min(hi, (gcur + 1) * U);
  float4_t acc[NT][2];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) acc[tt][0] = acc[tt][1] = float4_t{0.f, 0.f, 0.f, 0.f};

  // Group boundary.  Every wave of the workgroup flushes the same part at
  // the same point (they walk the same units), so the hand-off can use
  // workgroup barriers: one flag per contributing workgroup.  A part that
  // ends inside the range ends at its group's end, so only the range's last
  // part can be an owner's: the flushes inside the stage loop store or write
  // (kLast false: no hand-off loads there, none of their registers pending
  // across the loop), the one after it may also gather.
  uint32_t* lds_flag = lds_status + 1;  // owner: the poll's outcome, for all waves
  auto flush = [&](auto last_tag) {
    constexpr bool kLast = decltype(last_tag)::value;
    const int strip = kGroupWaves * gcur + wave;
    const int a = max(lo, gcur * U), b = min(hi, (gcur + 1) * U);
    const bool whole = a == gcur * U && b == (gcur + 1) * U;
    const bool owner = !whole && a == gcur * U;
    const __amdgpu_buffer_rsrc_t srs = coherent_rsrc(P.slots);
    uint32_t* flags = P.status + kWsStatusBytes / 4;  // one word per workgroup, zero between calls
    constexpr int kChunks = NT * 2 * 64;               // float4 chunks of one wave's sums
    // byte offset of chunk h of the sums of workgroup c's wave
    auto slot_off = [&](int c, int h) { return (uint32_t)(16 * ((c * kGroupWaves + wave) * kChunks + h * 64 + lane)); };
    if (!whole && !owner) {  // the first part of the range: stored for the group's first workgroup
      if (strip < P.strips) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
          for (int h = 0; h < 2; ++h) store16_sc1(srs, slot_off(p, 2 * tt + h), acc[tt][h]);
      }
      asm volatile("" ::: "memory");
      // the sums go out as 16-byte device-coherent stores (whole lines a
      // wave, where two 8-byte atomics a lane would write each line twice),
      // complete (vmcnt counts stores) in every wave before wave 0 raises
      // the flag
      wait_vmcnt<0>();
      lds_barrier();
      if (wave == 0) __hip_atomic_store(flags + p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      bool gave_up = false;
      if constexpr (kLast) {
        if (owner) {  // add the later workgroups' sums of this group, in workgroup order
          const int q_last = group_owner(P, (gcur + 1) * U - 1);
          if (wave == 0) {  // every later workgroup's flag, one lane each, polled together
            int polls = kMaxPolls;
            bool all = true;
            for (int c0 = p + 1; c0 <= q_last; c0 += 64) {
              const int c = c0 + lane;
              bool seen = c > q_last;
              for (;;) {
                if (!seen) seen = __hip_atomic_load(flags + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
                if (handoff_stop(__ballot(!seen) == 0ull, polls)) break;
                --polls;
                __builtin_amdgcn_s_sleep(1);
              }
              all = all && __ballot(!seen) == 0ull;
              if (c <= q_last) __hip_atomic_store(flags + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (!all && lane == 0)
              __hip_atomic_fetch_or(P.status, kWsStatusHandoffTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0) *lds_flag = all ? 1u : 0u;
          }
          lds_barrier();
          gave_up = status_from_lds(lds_flag) == 0u;
          if (strip < P.strips) {
            // device-coherent loads of kBatch workgroups' sums at a time, all
            // issued before the first add (past the last workgroup a batch
            // re-reads the last one's slot), added in workgroup order; then
            // the slots are cleared (the last one's again, past the end):
            // the workspace is left as found (zero), since the other kernels
            // sharing it take any non-zero slot word for a written partial
            constexpr int kBatch = 8 / NT;
            for (int c0 = p + 1; c0 <= q_last; c0 += kBatch) {
              float4_t t[kBatch][2 * NT];
#pragma unroll
              for (int i = 0; i < kBatch; ++i)
#pragma unroll
                for (int h = 0; h < 2 * NT; ++h) t[i][h] = load16_sc1(srs, slot_off(min(c0 + i, q_last), h));
              wait_vmcnt<0>();  // every load has read its slot before the slots are cleared
#pragma unroll
              for (int i = 0; i < kBatch; ++i)
                if (c0 + i <= q_last) {
#pragma unroll
                  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
                    for (int h = 0; h < 2; ++h) acc[tt][h] += t[i][2 * tt + h];
                }
#pragma unroll
              for (int i = 0; i < kBatch; ++i)
#pragma unroll
                for (int h = 0; h < 2 * NT; ++h)
                  store16_sc1(srs, slot_off(min(c0 + i, q_last), h), float4_t{0.f, 0.f, 0.f, 0.f});
            }
          }
        }
      }
      if (strip < P.strips) {
        const float poison = status_poison(status_from_lds(lds_status) | (gave_up ? 1u : 0u));
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 16 * tt + 4 * q + v;
            if (r < P.n) {
              float* yp = P.y + (int64_t)r * P.m + kStripCols * strip + 2 * j;
              const float y0 = acc[tt][0][v] + poison, y1 = acc[tt][1][v] + poison;
              if (P.y_vec8) {
                *reinterpret_cast<float2*>(yp) = float2{y0, y1};
              } else {
                yp[0] = y0;
                yp[1] = y1;
              }
            }
          }
      }
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) acc[tt][0] = acc[tt][1] = float4_t{0.f, 0.f, 0.f, 0.f};
  };

  struct UnitRegs {
    half8_t a[NT];
    uint4 sc;
    uint2 b;
  };
  auto load_unit = [&](UnitRegs& r, const uint8_t* wst, const uint8_t* xst, int k) {
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) r.a[tt] = *reinterpret_cast<const half8_t*>(xst + rx[tt][k]);
    r.sc = *reinterpret_cast<const uint4*>(wst + kUnitBytes * k + rsc);
    r.b = *reinterpret_cast<const uint2*>(wst + kUnitBytes * k + rpay);
  };
  auto math_unit = [&](const UnitRegs& r) {
    const uint32_t words[4] = {r.b.x, r.b.x >> 8, r.b.y, r.b.y >> 8};  // rows (0,1), (2,3), (4,5), (6,7)
    const uint32_t scp[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
    half8_t b0, b1;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const half2_t s2 = bitcast<half2_t>(scp[pp]);
      const half2_t lo2 = nib_lo_pair(words[pp], mw.lo) * s2;
      const half2_t hi2 = nib_hi_pair(words[pp], mw.hi) * s2;
      b0[2 * pp] = lo2[0];
      b0[2 * pp + 1] = lo2[1];
      b1[2 * pp] = hi2[0];
      b1[2 * pp + 1] = hi2[1];
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      acc[tt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a[tt], b0, acc[tt][0], 0, 0, 0);
      acc[tt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a[tt], b1, acc[tt][1], 0, 0, 0);
    }
  };

  for (int s = 0; s < nst; ++s) {
    if constexpr (kDepth == 2) {
      // the wave's own weights for stage s + 1 go out before the wait (its
      // ring slot held stage s - 1, which this wave has finished), the X
      // share after the barrier (every wave has finished reading stage
      // s - 1's X): the weights stay two stages ahead
      const bool more = s + 1 < nst;
      if (more) issue_w(s + 1);
      if (more) wait_vmcnt<kGroupWLoads>();  // stage s landed; W(s + 1) in flight
      else wait_vmcnt<0>();
      lds_barrier();  // every wave's copies of stage s have landed
      if (more) issue_x(s + 1);
    } else {
      // stages issued after this one (all waves alike)
      const int ahead = min(kDepth - 2, nst - 1 - s);
      if (ahead >= 2) wait_vmcnt<2 * (kGroupWLoads + 1)>();
      else if (ahead == 1) wait_vmcnt<kGroupWLoads + 1>();
      else wait_vmcnt<0>();
      // every wave's copies of stage s have landed, and every wave is done
      // with stage s - 1, whose buffers the next issue refills
      lds_barrier();
      if (s + kDepth - 1 < nst) issue(s + kDepth - 1);
    }
    const uint8_t* wst = wring + (s % kDepth) * kGroupWStage;
    const uint8_t* xst = xring + (s % kDepth) * G::kXStage;
    const int t0 = lo + kSU * s;
    const int kmax = min(kSU, hi - t0);
    int kb = part_end - t0;  // units k < kb belong to the current part (a stage meets at most one boundary)
    kb = kb <= 0 ? 0 : min(kmax, kb);
    auto run_units = [&](int k_begin, int k_end) {
#pragma unroll
      for (int k0 = 0; k0 < kSU; k0 += 2) {
        if (k0 >= k_begin && k0 + 2 <= k_end) {
          UnitRegs r0, r1;
          load_unit(r0, wst, xst, k0);
          load_unit(r1, wst, xst, k0 + 1);
          math_unit(r0);
          math_unit(r1);
        } else {
#pragma unroll
          for (int u = 0; u < 2; ++u)
            if (k0 + u >= k_begin && k0 + u < k_end) {
              UnitRegs r;
              load_unit(r, wst, xst, k0 + u);
              math_unit(r);
            }
        }
      }
    };
    run_units(0, kb);
    if (kb < kmax) {
      flush(FlushTag<false>{});
      ++gcur;
      part_end = min(hi, part_end + U);
      run_units(kb, kmax);
    }
  }
  if (hi > lo) flush(FlushTag<true>{});  // the last part
}

constexpr size_t kGroupMaxLds = 156 * 1024;

template <int NT, int kDepth>
static hipError_t launch_groups_one(const GroupParams& P, int wgs, hipStream_t stream) {
  const size_t lds = GroupGeom<NT>::template lds_bytes<kDepth>();
  if (lds > kGroupMaxLds) return hipErrorInvalidValue;
  hipLaunchKernelGGL((int4_gemm_strip_groups_kernel<NT, kDepth>), dim3(wgs), dim3(kGroupWaves * 64), lds, stream, P);
  return hipGetLastError();
}

int strip_groups_slot_bytes(int n) { return n <= 16 ? GroupGeom<1>::kSlotBytes : GroupGeom<2>::kSlotBytes; }

hipError_t launch_gemm_strip_groups(const uint16_t* x, const uint8_t* w, float* y, int n, int k, int m, int wgs,
                                    int depth, float* slots, uint32_t* status, hipStream_t stream) {
  GroupParams P = {};
  P.x = x; P.w = w; P.y = y; P.slots = slots; P.status = status;
  P.n = n; P.k = k; P.m = m;
  P.units = k / kUnitRows;
  P.strips = m / kStripCols;
  const int groups = (P.strips + kGroupWaves - 1) / kGroupWaves;
  const int total = groups * P.units;
  P.base = total / wgs;
  P.rem = total % wgs;
  P.y_vec8 = (reinterpret_cast<uintptr_t>(y) & 7) == 0 ? 1 : 0;
  const bool deep = depth >= 3;
  if (n <= 16) return deep ? launch_groups_one<1, 3>(P, wgs, stream) : launch_groups_one<1, 2>(P, wgs, stream);
  return deep ? launch_groups_one<2, 3>(P, wgs, stream) : launch_groups_one<2, 2>(P, wgs, stream);
}

// Records of W[K][M] from row order to strip order: one thread per 16-byte
// chunk of the output (record (g, b): chunk 0 = the 8 scales of rows 8b ..
// 8b+7, gathered from 8 row-order records; chunk c = 1..8 = payload bytes
// 2(c-1) and 2(c-1)+1 of rows 8b .. 8b+7, two bytes from each row's chunk).
__global__ void records_to_strips_kernel(const uint8_t* __restrict__ src, int64_t k, int64_t m,
                                         uint4* __restrict__ dst) {
  const int64_t strips = m / kStripCols, blocks = k / 8;
  const int64_t chunks = strips * blocks * 9;
  const int64_t gpr = m / kStripCols;  // groups per row
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < chunks; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rec = e / 9, c = e - rec * 9;
    const int64_t g = rec / blocks, b = rec - g * blocks;
    if (c == 0) {
      uint32_t h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t f0 = (8 * b + 2 * i) * gpr + g, f1 = f0 + gpr;  // flat groups of rows 8b+2i, 8b+2i+1
        const uint32_t s0 = *reinterpret_cast<const uint16_t*>(src + group_scale_offset(f0));
        const uint32_t s1 = *reinterpret_cast<const uint16_t*>(src + group_scale_offset(f1));
        h[i] = s0 | (s1 << 16);
      }
      dst[e] = uint4{h[0], h[1], h[2], h[3]};
    } else {
      // output bytes 0-7: byte j0 of rows 8b .. 8b+7, bytes 8-15: byte j0+1,
      // row i at position strip_row_pos(i)
      const int64_t j0 = 2 * (c - 1);
      uint32_t lo[2] = {0u, 0u}, hi[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t f = (8 * b + i) * gpr + g;
        const uint32_t two = *reinterpret_cast<const uint16_t*>(src + group_payload_offset(f) + j0);
        const int pos = strip_row_pos(i);
        lo[pos >> 2] |= (two & 0xFFu) << (8 * (pos & 3));
        hi[pos >> 2] |= (two >> 8) << (8 * (pos & 3));
      }
      dst[e] = uint4{lo[0], lo[1], hi[0], hi[1]};
    }
  }
}

// Strip order back to row order: one thread per 16-byte chunk of the output
// (row-order record R: chunk 0 = the scales of flat groups 8R .. 8R+7, chunk
// c = 1..8 = the 16 payload bytes of flat group 8R + c - 1), each byte
// gathered from its strip record.
__global__ void strips_to_records_kernel(const uint8_t* __restrict__ strips, int64_t k, int64_t m,
                                         uint4* __restrict__ dst) {
  const int64_t gpr = m / kStripCols, blocks = k / 8;  // groups per row, records per strip
  const int64_t chunks = (k * gpr / 8) * 9;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < chunks; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rec = e / 9, c = e - rec * 9;
    if (c == 0) {
      uint32_t h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t two[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int64_t f = 8 * rec + 2 * i + t, r = f / gpr, g = f - r * gpr;
          const uint8_t* sr = strips + (g * blocks + r / 8) * 144;
          two[t] = *reinterpret_cast<const uint16_t*>(sr + 2 * (r % 8));
        }
        h[i] = two[0] | (two[1] << 16);
      }
      dst[e] = uint4{h[0], h[1], h[2], h[3]};
    } else {
      const int64_t f = 8 * rec + c - 1, r = f / gpr, g = f - r * gpr;
      const uint8_t* sr = strips + (g * blocks + r / 8) * 144 + 16 + strip_row_pos((int)(r % 8));
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int jb = 0; jb < 16; ++jb) w[jb >> 2] |= (uint32_t)sr[8 * jb] << (8 * (jb & 3));
      dst[e] = uint4{w[0], w[1], w[2], w[3]};
    }
  }
}

hipError_t launch_strips_to_records(const uint8_t* strips, int k, int m, uint8_t* sb, hipStream_t stream) {
  const int64_t chunks = ((int64_t)k * (m / kStripCols) / 8) * 9;
  if (chunks == 0) return hipSuccess;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(strips_to_records_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, strips, (int64_t)k,
                     (int64_t)m, reinterpret_cast<uint4*>(sb));
  return hipGetLastError();
}

hipError_t launch_records_to_strips(const uint8_t* sb, int k, int m, uint8_t* strips, hipStream_t stream) {
  const int64_t chunks = (int64_t)(m / kStripCols) * (k / 8) * 9;
  if (chunks == 0) return hipSuccess;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(records_to_strips_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, sb, (int64_t)k,
                     (int64_t)m, reinterpret_cast<uint4*>(strips));
  return hipGetLastError();
}

}  // namespace moat
