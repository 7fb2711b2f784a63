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
//    [0,16) are the 8 fp16 scales of those rows' group g; byte 16 + 8j + i is
//    byte j of row 8b+i's 16 payload bytes of group g (column 32g + 2j in the
//    low nibble, 32g + 2j + 1 in the high nibble, each stored as q + 8): the
//    payload bytes column by column, so that the 8 rows of one column pair
//    are 8 consecutive bytes.
// A strip is one contiguous run of K x 18 bytes, and 32 rows of it (a "unit",
// one matrix-core K step) are 576 contiguous bytes.
//
// GEMM over strip order (int4_gemm_strips_kernel), for 1 <= N <= 8:
//  * the units of all strips form one stream (strip-major); workgroup p takes
//    an equal contiguous range of it (stream-K), which is one contiguous byte
//    range of the records.  When M/32 is between 128 and 256 the plan gives
//    every workgroup exactly one whole strip, and nothing is shared;
//  * the 4 waves of a workgroup take every 4th unit of its range; each keeps a
//    private LDS ring of `depth` stages of 16 units (9 KB, 9 global_load_lds
//    copies of 64 x 16 bytes) and a two-stage ring of the X rows those units
//    need, and keeps copying across strip boundaries: the ring never drains
//    until the range ends;
//  * per unit a lane (q, j) reads the 8 bytes of column pair j of rows
//    8q .. 8q+7 (record q, one 8-byte read) and the record's 8 row scales,
//    forms the two fp16 B operands of
//    v_mfma_f32_16x16x32_f16 for columns 2j and 2j+1 (magic-exponent nibble
//    decode, one v_pk_mul by the row-pair scales: fp16(f32(q - 8) * f32(s))
//    exactly), and the A operand is X[row j][32u + 8q .. +7] from the stage;
//  * where the range crosses a strip boundary the waves put their fp32
//    accumulators in a small LDS area apart from the ring, meet at one
//    barrier, and one wave adds the four in wave order and writes the part:
//    a whole strip goes to Y; the first part of a range (a strip that began
//    in an earlier workgroup's range) is stored encoded for that workgroup; the
//    last part of a range (a strip whose first unit it holds) is the
//    workgroup's own and, after its stream ends, it adds the later
//    workgroups' parts in workgroup order (polling, bounded, as the
//    record-stream kernel's hand-off does) and writes Y.  Results are
//    deterministic.
#include "stream_device.h"

namespace moat {

constexpr int kStripCols = 32;
constexpr int kUnitRows = 32;
constexpr int kUnitBytes = 576;  // 32 rows x 18 bytes: 4 records
constexpr int kStripMaxN = 8;

struct StripParams {
  const uint16_t* x;   // [n][k] fp16, 16-byte aligned
  const uint8_t* w;    // strip-order records
  float* y;            // [n][m] fp32
  float* slots;        // per workgroup n x 32 fp32 (encoded contributions); null when nothing is shared
  uint32_t* status;    // workspace status word (null when nothing is shared)
  int n, k, m;
  int units;           // units per strip, k / 32
  int base, rem;       // workgroup p covers units [p*base + min(p, rem), +base + (p < rem))
  int y_vec;           // y 16-byte aligned
};

// Geometry of a workgroup of W waves (4 or 8) staging NX rows of X.  Wave w
// takes units first + W*i of its workgroup's range; a stage holds 64 / W of
// them (the workgroup's 64 consecutive units per stage round), copied with
// ceil(36 * units / 64) global_load_lds_dwordx4 (1 KB each; 8 waves: the
// fifth copy's upper lanes re-load its lower lanes' chunks into a spare half
// kilobyte).  X: one row per copy with 4 waves (16 units x 64 B, rows 1088
// bytes apart), two rows per copy with 8 waves (8 units x 64 B each, rows 512
// bytes apart and the rows' unit and quarter order swizzled instead).
template <int NX, int W>
struct StripGeom {
  static constexpr int kStageUnits = 64 / W;
  static constexpr int kWLoads = (36 * kStageUnits + 63) / 64;  // 9 or 5
  static constexpr int kWStage = 1024 * kWLoads;
  static constexpr int kXRows = W == 4 ? NX : (NX < 2 ? 2 : NX);  // rows staged (8 waves: pairs)
  static constexpr int kXRowBytes = W == 4 ? 1088 : 512;
  static constexpr int kXLoads = W == 4 ? NX : kXRows / 2;
  static constexpr int kXStage = kXRows * kXRowBytes;
  template <int kDepth>
  static constexpr int wave_bytes() { return kDepth * kWStage + 2 * kXStage; }
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

// Output of one part of a strip by one wave (the part's sums of the four
// waves are in `sl`, wave-major): lanes l < n * 8 each hold four columns of
// one row.
template <int NX, int W>
__device__ __forceinline__ void strip_part_out(const StripParams& P, const float* sl, int p, int strip, bool whole,
                                               bool owner, int last_unit, float poison) {
  const int lane = threadIdx.x & 63;
  const int r = lane >> 3, c4 = 4 * (lane & 7);
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
    int polls = kMaxPolls;
    const float4_t zero = {0.f, 0.f, 0.f, 0.f};
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

template <int NX, int kDepth, int W>
__global__ void __launch_bounds__(W * 64) int4_gemm_strips_kernel(StripParams P) {
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

  // Weight copies: slot s = 64 i + lane of a stage carries chunk s % 36 of
  // the stage's unit s / 36 (slots past the stage's units re-load chunk
  // s % 36 of its first unit); the stage's units lie W units apart.  Units
  // past the range re-load the stage's first unit.
  uint32_t woff[G::kWLoads], wfirst[G::kWLoads];
  int wunit[G::kWLoads];
#pragma unroll
  for (int i = 0; i < G::kWLoads; ++i) {
    const int s = 64 * i + lane;
    wunit[i] = s < 36 * kSU ? s / 36 : 0;
    wfirst[i] = (uint32_t)(16 * (s % 36));
    woff[i] = (uint32_t)(W * kUnitBytes * wunit[i]) + wfirst[i];
  }
  // X copies (rows past N repeat row N - 1).  4 waves: copy n holds row n,
  // lane l = unit l / 4, 16-byte quarter (l & 3) ^ ((n >> 1) & 3).  8 waves:
  // copy c holds rows 2c (lanes 0-31) and 2c+1 (lanes 32-63), lane l = unit
  // ((l & 31) >> 2) ^ (row & 1), quarter (l & 3) ^ ((row >> 1) & 3).  Either
  // way the A-operand reads of 8 rows fall on 8 different 16-byte bank groups.
  uint32_t xoff[G::kXLoads];
  int xk;  // this lane's unit in an X copy
  if constexpr (W == 4) {
    xk = lane >> 2;
#pragma unroll
    for (int n = 0; n < G::kXLoads; ++n) {
      const int row = min(n, P.n - 1);
      const int quarter = (lane & 3) ^ ((n >> 1) & 3);
      xoff[n] = (uint32_t)(2 * (row * P.k + 8 * quarter));
    }
  } else {
    const int half = lane >> 5;
    xk = ((lane & 31) >> 2) ^ half;  // rows of a copy: 2c + half, whose parity is half
#pragma unroll
    for (int c = 0; c < G::kXLoads; ++c) {
      const int n = 2 * c + half;
      const int row = min(n, P.n - 1);
      const int quarter = (lane & 3) ^ ((n >> 1) & 3);
      xoff[c] = (uint32_t)(2 * (row * P.k + 8 * quarter));
    }
  }
  // LDS reads of a unit: record q's scales and the 8 bytes of column pair j
  // of its rows; X row j (rows past N read row N - 1, whose products are
  // never stored)
  const uint32_t rsc = 144 * q, rpay = 144 * q + 16 + 8 * j;
  const int xrow = min(j, P.n - 1);
  const uint32_t rxq = (uint32_t)(G::kXRowBytes * xrow + 16 * (q ^ ((xrow >> 1) & 3)));
  const int xpar = W == 4 ? 0 : (xrow & 1);  // 8 waves: unit k of row xrow sits at unit k ^ (xrow & 1)

  uint8_t* wring = smem + wave * G::template wave_bytes<kDepth>();
  uint8_t* xring = wring + kDepth * G::kWStage;
  const uint32_t wring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)wring;
  const uint32_t xring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)xring;
  float* slots = reinterpret_cast<float*>(smem + W * G::template wave_bytes<kDepth>());
  uint32_t* lds_status =
      reinterpret_cast<uint32_t*>(smem + W * G::template wave_bytes<kDepth>() + 2 * W * G::kSlotBytes);
  status_to_lds(P.status, lds_status);  // the wave's oldest copy: the first ring wait covers it

  const int first = lo + wave;  // this wave's units: first + W i
  const int cnt = first < hi ? (hi - first + W - 1) / W : 0;
  const int nst = (cnt + kSU - 1) / kSU;
  // strip-relative unit of this wave's first unit of stage s (scalar, kept
  // up to date stage by stage)
  int ub_issue = first % U;

  auto issue_w = [&](int s) {
    const int u0 = first + W * kSU * s;
    const uint8_t* base = P.w + (uint64_t)u0 * kUnitBytes;
    const uint32_t st = __builtin_amdgcn_readfirstlane(wring_lds + (s % kDepth) * G::kWStage);
#pragma unroll
    for (int i = 0; i < G::kWLoads; ++i)
      lds_dma16(base, u0 + W * wunit[i] < hi ? woff[i] : wfirst[i], st + 1024 * i);
  };
  auto issue_x = [&](int s, int ub) {  // ub: strip-relative unit of the stage's first unit
    int t = ub + W * xk;
    if (t >= U) t -= U;  // U >= 64 > W * xk
    const uint32_t st = __builtin_amdgcn_readfirstlane(xring_lds + (s & 1) * G::kXStage);
#pragma unroll
    for (int c = 0; c < G::kXLoads; ++c)
      lds_dma16(P.x, xoff[c] + 64u * (uint32_t)t, st + (W == 4 ? G::kXRowBytes : 2 * G::kXRowBytes) * c);
  };

#pragma unroll
  for (int s = 0; s < kDepth - 1; ++s)
    if (s < nst) issue_w(s);
  if (nst > 0) issue_x(0, ub_issue);
  else wait_vmcnt<0>();  // no ring wait will cover the status copy

  // parts of the range: one per strip it touches, in order
  const int strip0 = lo / U;
  const int nparts = hi > lo ? (hi - 1) / U - strip0 + 1 : 0;
  int part = 0;
  int part_end = min(hi, (strip0 + 1) * U);

  float4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};

  auto flush = [&](int pi) {
    float* sl = slots + ((pi & 1) * W + wave) * NX * kStripCols;
    if (q < 2) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = 4 * q + v;
        if (r < NX) *reinterpret_cast<float2*>(sl + r * kStripCols + 2 * j) = float2{acc0[v], acc1[v]};
      }
    }
    acc0 = float4_t{0.f, 0.f, 0.f, 0.f};
    acc1 = float4_t{0.f, 0.f, 0.f, 0.f};
    lds_barrier();
    if (wave == (pi & (W - 1))) {
      const int strip = strip0 + pi;
      const int a = max(lo, strip * U), b = min(hi, (strip + 1) * U);
      const bool whole = a == strip * U && b == (strip + 1) * U;
      const bool owner = !whole && a == strip * U;
      strip_part_out<NX, W>(P, slots + (pi & 1) * W * NX * kStripCols, p, strip, whole, owner,
                         (strip + 1) * U - 1, status_poison(status_from_lds(lds_status)));
    }
  };

  // One unit's LDS reads (X slice, the 8 row scales, the 8 bytes of column
  // pair j), then its arithmetic: the reads of a batch of units go out before
  // the first unit's arithmetic.
  struct UnitRegs {
    half8_t a;
    uint4 sc;
    uint2 b;
  };
  auto load_unit = [&](UnitRegs& r, const uint8_t* wu, const uint8_t* xst, int k) {
    r.a = *reinterpret_cast<const half8_t*>(xst + 64 * (k ^ xpar) + rxq);
    r.sc = *reinterpret_cast<const uint4*>(wu + rsc);
    r.b = *reinterpret_cast<const uint2*>(wu + rpay);
  };
  auto math_unit = [&](const UnitRegs& r) {
    const uint32_t scp[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};  // (s_{2p}, s_{2p+1}) per row pair
    half2_t lo2[4], hi2[4];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      // [row 2p byte, 0, row 2p+1 byte, 0]
      const uint32_t src = pp < 2 ? r.b.x : r.b.y;
      const uint32_t sel = (0x0Cu << 24) | ((uint32_t)(2 * (pp & 1) + 1) << 16) | (0x0Cu << 8) | (uint32_t)(2 * (pp & 1));
      const uint32_t wpair = __builtin_amdgcn_perm(0u, src, sel);
      const half2_t s2 = bitcast<half2_t>(scp[pp]);
      lo2[pp] = nib_lo_pair(wpair, mw.lo) * s2;
      hi2[pp] = nib_hi_pair(wpair, mw.hi) * s2;
    }
    half8_t b0, b1;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      b0[2 * pp] = lo2[pp][0];
      b0[2 * pp + 1] = lo2[pp][1];
      b1[2 * pp] = hi2[pp][0];
      b1[2 * pp + 1] = hi2[pp][1];
    }
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a, b0, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.a, b1, acc1, 0, 0, 0);
  };
  auto compute = [&](const uint8_t* wu, const uint8_t* xst, int k) {
    UnitRegs r;
    load_unit(r, wu, xst, k);
    math_unit(r);
  };

  constexpr int kLW = G::kWLoads, kLX = G::kXLoads;
  for (int s = 0; s < nst; ++s) {
    const bool w_more = s + kDepth - 1 < nst;
    const bool x_more = s + 1 < nst;
    int ub_next = ub_issue + W * kSU;
    while (ub_next >= U) ub_next -= U;
    if (w_more) issue_w(s + kDepth - 1);
    if (x_more) issue_x(s + 1, ub_next);
    ub_issue = ub_next;
    // copies issued after this stage's X: the next X and, further ahead, weights
    if (w_more) wait_vmcnt<kLW + kLX>();
    else if (x_more) wait_vmcnt<kLX>();
    else wait_vmcnt<0>();
    const uint8_t* wst = wring + (s % kDepth) * G::kWStage;
    const uint8_t* xst = xring + (s & 1) * G::kXStage;
    const int kmax = min(kSU, cnt - kSU * s);
    // units k < kb of this stage belong to the current part; with 64 or
    // more units per strip, a stage (units at most 60 apart) meets at most
    // one part boundary
    int kb = part_end - (first + W * kSU * s);
    kb = kb <= 0 ? 0 : min(kmax, (kb + W - 1) / W);
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
          for (int u = 0; u < kBatch; ++u) load_unit(r[u], wst + kUnitBytes * (k0 + u), xst, k0 + u);
#pragma unroll
          for (int u = 0; u < kBatch; ++u) math_unit(r[u]);
        } else {
#pragma unroll
          for (int u = 0; u < kBatch; ++u)
            if (k0 + u >= k_begin && k0 + u < k_end) compute(wst + kUnitBytes * (k0 + u), xst, k0 + u);
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
  }
  // the parts this wave has not flushed yet (always the last; also any it
  // holds no unit of)
  for (; part < nparts; ++part) flush(part);
}

// ---------------------------------------------------------------------------
// Host side.

template <int NX, int kDepth, int W>
static hipError_t launch_strips_one(const StripParams& P, int wgs, hipStream_t stream) {
  const size_t lds = StripGeom<NX, W>::template lds_bytes<kDepth>();
  if (lds > 156 * 1024) return hipErrorInvalidValue;  // never launch past the LDS
  hipLaunchKernelGGL((int4_gemm_strips_kernel<NX, kDepth, W>), dim3(wgs), dim3(W * 64), lds, stream, P);
  return hipGetLastError();
}

// X rows staged: N rounded up to 1, 2, 4 or 8.  Waves: 8 (two per SIMD, so
// that one wave's LDS and matrix-core latencies hide behind the other's
// arithmetic) up to 4 rows, 4 beyond (the LDS holds no more).  Ring depth:
// as deep as the LDS allows, 3 or 2.
int strips_rows_staged(int n) { return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : 8; }
int strips_waves(int n, int waves) {
  if (strips_rows_staged(n) == 8) return 4;
  return waves == 4 || waves == 8 ? waves : 8;
}
int strips_depth(int n, int waves, int depth) {
  const int nx = strips_rows_staged(n);
  const int w = strips_waves(n, waves);
  const int max_depth = w == 8 ? (nx <= 2 ? 3 : 2) : (nx <= 4 ? 3 : 2);
  return depth <= 0 || depth > max_depth ? max_depth : (depth < 2 ? 2 : depth);
}

hipError_t launch_gemm_strips(const uint16_t* x, const uint8_t* w, float* y, int n, int k, int m, int wgs, int depth,
                              int waves, float* slots, uint32_t* status, hipStream_t stream) {
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
  if (waves == 8) {
    if (nx == 1) return depth >= 3 ? launch_strips_one<1, 3, 8>(P, wgs, stream) : launch_strips_one<1, 2, 8>(P, wgs, stream);
    if (nx == 2) return depth >= 3 ? launch_strips_one<2, 3, 8>(P, wgs, stream) : launch_strips_one<2, 2, 8>(P, wgs, stream);
    return launch_strips_one<4, 2, 8>(P, wgs, stream);
  }
  if (nx == 1) return depth >= 3 ? launch_strips_one<1, 3, 4>(P, wgs, stream) : launch_strips_one<1, 2, 4>(P, wgs, stream);
  if (nx == 2) return depth >= 3 ? launch_strips_one<2, 3, 4>(P, wgs, stream) : launch_strips_one<2, 2, 4>(P, wgs, stream);
  if (nx == 4) return depth >= 3 ? launch_strips_one<4, 3, 4>(P, wgs, stream) : launch_strips_one<4, 2, 4>(P, wgs, stream);
  return launch_strips_one<8, 2, 4>(P, wgs, stream);
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
      // output byte e < 8: byte j0 of row 8b+e; e >= 8: byte j0+1 of row 8b+e-8
      const int64_t j0 = 2 * (c - 1);
      uint32_t lo[2] = {0u, 0u}, hi[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t f = (8 * b + i) * gpr + g;
        const uint32_t two = *reinterpret_cast<const uint16_t*>(src + group_payload_offset(f) + j0);
        lo[i >> 2] |= (two & 0xFFu) << (8 * (i & 3));
        hi[i >> 2] |= (two >> 8) << (8 * (i & 3));
      }
      dst[e] = uint4{lo[0], lo[1], hi[0], hi[1]};
    }
  }
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
