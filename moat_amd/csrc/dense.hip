// Dense fp16 decode product for gfx950: Y[N x M] (fp16) = X[N x K] (fp16) .
// W[K x M] (fp16, row-major), sums in fp32, each output rounded to fp16 once.
//
// The reference runs this product two ways, chosen per call by
// dispatchGEMM (antigravity-engine/src/transformer_engine.mm:463-500): the
// 8x8 simdgroup GEMM with half sums (antigravity-engine/src/shaders/
// batched_gemm.metal:74-109, N a multiple of 8) and, for one row, the GEMV
// with fp32 sums and a half result (antigravity-engine/src/shaders/
// transformer_ops.metal:270-286).  Here one kernel serves every N: the
// fp32 sums of the GEMV for all rows, which is also what the reference's
// CPU product computes (antigravity-engine/tests/test_batched_speed.py:31-42:
// X.f32 @ W.f32, cast to W's dtype).
//
// Layout and work split (HBM-bound: every weight byte is read once):
//  * a workgroup (4 waves) owns a block of 64 x WC columns and a contiguous
//    range of 32-row rounds.  WC = 4 for long rows (M >= 16384): wave w
//    takes the 64 columns 64w .. 64w+63, one 128-byte line of each row, over
//    every round, so the workgroup reads 512 contiguous bytes of a row at a
//    time.  WC = 1 below that, where 256-column blocks would be too few:
//    the four waves share 64 columns and take every 4th round.  A block's
//    rounds are split over `splits` workgroups when the blocks alone would
//    not fill the chip;
//  * each wave keeps 4 rounds of loads in flight.  Per round a lane loads
//    four 16-byte pieces of W (rows 4*rg .. 4*rg+3 of the round, columns
//    8*c8 .. 8*c8+7; eight lanes cover the wave's 128 bytes of a row) and,
//    for each 16-row tile of X, the 16 bytes of its MFMA A operand straight
//    from X (X is small and stays in L2);
//  * v_mfma_f32_16x16x32_f16 wants each lane's 8 B-operand values along K
//    (k = 8q .. 8q+7 of column j), while a row-major load gives 8 values
//    along M: the lane regroups its four rows into k-pairs (two per column)
//    and writes them to the wave's own LDS tile, column-major (80 bytes a
//    column: 32 rows of fp16 and 16 bytes of padding), from which each
//    lane reads its four B operands (16 columns each) as one 16-byte load;
//  * waves that share columns add their sums in LDS (in round order);
//    with one split the waves write Y.  With more, each wave stores its sums
//    (device-coherent) in its workspace slot and the workgroup counts itself
//    in the block's counter; the workgroup that arrives last loads every
//    split's sums, adds them in split order and writes Y, then resets the
//    counter.  No workgroup waits for another; the order of the sums is
//    fixed, so the bits do not depend on which workgroup arrives last, and
//    the plan does not depend on N (row r of any N equals the N = 1 call).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "superblock_device.h"

namespace moat {

namespace {

constexpr int kDenseWaves = 4;
constexpr int kDenseCols = 64;          // columns of a wave
constexpr int kDenseRoundRows = 32;     // rows of a round (one MFMA K step)
constexpr int kDenseColBytes = 80;      // a column of a wave's LDS tile: 32 fp16 rows + 16 padding bytes
constexpr int kDenseTileBytes = kDenseCols * kDenseColBytes;  // 5120 per wave
constexpr int kDenseDepth = 4;          // rounds a wave has in flight
constexpr int kDenseBatch = 4;          // splits whose sums the last workgroup loads at once

struct DenseParams {
  const uint16_t* x;   // [n][k]
  const uint16_t* w;   // [k][m]
  uint16_t* y;         // [n][m]
  float* slots;        // per (block, split, wave) NT x 4 x 64 lanes x 4 floats; null with one split
  uint32_t* counters;  // one word per block, zero between calls; null with one split
  int n, k, m;
  int rounds;          // ceil(k / 32)
  int per;             // rounds per split
  int splits;
};

template <int NT>
struct DenseRound {
  uint4 w[4];
  half8_t a[NT];
};

// Every lane loads from an address inside the matrices (rows and columns
// clamped), unmasked: the ring carries the loads as they arrive, so no
// wait falls on the ring's refills.  Past the last column or the last row
// of X the products land in outputs that are never stored; past row K the
// round's rows and X's k positions are zeroed when the round is used
// (dense_mask).
template <int NT>
__device__ __forceinline__ void dense_load(const DenseParams& P, int round, int col, bool col_ok, int rg, int q, int i,
                                           DenseRound<NT>& R) {
  const int k0 = round * kDenseRoundRows;
  const int colc = col_ok ? col : 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = k0 + 4 * rg + r;
    R.w[r] = *reinterpret_cast<const uint4*>(P.w + (int64_t)min(row, P.k - 1) * P.m + colc);
  }
  const int xk = k0 + 8 * q;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int xr = 16 * t + i;
    R.a[t] = *reinterpret_cast<const half8_t*>(P.x + (int64_t)min(xr, P.n - 1) * P.k + min(xk, P.k - 8));
  }
}

// Rows k >= K of a round (only the last round of a ragged K has them): W
// rows and X columns zeroed, so their products vanish.  Straight-line ANDs
// (no branch, nothing written into a register a load may still fill).
template <int NT>
__device__ __forceinline__ void dense_mask(const DenseParams& P, int round, int rg, int q, uint4 (&w)[4],
                                           half8_t (&a)[NT]) {
  const int k0 = round * kDenseRoundRows;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t keep = k0 + 4 * rg + r < P.k ? 0xFFFFFFFFu : 0u;
    w[r].x &= keep;
    w[r].y &= keep;
    w[r].z &= keep;
    w[r].w &= keep;
  }
  const uint32_t keep_x = k0 + 8 * q < P.k ? 0xFFFFFFFFu : 0u;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    uint4 v = __builtin_bit_cast(uint4, a[t]);
    v.x &= keep_x;
    v.y &= keep_x;
    v.z &= keep_x;
    v.w &= keep_x;
    a[t] = __builtin_bit_cast(half8_t, v);
  }
}

// The lane's 4 rows x 8 columns, written column-major: column 8*c8 + c gets
// rows 4*rg .. 4*rg+3 as 8 bytes at k offset 4*rg.
__device__ __forceinline__ void dense_stage(uint8_t* tile, int rg, int c8, const uint4 (&w)[4]) {
  const uint32_t* a0 = reinterpret_cast<const uint32_t*>(&w[0]);
  const uint32_t* a1 = reinterpret_cast<const uint32_t*>(&w[1]);
  const uint32_t* a2 = reinterpret_cast<const uint32_t*>(&w[2]);
  const uint32_t* a3 = reinterpret_cast<const uint32_t*>(&w[3]);
  uint8_t* base = tile + 8 * c8 * kDenseColBytes + 8 * rg;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint2 lo, hi;  // columns 2d (low halves) and 2d + 1 (high halves)
    lo.x = (a0[d] & 0xFFFFu) | (a1[d] << 16);
    lo.y = (a2[d] & 0xFFFFu) | (a3[d] << 16);
    hi.x = (a0[d] >> 16) | (a1[d] & 0xFFFF0000u);
    hi.y = (a2[d] >> 16) | (a3[d] & 0xFFFF0000u);
    *reinterpret_cast<uint2*>(base + (2 * d) * kDenseColBytes) = lo;
    *reinterpret_cast<uint2*>(base + (2 * d + 1) * kDenseColBytes) = hi;
  }
}

// LDS exchange between the lanes of one wave: the wave's LDS operations run
// in order; the fences keep the compiler from moving them across.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Device-coherent 16-byte accesses (cache policy SC1: written through to,
// and read from, the memory side, past the per-XCD L2) through a buffer
// resource on a wave's slot; a workgroup's sums travel this way instead of
// behind agent-scope fences, which write back and invalidate the L2.
typedef unsigned int dense_u32x4_t __attribute__((__vector_size__(16)));
constexpr int kDenseSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dense_rsrc(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ void dense_store_sc1(__amdgpu_buffer_rsrc_t r, int off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(dense_u32x4_t, v), r, off, 0, kDenseSc1);
}
__device__ __forceinline__ float4_t dense_load_sc1(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kDenseSc1));
}

// WC column groups of 64 a workgroup (1, 2 or 4): wave w reads group
// w % WC and every (4 / WC)-th round of the split from round w / WC; the
// 4 / WC waves of a group add their sums in LDS at the end, each finishing
// WC of the group's four 16-column tiles.
template <int WC>
constexpr int dense_lds_bytes(int nt) {
  return WC < 4 && kDenseWaves * nt * 4 * 64 * 16 > kDenseWaves * kDenseTileBytes ? kDenseWaves * nt * 4 * 64 * 16
                                                                                    : kDenseWaves * kDenseTileBytes;
}

template <int NT, int WC>
__global__ __launch_bounds__(256) void dense_gemm_kernel(DenseParams P) {
  constexpr int G = WC;                 // 16-column tiles a wave finishes
  constexpr int R = kDenseWaves / WC;   // waves sharing a column group
  __shared__ __attribute__((aligned(16))) uint8_t lds[dense_lds_bytes<WC>(NT)];
  __shared__ uint32_t last_flag;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.x, s = blockIdx.y;
  const int rg = lane >> 3, c8 = lane & 7;  // load role: rows 4rg..4rg+3, columns 8c8..8c8+7
  const int q = lane >> 4, i = lane & 15;   // MFMA role
  const int cg = wave % WC, ro = wave / WC;                 // column group, first round
  const int col0 = kDenseCols * (WC * b + cg);              // the wave's 64 columns
  const int col = col0 + 8 * c8;
  const bool col_ok = col < P.m;
  const int lo = s * P.per;
  const int hi = min(P.rounds, lo + P.per);
  uint8_t* tile = lds + wave * kDenseTileBytes;

  float4_t acc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[t][g] = float4_t{0.f, 0.f, 0.f, 0.f};

  // the wave's rounds: first, first + step, ... below hi, kDenseDepth of
  // them in flight (a ring of registers); a refill past the wave's last
  // round loads that round again (in the cache), so every pass issues the
  // same loads.  With WC = 4 the workgroup's four waves read 512 contiguous
  // bytes of each row together.
  constexpr int step = R;
  const int first = lo + ro;
  const int cnt = first < hi ? (hi - first + step - 1) / step : 0;
  if (cnt > 0) {
    const int last = first + step * (cnt - 1);
    DenseRound<NT> ring[kDenseDepth];
#pragma unroll
    for (int j = 0; j < kDenseDepth; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      dense_load<NT>(P, min(first + step * j, last), col, col_ok, rg, q, i, ring[j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // one round of the ring: entry j holds round first + step * (it + j)
    auto use = [&](int it, int j, bool live) {
      uint4 wv[4];
      half8_t a[NT];
#pragma unroll
      for (int r = 0; r < 4; ++r) wv[r] = ring[j].w[r];
#pragma unroll
      for (int t = 0; t < NT; ++t) a[t] = ring[j].a[t];
      dense_mask<NT>(P, first + step * (it + j), rg, q, wv, a);
      wave_lds_sync();  // the previous round's operand reads are done
      if (live) dense_stage(tile, rg, c8, wv);
      wave_lds_sync();
      if (live) {
        half8_t bop[4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
          bop[g] = *reinterpret_cast<const half8_t*>(tile + (16 * g + i) * kDenseColBytes + 16 * q);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int t = 0; t < NT; ++t)
            acc[t][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bop[g], acc[t][g], 0, 0, 0);
      }
    };
    // full passes: after each use the entry's registers are free and its
    // next round goes out in place (the scheduler keeps the ring's load
    // groups in this order, so the wait for an entry leaves the later
    // entries' loads in flight); the last pass issues no loads, so no
    // load is left for the end of the kernel to wait on
    int it = 0;
    for (; it + kDenseDepth < cnt; it += kDenseDepth) {
#pragma unroll
      for (int j = 0; j < kDenseDepth; ++j) {
        use(it, j, true);
        __builtin_amdgcn_sched_barrier(0);
        dense_load<NT>(P, min(first + step * (it + j + kDenseDepth), last), col, col_ok, rg, q, i, ring[j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int j = 0; j < kDenseDepth; ++j) use(it, j, it + j < cnt);
  }

  // fin[t][g]: the sums of the wave's output columns ycol0 + 16 g + i
  float4_t fin[NT][G];
  int ycol0;
  if constexpr (R == 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) fin[t][g] = acc[t][g];
    ycol0 = col0;
  } else {
    // the sums in LDS, [wave][t][tile][lane]; wave (cg, ro) adds tiles
    // ro * G .. ro * G + G - 1 of group cg over the group's R waves, in
    // round order
    __syncthreads();
    float4_t* red = reinterpret_cast<float4_t*>(lds);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) red[((wave * NT + t) * 4 + g) * 64 + lane] = acc[t][g];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int tile16 = ro * G + g;
        fin[t][g] = red[((cg * NT + t) * 4 + tile16) * 64 + lane];
#pragma unroll
        for (int v = 1; v < R; ++v) fin[t][g] += red[(((v * WC + cg) * NT + t) * 4 + tile16) * 64 + lane];
      }
    ycol0 = col0 + 16 * G * ro;
  }

  if (P.splits > 1) {
    // the wave's sums out (device-coherent), complete in every wave before
    // the workgroup counts itself; the last of the block's splits loads all
    // splits' sums (kDenseBatch splits at a time, every load issued before
    // the first add) and adds them in split order
    const __amdgpu_buffer_rsrc_t mine =
        dense_rsrc(P.slots + ((int64_t)(b * P.splits + s) * kDenseWaves + wave) * (NT * 1024));
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int g = 0; g < G; ++g) dense_store_sc1(mine, 16 * ((G * t + g) * 64 + lane), fin[t][g]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t before = __hip_atomic_fetch_add(P.counters + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = before == (uint32_t)(P.splits - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (last_flag == 0u) return;
    for (int s0 = 0; s0 < P.splits; s0 += kDenseBatch) {
      float4_t v[kDenseBatch][NT][G];
#pragma unroll
      for (int u = 0; u < kDenseBatch; ++u) {
        const int s2 = min(s0 + u, P.splits - 1);
        const __amdgpu_buffer_rsrc_t r =
            dense_rsrc(P.slots + ((int64_t)(b * P.splits + s2) * kDenseWaves + wave) * (NT * 1024));
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int g = 0; g < G; ++g) v[u][t][g] = dense_load_sc1(r, 16 * ((G * t + g) * 64 + lane));
      }
#pragma unroll
      for (int u = 0; u < kDenseBatch; ++u) {
        if (s0 + u < P.splits) {
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int g = 0; g < G; ++g) fin[t][g] = s0 + u == 0 ? v[u][t][g] : fin[t][g] + v[u][t][g];
        }
      }
    }
    if (threadIdx.x == 0) __hip_atomic_store(P.counters + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // D layout of v_mfma_f32_16x16x32_f16: lane (q, i) holds rows 4q..4q+3, column i
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int ycol = ycol0 + 16 * g + i;
    if (ycol < P.m) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * t + 4 * q + e;
          if (row < P.n) P.y[(int64_t)row * P.m + ycol] = __builtin_bit_cast(uint16_t, (_Float16)fin[t][g][e]);
        }
    }
  }
}

}  // namespace

// The workspace starts with a fixed area of counter words, one per block
// (so a counter never lies where another plan keeps split sums, which stay
// behind after a call); the split sums follow it.
constexpr int kDenseCounterWords = 4096;

int64_t dense_counter_bytes() { return (int64_t)kDenseCounterWords * 4; }

// Column groups of 64 a workgroup: 4 (256 columns) from m = 16384 -- long
// rows, where 512 contiguous bytes per row read keep the stream fast -- and
// 1 below, where 256-column blocks would be too few to fill the chip.
// (128-column blocks measured 0-9 % slower than 64 at m = 5504..14336.)
int dense_wc(int m) { return m >= 16384 ? 4 : 1; }

// Host-side plan, shared with the workspace query: blocks of 64 x WC
// columns; splits (when not given) the largest power of two that keeps
// blocks x splits within 256 (WC = 1) or 448 (WC = 4) workgroups, with at
// least 2 rounds a wave per split and at most 16 splits -- powers of two
// keep a split's rounds a multiple of the ring depth; one split when the
// blocks outnumber the counter words (m > 1048576: the blocks alone fill
// the chip).  (Measured, us at N = 1: K=2048 x M=5504 11.0 at 2 splits,
// 11.5 at 4, 12.3 at 6; K=3072 x M=8192 15.0 at 2, 17.7 at 4; K=8192 x
// M=28672 93.8 at 4, 99.2 at 2, 107.2 at 3, 109.8 at 5, 102.9 at 8;
// K=4096 x M=16384 31.1 at 4, 53.6 at 2, 38.6 at 3; K=2048 x M=32000 30.8
// at 2, 31.2 at 4, 34.9 at 3.)
void dense_plan(int k, int m, int splits_req, int* blocks, int* rounds, int* per, int* splits) {
  const int wc = dense_wc(m);
  const int nb = (m + kDenseCols * wc - 1) / (kDenseCols * wc);
  const int nr = (k + kDenseRoundRows - 1) / kDenseRoundRows;
  int sp = splits_req;
  if (sp <= 0) {
    const int most_wgs = wc == 4 ? 448 : 256;
    const int min_rounds = 2 * (kDenseWaves / wc);
    sp = 1;
    while (sp < 16 && (int64_t)nb * sp * 2 <= most_wgs && nr / (sp * 2) >= min_rounds) sp *= 2;
  }
  if (nb > kDenseCounterWords) sp = 1;
  if (sp > nr) sp = nr;
  const int pr = (nr + sp - 1) / sp;
  *blocks = nb;
  *rounds = nr;
  *per = pr;
  *splits = (nr + pr - 1) / pr;
}

int64_t dense_slot_bytes(int n, int blocks, int splits) {
  const int nt = n > 16 ? 2 : 1;
  return splits > 1 ? (int64_t)blocks * splits * kDenseWaves * nt * 1024 * (int64_t)sizeof(float) : 0;
}

// n <= 32 rows a launch; counters and slots as the plan needs (null with one split).
hipError_t launch_dense_gemm(const uint16_t* x, const uint16_t* w, uint16_t* y, int n, int k, int m, int splits_req,
                             float* slots, uint32_t* counters, hipStream_t stream) {
  DenseParams P;
  P.x = x;
  P.w = w;
  P.y = y;
  P.slots = slots;
  P.counters = counters;
  P.n = n;
  P.k = k;
  P.m = m;
  int blocks = 0;
  dense_plan(k, m, splits_req, &blocks, &P.rounds, &P.per, &P.splits);
  const dim3 grid(blocks, P.splits), block(256);
  const int wc = dense_wc(m);
  if (n > 16) {
    if (wc == 4) hipLaunchKernelGGL((dense_gemm_kernel<2, 4>), grid, block, 0, stream, P);
    else hipLaunchKernelGGL((dense_gemm_kernel<2, 1>), grid, block, 0, stream, P);
  } else {
    if (wc == 4) hipLaunchKernelGGL((dense_gemm_kernel<1, 4>), grid, block, 0, stream, P);
    else hipLaunchKernelGGL((dense_gemm_kernel<1, 1>), grid, block, 0, stream, P);
  }
  return hipGetLastError();
}

}  // namespace moat
