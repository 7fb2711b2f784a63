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
//  * a workgroup (4 waves) owns a 64-column block -- one 128-byte line of
//    each row -- and a contiguous range of 32-row rounds; the rounds of a
//    block are split over `splits` workgroups when the blocks alone would
//    not fill the chip;
//  * wave w takes every 4th round of the range.  Per round a lane loads four
//    16-byte pieces of W (rows 4*rg .. 4*rg+3 of the round, columns
//    8*c8 .. 8*c8+7; eight lanes cover a whole 128-byte line of a row) and,
//    for each 16-row tile of X, the 16 bytes of its MFMA A operand straight
//    from X (X is small and stays in L2);
//  * v_mfma_f32_16x16x32_f16 wants each lane's 8 B-operand values along K
//    (k = 8q .. 8q+7 of column j), while a row-major load gives 8 values
//    along M: the lane regroups its four rows into k-pairs (two per column)
//    and writes them to the wave's own LDS tile, column-major (80 bytes a
//    column: 32 rows of fp16 and 16 bytes of padding), from which each
//    lane reads its four B operands (16 columns each) as one 16-byte load;
//  * at the end the 4 waves' sums meet in LDS and wave w adds the column
//    group w in wave order.  With one split the workgroup writes Y.  With
//    more, it stores its sums (device-coherent) in its workspace slot and
//    counts itself in the block's counter; the workgroup that arrives last
//    adds every split's sums in split order and writes Y, then resets the
//    counter.  No workgroup waits for another; the order of the sums is
//    fixed, so the bits do not depend on which workgroup arrives last, and
//    the plan does not depend on N (row r of any N equals the N = 1 call).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "superblock_device.h"

namespace moat {

namespace {

constexpr int kDenseWaves = 4;
constexpr int kDenseCols = 64;          // columns of a block
constexpr int kDenseRoundRows = 32;     // rows of a round (one MFMA K step)
constexpr int kDenseColBytes = 80;      // a column of a wave's LDS tile: 32 fp16 rows + 16 padding bytes
constexpr int kDenseTileBytes = kDenseCols * kDenseColBytes;  // 5120 per wave
constexpr int kDenseDepth = 4;          // rounds a wave has in flight

struct DenseParams {
  const uint16_t* x;   // [n][k]
  const uint16_t* w;   // [k][m]
  uint16_t* y;         // [n][m]
  float* slots;        // per (block, split, wave) NT x 64 lanes x 4 floats; null with one split
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
// clamped) and zeroes what lies outside them, so the loads are not branched
// around and the ring's wait counts stay exact.
template <int NT>
__device__ __forceinline__ void dense_load(const DenseParams& P, int round, int col, bool col_ok, int rg, int q, int i,
                                           DenseRound<NT>& R) {
  const int k0 = round * kDenseRoundRows;
  const int colc = col_ok ? col : 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = k0 + 4 * rg + r;
    const uint4 v = *reinterpret_cast<const uint4*>(P.w + (int64_t)min(row, P.k - 1) * P.m + colc);
    const bool ok = col_ok && row < P.k;
    R.w[r] = make_uint4(ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u);
  }
  const int xk = k0 + 8 * q;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int xr = 16 * t + i;
    const half8_t v = *reinterpret_cast<const half8_t*>(P.x + (int64_t)min(xr, P.n - 1) * P.k + min(xk, P.k - 8));
    R.a[t] = (xr < P.n && xk < P.k) ? v : half8_t{};
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

template <int NT>
constexpr int dense_lds_bytes() {
  return kDenseWaves * kDenseTileBytes > kDenseWaves * NT * 4 * 64 * 16 ? kDenseWaves * kDenseTileBytes
                                                                         : kDenseWaves * NT * 4 * 64 * 16;
}

template <int NT>
__global__ __launch_bounds__(256) void dense_gemm_kernel(DenseParams P) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[dense_lds_bytes<NT>()];
  __shared__ uint32_t last_flag;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.x, s = blockIdx.y;
  const int rg = lane >> 3, c8 = lane & 7;  // load role: rows 4rg..4rg+3, columns 8c8..8c8+7
  const int q = lane >> 4, i = lane & 15;   // MFMA role
  const int col = kDenseCols * b + 8 * c8;
  const bool col_ok = col < P.m;
  const int lo = s * P.per;
  const int hi = min(P.rounds, lo + P.per);
  uint8_t* tile = lds + wave * kDenseTileBytes;

  float4_t acc[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[t][g] = float4_t{0.f, 0.f, 0.f, 0.f};

  // wave w: rounds first, first + 4, ... below hi, kDenseDepth of them in
  // flight (a ring of registers); a refill past the wave's last round loads
  // that round again (in the cache), so every pass issues the same loads
  const int first = lo + wave;
  const int cnt = first < hi ? (hi - first + kDenseWaves - 1) / kDenseWaves : 0;
  if (cnt > 0) {
    const int last = first + kDenseWaves * (cnt - 1);
    DenseRound<NT> ring[kDenseDepth];
#pragma unroll
    for (int j = 0; j < kDenseDepth; ++j)
      dense_load<NT>(P, min(first + kDenseWaves * j, last), col, col_ok, rg, q, i, ring[j]);
    for (int it = 0; it < cnt; it += kDenseDepth) {
#pragma unroll
      for (int j = 0; j < kDenseDepth; ++j) {
        const bool live = it + j < cnt;
        wave_lds_sync();  // the previous round's operand reads are done
        if (live) dense_stage(tile, rg, c8, ring[j].w);
        half8_t a[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) a[t] = ring[j].a[t];
        dense_load<NT>(P, min(first + kDenseWaves * (it + j + kDenseDepth), last), col, col_ok, rg, q, i, ring[j]);
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
      }
    }
  }

  // the 4 waves' sums in LDS, [wave][t][g][lane]; wave w adds column group w
  __syncthreads();
  float4_t* red = reinterpret_cast<float4_t*>(lds);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) red[((wave * NT + t) * 4 + g) * 64 + lane] = acc[t][g];
  __syncthreads();
  const int g = wave;
  float4_t sum[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    sum[t] = red[((0 * NT + t) * 4 + g) * 64 + lane];
#pragma unroll
    for (int v = 1; v < kDenseWaves; ++v) sum[t] += red[((v * NT + t) * 4 + g) * 64 + lane];
  }
  // D layout of v_mfma_f32_16x16x32_f16: lane (q, i) holds rows 4q..4q+3, column i
  const int ycol = kDenseCols * b + 16 * g + i;

  if (P.splits > 1) {
    // the sums out (device-coherent), complete in every wave before the
    // workgroup counts itself; the last of the block's splits reads them all
    const __amdgpu_buffer_rsrc_t mine =
        dense_rsrc(P.slots + ((int64_t)(b * P.splits + s) * kDenseWaves + g) * (NT * 256));
#pragma unroll
    for (int t = 0; t < NT; ++t) dense_store_sc1(mine, 16 * (64 * t + lane), sum[t]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t before = __hip_atomic_fetch_add(P.counters + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = before == (uint32_t)(P.splits - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (last_flag == 0u) return;
    float4_t tot[NT];
    for (int s2 = 0; s2 < P.splits; ++s2) {
      const __amdgpu_buffer_rsrc_t other =
          dense_rsrc(P.slots + ((int64_t)(b * P.splits + s2) * kDenseWaves + g) * (NT * 256));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float4_t v = s2 == s ? sum[t] : dense_load_sc1(other, 16 * (64 * t + lane));
        tot[t] = s2 == 0 ? v : tot[t] + v;
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) sum[t] = tot[t];
    if (threadIdx.x == 0) __hip_atomic_store(P.counters + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (ycol < P.m) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * t + 4 * q + e;
        if (row < P.n) P.y[(int64_t)row * P.m + ycol] = __builtin_bit_cast(uint16_t, (_Float16)sum[t][e]);
      }
  }
}

}  // namespace

// The workspace starts with a fixed area of counter words, one per block
// (so a counter never lies where another plan keeps split sums, which stay
// behind after a call); the split sums follow it.
constexpr int kDenseCounterWords = 4096;

int64_t dense_counter_bytes() { return (int64_t)kDenseCounterWords * 4; }

// Host-side plan, shared with the workspace query: blocks of 64 columns;
// splits (when not given) so that blocks x splits reaches about 512
// workgroups with at least 8 rounds (two a wave) per split; one split when
// the blocks outnumber the counter words (m > 262144: the blocks alone fill
// the chip).
void dense_plan(int k, int m, int splits_req, int* blocks, int* rounds, int* per, int* splits) {
  const int nb = (m + kDenseCols - 1) / kDenseCols;
  const int nr = (k + kDenseRoundRows - 1) / kDenseRoundRows;
  int sp = splits_req;
  if (sp <= 0) {
    sp = (512 + nb - 1) / nb;
    const int most = nr / 8 > 1 ? nr / 8 : 1;
    if (sp > most) sp = most;
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
  return splits > 1 ? (int64_t)blocks * splits * kDenseWaves * nt * 256 * (int64_t)sizeof(float) : 0;
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
  if (n > 16)
    hipLaunchKernelGGL(dense_gemm_kernel<2>, grid, block, 0, stream, P);
  else
    hipLaunchKernelGGL(dense_gemm_kernel<1>, grid, block, 0, stream, P);
  return hipGetLastError();
}

}  // namespace moat
