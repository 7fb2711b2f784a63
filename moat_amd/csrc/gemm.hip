// Batched INT4 superblock projection Y[N][M] = X[N][K] @ deq(W)[K][M] for gfx950.
//
// What it reproduces: the reference CPU path (dequantize the 144-byte stream,
// src/dequant.py:116-147, then a float32 matmul,
// antigravity-engine/tests/test_batched_speed.py:39-42); the reference's own
// GPU version of this product is the fused kernel
// antigravity-engine/src/shaders/batched_gemm.metal:116-169, which has no
// caller.  The weights are used as the bit-exact fp16 dequantized values and
// every product is accumulated in fp32, so the only difference from the CPU
// path is the summation order.
//
// Tiling (one wavefront = 64 lanes, lane = 16*q + j):
//  * a workgroup owns 128 consecutive columns of W (one column tile) and a
//    slice of its rows; lane j owns columns 8j..8j+7 of the tile, i.e. one
//    dword of one group per row, and lane group q owns rows 8q..8q+7 of each
//    32-row "round";
//  * per round a lane issues 8 dword loads (its 8 rows) and 8 fp16 scale
//    loads; for 16 lanes of a lane group those dwords are 64 contiguous
//    payload bytes of one row, so the wave reads 4 rows x 64 B per load;
//  * the nibbles are turned into (row t, row t+1) fp16 pairs per column
//    (v_perm_b32 + the magic-exponent trick + v_pk_mul by the scale pair);
//    for a column c the four pairs are exactly the 8-deep K slice a lane
//    contributes to a v_mfma_f32_16x16x32_f16 B operand (kk = 8q + t);
//  * MFMA variant: A operand = X[n][32r + 8q .. +7] for n = lane j (one
//    16-byte load), one MFMA per column c and 16-row block of X;
//  * DOT2 variant (no matrix cores): v_dot2_f32_f16 of each pair with the
//    matching X pair, then a shuffle reduction across the 4 lane groups;
//  * the 4 waves of a workgroup take interleaved rounds and are summed through
//    two LDS slots (32 KB at N = 32); with K split over `splits` workgroups, each writes an fp32 partial
//    and the last one to finish a column tile (device-scope counter) adds the
//    partials in split order, so results are deterministic.
#include "superblock_device.h"

namespace moat {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTileCols = 128;
constexpr int kRoundRows = 32;

struct GemmParams {
  const uint16_t* x;       // [N][K] fp16
  const uint8_t* sb;       // 144-byte records of W[K][M]
  float* y;                // [N][M] fp32
  float* partials;         // [splits][N][M] fp32 (splits > 1)
  uint32_t* counters;      // [col_tiles] (splits > 1), zero between calls
  int n, k, m;
  int splits;
  int rounds;              // ceil(k / 32)
  int x_vec;               // x is 16-byte aligned and k % 8 == 0: 16-byte X loads
};

// Per-lane loads for one 32-row round.
struct RoundData {
  uint32_t w[8];   // payload dword of rows 8q+t
  uint32_t s[4];   // fp16 scales of rows (2p, 2p+1) packed lo/hi
};

template <bool kMasked>
__device__ __forceinline__ void load_round(RoundData& d, const uint8_t* __restrict__ sb, uint64_t round_off,
                                           const uint32_t (&poff)[8], const uint32_t (&soff)[8],
                                           uint32_t scale_mask, int row0, int k) {
  const uint8_t* base = sb + round_off;
  uint32_t sc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (!kMasked || row0 + t < k) {
      d.w[t] = *reinterpret_cast<const uint32_t*>(base + poff[t]);
      sc[t] = *reinterpret_cast<const uint16_t*>(base + soff[t]);
    } else {
      d.w[t] = 0x88888888u;  // every nibble is 8, i.e. value 0
      sc[t] = 0;
    }
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) d.s[p] = (sc[2 * p] | (sc[2 * p + 1] << 16)) & scale_mask;
}

// X[n][kk .. kk+7] as 8 fp16 (zero outside [0,N) x [0,K)).
__device__ __forceinline__ half8_t load_x8(const uint16_t* __restrict__ x, int n, int nrows, int kk, int k,
                                           bool fast) {
  if (n >= nrows) return half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  const uint16_t* p = x + (int64_t)n * k + kk;
  if (fast) {
    return __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4*>(p));
  }
  half8_t v;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    v[t] = (kk + t < k) ? __builtin_bit_cast(_Float16, p[t]) : (_Float16)0.0f;
  }
  return v;
}

template <int NT>
struct MfmaAcc {
  float4_t c[NT][8];
};

template <int NT>
__device__ __forceinline__ void mfma_round(MfmaAcc<NT>& acc, const RoundData& d, const half8_t (&xa)[NT]) {
  half2_t pr[4][8];
#pragma unroll
  for (int p = 0; p < 4; ++p) dequant_row_pair(d.w[2 * p], d.w[2 * p + 1], bitcast<half2_t>(d.s[p]), pr[p]);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    half8_t b;
    b[0] = pr[0][c][0]; b[1] = pr[0][c][1];
    b[2] = pr[1][c][0]; b[3] = pr[1][c][1];
    b[4] = pr[2][c][0]; b[5] = pr[2][c][1];
    b[6] = pr[3][c][0]; b[7] = pr[3][c][1];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      acc.c[nt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[nt], b, acc.c[nt][c], 0, 0, 0);
    }
  }
}

template <int NN>
__device__ __forceinline__ void dot2_round(float (&acc)[NN][8], const RoundData& d, const half8_t (&xr)[NN]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    half2_t pr[8];
    dequant_row_pair(d.w[2 * p], d.w[2 * p + 1], bitcast<half2_t>(d.s[p]), pr);
#pragma unroll
    for (int nn = 0; nn < NN; ++nn) {
      const half2_t xp = {xr[nn][2 * p], xr[nn][2 * p + 1]};
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[nn][c] = __builtin_amdgcn_fdot2(pr[c], xp, acc[nn][c], false);
    }
  }
}

// Two LDS slots hold the tile: waves 2 and 3 store, then waves 0 and 1 add
// (wave w < 2 adds into slot w).  Each lane touches the same positions in
// both phases.
__device__ __forceinline__ void tile_put(float* red, int per_wave, int wave, int idx, float v, bool phase_add) {
  float* slot = red + (wave & 1) * per_wave;
  if (phase_add) slot[idx] += v;
  else slot[idx] = v;
}

// Sum the two LDS slots, then store to Y (one split) or to the
// partial buffer followed by the last-arriver reduction.
__device__ __forceinline__ void finish_tile(const GemmParams& P, float* red, int npad, int tile, int split) {
  const int tid = threadIdx.x;
  const int ncols = kTileCols;
  const int m0 = tile * kTileCols;
  const int per_wave = npad * ncols;
  if (P.splits == 1) {
    for (int idx = tid; idx < P.n * ncols; idx += kThreads) {
      const int n = idx / ncols, c = idx % ncols;
      if (m0 + c >= P.m) continue;
      const float v = red[n * ncols + c] + red[per_wave + n * ncols + c];
      P.y[(int64_t)n * P.m + m0 + c] = v;
    }
    return;
  }
  float* part = P.partials + (int64_t)split * P.n * P.m;
  for (int idx = tid; idx < P.n * ncols; idx += kThreads) {
    const int n = idx / ncols, c = idx % ncols;
    if (m0 + c >= P.m) continue;
    const float v = red[n * ncols + c] + red[per_wave + n * ncols + c];
    part[(int64_t)n * P.m + m0 + c] = v;
  }
  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&P.counters[tile], 1u);
    s_last = (prev == (uint32_t)(P.splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int idx = tid; idx < P.n * ncols; idx += kThreads) {
    const int n = idx / ncols, c = idx % ncols;
    if (m0 + c >= P.m) continue;
    const int64_t o = (int64_t)n * P.m + m0 + c;
    float v = 0.0f;
    for (int s = 0; s < P.splits; ++s) {
      v += __builtin_nontemporal_load(&P.partials[(int64_t)s * P.n * P.m + o]);
    }
    P.y[o] = v;
  }
  if (tid == 0) atomicExch(&P.counters[tile], 0u);
}

// Per-lane byte offsets of its 8 rows in round 0 (row = 8q + t).
__device__ __forceinline__ void lane_offsets(uint32_t (&poff)[8], uint32_t (&soff)[8], int q, int mcol, int m) {
  const uint32_t gpr = (uint32_t)(m >> 5);  // groups per row
  const uint32_t gcol = (uint32_t)(mcol >> 5);
  const uint32_t dw = (uint32_t)((mcol & 31) >> 1);  // byte offset of the lane's dword in the group chunk
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t g = (uint32_t)(8 * q + t) * gpr + gcol;
    poff[t] = (g >> 3) * kSbBytes + kSbHeader + ((g & 7) << 4) + dw;
    soff[t] = (g >> 3) * kSbBytes + ((g & 7) << 1);
  }
}

template <int NT>
__global__ void __launch_bounds__(kThreads) int4_gemm_mfma_kernel(GemmParams P) {
  extern __shared__ float red[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int mcol = tile * kTileCols + 8 * j;
  const bool col_ok = mcol < P.m;
  uint32_t poff[8], soff[8];
  lane_offsets(poff, soff, q, col_ok ? mcol : 0, P.m);
  const uint32_t smask = col_ok ? 0xFFFFFFFFu : 0u;
  const uint64_t round_bytes = (uint64_t)18 * (uint64_t)P.m;  // 32 rows of 0.5625 B per element

  const int r_begin = (int)((int64_t)split * P.rounds / P.splits);
  const int r_end = (int)((int64_t)(split + 1) * P.rounds / P.splits);
  const bool xfast_ok = P.x_vec != 0;

  MfmaAcc<NT> acc;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc.c[nt][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  RoundData cur, nxt;
  int r = r_begin + wave;
  if (r < r_end) {
    const int row0 = r * kRoundRows + 8 * q;
    if ((r + 1) * kRoundRows <= P.k) load_round<false>(cur, P.sb, r * round_bytes, poff, soff, smask, row0, P.k);
    else load_round<true>(cur, P.sb, r * round_bytes, poff, soff, smask, row0, P.k);
  }
  for (; r < r_end; r += kWaves) {
    const int rn = r + kWaves;
    if (rn < r_end) {
      const int row0n = rn * kRoundRows + 8 * q;
      if ((rn + 1) * kRoundRows <= P.k) load_round<false>(nxt, P.sb, rn * round_bytes, poff, soff, smask, row0n, P.k);
      else load_round<true>(nxt, P.sb, rn * round_bytes, poff, soff, smask, row0n, P.k);
    }
    const int kk = r * kRoundRows + 8 * q;
    const bool xfast = xfast_ok && (kk + 8 <= P.k);
    half8_t xa[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) xa[nt] = load_x8(P.x, nt * 16 + j, P.n, kk, P.k, xfast);
    mfma_round<NT>(acc, cur, xa);
    cur = nxt;
  }

  // D layout of v_mfma_f32_16x16x32_f16: lane (q, j) holds rows 4q..4q+3, column j.
  const int npad = NT * 16;
  const int per_wave = npad * kTileCols;
#pragma unroll
  for (int phase = 0; phase < 2; ++phase) {
    if ((wave >> 1) == 1 - phase) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            tile_put(red, per_wave, wave, (nt * 16 + 4 * q + v) * kTileCols + 8 * j + c, acc.c[nt][c][v], phase == 1);
    }
    __syncthreads();
  }
  finish_tile(P, red, npad, tile, split);
}

template <int NN>
__global__ void __launch_bounds__(kThreads) int4_gemm_dot2_kernel(GemmParams P) {
  extern __shared__ float red[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int mcol = tile * kTileCols + 8 * j;
  const bool col_ok = mcol < P.m;
  uint32_t poff[8], soff[8];
  lane_offsets(poff, soff, q, col_ok ? mcol : 0, P.m);
  const uint32_t smask = col_ok ? 0xFFFFFFFFu : 0u;
  const uint64_t round_bytes = (uint64_t)18 * (uint64_t)P.m;
  const int r_begin = (int)((int64_t)split * P.rounds / P.splits);
  const int r_end = (int)((int64_t)(split + 1) * P.rounds / P.splits);
  const bool xfast_ok = P.x_vec != 0;

  float acc[NN][8];
#pragma unroll
  for (int nn = 0; nn < NN; ++nn)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[nn][c] = 0.0f;

  RoundData cur, nxt;
  int r = r_begin + wave;
  if (r < r_end) {
    const int row0 = r * kRoundRows + 8 * q;
    if ((r + 1) * kRoundRows <= P.k) load_round<false>(cur, P.sb, r * round_bytes, poff, soff, smask, row0, P.k);
    else load_round<true>(cur, P.sb, r * round_bytes, poff, soff, smask, row0, P.k);
  }
  for (; r < r_end; r += kWaves) {
    const int rn = r + kWaves;
    if (rn < r_end) {
      const int row0n = rn * kRoundRows + 8 * q;
      if ((rn + 1) * kRoundRows <= P.k) load_round<false>(nxt, P.sb, rn * round_bytes, poff, soff, smask, row0n, P.k);
      else load_round<true>(nxt, P.sb, rn * round_bytes, poff, soff, smask, row0n, P.k);
    }
    const int kk = r * kRoundRows + 8 * q;
    const bool xfast = xfast_ok && (kk + 8 <= P.k);
    half8_t xr[NN];
#pragma unroll
    for (int nn = 0; nn < NN; ++nn) xr[nn] = load_x8(P.x, nn, P.n, kk, P.k, xfast);
    dot2_round<NN>(acc, cur, xr);
    cur = nxt;
  }

  // wavefront reduction over the 4 lane groups (lanes j, j+16, j+32, j+48)
#pragma unroll
  for (int nn = 0; nn < NN; ++nn)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float v = acc[nn][c];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[nn][c] = v;
    }
  const int npad = NN;
  const int per_wave = npad * kTileCols;
#pragma unroll
  for (int phase = 0; phase < 2; ++phase) {
    if ((wave >> 1) == 1 - phase && q == 0) {
#pragma unroll
      for (int nn = 0; nn < NN; ++nn)
#pragma unroll
        for (int c = 0; c < 8; ++c) tile_put(red, per_wave, wave, nn * kTileCols + 8 * j + c, acc[nn][c], phase == 1);
    }
    __syncthreads();
  }
  finish_tile(P, red, npad, tile, split);
}

}  // namespace moat

// ---------------------------------------------------------------------------
// Host-side launch (called from abi.cpp after argument validation).

namespace moat {

int gemm_col_tiles(int m) { return (m + kTileCols - 1) / kTileCols; }
int gemm_rounds(int k) { return (k + kRoundRows - 1) / kRoundRows; }

hipError_t launch_gemm(int algo, const uint16_t* x, const uint8_t* sb, float* y, int n, int k, int m,
                       int splits, float* partials, uint32_t* counters, hipStream_t stream) {
  GemmParams P;
  P.x = x; P.sb = sb; P.y = y; P.partials = partials; P.counters = counters;
  P.n = n; P.k = k; P.m = m; P.splits = splits; P.rounds = gemm_rounds(k);
  P.x_vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (k % 8) == 0) ? 1 : 0;
  dim3 grid(gemm_col_tiles(m), splits), block(kThreads);
  if (algo == 2) {
    if (n <= 16) {
      const size_t lds = (size_t)2 * 16 * kTileCols * sizeof(float);
      hipLaunchKernelGGL(int4_gemm_mfma_kernel<1>, grid, block, lds, stream, P);
    } else {
      const size_t lds = (size_t)2 * 32 * kTileCols * sizeof(float);
      hipLaunchKernelGGL(int4_gemm_mfma_kernel<2>, grid, block, lds, stream, P);
    }
  } else {
#define MOAT_DOT2_CASE(NNV)                                                               \
  case NNV: {                                                                             \
    const size_t lds = (size_t)2 * NNV * kTileCols * sizeof(float);                  \
    hipLaunchKernelGGL(int4_gemm_dot2_kernel<NNV>, grid, block, lds, stream, P);           \
    break;                                                                                \
  }
    switch (n) {
      MOAT_DOT2_CASE(1) MOAT_DOT2_CASE(2) MOAT_DOT2_CASE(3) MOAT_DOT2_CASE(4)
      MOAT_DOT2_CASE(5) MOAT_DOT2_CASE(6) MOAT_DOT2_CASE(7) MOAT_DOT2_CASE(8)
      default: return hipErrorInvalidValue;
    }
#undef MOAT_DOT2_CASE
  }
  return hipGetLastError();
}

}  // namespace moat
