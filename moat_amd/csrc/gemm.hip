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
//  * staged path (M % 64 == 0): per round a wave copies its 32 rows x 4
//    group chunks (2 KB of payload) and the 4 scales of each row (256 B)
//    straight from HBM into LDS with three global_load_lds instructions
//    (dwordx4 / dword per lane), then reads its MFMA operand layout back with
//    one ds_read_b32 per row: the load slots are ordered so that lane l's
//    dword of row t sits at byte 256*t + 4*l, which makes every read one
//    contiguous, conflict-free 256-byte LDS access.  Few, wide memory
//    instructions keep enough bytes in flight per CU to approach the HBM
//    rate; 4-byte loads straight into registers (the direct path, kept for
//    other M) cap far lower;
//  * a wave takes every 4th round of its workgroup's slice and issues the
//    loads of kBatch rounds before using any of them, so that a short slice
//    costs one memory latency rather than one latency per round;
//  * the nibbles are turned into (row t, row t+1) fp16 pairs per column
//    (v_perm_b32 + the magic-exponent trick + v_pk_mul by the scale pair);
//    for a column c the four pairs are exactly the 8-deep K slice a lane
//    contributes to a v_mfma_f32_16x16x32_f16 B operand (kk = 8q + t);
//  * MFMA kernel: A operand = X[n][32r + 8q .. +7] for n = lane j (one
//    16-byte load), one MFMA per column c and 16-row block of X;
//  * DOT2 kernel (no matrix cores): v_dot2_f32_f16 of each pair with the
//    matching X pair, then a shuffle reduction across the 4 lane groups;
//  * the 4 waves of a workgroup are summed through two LDS slots (32 KB at
//    N = 32); with K split over `splits` workgroups, each publishes an fp32
//    partial and the last one to finish a column tile adds the partials in
//    split order, so results are deterministic;
//  * workgroup ids are remapped so that each XCD (ids are dealt round-robin
//    to the 8 XCDs) works on one contiguous range of (split, tile) pairs:
//    neighbouring column tiles share 128-byte lines, which then meet in the
//    same L2.
#include "superblock_device.h"

namespace moat {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTileCols = 128;
constexpr int kRoundRows = 32;
constexpr int kXcds = 8;

// How a split-K workgroup hands its partial to the last one of its tile.
enum FinishMode : int {
  // partials written and read with device-scope atomic (sc1) accesses; the
  // writer waits for its stores to complete before the counter increment.
  kFinishDeviceAtomics = 0,
  // plain stores + agent-scope release/acquire fences (whole-L2 writeback
  // and invalidate in every workgroup)
  kFinishFences = 1,
  // plain stores only; a second kernel adds the partials
  kFinishSecondKernel = 2,
};

struct GemmParams {
  const uint16_t* x;       // [N][K] fp16
  const uint8_t* sb;       // 144-byte records of W[K][M]
  float* y;                // [N][M] fp32
  float* partials;         // [splits][N][M] fp32 (splits > 1)
  uint32_t* counters;      // [col_tiles] (splits > 1), zero between calls
  int n, k, m;
  int splits;
  int rounds;              // ceil(k / 32)
  int tiles;               // ceil(m / 128)
  int x_vec;               // x is 16-byte aligned and k % 8 == 0: 16-byte X loads
  int finish;              // FinishMode
};

// Per-lane loads for one 32-row round.
struct RoundData {
  uint32_t w[8];   // payload dword of rows 8q+t
  uint32_t s[4];   // fp16 scales of rows (2p, 2p+1) packed lo/hi
};

__device__ __forceinline__ void load_round(RoundData& d, const uint8_t* __restrict__ sb, uint64_t round_off,
                                           const uint32_t (&poff)[8], const uint32_t (&soff)[8],
                                           uint32_t scale_mask, int row0, int k, bool masked) {
  const uint8_t* base = sb + round_off;
  uint32_t sc[8];
  if (!masked) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      d.w[t] = *reinterpret_cast<const uint32_t*>(base + poff[t]);
      sc[t] = *reinterpret_cast<const uint16_t*>(base + soff[t]);
    }
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (row0 + t < k) {
        d.w[t] = *reinterpret_cast<const uint32_t*>(base + poff[t]);
        sc[t] = *reinterpret_cast<const uint16_t*>(base + soff[t]);
      } else {
        d.w[t] = 0x88888888u;  // every nibble is 8, i.e. value 0
        sc[t] = 0;
      }
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
__device__ __forceinline__ void mfma_round(float4_t (&acc)[NT][8], const RoundData& d, const half8_t (&xa)[NT]) {
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
      acc[nt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[nt], b, acc[nt][c], 0, 0, 0);
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
// (wave w adds into slot w & 1).  Each lane touches the same positions in
// both phases.
__device__ __forceinline__ void tile_put(float* red, int per_wave, int wave, int idx, float v, bool phase_add) {
  float* slot = red + (wave & 1) * per_wave;
  if (phase_add) slot[idx] += v;
  else slot[idx] = v;
}

__device__ __forceinline__ void store_partial(float* p, float v, int finish) {
  if (finish == kFinishDeviceAtomics) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

__device__ __forceinline__ float load_partial(const float* p, int finish) {
  if (finish == kFinishDeviceAtomics)
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}

// Sum the two LDS slots, then store to Y (one split) or publish the partial;
// the last workgroup of the tile to publish adds all partials in split order.
__device__ __forceinline__ void finish_tile(const GemmParams& P, float* red, int npad, int tile, int split) {
  const int tid = threadIdx.x;
  const int ncols = kTileCols;
  const int m0 = tile * kTileCols;
  const int per_wave = npad * ncols;
  if (P.splits == 1) {
    for (int idx = tid; idx < P.n * ncols; idx += kThreads) {
      const int n = idx / ncols, c = idx % ncols;
      if (m0 + c >= P.m) continue;
      P.y[(int64_t)n * P.m + m0 + c] = red[n * ncols + c] + red[per_wave + n * ncols + c];
    }
    return;
  }
  float* part = P.partials + (int64_t)split * P.n * P.m;
  for (int idx = tid; idx < P.n * ncols; idx += kThreads) {
    const int n = idx / ncols, c = idx % ncols;
    if (m0 + c >= P.m) continue;
    store_partial(&part[(int64_t)n * P.m + m0 + c], red[n * ncols + c] + red[per_wave + n * ncols + c], P.finish);
  }
  if (P.finish == kFinishSecondKernel) return;
  __shared__ int s_last;
  if (P.finish == kFinishFences) {
    __threadfence();
  } else {
    // the device-scope stores above must have completed before the counter moves
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
  }
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&P.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (uint32_t)(P.splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  if (P.finish == kFinishFences) __threadfence();
  for (int idx = tid; idx < P.n * ncols; idx += kThreads) {
    const int n = idx / ncols, c = idx % ncols;
    if (m0 + c >= P.m) continue;
    const int64_t o = (int64_t)n * P.m + m0 + c;
    float v = 0.0f;
    for (int s = 0; s < P.splits; ++s) v += load_partial(&P.partials[(int64_t)s * P.n * P.m + o], P.finish);
    P.y[o] = v;
  }
  if (tid == 0) __hip_atomic_store(&P.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-lane byte offsets of its 8 rows in round 0 (row = 8q + t).  Moving
// down 32 rows adds 32*M/32 = M groups; M % 8 == 0 keeps (g & 7) unchanged,
// so every later round is the same offsets plus 18*M bytes per round.
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

// blockIdx.x -> (tile, split): ids b and b+8 run on the same XCD, so deal
// contiguous logical ranges to each XCD; the logical index is split-major,
// keeping neighbouring tiles of one K slice together.
__device__ __forceinline__ void block_coords(const GemmParams& P, int& tile, int& split) {
  const int total = P.tiles * P.splits;
  const int b = blockIdx.x;
  const int per = total / kXcds;
  int logical = b;
  if (b < per * kXcds) logical = (b % kXcds) * per + b / kXcds;
  split = logical / P.tiles;
  tile = logical % P.tiles;
}

// ---------------------------------------------------------------------------
// LDS-staged front end.

constexpr int kStagePayload = 2048;  // 32 rows x 4 group chunks x 16 B
constexpr int kStageRound = kStagePayload + 256;  // + 32 rows x 4 fp16 scales

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Per-lane source offsets (round 0) of its three load slots:
//  payload slot s = 64*i + lane (i = 0, 1) holds row 8*((s>>2)&3) + (s>>4),
//  group (s & 3) of the tile; scale slot u = lane holds the fp16 pair of
//  groups (2*(u&1), 2*(u&1)+1) of row u >> 1.
struct StageOffsets {
  uint32_t pay[2];
  uint32_t sc;
  bool pay_ok[2];  // group inside the matrix (ragged last tile)
  bool sc_ok;
  int pay_row[2];  // row inside the round
  int sc_row;
};

__device__ __forceinline__ void stage_offsets(StageOffsets& o, int lane, int tile, int m) {
  const uint32_t gpr = (uint32_t)(m >> 5);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int s = 64 * i + lane;
    const int row = 8 * ((s >> 2) & 3) + (s >> 4);
    const uint32_t gcol = (uint32_t)(4 * tile + (s & 3));
    const uint32_t g = (uint32_t)row * gpr + gcol;
    o.pay[i] = (g >> 3) * kSbBytes + kSbHeader + ((g & 7) << 4);
    o.pay_ok[i] = gcol < gpr;
    o.pay_row[i] = row;
  }
  const int row = lane >> 1;
  const uint32_t gcol = (uint32_t)(4 * tile + 2 * (lane & 1));
  const uint32_t g = (uint32_t)row * gpr + gcol;  // even when M % 64 == 0, so the pair is 4-byte aligned
  o.sc = (g >> 3) * kSbBytes + ((g & 7) << 1);
  o.sc_ok = gcol < gpr;
  o.sc_row = row;
}

// Issue the three LDS copies of one round (rows >= k are not loaded).
__device__ __forceinline__ void stage_round(const StageOffsets& o, const uint8_t* __restrict__ sb, uint64_t round_off,
                                            int round_row0, int k, uint8_t* dst) {
  const uint8_t* base = sb + round_off;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (o.pay_ok[i] && round_row0 + o.pay_row[i] < k)
      __builtin_amdgcn_global_load_lds((const void*)(base + o.pay[i]), (lds_ptr_t)(dst + 1024 * i), 16, 0, 0);
  }
  if (o.sc_ok && round_row0 + o.sc_row < k)
    __builtin_amdgcn_global_load_lds((const void*)(base + o.sc), (lds_ptr_t)(dst + kStagePayload), 4, 0, 0);
}

// Read one round back in the register layout of RoundData.  Rows >= k and
// columns outside the matrix get scale 0 (their LDS bytes are stale, and
// every nibble times 0 is 0).
__device__ __forceinline__ void read_round(RoundData& d, const uint8_t* src, int lane, int q, int a, int round_row0,
                                           int k, uint32_t scale_mask) {
#pragma unroll
  for (int t = 0; t < 8; ++t) d.w[t] = *reinterpret_cast<const uint32_t*>(src + 256 * t + 4 * lane);
  const uint8_t* sc = src + kStagePayload + 2 * a;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int r0 = 8 * q + 2 * p;
    uint32_t lo = *reinterpret_cast<const uint16_t*>(sc + 8 * r0);
    uint32_t hi = *reinterpret_cast<const uint16_t*>(sc + 8 * (r0 + 1));
    if (round_row0 + r0 >= k) lo = 0;
    if (round_row0 + r0 + 1 >= k) hi = 0;
    d.s[p] = (lo | (hi << 16)) & scale_mask;
  }
}

template <int NT, int kBatch>
__global__ void __launch_bounds__(kThreads) int4_gemm_mfma_staged_kernel(GemmParams P) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4, a = j >> 2;
  int tile, split;
  block_coords(P, tile, split);
  const bool col_ok = tile * kTileCols + 8 * j < P.m;
  const uint32_t smask = col_ok ? 0xFFFFFFFFu : 0u;
  StageOffsets so;
  stage_offsets(so, lane, tile, P.m);
  const uint64_t round_bytes = (uint64_t)18 * (uint64_t)P.m;
  const int r_begin = (int)((int64_t)split * P.rounds / P.splits);
  const int r_end = (int)((int64_t)(split + 1) * P.rounds / P.splits);
  const bool xfast_ok = P.x_vec != 0;
  uint8_t* stage = smem + wave * kBatch * kStageRound;

  float4_t acc[NT][8];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[nt][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int rb = r_begin + wave; rb < r_end; rb += kWaves * kBatch) {
    half8_t xa[kBatch][NT];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int r = rb + i * kWaves;
      if (r < r_end) {
        stage_round(so, P.sb, r * round_bytes, r * kRoundRows, P.k, stage + i * kStageRound);
        const int row0 = r * kRoundRows + 8 * q;
        const bool xfast = xfast_ok && (row0 + 8 <= P.k);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) xa[i][nt] = load_x8(P.x, nt * 16 + j, P.n, row0, P.k, xfast);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the LDS copies of this batch have landed
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int r = rb + i * kWaves;
      if (r < r_end) {
        RoundData d;
        read_round(d, stage + i * kStageRound, lane, q, a, r * kRoundRows, P.k, smask);
        mfma_round<NT>(acc, d, xa[i]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // reads done before the next batch overwrites the stage
  }
  __syncthreads();  // the stage area is reused for the tile reduction

  float* red = reinterpret_cast<float*>(smem);
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
            tile_put(red, per_wave, wave, (nt * 16 + 4 * q + v) * kTileCols + 8 * j + c, acc[nt][c][v], phase == 1);
    }
    __syncthreads();
  }
  finish_tile(P, red, npad, tile, split);
}

template <int NN, int kBatch>
__global__ void __launch_bounds__(kThreads) int4_gemm_dot2_staged_kernel(GemmParams P) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4, a = j >> 2;
  int tile, split;
  block_coords(P, tile, split);
  const bool col_ok = tile * kTileCols + 8 * j < P.m;
  const uint32_t smask = col_ok ? 0xFFFFFFFFu : 0u;
  StageOffsets so;
  stage_offsets(so, lane, tile, P.m);
  const uint64_t round_bytes = (uint64_t)18 * (uint64_t)P.m;
  const int r_begin = (int)((int64_t)split * P.rounds / P.splits);
  const int r_end = (int)((int64_t)(split + 1) * P.rounds / P.splits);
  const bool xfast_ok = P.x_vec != 0;
  uint8_t* stage = smem + wave * kBatch * kStageRound;

  float acc[NN][8];
#pragma unroll
  for (int nn = 0; nn < NN; ++nn)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[nn][c] = 0.0f;

  for (int rb = r_begin + wave; rb < r_end; rb += kWaves * kBatch) {
    half8_t xr[kBatch][NN];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int r = rb + i * kWaves;
      if (r < r_end) {
        stage_round(so, P.sb, r * round_bytes, r * kRoundRows, P.k, stage + i * kStageRound);
        const int row0 = r * kRoundRows + 8 * q;
        const bool xfast = xfast_ok && (row0 + 8 <= P.k);
#pragma unroll
        for (int nn = 0; nn < NN; ++nn) xr[i][nn] = load_x8(P.x, nn, P.n, row0, P.k, xfast);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int r = rb + i * kWaves;
      if (r < r_end) {
        RoundData d;
        read_round(d, stage + i * kStageRound, lane, q, a, r * kRoundRows, P.k, smask);
        dot2_round<NN>(acc, d, xr[i]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
  }
  __syncthreads();

#pragma unroll
  for (int nn = 0; nn < NN; ++nn)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float v = acc[nn][c];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[nn][c] = v;
    }
  float* red = reinterpret_cast<float*>(smem);
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

// ---------------------------------------------------------------------------
// Direct front end (any M % 32 == 0): 4-byte loads straight into registers.

template <int NT, int kBatch>
__global__ void __launch_bounds__(kThreads) int4_gemm_mfma_kernel(GemmParams P) {
  extern __shared__ float red[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  int tile, split;
  block_coords(P, tile, split);
  const int mcol = tile * kTileCols + 8 * j;
  const bool col_ok = mcol < P.m;
  uint32_t poff[8], soff[8];
  lane_offsets(poff, soff, q, col_ok ? mcol : 0, P.m);
  const uint32_t smask = col_ok ? 0xFFFFFFFFu : 0u;
  const uint64_t round_bytes = (uint64_t)18 * (uint64_t)P.m;  // 32 rows of 0.5625 B per element

  const int r_begin = (int)((int64_t)split * P.rounds / P.splits);
  const int r_end = (int)((int64_t)(split + 1) * P.rounds / P.splits);
  const bool xfast_ok = P.x_vec != 0;

  float4_t acc[NT][8];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[nt][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int rb = r_begin + wave; rb < r_end; rb += kWaves * kBatch) {
    RoundData d[kBatch];
    half8_t xa[kBatch][NT];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int r = rb + i * kWaves;
      if (r < r_end) {
        const int row0 = r * kRoundRows + 8 * q;
        load_round(d[i], P.sb, r * round_bytes, poff, soff, smask, row0, P.k, (r + 1) * kRoundRows > P.k);
        const bool xfast = xfast_ok && (row0 + 8 <= P.k);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) xa[i][nt] = load_x8(P.x, nt * 16 + j, P.n, row0, P.k, xfast);
      }
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (rb + i * kWaves < r_end) mfma_round<NT>(acc, d[i], xa[i]);
    }
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
            tile_put(red, per_wave, wave, (nt * 16 + 4 * q + v) * kTileCols + 8 * j + c, acc[nt][c][v], phase == 1);
    }
    __syncthreads();
  }
  finish_tile(P, red, npad, tile, split);
}

template <int NN, int kBatch>
__global__ void __launch_bounds__(kThreads) int4_gemm_dot2_kernel(GemmParams P) {
  extern __shared__ float red[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4;
  int tile, split;
  block_coords(P, tile, split);
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

  for (int rb = r_begin + wave; rb < r_end; rb += kWaves * kBatch) {
    RoundData d[kBatch];
    half8_t xr[kBatch][NN];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int r = rb + i * kWaves;
      if (r < r_end) {
        const int row0 = r * kRoundRows + 8 * q;
        load_round(d[i], P.sb, r * round_bytes, poff, soff, smask, row0, P.k, (r + 1) * kRoundRows > P.k);
        const bool xfast = xfast_ok && (row0 + 8 <= P.k);
#pragma unroll
        for (int nn = 0; nn < NN; ++nn) xr[i][nn] = load_x8(P.x, nn, P.n, row0, P.k, xfast);
      }
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (rb + i * kWaves < r_end) dot2_round<NN>(acc, d[i], xr[i]);
    }
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

// Second kernel of kFinishSecondKernel: y = sum over splits of the partials.
__global__ void __launch_bounds__(256) splitk_sum_kernel(const float* __restrict__ partials, int splits,
                                                         int64_t nm, float* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nm; i += stride) {
    float v = 0.0f;
    for (int s = 0; s < splits; ++s) v += partials[(int64_t)s * nm + i];
    y[i] = v;
  }
}

// ---------------------------------------------------------------------------
// Host-side launch (called from abi.hip after argument validation).

int gemm_col_tiles(int m) { return (m + kTileCols - 1) / kTileCols; }
int gemm_rounds(int k) { return (k + kRoundRows - 1) / kRoundRows; }

static size_t reduce_lds(int npad) { return (size_t)2 * npad * kTileCols * sizeof(float); }

template <int B>
static hipError_t launch_gemm_batch(const GemmParams& P, int algo, bool staged, hipStream_t stream) {
  dim3 grid(P.tiles * P.splits), block(kThreads);
  const size_t stage_lds = (size_t)kWaves * B * kStageRound;
  auto lds_for = [&](int npad) { return staged ? (stage_lds > reduce_lds(npad) ? stage_lds : reduce_lds(npad)) : reduce_lds(npad); };
  if (algo == 2) {
    if (P.n <= 16) {
      if (staged) hipLaunchKernelGGL((int4_gemm_mfma_staged_kernel<1, B>), grid, block, lds_for(16), stream, P);
      else hipLaunchKernelGGL((int4_gemm_mfma_kernel<1, B>), grid, block, lds_for(16), stream, P);
    } else {
      if (staged) hipLaunchKernelGGL((int4_gemm_mfma_staged_kernel<2, B>), grid, block, lds_for(32), stream, P);
      else hipLaunchKernelGGL((int4_gemm_mfma_kernel<2, B>), grid, block, lds_for(32), stream, P);
    }
    return hipGetLastError();
  }
  switch (P.n) {
#define MOAT_DOT2_CASE(NNV)                                                                                  \
  case NNV:                                                                                                  \
    if (staged) hipLaunchKernelGGL((int4_gemm_dot2_staged_kernel<NNV, B>), grid, block, lds_for(NNV), stream, P); \
    else hipLaunchKernelGGL((int4_gemm_dot2_kernel<NNV, B>), grid, block, lds_for(NNV), stream, P);          \
    break;
    MOAT_DOT2_CASE(1) MOAT_DOT2_CASE(2) MOAT_DOT2_CASE(3) MOAT_DOT2_CASE(4)
    MOAT_DOT2_CASE(5) MOAT_DOT2_CASE(6) MOAT_DOT2_CASE(7) MOAT_DOT2_CASE(8)
#undef MOAT_DOT2_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemm(int algo, const uint16_t* x, const uint8_t* sb, float* y, int n, int k, int m, int splits,
                       int batch, int finish, int staged, float* partials, uint32_t* counters, hipStream_t stream) {
  GemmParams P;
  P.x = x; P.sb = sb; P.y = y; P.partials = partials; P.counters = counters;
  P.n = n; P.k = k; P.m = m; P.splits = splits; P.rounds = gemm_rounds(k); P.tiles = gemm_col_tiles(m);
  P.x_vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (k % 8) == 0) ? 1 : 0;
  P.finish = finish;
  const bool st = staged != 0 && (m % 64) == 0;
  hipError_t e;
  if (batch >= 4) e = launch_gemm_batch<4>(P, algo, st, stream);
  else if (batch == 2) e = launch_gemm_batch<2>(P, algo, st, stream);
  else e = launch_gemm_batch<1>(P, algo, st, stream);
  if (e != hipSuccess || splits == 1 || finish != kFinishSecondKernel) return e;
  const int64_t nm = (int64_t)n * m;
  int64_t blocks = (nm + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(splitk_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, partials, splits, nm, y);
  return hipGetLastError();
}

}  // namespace moat
