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
// Two kernels:
//  * int4_gemm_records_kernel (further down), the default whenever
//    M % 128 == 0, K % 32 == 0 and X rows are 16-byte aligned: 256-column
//    tiles of whole 144-byte records moved into LDS by DMA, matrix cores,
//    a stream-K split over (tile group, round) items with an in-kernel or
//    second-kernel hand-off; it also runs several matrices sharing X in one
//    launch and the gate/up pair with its SwiGLU epilogue;
//  * int4_gemm_kernel (this first part), every other shape (any
//    M % 32 == 0, ragged K, unaligned X) and the dot2 (no matrix core)
//    variant, described next.
//
// General kernel tiling (one wavefront = 64 lanes, lane = 16*q + j):
//  * a workgroup owns 128 consecutive columns of W (one column tile) and a
//    slice of its rows; lane j owns columns 8j..8j+7 of the tile, i.e. one
//    dword of one group per row, and lane group q owns rows 8q..8q+7 of each
//    32-row "round";
//  * a wave takes every 4th round of its workgroup's slice and issues the
//    loads of kBatch rounds before using any of them, so that a short slice
//    costs one memory latency rather than one latency per round; whole
//    batches run unconditionally and only the last round of the matrix is
//    masked;
//  * weight loads, three front ends:
//    - staged through LDS (M % 64 == 0): a round's 32 rows x 4 group chunks
//      (2 KB) and the 4 scales of each row (256 B) are fetched as three load
//      slots per lane (two 16-byte, one 4-byte) and put into a per-wave LDS
//      stage, either with plain vector loads + ds_write (kFrontVgprLds) or
//      with global_load_lds (kFrontLdsDma); the slots are ordered so that
//      lane l's dword of row t sits at byte 256*t + 4*l, making the read-back
//      one conflict-free 256-byte access per row;
//    - direct (any M % 32 == 0): 8 dword + 8 scale loads per lane and round
//      straight into registers;
//  * the nibbles are turned into (row t, row t+1) fp16 pairs per column
//    (v_perm_b32 + the magic-exponent trick + v_pk_mul by the scale pair);
//    for a column c the four pairs are exactly the 8-deep K slice a lane
//    contributes to a v_mfma_f32_16x16x32_f16 B operand (kk = 8q + t);
//  * MFMA compute: A operand = X[n][32r + 8q .. +7] for n = lane j (one
//    16-byte load), one MFMA per column c and 16-row block of X;
//  * DOT2 compute (no matrix cores): v_dot2_f32_f16 of each pair with the
//    matching X pair, then a shuffle reduction across the 4 lane groups;
//  * the 4 waves of a workgroup are summed through two LDS slots (32 KB at
//    N = 32); with K split over `splits` workgroups, each publishes an fp32
//    partial that a second kernel (default) or the last workgroup to finish
//    a column tile adds in split order, so results are deterministic;
//  * workgroup ids are remapped so that each XCD (ids are dealt round-robin
//    to the 8 XCDs) works on one contiguous range of (split, tile) pairs:
//    neighbouring column tiles share 128-byte lines, which then meet in the
//    same L2.
#include "stream_device.h"

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
  int tiles;               // column tiles of the launched kernel: ceil(m / 128), or ceil(m / 256) for records
  int x_vec;               // x is 16-byte aligned and k % 8 == 0: 16-byte X loads
  int finish;              // FinishMode
  int shift;               // records kernel: M % 256 == 128, odd rows start half-way into a record
  int rounds_base;         // rounds / splits: split s covers rounds [s*base + min(s, rem), +base + (s < rem))
  int rounds_rem;          // rounds % splits
  int y_vec;               // y and the partials are 16-byte aligned and m % 4 == 0: float4 stores
  int items_base;          // records kernel (stream-K): workgroup p covers items (tile * rounds + round)
  int items_rem;           //   [p*base + min(p, rem), +base + (p < rem))
  // Records kernel: where a tile's records lie.  Row order (the stream as
  // written): round stride 32 rows of M/256 records (18 * M bytes), tile
  // stride one record (144 bytes), rows M/256 records apart (rec_row_m = M).
  // Tile order (each 256-column tile's K rows of records contiguous, tiles
  // in column order): round stride 32 records (4608 bytes), tile stride K
  // records, rows one record apart (rec_row_m = 256).
  uint64_t rec_round_bytes;
  uint64_t rec_tile_bytes;
  int rec_row_m;
  // Record-stream kernel over several matrices of one shape that share X:
  // kModeMulti: tile t of the concatenated tile space is tile t - i*tiles of
  // matrix i = t / tiles (Y_i = X @ W_i); kModeSwiglu: tile group g pairs tile
  // g of matrix 0 (gate) with tile g of matrix 1 (up), and the output is
  // h = silu(X @ W_0) * (X @ W_1) in fp16.
  int mats;
  const uint8_t* sbm[4];
  float* ym[4];
  uint16_t* h;
  // Record-stream kernel with shared tile groups: the workspace's sticky
  // status word (kWsStatus*), read at the start of a call; when set, the call
  // writes NaN instead of results.  Null when the plan shares no tile group.
  uint32_t* status;
};

enum RecMode : int { kModeSingle = 0, kModeMulti = 1, kModeSwiglu = 2 };

// Uniform 4-way select (scalar compares, no indexed access to the arguments).
template <typename T>
__device__ __forceinline__ T select4(int i, T a0, T a1, T a2, T a3) {
  return i == 0 ? a0 : (i == 1 ? a1 : (i == 2 ? a2 : a3));
}

// h[r][c] = fp16(silu(g) * u), g = gu[r][c], u = gu[r][m + c] (rows ld floats
// apart): the SwiGLU step on the output of one GEMM over gate and up stored
// side by side, with swiglu4's arithmetic.  Four columns a thread.
__global__ void __launch_bounds__(256) swiglu_f32_kernel(const float* __restrict__ gu, int n, int m, int64_t ld,
                                                         uint16_t* __restrict__ h) {
  const int64_t quads = (int64_t)n * (m / 4);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < quads; e += stride) {
    const int64_t r = e / (m / 4);
    const int c = (int)(e - r * (m / 4)) * 4;
    const float4_t g = *reinterpret_cast<const float4_t*>(gu + r * ld + c);
    const float4_t u = *reinterpret_cast<const float4_t*>(gu + r * ld + m + c);
    *reinterpret_cast<uint2*>(h + r * m + c) = swiglu4(g, u);
  }
}

hipError_t launch_swiglu_f32(const float* gu, int n, int m, int64_t ld, uint16_t* h, hipStream_t stream) {
  const int64_t quads = (int64_t)n * (m / 4);
  if (quads == 0) return hipSuccess;
  int64_t blocks = (quads + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(swiglu_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, gu, n, m, ld, h);
  return hipGetLastError();
}

// Round range of split s (no device-side division).
__device__ __forceinline__ void split_rounds(const GemmParams& P, int split, int& r_begin, int& r_end) {
  r_begin = split * P.rounds_base + min(split, P.rounds_rem);
  r_end = r_begin + P.rounds_base + (split < P.rounds_rem ? 1 : 0);
}

// One 32-row round in registers: the lane's payload dword of rows 8q+t and
// the fp16 scales of rows (8q+2p, 8q+2p+1) packed lo/hi.
struct RoundData {
  uint32_t w[8];
  uint32_t s[4];
};

// ---------------------------------------------------------------------------
// Direct front end.

struct DirectOffsets {
  uint32_t pay[8];  // byte offset (round 0) of the lane's dword in row 8q+t
  uint32_t sc[8];   // byte offset (round 0) of the lane's scale in row 8q+t
};

// Moving down 32 rows adds 32*M/32 = M groups; M % 8 == 0 keeps (g & 7)
// unchanged, so round r is round 0 plus 18*M*r bytes.
__device__ __forceinline__ void direct_offsets(DirectOffsets& o, int q, int mcol, int m) {
  const uint32_t gpr = (uint32_t)(m >> 5);
  const uint32_t gcol = (uint32_t)(mcol >> 5);
  const uint32_t dw = (uint32_t)((mcol & 31) >> 1);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t g = (uint32_t)(8 * q + t) * gpr + gcol;
    o.pay[t] = (g >> 3) * kSbBytes + kSbHeader + ((g & 7) << 4) + dw;
    o.sc[t] = (g >> 3) * kSbBytes + ((g & 7) << 1);
  }
}

template <bool kMasked>
__device__ __forceinline__ void direct_round(RoundData& d, const DirectOffsets& o, const uint8_t* __restrict__ base,
                                             uint32_t scale_mask, int row0, int k) {
  uint32_t sc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (!kMasked || row0 + t < k) {
      d.w[t] = *reinterpret_cast<const uint32_t*>(base + o.pay[t]);
      sc[t] = *reinterpret_cast<const uint16_t*>(base + o.sc[t]);
    } else {
      d.w[t] = 0x88888888u;  // every nibble is 8, i.e. value 0
      sc[t] = 0;
    }
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) d.s[p] = (sc[2 * p] | (sc[2 * p + 1] << 16)) & scale_mask;
}

// ---------------------------------------------------------------------------
// LDS-staged front end.

constexpr int kStagePayload = 2048;               // 32 rows x 4 group chunks x 16 B
constexpr int kStageRound = kStagePayload + 256;  // + 32 rows x 4 fp16 scales


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
template <bool kMasked>
__device__ __forceinline__ void stage_round(const StageOffsets& o, const uint8_t* __restrict__ base, int round_row0,
                                            int k, uint8_t* dst) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (o.pay_ok[i] && (!kMasked || round_row0 + o.pay_row[i] < k))
      __builtin_amdgcn_global_load_lds((const void*)(base + o.pay[i]), (lds_ptr_t)(dst + 1024 * i), 16, 0, 0);
  }
  if (o.sc_ok && (!kMasked || round_row0 + o.sc_row < k))
    __builtin_amdgcn_global_load_lds((const void*)(base + o.sc), (lds_ptr_t)(dst + kStagePayload), 4, 0, 0);
}

// The same three slots loaded into registers (16-byte and 4-byte vector
// loads) and then written to the stage with ds_write: a plain dwordx4 load
// moves 1 KB per wave instruction, the widest the vector memory path takes.
struct SlotRegs {
  uint4 pay[2];
  uint32_t sc;
};

template <bool kMasked>
__device__ __forceinline__ void slot_load(SlotRegs& v, const StageOffsets& o, const uint8_t* __restrict__ base,
                                          int round_row0, int k) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (o.pay_ok[i] && (!kMasked || round_row0 + o.pay_row[i] < k))
      v.pay[i] = *reinterpret_cast<const uint4*>(base + o.pay[i]);
    else
      v.pay[i] = uint4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
  }
  v.sc = (o.sc_ok && (!kMasked || round_row0 + o.sc_row < k)) ? *reinterpret_cast<const uint32_t*>(base + o.sc) : 0u;
}

__device__ __forceinline__ void slot_store(const SlotRegs& v, uint8_t* dst, int lane) {
  *reinterpret_cast<uint4*>(dst + 16 * lane) = v.pay[0];
  *reinterpret_cast<uint4*>(dst + 1024 + 16 * lane) = v.pay[1];
  *reinterpret_cast<uint32_t*>(dst + kStagePayload + 4 * lane) = v.sc;
}

// Read one staged round back in the RoundData layout.  Columns outside the
// matrix (scale_mask) and, in a masked round, rows >= k get scale 0: their LDS
// bytes are stale, and any nibble times 0 is 0.  `sc_sel` is the v_perm
// selector that takes the fp16 of this lane's group from two row dwords.
template <bool kMasked>
__device__ __forceinline__ void read_round(RoundData& d, const uint8_t* src, int lane, int q, int a, uint32_t sc_sel,
                                           int round_row0, int k, uint32_t scale_mask) {
#pragma unroll
  for (int t = 0; t < 8; ++t) d.w[t] = *reinterpret_cast<const uint32_t*>(src + 256 * t + 4 * lane);
  const uint8_t* sc = src + kStagePayload + 4 * (a >> 1);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int r0 = 8 * q + 2 * p;
    const uint32_t lo = *reinterpret_cast<const uint32_t*>(sc + 8 * r0);
    const uint32_t hi = *reinterpret_cast<const uint32_t*>(sc + 8 * (r0 + 1));
    uint32_t v = __builtin_amdgcn_perm(hi, lo, sc_sel);
    if (kMasked) {
      if (round_row0 + r0 >= k) v &= 0xFFFF0000u;
      if (round_row0 + r0 + 1 >= k) v &= 0x0000FFFFu;
    }
    d.s[p] = v & scale_mask;
  }
}

// ---------------------------------------------------------------------------
// Compute.

// X[n][kk .. kk+7] as 8 fp16 (zero outside [0,N) x [0,K)).
__device__ __forceinline__ half8_t load_x8(const uint16_t* __restrict__ x, int n, int nrows, int kk, int k,
                                           bool fast) {
  if (n >= nrows) return half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  const uint16_t* p = x + (int64_t)n * k + kk;
  if (fast) return __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4*>(p));
  half8_t v;
#pragma unroll
  for (int t = 0; t < 8; ++t) v[t] = (kk + t < k) ? __builtin_bit_cast(_Float16, p[t]) : (_Float16)0.0f;
  return v;
}

// MFMA: NR 16-row blocks of X, lane j loads row nt*16 + j.
// DOT2: NR rows of X, every lane loads all of them.
template <bool kMfma, int NR>
__device__ __forceinline__ void load_x_round(half8_t (&xr)[NR], const GemmParams& P, int j, int row0, bool xfast) {
#pragma unroll
  for (int r = 0; r < NR; ++r) xr[r] = load_x8(P.x, kMfma ? r * 16 + j : r, P.n, row0, P.k, xfast);
}

template <bool kMfma, int NR>
struct Acc;
template <int NR>
struct Acc<true, NR> {
  float4_t c[NR][8];
};
template <int NR>
struct Acc<false, NR> {
  float c[NR][8];
};

template <bool kMfma, int NR>
__device__ __forceinline__ void compute_round(Acc<kMfma, NR>& acc, const RoundData& d, const half8_t (&xr)[NR],
                                              MagicWords mw) {
  if constexpr (kMfma) {
    half2_t pr[4][8];
#pragma unroll
    for (int p = 0; p < 4; ++p) dequant_row_pair(d.w[2 * p], d.w[2 * p + 1], bitcast<half2_t>(d.s[p]), pr[p], mw);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      half8_t b;
      b[0] = pr[0][c][0]; b[1] = pr[0][c][1];
      b[2] = pr[1][c][0]; b[3] = pr[1][c][1];
      b[4] = pr[2][c][0]; b[5] = pr[2][c][1];
      b[6] = pr[3][c][0]; b[7] = pr[3][c][1];
#pragma unroll
      for (int nt = 0; nt < NR; ++nt)
        acc.c[nt][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xr[nt], b, acc.c[nt][c], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      half2_t pr[8];
      dequant_row_pair(d.w[2 * p], d.w[2 * p + 1], bitcast<half2_t>(d.s[p]), pr, mw);
#pragma unroll
      for (int nn = 0; nn < NR; ++nn) {
        const half2_t xp = {xr[nn][2 * p], xr[nn][2 * p + 1]};
#pragma unroll
        for (int c = 0; c < 8; ++c) acc.c[nn][c] = __builtin_amdgcn_fdot2(pr[c], xp, acc.c[nn][c], false);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Epilogue.

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

// Sum the two LDS slots (each [npad][kCols] floats), then store to Y (one
// split) or publish the partial; the last workgroup of the tile to publish
// adds all partials in split order.
template <int kCols = kTileCols>
__device__ __forceinline__ void finish_tile(const GemmParams& P, float* red, int npad, int tile, int split) {
  const int tid = threadIdx.x;
  const int ncols = kCols;
  const int m0 = tile * kCols;
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
    // leave the workspace at zero for the calls that share it
    for (int s = 0; s < P.splits; ++s) store_partial(&P.partials[(int64_t)s * P.n * P.m + o], 0.0f, P.finish);
    P.y[o] = v;
  }
  if (tid == 0) __hip_atomic_store(&P.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// blockIdx.x -> (tile, split): ids b and b+8 run on the same XCD, so deal
// contiguous logical ranges to each XCD; the logical index is split-major,
// keeping neighbouring tiles of one K slice together.
__device__ __forceinline__ void block_coords(const GemmParams& P, int& tile, int& split) {
  const int total = P.tiles * P.splits;  // P.tiles: column tiles of the launched kernel
  const int b = blockIdx.x;
  const int per = total / kXcds;
  int logical = b;
  if (b < per * kXcds) logical = (b % kXcds) * per + b / kXcds;
  split = logical / P.tiles;
  tile = logical % P.tiles;
}

// ---------------------------------------------------------------------------
// The kernel: kMfma selects MFMA (NR = 16-row blocks of X) or dot2 (NR = rows
// of X); kFront selects how weights reach the registers.

enum Front : int {
  kFrontDirect = 0,   // 4-byte loads straight into the operand layout
  kFrontLdsDma = 1,   // global_load_lds into the stage, ds_read back
  kFrontVgprLds = 2,  // dwordx4 loads, ds_write into the stage, ds_read back
  kFrontRecords = 3,  // the record-stream kernel (int4_gemm_records_kernel)
};

template <bool kMfma, int NR, int kBatch, int kFront>
__global__ void __launch_bounds__(kThreads) int4_gemm_kernel(GemmParams P) {
  constexpr bool kStaged = kFront != kFrontDirect;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, q = lane >> 4, a = j >> 2;
  int tile, split;
  block_coords(P, tile, split);
  const int mcol = tile * kTileCols + 8 * j;
  const bool col_ok = mcol < P.m;
  const uint32_t smask = col_ok ? 0xFFFFFFFFu : 0u;
  const uint64_t round_bytes = (uint64_t)18 * (uint64_t)P.m;  // 32 rows of 0.5625 B per element
  int r_begin, r_end;
  split_rounds(P, split, r_begin, r_end);
  const bool xfast_ok = P.x_vec != 0;
  const MagicWords mw = magic_words();

  StageOffsets so;
  DirectOffsets dof;
  uint32_t sc_sel = 0;
  uint8_t* stage = smem + wave * kBatch * kStageRound;
  if constexpr (kStaged) {
    stage_offsets(so, lane, tile, P.m);
    sc_sel = (a & 1) ? 0x07060302u : 0x05040100u;
  } else {
    direct_offsets(dof, q, col_ok ? mcol : 0, P.m);
  }

  Acc<kMfma, NR> acc;
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if constexpr (kMfma) acc.c[r][c] = float4_t{0.f, 0.f, 0.f, 0.f};
      else acc.c[r][c] = 0.0f;
    }

  // whole batches: every round present and inside K
  const int full_rounds = P.k / kRoundRows;  // rounds with no row past K
  const int r_full_end = r_end < full_rounds ? r_end : full_rounds;
  int r = r_begin + wave;
  for (; r + (kBatch - 1) * kWaves < r_full_end; r += kWaves * kBatch) {
    half8_t xr[kBatch][NR];
    RoundData d[kStaged ? 1 : kBatch];
    SlotRegs sr[kFront == kFrontVgprLds ? kBatch : 1];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int ri = r + i * kWaves;
      const uint8_t* base = P.sb + ri * round_bytes;
      if constexpr (kFront == kFrontLdsDma) stage_round<false>(so, base, ri * kRoundRows, P.k, stage + i * kStageRound);
      else if constexpr (kFront == kFrontVgprLds) slot_load<false>(sr[i], so, base, ri * kRoundRows, P.k);
      else direct_round<false>(d[i], dof, base, smask, ri * kRoundRows + 8 * q, P.k);
      load_x_round<kMfma, NR>(xr[i], P, j, ri * kRoundRows + 8 * q, xfast_ok);
    }
    if constexpr (kFront == kFrontLdsDma) __builtin_amdgcn_s_waitcnt(0);  // this batch's LDS copies have landed
    if constexpr (kFront == kFrontVgprLds) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) slot_store(sr[i], stage + i * kStageRound, lane);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if constexpr (kStaged) {
        read_round<false>(d[0], stage + i * kStageRound, lane, q, a, sc_sel, 0, P.k, smask);
        compute_round<kMfma, NR>(acc, d[0], xr[i], mw);
      } else {
        compute_round<kMfma, NR>(acc, d[i], xr[i], mw);
      }
    }
    if constexpr (kFront == kFrontLdsDma) __builtin_amdgcn_s_waitcnt(0);  // reads done before the stage is refilled
  }
  // remaining rounds one at a time; only a round reaching past K is masked
  for (; r < r_end; r += kWaves) {
    const uint8_t* base = P.sb + r * round_bytes;
    const int row0 = r * kRoundRows;
    const bool masked = row0 + kRoundRows > P.k;
    half8_t xr[1][NR];
    RoundData d;
    load_x_round<kMfma, NR>(xr[0], P, j, row0 + 8 * q, xfast_ok && row0 + 8 * q + 8 <= P.k);
    if constexpr (kStaged) {
      if constexpr (kFront == kFrontLdsDma) {
        if (masked) stage_round<true>(so, base, row0, P.k, stage);
        else stage_round<false>(so, base, row0, P.k, stage);
        __builtin_amdgcn_s_waitcnt(0);
      } else {
        SlotRegs v;
        if (masked) slot_load<true>(v, so, base, row0, P.k);
        else slot_load<false>(v, so, base, row0, P.k);
        slot_store(v, stage, lane);
      }
      if (masked) read_round<true>(d, stage, lane, q, a, sc_sel, row0, P.k, smask);
      else read_round<false>(d, stage, lane, q, a, sc_sel, row0, P.k, smask);
    } else {
      if (masked) direct_round<true>(d, dof, base, smask, row0 + 8 * q, P.k);
      else direct_round<false>(d, dof, base, smask, row0 + 8 * q, P.k);
    }
    compute_round<kMfma, NR>(acc, d, xr[0], mw);
    if constexpr (kFront == kFrontLdsDma) __builtin_amdgcn_s_waitcnt(0);
  }
  if constexpr (kStaged) __syncthreads();  // the stage area is reused for the tile reduction

  float* red = reinterpret_cast<float*>(smem);
  if constexpr (kMfma) {
    // D layout of v_mfma_f32_16x16x32_f16: lane (q, j) holds rows 4q..4q+3, column j.
    const int npad = NR * 16;
    const int per_wave = npad * kTileCols;
#pragma unroll
    for (int phase = 0; phase < 2; ++phase) {
      if ((wave >> 1) == 1 - phase) {
#pragma unroll
        for (int nt = 0; nt < NR; ++nt)
#pragma unroll
          for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              tile_put(red, per_wave, wave, (nt * 16 + 4 * q + v) * kTileCols + 8 * j + c, acc.c[nt][c][v],
                       phase == 1);
      }
      __syncthreads();
    }
    finish_tile(P, red, npad, tile, split);
  } else {
    // wavefront reduction over the 4 lane groups (lanes j, j+16, j+32, j+48)
#pragma unroll
    for (int nn = 0; nn < NR; ++nn)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float v = acc.c[nn][c];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        acc.c[nn][c] = v;
      }
    const int npad = NR;
    const int per_wave = npad * kTileCols;
#pragma unroll
    for (int phase = 0; phase < 2; ++phase) {
      if ((wave >> 1) == 1 - phase && q == 0) {
#pragma unroll
        for (int nn = 0; nn < NR; ++nn)
#pragma unroll
          for (int c = 0; c < 8; ++c)
            tile_put(red, per_wave, wave, nn * kTileCols + 8 * j + c, acc.c[nn][c], phase == 1);
      }
      __syncthreads();
    }
    finish_tile(P, red, npad, tile, split);
  }
}

// ---------------------------------------------------------------------------
// Record-stream kernel: M % 128 == 0, K % 32 == 0, X rows 16-byte aligned.
//
// A workgroup (4 or 8 waves) owns a group of 1, 2 or 4 adjacent 256-column
// tiles and a run of (tile group, round) items (stream-K); the waves of one
// tile take every (waves per tile)-th round of the run's segment in that
// group.  In every row the tile's bytes are whole
// 16-byte chunks of at most two records:
//  * a row that starts on a record boundary (every row when M % 256 == 0,
//    the even rows when M % 256 == 128) needs the record's header and its 8
//    payload chunks;
//  * a row that starts half-way into record s needs the header of s (the
//    tile's groups 0-3 have their scales at bytes 8..15), payload chunks 4-7
//    of s, the header of s+1 (groups 4-7 at bytes 0..7) and payload chunks
//    0-3 of s+1, the last nine being one contiguous 144-byte window.
// A round (32 rows) therefore needs at most 10 chunks per row; the stage
// gives each row 11 chunk slots (176 bytes: rows 8 apart, which the four
// lane groups of an LDS read address together, then fall on different
// banks), 6 KB per round, plus the round's X slice (16 rows x 32 fp16 per
// 16-row block of X).  Both are moved
// with global_load_lds (16 bytes per lane, straight into LDS) into a
// per-wave ring of kDepth stages: the wave keeps kDepth - 1 rounds in flight
// while it computes one, and waits for a round with an explicit vmcnt.
// Whole records per row touch the fewest 128-byte lines per instruction of
// any layout of this stream.
constexpr int kRecCols = 256;
// LDS a workgroup may take on gfx950 (160 KB), less room for the kernels'
// static __shared__ words.
constexpr size_t kMaxDynamicLds = 156 * 1024;
constexpr int kRecSlotsPerRow = 11;
constexpr int kRecRowBytes = 16 * kRecSlotsPerRow;                                  // 176
constexpr int kRecWeightLoads = (kRoundRows * kRecRowBytes + 1023) / 1024;          // 6 loads of 64 x 16 bytes
constexpr int kRecWeightBytes = kRecWeightLoads * 1024;                             // 6144

template <int NR>
struct RecGeom {
  static constexpr int kStageBytes = kRecWeightBytes + NR * 1024;  // + X: NR loads of 64 x 16 bytes
  static constexpr int kLoads = kRecWeightLoads + NR;               // vector-memory instructions per round
};

// Source offsets of a lane's weight slots, relative to the first record the
// tile touches in the round (byte 144 * tile of the round): slot s = 64*i +
// lane carries chunk c = s % 11 of row s / 11 and lands at byte 16*s of the
// stage, so row t starts at byte 176*t.  Apart from the tile's base, which is
// wave-uniform and travels in scalar registers, the offsets depend on the lane
// and on M only; a 128-column last tile (M % 256 == 128) has its own set.
// Slots that carry nothing the tile needs (chunk 9 of an aligned row, chunk 10,
// the slots past row 31, groups 4-7 in a 128-column tile) re-load the row's
// first header chunk: every round issues the same instructions, which keeps
// the vmcnt arithmetic exact, and every address stays inside the stream.
struct RecSlots {
  uint32_t full[kRecWeightLoads];  // 256-column tile
  uint32_t half[kRecWeightLoads];  // 128-column last tile
};

__device__ __forceinline__ void rec_slots(RecSlots& s, int lane, int m) {
  const uint32_t halves_per_row = (uint32_t)m >> 7;  // 128-column halves of a row
#pragma unroll
  for (int i = 0; i < kRecWeightLoads; ++i) {
    const int slot = 64 * i + lane;
    const int row = min(slot / kRecSlotsPerRow, kRoundRows - 1);
    const int c = slot < kRoundRows * kRecSlotsPerRow ? slot % kRecSlotsPerRow : kRecSlotsPerRow - 1;
    const uint32_t halves = (uint32_t)row * halves_per_row;  // row start, in 128-column units
    const uint32_t head = (halves >> 1) * kSbBytes;          // the record the row starts in
    const bool shifted = halves & 1;                         // ... half-way in
    // aligned row: header, then payload chunk c-1 at 16*c (c = 1..8).
    // shifted row: header of s, chunks 4-7 of s (c = 1..4), header of s+1
    // (c = 5) and chunks 0-3 of s+1 (c = 6..9): one window from byte 80.
    const uint32_t pay = 16 * c + (shifted ? 64 : 0);
    const int last_full = shifted ? 9 : 8;
    s.full[i] = head + ((c >= 1 && c <= last_full) ? pay : 0u);
    s.half[i] = head + ((c >= 1 && c <= 4) ? pay : 0u);
  }
}

template <int NR>
__device__ __forceinline__ void rec_issue(const uint32_t (&woff)[kRecWeightLoads], const uint8_t* wround,
                                          const uint8_t* xround, const uint32_t (&xoff)[NR], uint32_t stage) {
#pragma unroll
  for (int i = 0; i < kRecWeightLoads; ++i) lds_dma16(wround, woff[i], stage + 1024 * i);
#pragma unroll
  for (int nt = 0; nt < NR; ++nt) lds_dma16(xround, xoff[nt], stage + kRecWeightBytes + 1024 * nt);
}

// Per-lane LDS read offsets inside a stage: payload (8 bytes = the lane's 16
// columns) and fp16 scale of a row, for rows that start on a record boundary
// ([0]) and rows that start half-way into one ([1]).
struct RecReads {
  uint32_t pay[2];
  uint32_t sc[2];
  uint32_t x;
};

// Accumulators of one wave: 16 MFMA column blocks (block c = columns 16j + c
// for lane column j) per 16-row block of X.
template <int NR>
struct RecAcc {
  float4_t c[NR][16];
};

template <int NR>
__device__ __forceinline__ void rec_compute(RecAcc<NR>& acc, const uint8_t* st, const RecReads& rd, int q,
                                            uint32_t smask, MagicWords mw) {
  half8_t xr[NR];
#pragma unroll
  for (int nt = 0; nt < NR; ++nt)
    xr[nt] = *reinterpret_cast<const half8_t*>(st + kRecWeightBytes + 1024 * nt + rd.x);
  const uint8_t* rows = st + kRecRowBytes * 8 * q;  // rows 8q .. 8q+7 of the round
  uint2 w[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const uint2*>(rows + kRecRowBytes * u + rd.pay[u & 1]);
  uint32_t sp[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t lo = *reinterpret_cast<const uint16_t*>(rows + kRecRowBytes * (2 * p) + rd.sc[0]);
    const uint32_t hi = *reinterpret_cast<const uint16_t*>(rows + kRecRowBytes * (2 * p + 1) + rd.sc[1]);
    sp[p] = (lo | (hi << 16)) & smask;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    half2_t pr[4][8];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t a = h ? w[2 * p].y : w[2 * p].x;
      const uint32_t b = h ? w[2 * p + 1].y : w[2 * p + 1].x;
      dequant_row_pair(a, b, bitcast<half2_t>(sp[p]), pr[p], mw);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      half8_t b;
      b[0] = pr[0][c][0]; b[1] = pr[0][c][1];
      b[2] = pr[1][c][0]; b[3] = pr[1][c][1];
      b[4] = pr[2][c][0]; b[5] = pr[2][c][1];
      b[6] = pr[3][c][0]; b[7] = pr[3][c][1];
#pragma unroll
      for (int nt = 0; nt < NR; ++nt)
        acc.c[nt][8 * h + c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xr[nt], b, acc.c[nt][8 * h + c], 0, 0, 0);
    }
  }
}

// Work split.  A workgroup covers kC adjacent 256-column tiles (a "tile
// group"): wave w works on tile w % kC of the group and takes every
// (4 / kC)-th round, so the waves of one tile share its K range and meet in
// an LDS reduction, and each row the workgroup reads is kC whole records
// long (wider runs of a row per CU use the 128-byte lines better).  The items
// are (tile group, round) pairs in group-major order; workgroup p takes a
// contiguous range (stream-K), and runs it as segments, one per tile group
// it touches.  A segment covering a whole group writes Y; any other segment
// writes fp32 partials into slots 2p (the workgroup's first segment) or
// 2p + 1 (its last), and the fix-up kernel adds the partials of each shared
// group in workgroup order, so results are deterministic.
__device__ __forceinline__ void streamk_range(const GemmParams& P, int p, int& lo, int& hi) {
  lo = p * P.items_base + min(p, P.items_rem);
  hi = lo + P.items_base + (p < P.items_rem ? 1 : 0);
}

// Workgroup whose range holds item i.
__device__ __forceinline__ int streamk_owner(const GemmParams& P, int i) {
  const int big = P.items_rem * (P.items_base + 1);
  return i < big ? i / (P.items_base + 1) : P.items_rem + (i - big) / P.items_base;
}

// LDS position (floats) of D[row][col] of one tile inside a reduction slot:
// four consecutive columns form one 16-byte quad, and the quads of column
// group jj = col / 16 are rotated by jj / 4, so that any 8 consecutive lanes
// of a row address 8 different 16-byte bank groups.
__device__ __forceinline__ int red_pos(int row, int jj, int u) {
  return row * kRecCols + 16 * jj + 4 * ((u + (jj >> 2)) & 3);
}

// Where a tile group's results go: tile tl of the group covers columns
// m0 + tl*256 .. of `y` (single matrix: adjacent tiles; several matrices: one
// tile of matrix i); with SwiGLU both tiles (gate, up) cover columns m0 ..
// and the group writes h.
struct RecOut {
  float* y;
  int m0;
  float poison;  // added to every result: NaN when the workspace's status was set at the start of the call
};

template <int kMode>
__device__ __forceinline__ int rec_col(const RecOut& o, int tl, int qd) {
  return o.m0 + (kMode == kModeSwiglu ? 0 : tl * kRecCols) + 4 * qd;
}

template <int kMode>
__device__ __forceinline__ void rec_put_y(const GemmParams& P, const RecOut& o, int row, int col, float4_t v) {
  v = poisoned(v, o.poison);
  float* yp = o.y + (int64_t)row * P.m + col;
  if (P.y_vec) {
    *reinterpret_cast<float4_t*>(yp) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) yp[e] = v[e];
  }
}

__device__ __forceinline__ void rec_put_h(const GemmParams& P, const RecOut& o, int row, int col, float4_t g,
                                          float4_t u) {
  g = poisoned(g, o.poison);
  *reinterpret_cast<uint2*>(P.h + (int64_t)row * P.m + col) = swiglu4(g, u);  // m % 128 == 0: 8-byte aligned
}

// Sum of the `nslots` LDS slots of tile tl at quad (row, qd) (slot s of tile tl
// at red + (tl * nslots + s) * per_slot), in wave order.
__device__ __forceinline__ float4_t rec_lds_sum(const float* red, int per_slot, int nslots, int tl, int row, int qd) {
  const float* base = red + tl * nslots * per_slot + red_pos(row, qd >> 2, qd & 3);
  float4_t v = *reinterpret_cast<const float4_t*>(base);
  for (int sl = 1; sl < nslots; ++sl) v += *reinterpret_cast<const float4_t*>(base + sl * per_slot);
  return v;
}

// Output of a tile group: tile tl of the group sums its LDS slots and goes to
// Y (part == nullptr; with SwiGLU the two tiles' sums combine into h) or to
// the partial slot part + tl * per_slot, plain (for the fix-up kernel) or
// encoded and device-coherent (for the owner of the group).  The whole
// workgroup stores, one 4-column quad per thread and step.
template <int kC, int kW, int kMode>
__device__ __forceinline__ void rec_store(const GemmParams& P, const float* red, int per_slot, int nslots,
                                          const RecOut& o, float* part, bool coherent) {
  if (kMode == kModeSwiglu && !part) {
    for (int idx = threadIdx.x; idx < P.n * 64; idx += kW * 64) {
      const int row = idx >> 6, qd = idx & 63;
      const int col = rec_col<kMode>(o, 0, qd);
      if (col >= P.m) continue;
      rec_put_h(P, o, row, col, rec_lds_sum(red, per_slot, nslots, 0, row, qd),
                rec_lds_sum(red, per_slot, nslots, 1, row, qd));
    }
    return;
  }
  const int total = kC * P.n * 64;
  for (int idx = threadIdx.x; idx < total; idx += kW * 64) {
    const int tl = kC == 1 ? 0 : idx / (P.n * 64);
    const int w = idx - tl * P.n * 64;
    const int row = w >> 6, qd = w & 63;
    const int col = rec_col<kMode>(o, tl, qd);
    if (col >= P.m) continue;
    const float4_t v = rec_lds_sum(red, per_slot, nslots, tl, row, qd);
    if (part) {
      float* pp = part + tl * per_slot + row * kRecCols + 4 * qd;
      if (coherent) store_sc1(pp, enc_partial(v));
      else *reinterpret_cast<float4_t*>(pp) = v;
    } else {
      rec_put_y<kMode>(P, o, row, col, v);
    }
  }
}

// In-kernel hand-off, run by the owner of a shared tile group (the workgroup
// whose range holds the group's last round; it processes that segment last,
// after every contribution it makes to other groups).  The contributors
// p0 .. owner-1 have stored their partials encoded, each before any wait of
// its own; the owner reads them device-coherently, polls again while any
// word reads "not written", adds them in workgroup order and its own partial
// (the LDS slots) last -- the fix-up kernel's order, so both hand-offs give
// the same bits -- writes Y and clears the chunks it read.
//
// A thread takes kQ of its quads at a time and kCB contributors of each: the
// kQ * kCB = 16 loads go out together, one memory round trip per batch.
template <int kQ, int kCB, int kC, int kW, int kMode>
__device__ __forceinline__ void rec_gather_batched(const GemmParams& P, float* red, int per_slot, int nslots,
                                                   int tg, const RecOut& o, int owner, int p0, int& polls) {
  static_assert(kQ * kCB == 16, "one batch is 16 loads");
  const int item0 = tg * P.rounds;
  const int total = kC * P.n * 64;
  const float4_t zero = {0.f, 0.f, 0.f, 0.f};
  const uint32_t slot_bytes = (uint32_t)(kC * per_slot * sizeof(float));  // partials of one workgroup segment
  for (int first = threadIdx.x; first < total; first += kQ * kW * 64) {
    uint32_t off[kQ];  // byte offset of quad j inside a slot
    bool ok[kQ];
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
      const int idx = first + j * kW * 64;
      const int tl = kC == 1 ? 0 : idx / (P.n * 64);
      const int w = idx - tl * P.n * 64;
      const int row = w >> 6, qd = w & 63;
      ok[j] = idx < total && rec_col<kMode>(o, tl, qd) < P.m;
      off[j] = ok[j] ? (uint32_t)(4 * (tl * per_slot + row * kRecCols + 4 * qd)) : 0u;  // outside: a harmless read
    }
    float4_t v[kQ];
#pragma unroll
    for (int j = 0; j < kQ; ++j) v[j] = zero;
    for (int c0 = p0; c0 < owner; c0 += kCB) {
      uint32_t a[16];
#pragma unroll
      for (int i = 0; i < kCB; ++i) {
        const int pp = min(c0 + i, owner - 1);  // past the last contributor: re-read it, not added
        const int lo_p = pp * P.items_base + min(pp, P.items_rem);
        const uint32_t slot = (uint32_t)(2 * pp + (lo_p < item0 ? 1 : 0)) * slot_bytes;
#pragma unroll
        for (int j = 0; j < kQ; ++j) a[j * kCB + i] = slot + off[j];
      }
      float4_t t[16];
      load16_sc1(t, P.partials, a);
      // a chunk still unwritten: load the whole batch again (one round trip
      // for all of them) after a short sleep
      bool ready;
      for (;;) {
        ready = true;
#pragma unroll
        for (int j = 0; j < kQ; ++j)
#pragma unroll
          for (int i = 0; i < kCB; ++i)
            if (ok[j] && c0 + i < owner) ready = ready && partial_ready(t[j * kCB + i]);
        if (handoff_stop(ready, polls)) break;
        --polls;
        __builtin_amdgcn_s_sleep(1);
        load16_sc1(t, P.partials, a);
      }
      // out of polls: record it (every later call on this workspace writes
      // NaN until it is cleared) and add what there is (a missing chunk
      // decodes to NaN)
      if (handoff_gave_up(ready, polls)) __hip_atomic_fetch_or(P.status, kWsStatusHandoffTimeout, __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int j = 0; j < kQ; ++j)
#pragma unroll
        for (int i = 0; i < kCB; ++i)  // in workgroup order
          if (ok[j] && c0 + i < owner) v[j] += dec_partial(t[j * kCB + i]);
      // clear every chunk of the batch: after a give-up this also removes a
      // late partial that landed between the last poll and here (one that
      // lands later stays, and the status word covers it)
#pragma unroll
      for (int j = 0; j < kQ; ++j)
#pragma unroll
        for (int i = 0; i < kCB; ++i)
          if (ok[j] && c0 + i < owner) store_sc1_at(P.partials, a[j * kCB + i], zero);
    }
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
      if (!ok[j]) continue;
      const int idx = first + j * kW * 64;
      const int tl = kC == 1 ? 0 : idx / (P.n * 64);
      const int w = idx - tl * P.n * 64;
      const int row = w >> 6, qd = w & 63;
      v[j] += rec_lds_sum(red, per_slot, nslots, tl, row, qd);
      if (kMode == kModeSwiglu) {
        // the group's sum of tile tl replaces its first LDS slot; h follows
        // once both tiles are summed
        *reinterpret_cast<float4_t*>(red + tl * nslots * per_slot + red_pos(row, qd >> 2, qd & 3)) = v[j];
      } else {
        rec_put_y<kMode>(P, o, row, rec_col<kMode>(o, tl, qd), v[j]);
      }
    }
  }
}

// Batch shape by contributor count: as many of a thread's quads per batch as
// 16 loads allow with every contributor (up to 8) in it.
template <int kC, int kW, int kMode>
__device__ __forceinline__ void rec_gather(const GemmParams& P, float* red, int per_slot, int nslots, int tg,
                                           const RecOut& o, int owner) {
  const int p0 = streamk_owner(P, tg * P.rounds);
  int polls = kMaxPolls;  // this thread's budget of repeated loads
  const int contributors = owner - p0;
  if (contributors <= 2)
    rec_gather_batched<8, 2, kC, kW, kMode>(P, red, per_slot, nslots, tg, o, owner, p0, polls);
  else if (contributors <= 4)
    rec_gather_batched<4, 4, kC, kW, kMode>(P, red, per_slot, nslots, tg, o, owner, p0, polls);
  else
    rec_gather_batched<2, 8, kC, kW, kMode>(P, red, per_slot, nslots, tg, o, owner, p0, polls);
  if (kMode == kModeSwiglu) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < P.n * 64; idx += kW * 64) {
      const int row = idx >> 6, qd = idx & 63;
      const int col = rec_col<kMode>(o, 0, qd);
      if (col >= P.m) continue;
      rec_put_h(P, o, row, col, *reinterpret_cast<const float4_t*>(red + red_pos(row, qd >> 2, qd & 3)),
                *reinterpret_cast<const float4_t*>(red + nslots * per_slot + red_pos(row, qd >> 2, qd & 3)));
    }
  }
}

template <int NR, int kDepth, int kC, int kW, int kMode>
__global__ void __launch_bounds__(kW * 64) int4_gemm_records_kernel(GemmParams P) {
  using G = RecGeom<NR>;
  static_assert(kMode == kModeSingle || (kMode == kModeMulti && kC == 1) || (kMode == kModeSwiglu && kC == 2),
                "several matrices: one tile per group; SwiGLU: gate and up tile per group");
  constexpr int kShare = kW / kC;  // waves per tile
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // fetch every argument now, in one batch of scalar loads, rather than at
  // first use (each late load is another serial trip to memory)
  asm volatile("" : : "s"(P.x), "s"(P.sb), "s"(P.y), "s"(P.partials), "s"(P.n), "s"(P.k), "s"(P.m),
               "s"(P.rounds), "s"(P.shift), "s"(P.y_vec), "s"(P.items_base), "s"(P.items_rem), "s"(P.tiles),
               "s"(P.finish), "s"(P.splits));
  if (kMode != kModeSingle)
    asm volatile("" : : "s"(P.sbm[0]), "s"(P.sbm[1]), "s"(P.sbm[2]), "s"(P.sbm[3]), "s"(P.ym[0]), "s"(P.ym[1]),
                 "s"(P.ym[2]), "s"(P.ym[3]), "s"(P.h));
  const int lane = threadIdx.x & 63;
  // wave index as a scalar: the round loop below is then uniform control flow
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tl = wave % kC, kpart = wave / kC;
  const int j = lane & 15, q = lane >> 4;
  const int g = j >> 1;  // lane j owns columns 16j .. 16j+15 of a tile (group j/2)
  const MagicWords mw = magic_words();
  RecReads rd;
  rd.pay[0] = 16 + 16 * g + 8 * (j & 1);
  rd.sc[0] = 2 * g;
  if (P.shift) {
    rd.pay[1] = (g >= 4 ? 32 : 16) + 16 * g + 8 * (j & 1);
    rd.sc[1] = (g < 4 ? 8 : 72) + 2 * g;
  } else {
    rd.pay[1] = rd.pay[0];
    rd.sc[1] = rd.sc[0];
  }
  rd.x = 64 * j + 16 * (q ^ (j & 3) ^ ((j >> 2) & 3));
  // X slice loads: lane l fetches row 16*nt + l/4 (rows past N repeat row N-1;
  // their products land in output rows that are never stored), 8 fp16 at
  // column 8 * ((l & 3) ^ ((l >> 2) & 3) ^ ((l >> 4) & 3)) of the round: the
  // read-back (lane (q, j): row j, columns 8q..8q+7) then spreads any 8
  // consecutive lanes over 8 different 16-byte bank groups
  uint32_t xoff[NR];
#pragma unroll
  for (int nt = 0; nt < NR; ++nt) {
    const int row = min(16 * nt + (lane >> 2), P.n - 1);
    const int chunk = (lane & 3) ^ ((lane >> 2) & 3) ^ ((lane >> 4) & 3);
    xoff[nt] = (uint32_t)(2 * (row * P.k + 8 * chunk));
  }
  // Workgroup ids are dealt round-robin to the 8 XCDs: give each XCD one
  // contiguous run of ranges, so that neighbouring tiles, which share the
  // 128-byte lines at their edges, meet in its L2.  Within a run the range
  // order is the dispatch order, so the owner of a tile group (its highest
  // range, which waits in the in-kernel hand-off) starts after the
  // contributors it waits for; only a group that straddles two runs (at most
  // 7) can have an owner dispatched before a contributor, and those few
  // waiting owners cannot hold back the dispatch of the rest.  (The workgroup
  // count is P.splits: the grid size would be one more serial load from the
  // dispatch's hidden arguments.)
  const int nwg = P.splits, b = blockIdx.x, per = nwg / kXcds;
  const int p = b < per * kXcds ? (b % kXcds) * per + b / kXcds : b;
  int lo, hi;
  streamk_range(P, p, lo, hi);

  // the status word's copies first in LDS, the ring and reduction slots after
  uint32_t* lds_status = reinterpret_cast<uint32_t*>(smem);
  uint8_t* const lds0 = smem + kStatusLdsBytes;
  status_to_lds(P.status, lds_status);  // read once the segment's ring has drained
  const uint64_t round_bytes = P.rec_round_bytes;
  RecSlots slots;
  rec_slots(slots, lane, P.rec_row_m);
  uint8_t* ring = lds0 + wave * kDepth * G::kStageBytes;
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(lds_ptr_t)ring;  // LDS byte address (wave-uniform)
  float* red = reinterpret_cast<float*>(lds0);
  const int per_slot = P.n * kRecCols;
  constexpr int kSlots = kShare;  // reduction slots per tile: one per wave

  // Segments (the range's pieces in one tile group) run from the last to the
  // first: the segment that ends a tile group (its owner's) then runs last in
  // its workgroup, and the segments that contribute to it run first in theirs.
  for (int seg_hi = hi; seg_hi > lo;) {
    const int tg = (seg_hi - 1) / P.rounds;
    const int seg_lo = max(lo, tg * P.rounds);
    const int r0 = seg_lo - tg * P.rounds;
    const int r1 = seg_hi - tg * P.rounds;
    // this wave's tile: its matrix, its index in that matrix, its records
    int mat = 0, ltile = tg * kC + tl;
    if (kMode == kModeMulti) {
      mat = (ltile >= P.tiles) + (ltile >= 2 * P.tiles) + (ltile >= 3 * P.tiles);
      ltile -= mat * P.tiles;
    } else if (kMode == kModeSwiglu) {
      mat = tl;
      ltile = tg;
    }
    const bool has_tile = ltile < P.tiles && mat < (kMode == kModeSingle ? 1 : P.mats);  // the last group may be short
    const int groups = has_tile ? min(8, (P.m - kRecCols * ltile) >> 5) : 0;  // 4 or 8 (M % 128 == 0)
    const uint32_t smask = g < groups ? 0xFFFFFFFFu : 0u;
    uint32_t woff[kRecWeightLoads];
#pragma unroll
    for (int i = 0; i < kRecWeightLoads; ++i) woff[i] = groups < 8 ? slots.half[i] : slots.full[i];
    const uint8_t* wmat = kMode == kModeSingle ? P.sb : select4(mat, P.sbm[0], P.sbm[1], P.sbm[2], P.sbm[3]);
    const uint8_t* wtile = wmat + P.rec_tile_bytes * (uint64_t)(has_tile ? ltile : 0);
    // where the group's results go (the group's first tile)
    RecOut out;
    if (kMode == kModeSingle) {
      out.y = P.y;
      out.m0 = tg * kC * kRecCols;
    } else if (kMode == kModeMulti) {
      out.y = select4(mat, P.ym[0], P.ym[1], P.ym[2], P.ym[3]);
      out.m0 = ltile * kRecCols;
    } else {
      out.y = nullptr;
      out.m0 = tg * kRecCols;
    }

    RecAcc<NR> acc;
#pragma unroll
    for (int nt = 0; nt < NR; ++nt)
#pragma unroll
      for (int c = 0; c < 16; ++c) acc.c[nt][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int first = r0 + kpart;
    const int cnt = (has_tile && first < r1) ? (r1 - first + kShare - 1) / kShare : 0;
    auto issue = [&](int i) {
      const int r = first + kShare * i;
      rec_issue<NR>(woff, wtile + (uint64_t)r * round_bytes, reinterpret_cast<const uint8_t*>(P.x) + 64 * r, xoff,
                    __builtin_amdgcn_readfirstlane(ring_lds + (i % kDepth) * G::kStageBytes));
    };
#pragma unroll
    for (int i = 0; i < kDepth - 1; ++i)
      if (i < cnt) issue(i);
    for (int i = 0; i < cnt; ++i) {
      if (i + kDepth - 1 < cnt) {
        issue(i + kDepth - 1);
        wait_vmcnt<(kDepth - 1) * G::kLoads>();
      } else {
        const int after = cnt - 1 - i;  // rounds issued after round i: 0 .. kDepth - 2
        if (kDepth >= 5 && after == 4) wait_vmcnt<(kDepth >= 5 ? 4 * G::kLoads : 0)>();
        else if (kDepth >= 4 && after == 3) wait_vmcnt<(kDepth >= 4 ? 3 * G::kLoads : 0)>();
        else if (kDepth >= 3 && after == 2) wait_vmcnt<(kDepth >= 3 ? 2 * G::kLoads : 0)>();
        else if (kDepth >= 2 && after == 1) wait_vmcnt<(kDepth >= 2 ? G::kLoads : 0)>();
        else wait_vmcnt<0>();
      }
      rec_compute<NR>(acc, ring + (i % kDepth) * G::kStageBytes, rd, q, smask, mw);
    }
    __syncthreads();  // the ring is reused for the reduction
    wait_vmcnt<0>();  // the ring has drained: free
    out.poison = status_poison(status_from_lds(lds_status));

    // Waves of one tile add up through LDS: each stores its accumulators in
    // its own slot of the tile, and the store below sums the slots in wave
    // order.  Lane (q, j) holds D[16*nt + 4q + v][16j + c]; 4 columns per
    // access.
    {
      float* slot = red + (tl * kSlots + kpart) * per_slot;
#pragma unroll
      for (int nt = 0; nt < NR; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = nt * 16 + 4 * q + v;
          if (row < P.n) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float4_t val = {acc.c[nt][4 * u][v], acc.c[nt][4 * u + 1][v], acc.c[nt][4 * u + 2][v],
                                    acc.c[nt][4 * u + 3][v]};
              *reinterpret_cast<float4_t*>(slot + red_pos(row, j, u)) = val;
            }
          }
        }
    }
    __syncthreads();
    const bool whole = r0 == 0 && r1 == P.rounds;
    const int pslot = 2 * p + (seg_lo == lo ? 0 : 1);
    const bool in_kernel = P.finish != kFinishSecondKernel;
    if (!whole && in_kernel && r1 == P.rounds) {
      rec_gather<kC, kW, kMode>(P, red, per_slot, kSlots, tg, out, p);  // this workgroup owns the group
    } else {
      rec_store<kC, kW, kMode>(P, red, per_slot, kSlots, out,
                               whole ? nullptr : P.partials + (int64_t)pslot * kC * per_slot, in_kernel);
    }
    __syncthreads();  // LDS is the next segment's ring
    seg_hi = seg_lo;
  }
}

// Sum of tile tl's partials of tile group tg at quad (row, qd) over the
// contributing workgroups p0 .. p1, in workgroup order; the slots are left at
// zero (the in-kernel hand-off reads zero as empty).  The partials are
// independent loads: 8 go out before any add (a load-then-add loop would pay
// one memory round trip per partial).
__device__ __forceinline__ float4_t fixup_sum(const GemmParams& P, int group_tiles, int item0, int p0, int p1, int tl,
                                              int row, int qd) {
  const int per_slot = P.n * kRecCols;
  float4_t v = {0.f, 0.f, 0.f, 0.f};
  const int64_t off = (int64_t)tl * per_slot + row * kRecCols + 4 * qd;
  for (int p8 = p0; p8 <= p1; p8 += 8) {
    float4_t t[8];
    float4_t* a[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int pp = min(p8 + i, p1);  // past the end: re-read the last one, added as 0 below
      const int lo_p = pp * P.items_base + min(pp, P.items_rem);
      const int pslot = 2 * pp + (lo_p < item0 ? 1 : 0);
      a[i] = reinterpret_cast<float4_t*>(P.partials + (int64_t)pslot * group_tiles * per_slot + off);
      t[i] = *a[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)  // in workgroup order
      if (p8 + i <= p1) v += t[i];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (p8 + i <= p1) *a[i] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  return v;
}

// Fix-up of the tile groups that several workgroups share: Y = sum of their
// partials in workgroup order (with SwiGLU, h from the gate and up sums).
// One thread per 4-column quad of a tile (of a gate/up pair).
__global__ void __launch_bounds__(256) streamk_fixup_kernel(GemmParams P, int group_tiles, int mode) {
  const float poison =
      status_poison(P.status ? __hip_atomic_load(P.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u);
  const int per_tile = P.n * 64;
  const int tiles = mode == kModeMulti ? P.mats * P.tiles : P.tiles;  // tiles (gate/up pairs) to cover
  const int total = tiles * per_tile;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const int tile = e / per_tile, w = e - tile * per_tile;
    const int row = w >> 6, qd = w & 63;
    const int tg = mode == kModeSwiglu ? tile : tile / group_tiles;
    const int item0 = tg * P.rounds;
    const int p0 = streamk_owner(P, item0), p1 = streamk_owner(P, item0 + P.rounds - 1);
    if (p0 == p1) continue;  // one workgroup covered the group and wrote it
    if (mode == kModeSwiglu) {
      const int col = tile * kRecCols + 4 * qd;
      if (col >= P.m) continue;
      const float4_t gsum = poisoned(fixup_sum(P, 2, item0, p0, p1, 0, row, qd), poison);
      const float4_t usum = fixup_sum(P, 2, item0, p0, p1, 1, row, qd);
      *reinterpret_cast<uint2*>(P.h + (int64_t)row * P.m + col) = swiglu4(gsum, usum);
      continue;
    }
    const int tl = tile - tg * group_tiles;
    int mat = 0, ltile = tile;
    if (mode == kModeMulti) {
      mat = (tile >= P.tiles) + (tile >= 2 * P.tiles) + (tile >= 3 * P.tiles);
      ltile = tile - mat * P.tiles;
    }
    const int col = ltile * kRecCols + 4 * qd;
    if (col >= P.m) continue;
    const float4_t v = poisoned(fixup_sum(P, group_tiles, item0, p0, p1, tl, row, qd), poison);
    float* yp = (mode == kModeMulti ? select4(mat, P.ym[0], P.ym[1], P.ym[2], P.ym[3]) : P.y) +
                (int64_t)row * P.m + col;
    if (P.y_vec) {
      *reinterpret_cast<float4_t*>(yp) = v;
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) yp[k] = v[k];
    }
  }
}

// Second kernel of kFinishSecondKernel: y = sum over splits of the partials.
__global__ void __launch_bounds__(256) splitk_sum_kernel(float* __restrict__ partials, int splits, int64_t nm,
                                                         float* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nm; i += stride) {
    // 8 independent loads in flight before any add, summed in split order
    float v = 0.0f;
    for (int s8 = 0; s8 < splits; s8 += 8) {
      float t[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) t[k] = partials[(int64_t)min(s8 + k, splits - 1) * nm + i];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (s8 + k < splits) v += t[k];
#pragma unroll
      for (int k = 0; k < 8; ++k)  // leave the workspace at zero for the calls that share it
        if (s8 + k < splits) partials[(int64_t)(s8 + k) * nm + i] = 0.0f;
    }
    y[i] = v;
  }
}

// ---------------------------------------------------------------------------
// Host-side launch (called from abi.hip after argument validation).

int gemm_col_tiles(int m) { return (m + kTileCols - 1) / kTileCols; }
int gemm_rounds(int k) { return (k + kRoundRows - 1) / kRoundRows; }

static size_t reduce_lds(int npad) { return (size_t)2 * npad * kTileCols * sizeof(float); }

template <bool kMfma, int NR, int B, int kFront>
static void launch_one(const GemmParams& P, hipStream_t stream) {
  const size_t red = reduce_lds(kMfma ? NR * 16 : NR);
  const size_t stg = kFront != kFrontDirect ? (size_t)kWaves * B * kStageRound : 0;
  hipLaunchKernelGGL((int4_gemm_kernel<kMfma, NR, B, kFront>), dim3(P.tiles * P.splits), dim3(kThreads),
                     red > stg ? red : stg, stream, P);
}

template <int B, int kFront>
static hipError_t launch_gemm_variant(const GemmParams& P, int algo, hipStream_t stream) {
  if (algo == 2) {
    if (P.n <= 16) launch_one<true, 1, B, kFront>(P, stream);
    else launch_one<true, 2, B, kFront>(P, stream);
    return hipGetLastError();
  }
  switch (P.n) {
    case 1: launch_one<false, 1, B, kFront>(P, stream); break;
    case 2: launch_one<false, 2, B, kFront>(P, stream); break;
    case 3: launch_one<false, 3, B, kFront>(P, stream); break;
    case 4: launch_one<false, 4, B, kFront>(P, stream); break;
    case 5: launch_one<false, 5, B, kFront>(P, stream); break;
    case 6: launch_one<false, 6, B, kFront>(P, stream); break;
    case 7: launch_one<false, 7, B, kFront>(P, stream); break;
    case 8: launch_one<false, 8, B, kFront>(P, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int kFront>
static hipError_t launch_front(const GemmParams& P, int algo, int batch, hipStream_t stream) {
  if (batch >= 4) return launch_gemm_variant<4, kFront>(P, algo, stream);
  if (batch == 2) return launch_gemm_variant<2, kFront>(P, algo, stream);
  return launch_gemm_variant<1, kFront>(P, algo, stream);
}

// Reduction slots of one tile: one per wave that shares it.
constexpr int rec_slots_per_tile(int waves, int group_tiles) { return waves / group_tiles; }

template <int NR, int kDepth, int kC, int kW, int kMode>
static hipError_t launch_records_one(const GemmParams& P, int wgs, hipStream_t stream) {
  const size_t ring = (size_t)kW * kDepth * RecGeom<NR>::kStageBytes;
  const size_t red = (size_t)kC * rec_slots_per_tile(kW, kC) * P.n * kRecCols * sizeof(float);
  const size_t lds = (ring > red ? ring : red) + kStatusLdsBytes;
  if (lds > kMaxDynamicLds) return hipErrorInvalidValue;  // never launch past the LDS
  hipLaunchKernelGGL((int4_gemm_records_kernel<NR, kDepth, kC, kW, kMode>), dim3(wgs), dim3(kW * 64), lds, stream,
                     P);
  return hipGetLastError();
}

template <int NR, int kC, int kW>
static hipError_t launch_records_depth(const GemmParams& P, int wgs, int depth, hipStream_t stream) {
  // the ring must fit: clamp the depth (kW waves x depth stages)
  const int max_depth = (int)((kMaxDynamicLds - kStatusLdsBytes) / ((size_t)kW * RecGeom<NR>::kStageBytes));
  if (depth > max_depth) depth = max_depth;
  if (depth >= 5) return launch_records_one<NR, 5, kC, kW, kModeSingle>(P, wgs, stream);
  if (depth == 4) return launch_records_one<NR, 4, kC, kW, kModeSingle>(P, wgs, stream);
  if (depth == 3) return launch_records_one<NR, 3, kC, kW, kModeSingle>(P, wgs, stream);
  if (depth == 2) return launch_records_one<NR, 2, kC, kW, kModeSingle>(P, wgs, stream);
  return launch_records_one<NR, 1, kC, kW, kModeSingle>(P, wgs, stream);
}

template <int NR, int kW>
static hipError_t launch_records_group(const GemmParams& P, int wgs, int depth, int group_tiles, hipStream_t stream) {
  if (group_tiles == 4) return launch_records_depth<NR, 4, kW>(P, wgs, depth, stream);
  if (group_tiles == 2) return launch_records_depth<NR, 2, kW>(P, wgs, depth, stream);
  return launch_records_depth<NR, 1, kW>(P, wgs, depth, stream);
}

// 8 waves hold at most 256 registers per lane, too few for the accumulators
// of 32 rows: those run on 4 waves (the plan never asks otherwise)
template <int NR>
static hipError_t launch_records(const GemmParams& P, int wgs, int depth, int group_tiles, int waves,
                                 hipStream_t stream) {
  if (NR == 1 && waves == 8) return launch_records_group<1, 8>(P, wgs, depth, group_tiles, stream);
  if (waves != 4) return hipErrorInvalidValue;
  return launch_records_group<NR, 4>(P, wgs, depth, group_tiles, stream);
}

// Several matrices (one tile per group) or SwiGLU pairs (gate and up tile per
// group): 4 waves, ring depth 2 or 3.
template <int NR, int kMode>
static hipError_t launch_records_fused(const GemmParams& P, int wgs, int depth, hipStream_t stream) {
  constexpr int kC = kMode == kModeSwiglu ? 2 : 1;
  if (depth >= 3) return launch_records_one<NR, 3, kC, 4, kMode>(P, wgs, stream);
  return launch_records_one<NR, 2, kC, 4, kMode>(P, wgs, stream);
}

bool gemm_records_eligible(int k, int m) { return (m % 128) == 0 && (k % kRoundRows) == 0; }

// Dynamic LDS of one record-stream workgroup (after the depth clamp).
int gemm_records_tiles(int m) { return (m + kRecCols - 1) / kRecCols; }
int gemm_records_groups(int m, int group_tiles) { return (gemm_records_tiles(m) + group_tiles - 1) / group_tiles; }

// Workgroups of a stream-K launch share tile groups unless every range is a
// whole number of groups.
bool gemm_groups_shared(int64_t groups, int64_t rounds, int wgs) {
  const int64_t items = groups * rounds;
  const int64_t base = items / wgs, rem = items % wgs;
  return !(rem == 0 && base % rounds == 0);
}

bool gemm_records_shares_tiles(int k, int m, int group_tiles, int wgs) {
  return gemm_groups_shared(gemm_records_groups(m, group_tiles), k / kRoundRows, wgs);
}

// Tile groups of a fused launch: `mats` matrices of one tile each per group,
// or (SwiGLU) one gate/up pair per group.
int gemm_fused_groups(int mode, int mats, int m) {
  return mode == kModeSwiglu ? gemm_records_tiles(m) : mats * gemm_records_tiles(m);
}

bool gemm_fused_shares_tiles(int mode, int mats, int k, int m, int wgs) {
  return gemm_groups_shared(gemm_fused_groups(mode, mats, m), k / kRoundRows, wgs);
}

hipError_t launch_gemm(int algo, const uint16_t* x, const uint8_t* sb, float* y, int n, int k, int m, int splits,
                       int batch, int finish, int front, int group, int waves, float* partials, uint32_t* counters,
                       uint32_t* status, int tile_order, hipStream_t stream) {
  GemmParams P = {};
  P.x = x; P.sb = sb; P.y = y; P.partials = partials; P.counters = counters; P.status = status;
  P.n = n; P.k = k; P.m = m; P.splits = splits; P.rounds = gemm_rounds(k); P.tiles = gemm_col_tiles(m);
  P.x_vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (k % 8) == 0) ? 1 : 0;
  P.finish = finish;
  P.shift = 0;
  P.rounds_base = P.rounds / splits;
  P.rounds_rem = P.rounds % splits;
  P.y_vec = ((reinterpret_cast<uintptr_t>(y) & 15) == 0 && (reinterpret_cast<uintptr_t>(partials) & 15) == 0 &&
             (m % 4) == 0) ? 1 : 0;
  hipError_t e;
  if (front == kFrontRecords) {
    // matrix cores only, whole 32-row rounds, 128-column halves of records and
    // 16-byte X rows; anything else takes the general kernel's staged front end
    if (algo == 2 && gemm_records_eligible(k, m) && P.x_vec) {
      // `splits` is the stream-K workgroup count here
      const int wgs = splits, group_tiles = group;
      P.tiles = gemm_records_tiles(m);
      P.shift = (m % kRecCols) != 0;
      const int items = gemm_records_groups(m, group_tiles) * P.rounds;
      P.items_base = items / wgs;
      P.items_rem = items % wgs;
      P.y_vec = ((reinterpret_cast<uintptr_t>(y) & 15) == 0) ? 1 : 0;
      if (tile_order) {  // the caller has checked M % 256 == 0
        P.rec_round_bytes = (uint64_t)kRoundRows * kSbBytes;
        P.rec_tile_bytes = (uint64_t)k * kSbBytes;
        P.rec_row_m = kRecCols;
      } else {
        P.rec_round_bytes = (uint64_t)18 * (uint64_t)m;
        P.rec_tile_bytes = kSbBytes;
        P.rec_row_m = m;
      }
      e = P.n <= 16 ? launch_records<1>(P, wgs, batch, group_tiles, waves, stream)
                    : launch_records<2>(P, wgs, batch, group_tiles, waves, stream);
      if (e != hipSuccess || !gemm_records_shares_tiles(k, m, group_tiles, wgs) || finish != kFinishSecondKernel)
        return e;
      const int quads = P.tiles * P.n * 64;
      int blocks = (quads + 255) / 256;
      if (blocks > 2048) blocks = 2048;
      hipLaunchKernelGGL(streamk_fixup_kernel, dim3(blocks), dim3(256), 0, stream, P, group_tiles, (int)kModeSingle);
      return hipGetLastError();
    }
    // the planner gives the record-stream front end only to shapes and
    // inputs it takes (its workgroup count and workspace are not the
    // general kernel's)
    return hipErrorInvalidValue;
  }
  // the staged front ends need M % 64 == 0 (4-byte aligned scale pairs)
  if ((m % 64) != 0) front = kFrontDirect;
  if (front == kFrontLdsDma) e = launch_front<kFrontLdsDma>(P, algo, batch, stream);
  else if (front == kFrontVgprLds) e = launch_front<kFrontVgprLds>(P, algo, batch, stream);
  else e = launch_front<kFrontDirect>(P, algo, batch, stream);
  if (e != hipSuccess || splits == 1 || finish != kFinishSecondKernel) return e;
  const int64_t nm = (int64_t)n * m;
  int64_t blocks = (nm + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(splitk_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, partials, splits, nm, y);
  return hipGetLastError();
}

// Record-stream GEMM of `mats` matrices of one shape sharing X (mode
// kModeMulti: Y_i = X @ W_i) or of a gate/up pair (kModeSwiglu: h =
// silu(X @ W_0) * (X @ W_1) in fp16).  The caller has checked the shape
// (m % 128 == 0, k % 32 == 0, x 16-byte aligned).
hipError_t launch_gemm_fused(int mode, const uint16_t* x, const uint8_t* const* sbs, float* const* ys, uint16_t* h,
                             int mats, int n, int k, int m, int wgs, int depth, int finish, float* partials,
                             uint32_t* status, hipStream_t stream) {
  GemmParams P = {};
  P.x = x; P.sb = sbs[0]; P.y = ys ? ys[0] : nullptr; P.partials = partials; P.counters = nullptr; P.status = status;
  P.n = n; P.k = k; P.m = m; P.splits = wgs; P.rounds = gemm_rounds(k);
  P.tiles = gemm_records_tiles(m);
  P.x_vec = 1;
  P.finish = finish;
  P.shift = (m % kRecCols) != 0;
  const int items = gemm_fused_groups(mode, mats, m) * P.rounds;
  P.items_base = items / wgs;
  P.items_rem = items % wgs;
  P.mats = mats;
  P.rec_round_bytes = (uint64_t)18 * (uint64_t)m;
  P.rec_tile_bytes = kSbBytes;
  P.rec_row_m = m;
  int y_vec = 1;
  for (int i = 0; i < 4; ++i) {
    P.sbm[i] = sbs[i < mats ? i : 0];
    P.ym[i] = ys ? ys[i < mats ? i : 0] : nullptr;
    if (ys && i < mats && (reinterpret_cast<uintptr_t>(ys[i]) & 15) != 0) y_vec = 0;
  }
  P.y_vec = y_vec;
  P.h = h;
  hipError_t e;
  if (mode == kModeSwiglu)
    e = n <= 16 ? launch_records_fused<1, kModeSwiglu>(P, wgs, depth, stream)
                : launch_records_fused<2, kModeSwiglu>(P, wgs, depth, stream);
  else
    e = n <= 16 ? launch_records_fused<1, kModeMulti>(P, wgs, depth, stream)
                : launch_records_fused<2, kModeMulti>(P, wgs, depth, stream);
  if (e != hipSuccess || !gemm_fused_shares_tiles(mode, mats, k, m, wgs) || finish != kFinishSecondKernel) return e;
  const int tiles = mode == kModeMulti ? mats * P.tiles : P.tiles;
  const int quads = tiles * n * 64;
  int blocks = (quads + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(streamk_fixup_kernel, dim3(blocks), dim3(256), 0, stream, P, mode == kModeSwiglu ? 2 : 1, mode);
  return hipGetLastError();
}

// Records of W[K][M] (M % 256 == 0) from row order to tile order: record
// (row r, tile j) moves from r * (M/256) + j to j * K + r.  One thread per
// 16-byte chunk (9 per record), reading the source in order.
__global__ void records_to_tiles_kernel(const uint4* __restrict__ src, int64_t k, int64_t tiles, uint4* __restrict__ dst) {
  const int64_t chunks = k * tiles * 9;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rec = i / 9, c = i - rec * 9;
    const int64_t r = rec / tiles, j = rec - r * tiles;
    dst[(j * k + r) * 9 + c] = src[i];
  }
}

hipError_t launch_records_to_tiles(const uint8_t* sb, int k, int m, uint8_t* tiles, hipStream_t stream) {
  const int64_t chunks = (int64_t)k * (m / kRecCols) * 9;
  if (chunks == 0) return hipSuccess;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(records_to_tiles_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const uint4*>(sb), (int64_t)k, (int64_t)(m / kRecCols), reinterpret_cast<uint4*>(tiles));
  return hipGetLastError();
}

}  // namespace moat
