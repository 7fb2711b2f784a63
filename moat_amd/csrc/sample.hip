// Batched token sampling over LM-head logits: the table ("LUT") softmax of the
// reference's numpy sampler, then greedy argmax or a draw from the k most
// probable tokens (antigravity-engine/src/batch_generator.py:187-253,
// antigravity-engine/src/attention.py:60-135).
//
// One workgroup of 1024 threads per row (V <= 32768): thread t holds the
// logits t + 1024 j (j < 32) in registers after one coalesced pass; the fp16
// exp table (up to 32768 entries, 64 KB) and the row's fp16 table values, then
// probabilities, sit in LDS (64 KB, padded to 32768 entries so that every
// thread stores all 32 of its slots).  Per-element work is branch-free: a
// CU's 16 waves share one scalar unit, and per-element branches (exec-mask
// updates) made it the bottleneck.  Steps, with the reference's arithmetic:
//   1. x (f32/f16/f64) divided by the temperature in its own dtype (fp16:
//      divide in f32, round to fp16), then rounded to f32; the row maximum
//      (NaN-propagating); greedy: the first index of the raw maximum.
//   2. table index size-1-trunc(min(|x - max| / step, size-1)) (f32 division,
//      correctly rounded) -> e, the table's fp16 value.
//   3. sum of e in numpy's float32 order: pairwise sums of 8192-element chunks
//      (the reduction buffer) added in sequence from 0; inside a chunk,
//      halves split at multiples of 8 down to blocks of at most 128, each
//      summed with 8 strided accumulators, then its tail.  Per chunk: 8
//      chains per leaf (one thread each), one lane of a wave per node one
//      level above the leaves (up to 64), shuffles for the levels above.
//   4. p = fp16(e / sum) (f32 division).
//   5. greedy: log of p[argmax] (float32 log, then fp16, as numpy's fp16 log);
//      sampling: the k largest p by (p descending, index ascending): the
//      k-th largest fp16 key found bit by bit from workgroup counts, ties at
//      it taken in index order (thread t re-reads elements 32t..32t+31 from
//      LDS, and a scan of the threads' tie counts ranks them); wave 0 orders the k
//      entries, sums them in numpy's order (8 accumulators), normalises in
//      f32, forms the f64 cumulative sum over its last entry and takes the
//      first entry above the row's uniform draw; log of the full-softmax p of
//      that token.
// A row whose maximum is NaN or infinite (where the reference's table index
// is undefined) gets the argmax rule's token (first NaN, else first maximum
// of the raw logits) and a NaN log-probability, and NaN probabilities.
#include <math.h>
#include <stdint.h>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace moat {
namespace {

constexpr int kSThreads = 1024;
constexpr int kSWaves = kSThreads / 64;
constexpr int kSMaxV = 32768;
constexpr int kSPer = kSMaxV / kSThreads;  // elements per thread: t + 1024 j
constexpr int kSMaxLut = 32768;
constexpr int kSChunk = 8192;  // numpy's reduction buffer (np.getbufsize() default)
constexpr int kSMaxChunks = kSMaxV / kSChunk;
constexpr int kSSlots = 128;          // leaves per chunk: at most 64 nodes one level up, two children each
constexpr int kSNodes = kSSlots / 2;  // one wave per chunk holds those nodes
constexpr int kSMaxK = 64;
constexpr int kNone = 0x7FFFFFFF;
// The row's LDS copy skips 8 entries (16 bytes) after every 128 so that the
// sum's chains, which read leaves about 128 entries apart, fall on different
// banks.
constexpr int kSERow = kSMaxV + (kSMaxV >> 7) * 8;
__device__ __forceinline__ int epos(int i) { return i + ((i >> 7) << 3); }

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

enum SampleMode { kModeProbs = 0, kModeGreedy = 1, kModeSample = 2 };

struct SampleShared {
  uint16_t lut[kSMaxLut];
  uint16_t e[kSERow];  // table value of each element, then its probability (fp16 bits), at epos(i)
  float chain[kSMaxChunks][kSSlots][8];
  float chunk_sum[kSMaxChunks];
  float wave_f[kSWaves];
  int wave_i[2][kSWaves];
  double wave_d[kSWaves];
  int wc[kSWaves][kSMaxK];  // each wave's k first entries (indices) in the selection order
  uint32_t wcount[kSWaves];
  int cand[kSMaxK];
};

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// value as float32 (logits are converted as numpy's astype(float32): RNE)
__device__ __forceinline__ float conv(float r) { return r; }
__device__ __forceinline__ float conv(double r) { return (float)r; }
__device__ __forceinline__ float conv(uint16_t r) { return h2f(r); }
// logits / T in the logits' dtype (T already rounded to it), then as float32
__device__ __forceinline__ float scale_conv(float r, double t) { return __fdiv_rn(r, (float)t); }
__device__ __forceinline__ float scale_conv(double r, double t) { return (float)__ddiv_rn(r, t); }
__device__ __forceinline__ float scale_conv(uint16_t r, double t) { return h2f(f2h(__fdiv_rn(h2f(r), (float)t))); }
// a / b rounded to nearest even from r = RN(1 / b), b > 0, by Markstein's FMA
// sequence: q0 = RN(a r), rem = a - q0 b (exact), q = RN(q0 + rem r).  It is
// the correctly rounded quotient when a and q0 are 0 or in [2^-100, 2^100]
// (tests/test_markstein_division.py checks it against IEEE division over a
// whole binade of dividends for the table step, sums, hard and random
// divisor significands); it can miss by an ulp when the quotient is
// subnormal and gives NaN when it overflows.  `fast` says whether a and q0 are in the range.  Used where
// neither case changes the result: the table index (a quotient below 1 is
// index 0, one above 2^100 the last index) and e / sum (always in range).
__device__ __forceinline__ float div_markstein(float a, float b, float r, bool& fast) {
  asm volatile("" : "+v"(a));  // a converted on its own (no mixed-precision fma)
  const float q0 = a * r;
  const float rem = __builtin_fmaf(-q0, b, a);
  const float aa = fabsf(a), aq = fabsf(q0);
  fast = aa == 0.f || (aa >= 0x1p-100f && aa <= 0x1p100f && aq >= 0x1p-100f && aq <= 0x1p100f);
  float q = __builtin_fmaf(rem, r, q0);
  // the float32 quotient as such: fused with a following fp16 conversion
  // (v_fma_mixlo_f16) it would be rounded once, to fp16, instead of twice
  asm volatile("" : "+v"(q));
  return q;
}
// raw value for an argmax (exact in double for every input dtype)
__device__ __forceinline__ double raw_d(float r) { return (double)r; }
__device__ __forceinline__ double raw_d(double r) { return r; }
__device__ __forceinline__ double raw_d(uint16_t r) { return (double)h2f(r); }

__device__ __forceinline__ float rl(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ __forceinline__ int rl(int x, int l) { return __builtin_amdgcn_readlane(x, l); }
__device__ __forceinline__ double rl(double x, int l) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(x);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Wave sum by DPP (quad permutes, row shifts, row broadcasts); the total
// lands in lane 63.
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ float wave_max(float v) {  // NaN-propagating
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    v = (isnan(v) || isnan(w)) ? NAN : fmaxf(v, w);
  }
  return v;
}

__device__ __forceinline__ int wave_min(int v) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

// Workgroup minimum of one int per thread (one barrier; slot `b` of the
// per-wave array alternates between consecutive uses).
__device__ __forceinline__ int block_min(SampleShared& S, int v, int b) {
  v = wave_min(v);
  if ((threadIdx.x & 63) == 0) S.wave_i[b][threadIdx.x >> 6] = v;
  __syncthreads();
  int m = S.wave_i[b][0];
#pragma unroll
  for (int w = 1; w < kSWaves; ++w) m = min(m, S.wave_i[b][w]);
  return m;
}

// Exclusive prefix sum over the wave's lanes; `total` gets the wave's sum.
__device__ __forceinline__ uint32_t wave_prefix(uint32_t v, uint32_t& total) {
  const int lane = threadIdx.x & 63;
  uint32_t inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = __shfl_up(inc, o, 64);
    inc += lane >= o ? u : 0u;
  }
  total = (uint32_t)rl((int)inc, 63);
  return inc - v;
}

// Wave count of encoded keys >= c (c in 1..0x7FFF): key - c in 16 bits has
// its top bit set exactly when key < c.
template <int kN>
__device__ __forceinline__ uint32_t wave_count_ge(const us2 (&ek)[kN / 2], uint32_t c) {
  const us2 cc = {(unsigned short)c, (unsigned short)c};
  us2 lt = {0, 0};
#pragma unroll
  for (int h = 0; h < kN / 2; ++h) lt += (us2)((ek[h] - cc) >> (us2){15, 15});
  return wave_sum((uint32_t)kN - lt.x - lt.y);
}

// The wave's first kk entries in the order (key descending, position
// ascending), position = kN * lane + slot: returns this lane's slots taken.
// Encoded keys are the fp16 key + 1, 0 for no entry; with fewer than kk
// entries the wave takes all of them.
template <int kN>
__device__ __forceinline__ uint32_t wave_select(const us2 (&ek)[kN / 2], uint32_t kk) {
  uint32_t thr = 0;  // the kk-th largest encoded key
  for (int bit = 14; bit >= 0; --bit) {
    const uint32_t c = thr | (1u << bit);
    if (wave_count_ge<kN>(ek, c) >= kk) thr = c;
  }
  uint32_t above = 0, ties = 0;
#pragma unroll
  for (int h = 0; h < kN / 2; ++h) {
    above |= (ek[h].x > thr ? 1u : 0u) << (2 * h);
    above |= (ek[h].y > thr ? 1u : 0u) << (2 * h + 1);
    ties |= (ek[h].x == thr ? 1u : 0u) << (2 * h);
    ties |= (ek[h].y == thr ? 1u : 0u) << (2 * h + 1);
  }
  const uint32_t n_above = wave_sum((uint32_t)__popc(above));
  const uint32_t need = thr ? kk - n_above : 0u;  // ties at thr, lowest positions first
  uint32_t n_ties;
  const uint32_t pre = wave_prefix((uint32_t)__popc(ties), n_ties);
  uint32_t take = above;
  if (pre < need) {
    uint32_t left = min((uint32_t)__popc(ties), need - pre), x = ties;
    while (left--) {
      const uint32_t lowest = x & (0u - x);
      take |= lowest;
      x ^= lowest;
    }
  }
  return take;
}

// The row's draw in [0, 1): 53 bits of SplitMix64's output mix of
// seed + (row + 1) * 0x9E3779B97F4A7C15.
__device__ __forceinline__ double row_uniform(uint64_t seed, int row) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(row + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (double)(z >> 11) * 0x1.0p-53;
}

// Depth below a chunk's root at which every node is a leaf of at most 128
// elements (q blocks of 8 plus an r-element tail on the rightmost node; the
// rightmost node at depth d has ceil(q / 2^d) blocks, the largest).
__device__ __forceinline__ int leaf_depth(int q, int r) {
  if (8 * q + r <= 128) return 0;
  int d = 1;
  while (8 * ((q + (1 << d) - 1) >> d) + r > 128) ++d;
  return d;
}

// Node i at depth d: numpy's split puts floor(n/2) blocks on the left.
__device__ __forceinline__ void walk(int i, int d, int q, int& a0, int& sz) {
  a0 = 0;
  sz = q;
  for (int l = d - 1; l >= 0; --l) {
    const int h = sz >> 1;
    const bool right = (i >> l) & 1;
    a0 += right ? h : 0;
    sz = right ? sz - h : h;
  }
}

__device__ __forceinline__ float leaf_value(const SampleShared& S, int c, int slot, int tail_from, int tail) {
  const float* r = S.chain[c][slot];
  float v = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
  for (int k = 0; k < 7; ++k) {
    const float x = h2f(S.e[epos(min(tail_from + k, kSMaxV - 1))]);
    v = k < tail ? v + x : v;
  }
  return v;
}

// numpy's float32 sum of the row's e values (S.e[0..v)); every thread gets it.
__device__ float row_sum(SampleShared& S, int v) {
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int nchunks = (v + kSChunk - 1) / kSChunk;
  // chains: thread t is accumulator j = t % 8 of leaf slot t / 8, in every chunk
  const int slot = t >> 3, j = t & 7, i = slot >> 1, ch = slot & 1;
  for (int c = 0; c < nchunks; ++c) {
    const int base = c * kSChunk, nc = min(kSChunk, v - base), q = nc >> 3, r = nc & 7;
    if (nc == kSChunk) {
      // a whole chunk: 64 leaves of 16 blocks (32 nodes of 32 blocks, halved)
      if (slot < 64) {
        const uint16_t* ep = S.e + epos(base + 128 * slot) + j;
        float acc = h2f(ep[0]);
#pragma unroll
        for (int k = 1; k < 16; ++k) acc = acc + h2f(ep[8 * k]);
        S.chain[c][slot][j] = acc;
      }
      continue;
    }
    if (nc < 8) continue;
    const int d = leaf_depth(q, r);
    const int p = d ? 1 << (d - 1) : 1;
    int a0, sz;
    walk(i, d ? d - 1 : 0, q, a0, sz);
    const bool leaf = d == 0 || 8 * sz + (i == p - 1 ? r : 0) <= 128;
    const int h = sz >> 1;
    const int b0 = (leaf || !ch) ? a0 : a0 + h;
    const int b1 = leaf ? a0 + sz : (ch ? a0 + sz : a0 + h);
    const int from = base + j;
    float acc = h2f(S.e[epos(min(from + 8 * b0, kSMaxV - 1))]);
#pragma unroll
    for (int k = 1; k < 16; ++k) {
      const float x = h2f(S.e[epos(min(from + 8 * (b0 + k), kSMaxV - 1))]);
      acc = b0 + k < b1 ? acc + x : acc;
    }
    S.chain[c][slot][j] = acc;  // slots past the chunk's leaves are never read
  }
  __syncthreads();
  // nodes one level above the leaves: wave c, lane i; then the levels above
  if (wv < nchunks) {
    const int c = wv;
    const int base = c * kSChunk, nc = min(kSChunk, v - base), q = nc >> 3, r = nc & 7;
    float nv = 0.f;
    int p = 1;
    if (nc < 8) {
#pragma unroll
      for (int k = 0; k < 7; ++k) {
        const float x = h2f(S.e[epos(min(base + k, kSMaxV - 1))]);
        nv = (lane == 0 && k < nc) ? nv + x : nv;
      }
    } else {
      const int d = leaf_depth(q, r);
      p = d ? 1 << (d - 1) : 1;
      int a0, sz;
      walk(lane, d ? d - 1 : 0, q, a0, sz);
      const bool last = lane == p - 1;
      const int tail = last ? r : 0;
      const int tail_from = base + 8 * q;
      const bool leaf = d == 0 || 8 * sz + tail <= 128;
      const int ls = min(2 * lane, kSSlots - 2);
      const float left = leaf_value(S, c, ls, tail_from, leaf ? tail : 0);
      const float right = leaf_value(S, c, ls + 1, tail_from, tail);
      nv = leaf ? left : left + right;
      nv = lane < p ? nv : 0.f;
    }
    for (int m = p; m > 1; m >>= 1) {
      const float a = __shfl(nv, 2 * lane, 64);
      const float b = __shfl(nv, 2 * lane + 1, 64);
      nv = a + b;
    }
    if (lane == 0) S.chunk_sum[c] = nv;
  }
  __syncthreads();
  float s = 0.f;
  for (int c = 0; c < nchunks; ++c) s = s + S.chunk_sum[c];
  return s > 0.f ? s : 1.f;
}

// Token for a row whose maximum is not finite: np.argmax of the raw logits
// (first NaN, else first maximum).  Rare; re-reads the row.
template <typename T>
__device__ int raw_argmax(SampleShared& S, const T* xr, int v) {
  int first_nan = kNone;
  double best = -INFINITY;
  for (int i = threadIdx.x; i < v; i += kSThreads) {
    const double r = raw_d(xr[i]);
    if (isnan(r)) first_nan = min(first_nan, i);
    else best = fmax(best, r);
  }
  for (int o = 32; o > 0; o >>= 1) best = fmax(best, __shfl_xor(best, o, 64));
  if ((threadIdx.x & 63) == 0) S.wave_d[threadIdx.x >> 6] = best;
  const int fn = block_min(S, first_nan, 0);
  if (fn != kNone) return fn;
  double m = S.wave_d[0];
  for (int w = 1; w < kSWaves; ++w) m = fmax(m, S.wave_d[w]);
  int first = kNone;
  for (int i = threadIdx.x; i < v; i += kSThreads)
    if (raw_d(xr[i]) == m) first = min(first, i);
  return block_min(S, first, 1);
}

template <typename T, bool kScaled>
__global__ void __launch_bounds__(kSThreads) lut_sample_kernel(const T* __restrict__ x, int v, double temp,
                                                               const uint16_t* __restrict__ lut, int lut_size,
                                                               float step, int mode, int top_k, uint64_t seed,
                                                               int32_t* __restrict__ tokens,
                                                               float* __restrict__ logprobs,
                                                               uint16_t* __restrict__ probs) {
  __shared__ SampleShared S;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int row = blockIdx.x;
  const T* xr = x + (int64_t)row * v;

  // 1. every load issued before any use: the row (indices past its end read
  // its last element, unused) and the table
  T raw[kSPer];
#pragma unroll
  for (int j = 0; j < kSPer; ++j) raw[j] = xr[min(t + j * kSThreads, v - 1)];
  for (int i = t; i < lut_size; i += kSThreads) S.lut[i] = lut[i];

  // scaled values as float32, -inf past the row's end (x / T divides in full:
  // arbitrary logits can put the quotient where Markstein's sequence is not
  // exact)
  float xs[kSPer];
#pragma unroll
  for (int j = 0; j < kSPer; ++j) xs[j] = kScaled ? scale_conv(raw[j], temp) : conv(raw[j]);
  float mx = -INFINITY;
  bool nan_seen = false;
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const bool ok = t + j * kSThreads < v;
    nan_seen = nan_seen || (ok && isnan(xs[j]));
    xs[j] = ok ? xs[j] : -INFINITY;
    mx = fmaxf(mx, xs[j]);
  }
  const float wm = wave_max(nan_seen ? NAN : mx);
  if (lane == 0) S.wave_f[wv] = wm;
  if (t < kSMaxK) S.cand[t] = 0;
  __syncthreads();
  float m = S.wave_f[0];
#pragma unroll
  for (int w = 1; w < kSWaves; ++w) {
    const float o = S.wave_f[w];
    m = (isnan(m) || isnan(o)) ? NAN : fmaxf(m, o);
  }

  if (!isfinite(m)) {
    if (probs)
      for (int i = t; i < v; i += kSThreads) probs[(int64_t)row * v + i] = 0x7E00;
    if (mode != kModeProbs) {
      const int tok = raw_argmax(S, xr, v);
      if (t == 0) {
        tokens[row] = tok;
        logprobs[row] = NAN;
      }
    }
    return;
  }

  // greedy: the first index of the raw maximum (the values are the raw ones
  // converted; for f64, candidates equal in float32 are compared in float64)
  int tok = 0;
  if (!kScaled && mode == kModeGreedy) {
    int first = kNone;
    double bd = -INFINITY;
#pragma unroll
    for (int j = 0; j < kSPer; ++j) {
      const int i = t + j * kSThreads;
      const bool cnd = xs[j] == m;
      if (sizeof(T) == 8) {
        const double r = raw_d(raw[j]);
        const bool better = cnd && (first == kNone || r > bd);
        bd = better ? r : bd;
        first = better ? i : first;
      } else {
        first = (cnd && first == kNone) ? i : first;
      }
    }
    if (sizeof(T) == 8) {
      // the largest double with its first index, over the workgroup
      for (int o = 32; o > 0; o >>= 1) {
        const double ob = __shfl_xor(bd, o, 64);
        const int oi = __shfl_xor(first, o, 64);
        const bool take = oi != kNone && (first == kNone || ob > bd || (ob == bd && oi < first));
        bd = take ? ob : bd;
        first = take ? oi : first;
      }
      if (lane == 0) {
        S.wave_d[wv] = bd;
        S.wave_i[1][wv] = first;
      }
      __syncthreads();
      double bb = S.wave_d[0];
      int bi = S.wave_i[1][0];
      for (int w = 1; w < kSWaves; ++w) {
        const double ob = S.wave_d[w];
        const int oi = S.wave_i[1][w];
        const bool take = oi != kNone && (bi == kNone || ob > bb || (ob == bb && oi < bi));
        bb = take ? ob : bb;
        bi = take ? oi : bi;
      }
      tok = bi;
    } else {
      tok = block_min(S, first, 1);
    }
  }

  // 2. table values (every lookup issued before the stores); element
  // t + 1024 j sits at epos(t) + 1088 j
  const float top = (float)(lut_size - 1);
  uint16_t* const my_e = S.e + epos(t);
  {
    // |x - max| / step by Markstein's sequence: outside its range the
    // quotient is either below 1 (index 0 either way) or far above the last
    // index (NaN or huge here, clamped to it)
    const float rs = __fdiv_rn(1.0f, step);
    uint16_t tv[kSPer];
#pragma unroll
    for (int j = 0; j < kSPer; ++j) {
      bool fast;
      const float a = div_markstein(fabsf(xs[j] - m), step, rs, fast);
      tv[j] = S.lut[lut_size - 1 - (int)(a == a ? fminf(a, top) : top)];
    }
#pragma unroll
    for (int j = 0; j < kSPer; ++j) my_e[1088 * j] = tv[j];
  }
  __syncthreads();

  // 3. numpy-order sum
  const float sum = row_sum(S, v);

  if (mode == kModeGreedy) {
    if (t == 0) {
      // the maximum's table value is the table's last entry (|x - max| = 0)
      const float p = h2f(f2h(__fdiv_rn(h2f(S.lut[lut_size - 1]), sum)));
      tokens[row] = tok;
      logprobs[row] = h2f(f2h((float)log((double)p)));  // f32 log, then fp16 (numpy's fp16 log)
    }
    return;
  }

  // 4. probabilities (each thread rewrites its own slots); e / sum by
  // Markstein's sequence, always in its range (e is 0 or at least 2^-24 and
  // at most 1; 1 <= sum <= 32768, the maximum's table value being 1)
  const float rsum = __fdiv_rn(1.0f, sum);
  bool fast;
  if (mode == kModeProbs) {
#pragma unroll
    for (int j = 0; j < kSPer; ++j) {
      const int i = t + j * kSThreads;
      if (i < v) probs[(int64_t)row * v + i] = f2h(div_markstein(h2f(my_e[1088 * j]), sum, rsum, fast));
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < kSPer; ++j) my_e[1088 * j] = f2h(div_markstein(h2f(my_e[1088 * j]), sum, rsum, fast));

  // 5. the k largest p, index order among equal p: each wave takes the first
  // k entries of its own 2048 (thread t re-reads elements 32t .. 32t+31 of
  // the row from LDS, so that a wave's entries are in index order); the k
  // first of the whole row are among those 16 lists, which wave 0 selects
  // from.  Keys are encoded as the fp16 bits + 1 (0: past the row's end);
  // list entries are key << 16 | index.
  __syncthreads();
  const uint32_t kk = (uint32_t)min(top_k, v);
  {
    us2 ek[kSPer / 2];
#pragma unroll
    for (int q4 = 0; q4 < kSPer / 8; ++q4) {
      const uint4 w = *reinterpret_cast<const uint4*>(S.e + epos(kSPer * t) + 8 * q4);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int i0 = kSPer * t + 8 * q4 + 2 * h;
        ek[4 * q4 + h].x = i0 < v ? (unsigned short)((ws[h] & 0xFFFF) + 1) : (unsigned short)0;
        ek[4 * q4 + h].y = i0 + 1 < v ? (unsigned short)((ws[h] >> 16) + 1) : (unsigned short)0;
      }
    }
    // lower bound of the wave's k-th largest key: the k-th largest of the 64
    // lane maxima (k lanes each hold a key at least that large), by ballots
    us2 m2 = ek[0];
#pragma unroll
    for (int h = 1; h < kSPer / 2; ++h) m2 = __builtin_elementwise_max(m2, ek[h]);
    const uint32_t lmax = max((uint32_t)m2.x, (uint32_t)m2.y);
    uint32_t lb = 0;
    for (int bit = 14; bit >= 0; --bit) {
      const uint32_t c = lb | (1u << bit);
      if ((uint32_t)__popcll(__ballot(lmax >= c)) >= kk) lb = c;
    }
    lb = max(lb, 1u);
    uint32_t cm = 0;  // this lane's candidates: keys >= lb
#pragma unroll
    for (int h = 0; h < kSPer / 2; ++h) {
      cm |= (ek[h].x >= lb ? 1u : 0u) << (2 * h);
      cm |= (ek[h].y >= lb ? 1u : 0u) << (2 * h + 1);
    }
    uint32_t n_cand;
    uint32_t at = wave_prefix((uint32_t)__popc(cm), n_cand);
    uint32_t take;
    uint32_t pos[4];
    if (n_cand <= 256) {
      // compact the candidates (in index order) into this wave's 256-entry
      // list (the sum's chain area, free now), then select exactly among them
      uint32_t* list = reinterpret_cast<uint32_t*>(&S.chain[0][0][0]) + 256 * wv;
      for (uint32_t mm = cm; mm;) {
        const int jj = __ffs(mm) - 1;
        mm &= mm - 1;
        const int i = kSPer * t + jj;
        list[at++] = ((uint32_t)S.e[epos(i)] + 1u) << 16 | (uint32_t)i;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      us2 ck[2];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t e = 4 * lane + h;
        const uint32_t val = e < n_cand ? list[e] : 0u;
        pos[h] = val;
        if (h & 1) ck[h >> 1].y = (unsigned short)(val >> 16);
        else ck[h >> 1].x = (unsigned short)(val >> 16);
      }
      take = wave_select<4>(ck, kk);
    } else {
      // many equal keys near the top (e.g. a flat row): search all 32 per lane
      take = wave_select<kSPer>(ek, kk);
    }
    uint32_t total;
    at = wave_prefix((uint32_t)__popc(take), total);
    if (n_cand <= 256) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
        if ((take >> h) & 1u) S.wc[wv][at++] = (int)pos[h];
    } else {
      while (take) {  // few lanes hold any of the wave's k entries
        const int jj = __ffs(take) - 1;
        take &= take - 1;
        const int i = kSPer * t + jj;
        S.wc[wv][at++] = (int)(((uint32_t)S.e[epos(i)] + 1u) << 16 | (uint32_t)i);
      }
    }
    if (lane == 0) S.wcount[wv] = total;
  }
  __syncthreads();
  if (wv != 0) return;
  {
    // wave 0: the 16 lists, 16 entries per lane, in index order
    us2 ek[8];
    int ent[16];
    const uint32_t cnt = S.wcount[lane >> 2];  // a lane's 16 entries lie in list lane / 4
#pragma unroll
    for (int h = 0; h < 16; ++h) {
      const int p = (16 * lane + h) & 63;
      ent[h] = (uint32_t)p < cnt ? S.wc[lane >> 2][p] : 0;
      const unsigned short k = (unsigned short)((uint32_t)ent[h] >> 16);
      if (h & 1) ek[h >> 1].y = k;
      else ek[h >> 1].x = k;
    }
    const uint32_t take = wave_select<16>(ek, kk);
    uint32_t total;
    uint32_t at = wave_prefix((uint32_t)__popc(take), total);
#pragma unroll
    for (int h = 0; h < 16; ++h)
      if ((take >> h) & 1) S.cand[at++] = ent[h];
    // the wave's LDS writes before its reads of them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }

  // 6. wave 0: order the k entries (p descending, index ascending), lane r
  // takes rank r; their sum in numpy's order; the draw
  const int kc = (int)kk;
  const bool live = lane < kc;
  const uint32_t ce = live ? (uint32_t)S.cand[lane] : 0u;
  const int mi = (int)(ce & 0xFFFFu);
  const int mk = live ? (int)(ce >> 16) - 1 : -1;  // the fp16 bits of p
  int rank = 0;
  for (int o = 0; o < kc; ++o) {
    const int ok = rl(mk, o), oi = rl(mi, o);
    rank += (ok > mk || (ok == mk && oi < mi)) ? 1 : 0;
  }
  const int dst = 4 * (live ? rank : lane);
  const int sidx = __builtin_amdgcn_ds_permute(dst, mi);
  const int skey = __builtin_amdgcn_ds_permute(dst, mk);
  const float pk = live ? h2f((uint16_t)skey) : 0.f;
  float s;
  if (kc < 8) {
    s = 0.f;
    for (int o = 0; o < kc; ++o) s = s + rl(pk, o);
  } else {
    const int full = kc - kc % 8;
    float acc = pk;  // lane j < 8: accumulator j, starting at entry j
    for (int bb = 8; bb < full; bb += 8) acc = acc + __shfl(pk, bb + (lane & 7), 64);
    s = ((rl(acc, 0) + rl(acc, 1)) + (rl(acc, 2) + rl(acc, 3))) + ((rl(acc, 4) + rl(acc, 5)) + (rl(acc, 6) + rl(acc, 7)));
    for (int o = full; o < kc; ++o) s = s + rl(pk, o);
  }
  // cumulative distribution in f64, in order (lane r: entries 0..r), over its last entry
  const double pn = live ? (s > 0.f ? (double)__fdiv_rn(pk, s) : 1.0 / (double)kc) : 0.0;
  double c = 0.0;
  for (int o = 0; o < kc; ++o) {
    const double xo = rl(pn, o);
    c = o <= lane ? c + xo : c;
  }
  const double total = rl(c, kc - 1);
  const double u = row_uniform(seed, row);
  const unsigned long long hit = __ballot(live && __ddiv_rn(c, total) > u);
  const int pick = hit ? __ffsll((long long)hit) - 1 : kc - 1;
  const int tk = rl(sidx, pick);
  const float pc = rl(pk, pick);
  if (lane == 0) {
    tokens[row] = tk;
    logprobs[row] = pc >= 1e-10f ? (float)log((double)pc) : (float)-23.025850929940457;  // log(1e-10)
  }
}

__global__ void lut_lookup_kernel(const float* __restrict__ x, int64_t n, const uint16_t* __restrict__ lut,
                                  int lut_size, float step, uint16_t* __restrict__ out) {
  const float top = (float)(lut_size - 1);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float a = __fdiv_rn(fabsf(x[i]), step);
    // NaN: numpy's index is undefined; give NaN
    out[i] = isnan(a) ? (uint16_t)0x7E00 : lut[lut_size - 1 - (int)fminf(a, top)];
  }
}

template <typename T>
hipError_t launch_typed(const void* x, int n, int v, double temp, int scaled, const uint16_t* lut, int lut_size,
                        float step, int mode, int top_k, uint64_t seed, int32_t* tokens, float* logprobs,
                        uint16_t* probs, hipStream_t st) {
  const dim3 grid(n), block(kSThreads);
  if (scaled)
    hipLaunchKernelGGL((lut_sample_kernel<T, true>), grid, block, 0, st, static_cast<const T*>(x), v, temp, lut,
                       lut_size, step, mode, top_k, seed, tokens, logprobs, probs);
  else
    hipLaunchKernelGGL((lut_sample_kernel<T, false>), grid, block, 0, st, static_cast<const T*>(x), v, temp, lut,
                       lut_size, step, mode, top_k, seed, tokens, logprobs, probs);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_lut_sample(const void* x, int dtype, int n, int v, double temp, int scaled, const uint16_t* lut,
                             int lut_size, float step, int mode, int top_k, uint64_t seed, int32_t* tokens,
                             float* logprobs, uint16_t* probs, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  switch (dtype) {
    case 0:
      return launch_typed<float>(x, n, v, temp, scaled, lut, lut_size, step, mode, top_k, seed, tokens, logprobs,
                                 probs, st);
    case 1:
      return launch_typed<uint16_t>(x, n, v, temp, scaled, lut, lut_size, step, mode, top_k, seed, tokens,
                                    logprobs, probs, st);
    default:
      return launch_typed<double>(x, n, v, temp, scaled, lut, lut_size, step, mode, top_k, seed, tokens,
                                  logprobs, probs, st);
  }
}

hipError_t launch_lut_lookup(const float* x, int64_t n, const uint16_t* lut, int lut_size, float step, uint16_t* out,
                             hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  const int grid = (int)(blocks < 4096 ? blocks : 4096);
  hipLaunchKernelGGL(lut_lookup_kernel, dim3(grid), dim3(256), 0, st, x, n, lut, lut_size, step, out);
  return hipGetLastError();
}

}  // namespace moat
