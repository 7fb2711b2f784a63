// Batched token sampling over LM-head logits: the table ("LUT") softmax of the
// reference's numpy sampler, then greedy argmax or a draw from the k most
// probable tokens (antigravity-engine/src/batch_generator.py:187-253,
// antigravity-engine/src/attention.py:60-135).
//
// A row is cut into chunks of 8192 logits -- the pieces numpy's float32 sum
// runs over -- and each chunk is a 1024-thread workgroup (logits t + 1024 j,
// j < 8, of the chunk in thread t), so a row spreads over ceil(V / 8192) CUs;
// V is bounded by the row merge (64 chunks: V <= 524288).  Launches, passing
// results through the caller's workspace (a row of one 8192-logit chunk
// skips K1; greedy skips K3):
//   K1 chunk_stats   (rows of more than one chunk) per chunk: the raw maximum
//                    (in double, NaN skipped) with its first index, and the
//                    first NaN;
//   K2 chunk_sum     per chunk: the row's maximum from K1 (a row of one
//                    chunk: its own, with K1's statistics); x / T in the
//                    logits' dtype (fp16: f32 division rounded to fp16), as float32
//                    (x / T is monotone, so the scaled maximum is the
//                    maximum's quotient); table index
//                    size-1-trunc(min(|x - max| / step, size-1)) -> e (fp16);
//                    the chunk's sum of e in numpy's pairwise order (halves
//                    split at multiples of 8 down to blocks of at most 128,
//                    each summed with 8 strided accumulators, then its tail:
//                    8 chains per leaf, one lane per node one level above the
//                    leaves, DPP for the levels above).  Greedy: the row's
//                    last workgroup to finish writes np.argmax's token (from
//                    the chunk statistics) and the fp16 log of its p;
//   K3 chunk_select  per chunk: the row's sum (the chunk sums added in order
//                    from 0, as numpy adds its pieces), p = fp16(e / sum);
//                    the softmax output, or the chunk's first k entries in
//                    the order (p descending, index ascending).  The row's
//                    last workgroup to finish draws: the row's first k from
//                    the chunk lists, their sum in numpy's order (8
//                    accumulators), normalised in f32, the f64 cumulative
//                    distribution over its last entry, the first entry above
//                    the row's uniform draw, and the float32 log of its
//                    full-softmax p.
// "Last to finish" is a per-row counter in the workspace (K1 zeroes it; the
// row's last workgroup leaves it at zero too): the writer wave
// publishes its results with sc1 stores (written through the per-XCD L2s to
// the coherence point) and waits for them to complete before a relaxed
// agent-scope increment; the workgroup that brings the counter to the chunk
// count reads every chunk's results with sc1 loads (past the L2s) and puts
// the counter back to zero.  (Agent-scope fences would write back and
// invalidate whole L2s instead.)  The k-entry selections run per wave, bit
// by bit on 16-bit keys (the fp16 bits of p, plus 1) with packed compares and
// DPP wave sums, ties in index order; wave 0 merges the 16 wave lists.
// Per-element work is branch-free: a CU's 16 waves share one scalar unit, and
// per-element branches (exec-mask updates) make it the bottleneck.  A row whose maximum
// is NaN or infinite (where the reference's table index is undefined) gets
// np.argmax's token (first NaN, else first maximum of the raw logits), a NaN
// log-probability and NaN probabilities.
#include <math.h>
#include <stdint.h>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace moat {
namespace {

constexpr int kT = 1024;        // threads per workgroup
constexpr int kW = kT / 64;     // waves
constexpr int kCh = 8192;       // numpy's reduction buffer (np.getbufsize() default)
constexpr int kPer = kCh / kT;  // logits of a chunk per thread: t + 1024 j
constexpr int kMaxChunks = 64;  // the row merge holds 64 chunk lists (4 entries per thread)
constexpr int kSlots = 128;     // leaves per chunk: at most 64 nodes one level up, two children each
constexpr int kMaxK = 64;
constexpr int kNone = 0x7FFFFFFF;
// The chunk's LDS copy skips 8 entries (16 bytes) after every 128 so that the
// sum's chains, which read leaves about 128 entries apart, fall on different
// banks.
constexpr int kERow = kCh + (kCh >> 7) * 8;
__device__ __forceinline__ int epos(int i) { return i + ((i >> 7) << 3); }

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

enum SampleMode { kModeProbs = 0, kModeGreedy = 1, kModeSample = 2 };

// Workspace of one call; per row r and chunk c at r * nch + c.
struct SampleWs {
  uint32_t* cnt;    // [n] workgroups of the row done (zeroed by K1)
  double* cmax;     // chunk maximum of the raw logits (NaN skipped; -inf if none)
  int* cnan;        // first NaN index in the chunk, or kNone
  int* cfirst;      // first index of the chunk maximum, or kNone
  float* csum;      // numpy-order sum of the chunk's table values
  uint32_t* ccnt;   // entries in the chunk list
  uint64_t* clist;  // [.][64] (fp16 key + 1) << 32 | index, in index order
  int* rowbad;      // [n] the row's maximum (after T) is not finite
  uint16_t* e;      // [n][v] table values (softmax: the output, rewritten as p)
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
// raw value as double (exact for every input dtype), and back
__device__ __forceinline__ double raw_d(float r) { return (double)r; }
__device__ __forceinline__ double raw_d(double r) { return r; }
__device__ __forceinline__ double raw_d(uint16_t r) { return (double)h2f(r); }
template <typename T>
__device__ __forceinline__ T from_d(double d);
template <>
__device__ __forceinline__ float from_d<float>(double d) { return (float)d; }
template <>
__device__ __forceinline__ double from_d<double>(double d) { return d; }
template <>
__device__ __forceinline__ uint16_t from_d<uint16_t>(double d) { return f2h((float)d); }

// a / b rounded to nearest even from r = RN(1 / b), b > 0, by Markstein's FMA
// sequence: q0 = RN(a r), rem = a - q0 b (exact), q = RN(q0 + rem r).  It is
// the correctly rounded quotient when a and q0 are 0 or in [2^-100, 2^100]
// (tests/test_markstein_division.py checks it against IEEE division over a
// whole binade of dividends for the table step, sums, hard and random
// divisor significands); it can miss by an ulp when the quotient is
// subnormal and gives NaN when it overflows.  Used where neither case
// changes the result: the table index (a quotient below 1 is index 0, one
// above 2^100 the last index) and e / sum (always in range).
__device__ __forceinline__ float div_markstein(float a, float b, float r) {
  asm volatile("" : "+v"(a));  // a converted on its own (no mixed-precision fma)
  const float q0 = a * r;
  const float rem = __builtin_fmaf(-q0, b, a);
  float q = __builtin_fmaf(rem, r, q0);
  // the float32 quotient as such: fused with a following fp16 conversion
  // (v_fma_mixlo_f16) it would be rounded once, to fp16, instead of twice
  asm volatile("" : "+v"(q));
  return q;
}

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

// Results handed to the row's last workgroup within a launch: sc1 stores and
// loads (relaxed agent-scope atomics).
template <typename V>
__device__ __forceinline__ void publish(V* p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ V fetch(const V* p) {
  return __hip_atomic_load(const_cast<V*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// v from another lane by DPP (`kCtrl`), or `old` where the source lane is
// out of its row or the row is masked off (`kRows`).
template <int kCtrl, int kRows>
__device__ __forceinline__ int dpp(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, kCtrl, kRows, 0xF, false);
}
template <int kCtrl, int kRows>
__device__ __forceinline__ double dpp_d(double old, double v) {
  const long long b = __double_as_longlong(v), o = __double_as_longlong(old);
  const int lo = dpp<kCtrl, kRows>((int)o, (int)b);
  const int hi = dpp<kCtrl, kRows>((int)(o >> 32), (int)(b >> 32));
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
template <int kCtrl, int kRows>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(dpp<kCtrl, kRows>(__float_as_int(old), __float_as_int(v)));
}

// Full-wave reductions by DPP: quad permutes [1,0,3,2] and [2,3,0,1], row
// shifts right by 4 and 8, broadcasts of lane 15 to rows 1 and 3 and of lane
// 31 to rows 2 and 3; the result lands in lane 63 and is read from there.
#define MOAT_WAVE_REDUCE(v, id, op, dp) \
  v = op(v, dp<0xB1, 0xF>(id, v));      \
  v = op(v, dp<0x4E, 0xF>(id, v));      \
  v = op(v, dp<0x114, 0xF>(id, v));     \
  v = op(v, dp<0x118, 0xF>(id, v));     \
  v = op(v, dp<0x142, 0xA>(id, v));     \
  v = op(v, dp<0x143, 0xC>(id, v))

__device__ __forceinline__ int add_i(int a, int b) { return a + b; }
__device__ __forceinline__ int min_i(int a, int b) { return min(a, b); }
__device__ __forceinline__ double max_d(double a, double b) { return fmax(a, b); }

__device__ __forceinline__ uint32_t wave_sum(uint32_t u) {
  int v = (int)u;
  MOAT_WAVE_REDUCE(v, 0, add_i, dpp);
  return (uint32_t)rl(v, 63);
}
__device__ __forceinline__ int wave_min(int v) {
  MOAT_WAVE_REDUCE(v, kNone, min_i, dpp);
  return rl(v, 63);
}
__device__ __forceinline__ double wave_max(double v) {  // NaN-free inputs
  MOAT_WAVE_REDUCE(v, -INFINITY, max_d, dpp_d);
  return rl(v, 63);
}

// The wave's largest raw value (NaN skipped) with its least index (kNone: no
// value), by DPP; every lane gets both.
__device__ __forceinline__ void wave_argmax(double& best, int& idx) {
#define MOAT_ARGMAX_STEP(C, R)                                                       \
  {                                                                                  \
    const double ob = dpp_d<C, R>(-INFINITY, best);                                  \
    const int oi = dpp<C, R>(kNone, idx);                                            \
    const bool take = oi != kNone && (idx == kNone || ob > best || (ob == best && oi < idx)); \
    best = take ? ob : best;                                                         \
    idx = take ? oi : idx;                                                           \
  }
  MOAT_ARGMAX_STEP(0xB1, 0xF)
  MOAT_ARGMAX_STEP(0x4E, 0xF)
  MOAT_ARGMAX_STEP(0x114, 0xF)
  MOAT_ARGMAX_STEP(0x118, 0xF)
  MOAT_ARGMAX_STEP(0x142, 0xA)
  MOAT_ARGMAX_STEP(0x143, 0xC)
#undef MOAT_ARGMAX_STEP
  best = rl(best, 63);
  idx = rl(idx, 63);
}

// Folds element i (raw value d, valid if ok) into a running (max, its first
// index, first NaN); elements come in increasing index order.
__device__ __forceinline__ void fold_argmax(double d, int i, bool ok, double& best, int& idx, int& fnan) {
  const bool isn = isnan(d);
  fnan = (ok && isn && fnan == kNone) ? i : fnan;
  const bool take = ok && !isn && (idx == kNone || d > best);
  best = take ? d : best;
  idx = take ? i : idx;
}

// Workgroup (max, first index, first NaN) from every thread's; two barriers'
// worth of LDS (`sd`, `si`), every thread gets the result.
__device__ __forceinline__ void block_argmax(double& best, int& idx, int& fnan, double* sd, int (*si)[kW]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  wave_argmax(best, idx);
  fnan = wave_min(fnan);
  if (lane == 0) {
    sd[wv] = best;
    si[0][wv] = idx;
    si[1][wv] = fnan;
  }
  __syncthreads();
  best = -INFINITY;
  idx = kNone;
  fnan = kNone;
#pragma unroll
  for (int w = 0; w < kW; ++w) {  // waves in index order: ties keep the lower index
    const double ob = sd[w];
    const int oi = si[0][w];
    const bool take = oi != kNone && (idx == kNone || ob > best || (ob == best && oi < idx));
    best = take ? ob : best;
    idx = take ? oi : idx;
    fnan = min(fnan, si[1][w]);
  }
}

// Exclusive prefix sum over the wave's lanes of v < 2^kBits, by bit planes
// (ballot and lane-masked bit counts); `total` gets the wave's sum.
template <int kBits>
__device__ __forceinline__ uint32_t wave_prefix(uint32_t v, uint32_t& total) {
  uint32_t pre = 0, tot = 0;
#pragma unroll
  for (int b = 0; b < kBits; ++b) {
    const unsigned long long m = __ballot((v >> b) & 1u);
    pre += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << b;
    tot += (uint32_t)__popcll(m) << b;
  }
  total = tot;
  return pre;
}

template <int kN>
struct Bits {  // bits of a count 0..kN
  static constexpr int value = kN < 2 ? 1 : 1 + Bits<kN / 2>::value;
};
template <>
struct Bits<1> {
  static constexpr int value = 1;
};

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
// Encoded keys are the fp16 key + 1 (at most 0x7FFF), 0 for no entry; a wave
// with at most kk entries takes all of them without a search.
template <int kN>
__device__ __forceinline__ uint32_t wave_select(const us2 (&ek)[kN / 2], uint32_t kk) {
  uint32_t thr = 0;  // the kk-th largest encoded key
  if (wave_count_ge<kN>(ek, 1) > kk) {
    for (int bit = 14; bit >= 0; --bit) {
      const uint32_t c = thr | (1u << bit);
      if (wave_count_ge<kN>(ek, c) >= kk) thr = c;
    }
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
  const uint32_t pre = wave_prefix<Bits<kN>::value>((uint32_t)__popc(ties), n_ties);
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

__device__ __forceinline__ float leaf_value(const float (*chain)[8], const uint16_t* se, int slot, int tail_from,
                                            int tail) {
  const float* r = chain[slot];
  float v = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
  for (int k = 0; k < 7; ++k) {
    const float x = h2f(se[epos(min(tail_from + k, kCh - 1))]);
    v = k < tail ? v + x : v;
  }
  return v;
}

// The row's sum of table values: the chunk sums added in order from 0.  The
// calling wave's lanes load them; every lane gets the sum.
__device__ __forceinline__ float row_total(const SampleWs& ws, int64_t rc, int nch) {
  const int lane = threadIdx.x & 63;
  const float cs = lane < nch ? fetch(ws.csum + rc + lane) : 0.f;
  float s = 0.f;
  for (int c = 0; c < nch; ++c) s = s + rl(cs, c);
  return s > 0.f ? s : 1.f;
}

// Marks the calling workgroup done with row r; true in the row's last one
// (every thread), whose sc1 loads then see every other workgroup's published
// results, and which has put the counter back to zero.  Wave 0 holds the
// workgroup's published results; every thread must call.
__device__ bool row_done(const SampleWs& ws, int r, int nch, int* s_last) {
  if (nch == 1) return true;
  const int t = threadIdx.x;
  if (t < 64) {
    // wave 0's sc1 stores complete before the counter moves
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    if (t == 0)
      *s_last = __hip_atomic_fetch_add(&ws.cnt[r], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                (uint32_t)(nch - 1);
  }
  __syncthreads();
  if (!*s_last) return false;
  if (t == 0) __hip_atomic_store(&ws.cnt[r], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// np.argmax of the raw row from the chunk statistics: the first NaN, else the
// least first index among the chunks holding the maximum (the calling wave).
__device__ __forceinline__ int row_argmax(const SampleWs& ws, int64_t rc, int nch) {
  const int lane = threadIdx.x & 63;
  const bool ok = lane < nch;
  double best = ok ? fetch(ws.cmax + rc + lane) : -INFINITY;
  int idx = ok ? fetch(ws.cfirst + rc + lane) : kNone;
  const int fnan = wave_min(ok ? fetch(ws.cnan + rc + lane) : kNone);
  wave_argmax(best, idx);
  return fnan != kNone ? fnan : idx;
}

// ---- K1: chunk statistics (rows of more than kFuse chunks) ---------------

template <typename T>
__global__ void __launch_bounds__(kT) chunk_stats_kernel(const T* __restrict__ x, int v, int nch, SampleWs ws) {
  __shared__ double sd[kW];
  __shared__ int si[2][kW];
  const int t = threadIdx.x;
  const int r = blockIdx.x, c = blockIdx.y;
  const int base = c * kCh, nc = min(kCh, v - base);
  const T* xc = x + (int64_t)r * v + base;
  T raw[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) raw[j] = xc[min(t + kT * j, nc - 1)];
  double best = -INFINITY;
  int idx = kNone, fnan = kNone;
#pragma unroll
  for (int j = 0; j < kPer; ++j) fold_argmax(raw_d(raw[j]), base + t + kT * j, t + kT * j < nc, best, idx, fnan);
  block_argmax(best, idx, fnan, sd, si);
  if (t == 0) {
    const int64_t at = (int64_t)r * nch + c;
    publish(ws.cmax + at, best);
    publish(ws.cnan + at, fnan);
    publish(ws.cfirst + at, idx);
    // the row's counter starts from zero in the launches that follow (only
    // rows of more than one chunk, which all run K1, use it)
    if (c == 0) ws.cnt[r] = 0u;
  }
}

// ---- K2: the row's maximum, table values and the chunk sums --------------

// kOne: a row of one chunk (no K1: the chunk's statistics are the row's).
template <typename T, bool kScaled, bool kOne>
__global__ void __launch_bounds__(kT) chunk_sum_kernel(const T* __restrict__ x, int v, int nch, double temp,
                                                       const uint16_t* __restrict__ lut, int lut_size, float step,
                                                       int mode, int32_t* __restrict__ tokens,
                                                       float* __restrict__ logprobs, SampleWs ws) {
  __shared__ uint16_t se[kERow];
  __shared__ float chain[kSlots][8];
  __shared__ double sd[kW];
  __shared__ int si[2][kW];
  __shared__ int s_last;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int r = blockIdx.x, c = blockIdx.y;
  const int base = c * kCh, nc = min(kCh, v - base);
  const int64_t rc = (int64_t)r * nch;
  const T* xr = x + (int64_t)r * v;
  T raw[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) raw[j] = xr[base + min(t + kT * j, nc - 1)];
  // the row's raw maximum (NaN skipped) and whether it holds a NaN
  double mraw;
  bool anynan;
  if (kOne) {
    // the chunk's statistics (for np.argmax) are the row's
    double best = -INFINITY;
    int idx = kNone, fn = kNone;
#pragma unroll
    for (int j = 0; j < kPer; ++j) fold_argmax(raw_d(raw[j]), base + t + kT * j, t + kT * j < nc, best, idx, fn);
    block_argmax(best, idx, fn, sd, si);
    mraw = best;
    anynan = fn != kNone;
    if (t == 0) {
      publish(ws.cmax + rc + c, best);
      publish(ws.cnan + rc + c, fn);
      publish(ws.cfirst + rc + c, idx);
    }
  } else {
    // from K1's chunk statistics (every wave reduces the same values)
    const bool ok = lane < nch;
    mraw = wave_max(ok ? ws.cmax[rc + lane] : -INFINITY);
    anynan = wave_min(ok ? ws.cnan[rc + lane] : kNone) != kNone;
  }
  // the maximum after T: x / T is monotone, so it is the maximum's quotient
  const T mt = from_d<T>(mraw);
  const float m = anynan ? NAN : (kScaled ? scale_conv(mt, temp) : conv(mt));
  const bool bad = !isfinite(m);
  if (t == 0 && c == 0) ws.rowbad[r] = bad ? 1 : 0;
  if (!bad) {
    // table values; |x - max| / step by Markstein's sequence: outside its
    // range the quotient is below 1 (index 0 either way) or far above the
    // last index (NaN or huge here, clamped to it)
    const float top = (float)(lut_size - 1), rs = __fdiv_rn(1.0f, step);
    uint16_t ev[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const float xs = t + kT * j < nc ? (kScaled ? scale_conv(raw[j], temp) : conv(raw[j])) : -INFINITY;
      const float a = div_markstein(fabsf(xs - m), step, rs);
      ev[j] = lut[lut_size - 1 - (int)(a == a ? fminf(a, top) : top)];
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) se[epos(t + kT * j)] = ev[j];
    if (mode != kModeGreedy) {
      uint16_t* er = ws.e + (int64_t)r * v + base;
#pragma unroll
      for (int j = 0; j < kPer; ++j)
        if (t + kT * j < nc) er[t + kT * j] = ev[j];
    }
    __syncthreads();
    // chains: thread t is accumulator t % 8 of leaf slot t / 8
    const int q = nc >> 3, rr = nc & 7;
    const int slot = t >> 3, j8 = t & 7;
    if (nc == kCh) {
      // a whole chunk: 64 leaves of 16 blocks (32 nodes of 32 blocks, halved)
      if (slot < 64) {
        const uint16_t* ep = se + epos(128 * slot) + j8;
        float acc = h2f(ep[0]);
#pragma unroll
        for (int k = 1; k < 16; ++k) acc = acc + h2f(ep[8 * k]);
        chain[slot][j8] = acc;
      }
    } else if (nc >= 8) {
      const int d = leaf_depth(q, rr);
      const int p = d ? 1 << (d - 1) : 1;
      const int i = slot >> 1, ch = slot & 1;
      int a0, sz;
      walk(i, d ? d - 1 : 0, q, a0, sz);
      const bool leaf = d == 0 || 8 * sz + (i == p - 1 ? rr : 0) <= 128;
      const int h = sz >> 1;
      const int b0 = (leaf || !ch) ? a0 : a0 + h;
      const int b1 = leaf ? a0 + sz : (ch ? a0 + sz : a0 + h);
      float acc = h2f(se[epos(min(j8 + 8 * b0, kCh - 1))]);
#pragma unroll
      for (int k = 1; k < 16; ++k) {
        const float xk = h2f(se[epos(min(j8 + 8 * (b0 + k), kCh - 1))]);
        acc = b0 + k < b1 ? acc + xk : acc;
      }
      chain[slot][j8] = acc;  // slots past the chunk's leaves are never read
    }
    __syncthreads();
    if (wv == 0) {
      // nodes one level above the leaves (lane i; at most 64, a power of two,
      // 0 past the last), then pairs of neighbours up to the root: DPP within
      // rows of 16 lanes, the four row sums last (adding +0 to a sum of
      // non-negative values leaves it unchanged)
      float nv = 0.f;
      if (nc < 8) {
#pragma unroll
        for (int k = 0; k < 7; ++k) {
          const float xk = h2f(se[epos(k)]);
          nv = (lane == 0 && k < nc) ? nv + xk : nv;
        }
      } else {
        const int d = leaf_depth(q, rr);
        const int p = d ? 1 << (d - 1) : 1;
        int a0, sz;
        walk(lane, d ? d - 1 : 0, q, a0, sz);
        const int tail = lane == p - 1 ? rr : 0;
        const bool leaf = d == 0 || 8 * sz + tail <= 128;
        const int ls = min(2 * lane, kSlots - 2);
        const float left = leaf_value(chain, se, ls, 8 * q, leaf ? tail : 0);
        const float right = leaf_value(chain, se, ls + 1, 8 * q, tail);
        nv = leaf ? left : left + right;
        nv = lane < p ? nv : 0.f;
      }
      nv = nv + dpp_f<0xB1, 0xF>(0.f, nv);   // lane 2i: nodes 2i, 2i+1
      nv = nv + dpp_f<0x4E, 0xF>(0.f, nv);   // lane 4i: + lane 4i+2
      nv = nv + dpp_f<0x104, 0xF>(0.f, nv);  // lane 8i: + lane 8i+4 (row_shl:4)
      nv = nv + dpp_f<0x108, 0xF>(0.f, nv);  // lane 16i: + lane 16i+8 (row_shl:8)
      const float s = (rl(nv, 0) + rl(nv, 16)) + (rl(nv, 32) + rl(nv, 48));
      if (lane == 0) publish(ws.csum + rc + c, s);
    }
  }
  if (mode != kModeGreedy) return;
  // greedy: the row's last workgroup writes the token and fp16(log p) of it
  if (!row_done(ws, r, nch, &s_last)) return;
  if (wv == 0) {
    const int tok = row_argmax(ws, rc, nch);
    float lp = NAN;
    if (!bad) {
      // the maximum's table value is the table's last entry (|x - max| = 0)
      const float p = h2f(f2h(__fdiv_rn(h2f(lut[lut_size - 1]), row_total(ws, rc, nch))));
      lp = h2f(f2h((float)log((double)p)));  // f32 log, then fp16 (numpy's fp16 log)
    }
    if (lane == 0) {
      tokens[r] = tok;
      logprobs[r] = lp;
    }
  }
}

// The calling wave's first kk entries of 4 lists of (key + 1) << 32 | index
// entries in index order (list i: cnt[i] entries at lists[i]), 4 positions a
// lane (list lane / 16), written in index order to `out` (LDS, or the
// workspace with sc1 stores when kPublish); `total` gets their count.
template <bool kPublish>
__device__ __forceinline__ void select_lists(const uint64_t (*lists)[kMaxK], const uint32_t* cnt, uint32_t kk,
                                             uint32_t& total, uint64_t* out) {
  const int lane = threadIdx.x & 63;
  const int li = lane >> 4;
  const uint32_t n = cnt[li];
  us2 ek[2];
  uint64_t ent[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const uint32_t s = (4 * lane + h) & 63;
    ent[h] = s < n ? lists[li][s] : 0ull;
    const unsigned short k = (unsigned short)(ent[h] >> 32);
    if (h & 1) ek[h >> 1].y = k;
    else ek[h >> 1].x = k;
  }
  const uint32_t take = wave_select<4>(ek, kk);
  uint32_t at = wave_prefix<3>((uint32_t)__popc(take), total);
#pragma unroll
  for (int h = 0; h < 4; ++h)
    if (((take >> h) & 1u) && at < kMaxK) {
      if (kPublish) publish(out + at, ent[h]);
      else out[at] = ent[h];
      ++at;
    }
  total = min(total, (uint32_t)kMaxK);
}

// The row's draw from its chunk lists (every thread of the workgroup calls):
// chunk list c's entry s at position 64 c + s, 4 a thread; each wave takes
// the first kk of its 256 positions, wave 0 the first kk of the 16 wave
// lists (a row of at most 4 chunks: wave 0 alone, from its 256 positions),
// orders them (p descending, index ascending), sums them in numpy's order
// and draws.
__device__ void draw_row(const SampleWs& ws, int r, int nch, uint32_t kk, uint64_t seed, int32_t* tokens,
                         float* logprobs, uint64_t (*wl)[kMaxK], uint32_t* wcnt, uint64_t* cand) {
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t rc = (int64_t)r * nch;
  if (t < kMaxK) cand[t] = 0ull;
  const bool one_wave = nch <= 4;
  if (one_wave && wv != 0) return;
  {
    us2 ek[2];
    uint64_t ent[4];
    const int c = t >> 4;  // positions 4 t .. 4 t + 3 lie in list t / 16
    const uint32_t cnt = c < nch ? fetch(ws.ccnt + rc + c) : 0u;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const uint32_t s = (4 * t + h) & 63;
      ent[h] = s < cnt ? fetch(ws.clist + (rc + c) * kMaxK + s) : 0ull;
      const unsigned short k = (unsigned short)(ent[h] >> 32);
      if (h & 1) ek[h >> 1].y = k;
      else ek[h >> 1].x = k;
    }
    const uint32_t take = wave_select<4>(ek, kk);
    uint32_t total;
    uint32_t at = wave_prefix<3>((uint32_t)__popc(take), total);
    uint64_t* dst = one_wave ? cand : wl[wv];
#pragma unroll
    for (int h = 0; h < 4; ++h)
      if (((take >> h) & 1u) && at < kMaxK) dst[at++] = ent[h];
    if (lane == 0) wcnt[wv] = min(total, (uint32_t)kMaxK);
  }
  if (!one_wave) __syncthreads();
  if (wv != 0) return;
  if (!one_wave) {
    us2 ek[8];
    uint64_t ent[16];
    const uint32_t cnt = wcnt[lane >> 2];  // a lane's 16 entries lie in list lane / 4
#pragma unroll
    for (int h = 0; h < 16; ++h) {
      const int pp = (16 * lane + h) & 63;
      ent[h] = (uint32_t)pp < cnt ? wl[lane >> 2][pp] : 0ull;
      const unsigned short k = (unsigned short)(ent[h] >> 32);
      if (h & 1) ek[h >> 1].y = k;
      else ek[h >> 1].x = k;
    }
    const uint32_t take = wave_select<16>(ek, kk);
    uint32_t total;
    uint32_t at = wave_prefix<5>((uint32_t)__popc(take), total);
#pragma unroll
    for (int h = 0; h < 16; ++h)
      if (((take >> h) & 1u) && at < kMaxK) cand[at++] = ent[h];
  }
  // the wave's LDS writes before its reads of them
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // lane q takes rank q; the sum in numpy's order; the draw
  const int kc = (int)kk;
  const bool live = lane < kc;
  const uint64_t ce = live ? cand[lane] : 0ull;
  const int mi = (int)(uint32_t)ce;
  const uint32_t mk = (uint32_t)(ce >> 32) - 1u;  // the fp16 bits of p (live lanes)
  // rank in (p descending, index ascending), radix style from the top key
  // bit: `eq` holds the live lanes whose key agrees with this lane's so far,
  // and the lanes that leave it with a 1 where this lane has a 0 rank above
  // it; the entries are in index order (lists merged in position order), so
  // equal keys rank by lane
  const unsigned long long live_m = __ballot(live);
  unsigned long long eq = live_m;
  uint32_t rank = 0;
#pragma unroll
  for (int b = 14; b >= 0; --b) {
    const bool one = (mk >> b) & 1u;
    const unsigned long long ones = __ballot(live && one);
    rank += one ? 0u : (uint32_t)__popcll(eq & ones);
    eq = one ? (eq & ones) : (eq & ~ones);
  }
  rank += __builtin_amdgcn_mbcnt_hi((uint32_t)(eq >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)eq, 0u));
  const int dst = 4 * (live ? (int)rank : lane);
  const int sidx = __builtin_amdgcn_ds_permute(dst, mi);
  const int skey = __builtin_amdgcn_ds_permute(dst, (int)mk);
  const float pk = live ? h2f((uint16_t)skey) : 0.f;
  float s;
  if (kc < 8) {
    s = 0.f;
    for (int o = 0; o < kc; ++o) s = s + rl(pk, o);
  } else {
    // accumulator j < 8: entries j, j + 8, ... of the full blocks of 8, in
    // order; lane 8 j + i holds entry 8 i + j (one permute), and lane 8 j adds
    // lanes 8 j + 1 .. 8 j + 7 (row_shl) of its row in sequence
    const int blocks = kc / 8;
    const int src = 8 * (lane & 7) + (lane >> 3);
    const float tp = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * src, __float_as_int(pk)));
    const float z = 0.f;
    float acc = tp;
    float x1 = dpp_f<0x101, 0xF>(z, tp), x2 = dpp_f<0x102, 0xF>(z, tp), x3 = dpp_f<0x103, 0xF>(z, tp);
    float x4 = dpp_f<0x104, 0xF>(z, tp), x5 = dpp_f<0x105, 0xF>(z, tp), x6 = dpp_f<0x106, 0xF>(z, tp);
    float x7 = dpp_f<0x107, 0xF>(z, tp);
    acc = blocks > 1 ? acc + x1 : acc;
    acc = blocks > 2 ? acc + x2 : acc;
    acc = blocks > 3 ? acc + x3 : acc;
    acc = blocks > 4 ? acc + x4 : acc;
    acc = blocks > 5 ? acc + x5 : acc;
    acc = blocks > 6 ? acc + x6 : acc;
    acc = blocks > 7 ? acc + x7 : acc;
    s = ((rl(acc, 0) + rl(acc, 8)) + (rl(acc, 16) + rl(acc, 24))) +
        ((rl(acc, 32) + rl(acc, 40)) + (rl(acc, 48) + rl(acc, 56)));
    for (int o = 8 * blocks; o < kc; ++o) s = s + rl(pk, o);
  }
  // cumulative distribution in f64, in order (lane q: entries 0..q), over
  // its last entry; entries past kc are +0, which leaves a sum unchanged
  const double pn = live ? (s > 0.f ? (double)__fdiv_rn(pk, s) : 1.0 / (double)kc) : 0.0;
  double cdf = 0.0;
#pragma unroll
  for (int o = 0; o < kMaxK; ++o) {
    const double xo = rl(pn, o);
    cdf = o <= lane ? cdf + xo : cdf;
  }
  const double total = rl(cdf, kc - 1);
  const double u = row_uniform(seed, r);
  const unsigned long long hit = __ballot(live && __ddiv_rn(cdf, total) > u);
  const int pick = hit ? __ffsll((long long)hit) - 1 : kc - 1;
  const int tk = rl(sidx, pick);
  const float pc = rl(pk, pick);
  if (lane == 0) {
    tokens[r] = tk;
    logprobs[r] = pc >= 1e-10f ? (float)log((double)pc) : (float)-23.025850929940457;  // log(1e-10)
  }
}

// ---- K3: probabilities; the chunk's first k entries; the draw ------------

__global__ void __launch_bounds__(kT) chunk_select_kernel(int v, int nch, int top_k, int mode, uint64_t seed,
                                                          uint16_t* __restrict__ probs, int32_t* __restrict__ tokens,
                                                          float* __restrict__ logprobs, SampleWs ws) {
  __shared__ __align__(16) uint16_t sp[kERow];
  __shared__ uint64_t wl[kW][kMaxK];
  __shared__ uint32_t wcnt[kW];
  __shared__ uint64_t wl2[4][kMaxK];
  __shared__ uint32_t wcnt2[4];
  __shared__ uint64_t cand[kMaxK];
  __shared__ float s_sum;
  __shared__ int s_last;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int r = blockIdx.x, c = blockIdx.y;
  const int base = c * kCh, nc = min(kCh, v - base);
  const int64_t rc = (int64_t)r * nch;
  const uint32_t kk = (uint32_t)min(top_k, v);
  const bool bad = ws.rowbad[r] != 0;
  if (bad && mode == kModeProbs) {
    for (int i = t; i < nc; i += kT) probs[(int64_t)r * v + base + i] = 0x7E00;
    return;
  }
  if (!bad) {
    const uint16_t* er = ws.e + (int64_t)r * v + base;
    uint16_t ev[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) ev[j] = er[min(t + kT * j, nc - 1)];
    if (wv == 0) {
      const float s = row_total(ws, rc, nch);
      if (lane == 0) s_sum = s;
    }
    __syncthreads();
    const float sum = s_sum, rsum = __fdiv_rn(1.0f, sum);
    // e / sum by Markstein's sequence, always in its range (e is 0 or at
    // least 2^-24 and at most 1; 1 <= sum, the maximum's table value being 1)
    if (mode == kModeProbs) {
      uint16_t* pr = probs + (int64_t)r * v + base;
#pragma unroll
      for (int j = 0; j < kPer; ++j)
        if (t + kT * j < nc) pr[t + kT * j] = f2h(div_markstein(h2f(ev[j]), sum, rsum));
      return;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) sp[epos(t + kT * j)] = f2h(div_markstein(h2f(ev[j]), sum, rsum));
    __syncthreads();
    // per wave: its 512 entries in index order (thread t re-reads entries
    // 8t .. 8t+7 of the chunk), the first kk in the order (p descending,
    // index ascending); keys are the fp16 bits + 1, 0 past the chunk's end
    {
      const uint4 w4 = *reinterpret_cast<const uint4*>(sp + epos(kPer * t));
      const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
      us2 ek[kPer / 2];
#pragma unroll
      for (int h = 0; h < kPer / 2; ++h) {
        const int i0 = kPer * t + 2 * h;
        ek[h].x = i0 < nc ? (unsigned short)((wd[h] & 0xFFFF) + 1) : (unsigned short)0;
        ek[h].y = i0 + 1 < nc ? (unsigned short)((wd[h] >> 16) + 1) : (unsigned short)0;
      }
      const uint32_t take = wave_select<kPer>(ek, kk);
      uint32_t total;
      uint32_t at = wave_prefix<Bits<kPer>::value>((uint32_t)__popc(take), total);
#pragma unroll
      for (int h = 0; h < kPer; ++h)
        if (((take >> h) & 1u) && at < kMaxK) {
          const uint32_t key = (h & 1) ? ek[h >> 1].y : ek[h >> 1].x;
          wl[wv][at++] = (uint64_t)key << 32 | (uint32_t)(base + kPer * t + h);
        }
      if (lane == 0) wcnt[wv] = min(total, (uint32_t)kMaxK);
    }
    __syncthreads();
    // the 16 wave lists (index order) merged in two steps: waves 0..3 each
    // take the first kk of 4 lists, then wave 0 the first kk of those 4
    if (wv < 4) {
      uint32_t total;
      select_lists<false>(wl + 4 * wv, wcnt + 4 * wv, kk, total, wl2[wv]);
      if (lane == 0) wcnt2[wv] = total;
    }
    __syncthreads();
    if (wv == 0) {
      uint32_t total;
      select_lists<true>(wl2, wcnt2, kk, total, ws.clist + (rc + c) * kMaxK);
      if (lane == 0) publish(ws.ccnt + rc + c, min(total, (uint32_t)kMaxK));
    }
  }
  // the row's last workgroup draws
  if (!row_done(ws, r, nch, &s_last)) return;
  if (bad) {
    if (wv == 0) {
      const int tok = row_argmax(ws, rc, nch);
      if (lane == 0) {
        tokens[r] = tok;
        logprobs[r] = NAN;
      }
    }
    return;
  }
  __syncthreads();  // wl and wcnt are reused
  draw_row(ws, r, nch, kk, seed, tokens, logprobs, wl, wcnt, cand);
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

template <typename T, bool kScaled>
void launch_sum(const T* x, int n, int v, int nch, double temp, const uint16_t* lut, int lut_size, float step,
                int mode, int32_t* tokens, float* logprobs, const SampleWs& ws, hipStream_t st) {
  const dim3 grid(n, nch), block(kT);
  if (nch == 1) {
    hipLaunchKernelGGL((chunk_sum_kernel<T, kScaled, true>), grid, block, 0, st, x, v, nch, temp, lut, lut_size,
                       step, mode, tokens, logprobs, ws);
  } else {
    hipLaunchKernelGGL(chunk_stats_kernel<T>, grid, block, 0, st, x, v, nch, ws);
    hipLaunchKernelGGL((chunk_sum_kernel<T, kScaled, false>), grid, block, 0, st, x, v, nch, temp, lut, lut_size,
                       step, mode, tokens, logprobs, ws);
  }
}

template <typename T>
void launch_front(const void* x, int n, int v, int nch, double temp, int scaled, const uint16_t* lut, int lut_size,
                  float step, int mode, int32_t* tokens, float* logprobs, const SampleWs& ws, hipStream_t st) {
  const T* xt = static_cast<const T*>(x);
  if (scaled) launch_sum<T, true>(xt, n, v, nch, temp, lut, lut_size, step, mode, tokens, logprobs, ws, st);
  else launch_sum<T, false>(xt, n, v, nch, temp, lut, lut_size, step, mode, tokens, logprobs, ws, st);
}

// Byte offsets of the workspace arrays (256-byte aligned; the row counters
// first) and the total.
struct WsLayout {
  int64_t off[9];
  int64_t bytes;
};

WsLayout ws_layout(int n, int v, bool with_e) {
  const int64_t per = (int64_t)n * ((v + kCh - 1) / kCh);
  const int64_t sizes[9] = {4 * (int64_t)n, 8 * per, 4 * per, 4 * per, 4 * per, 4 * per, 8 * per * kMaxK,
                            4 * (int64_t)n, with_e ? 2 * (int64_t)n * v : 0};
  WsLayout l;
  int64_t o = 0;
  for (int i = 0; i < 9; ++i) {
    l.off[i] = o;
    o += (sizes[i] + 255) / 256 * 256;
  }
  l.bytes = o;
  return l;
}

}  // namespace

int sample_max_vocab() { return kMaxChunks * kCh; }

// Workspace of a sampling call (with_e) or a softmax call, whose table values
// go to the output buffer.
int64_t sample_workspace_bytes(int n, int v, bool with_e) {
  return n > 0 && v > 0 ? ws_layout(n, v, with_e).bytes : 0;
}

hipError_t launch_lut_sample(const void* x, int dtype, int n, int v, double temp, int scaled, const uint16_t* lut,
                             int lut_size, float step, int mode, int top_k, uint64_t seed, int32_t* tokens,
                             float* logprobs, uint16_t* probs, void* workspace, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const WsLayout l = ws_layout(n, v, mode != kModeProbs);
  uint8_t* w = static_cast<uint8_t*>(workspace);
  const SampleWs ws = {reinterpret_cast<uint32_t*>(w + l.off[0]),
                       reinterpret_cast<double*>(w + l.off[1]),
                       reinterpret_cast<int*>(w + l.off[2]),
                       reinterpret_cast<int*>(w + l.off[3]),
                       reinterpret_cast<float*>(w + l.off[4]),
                       reinterpret_cast<uint32_t*>(w + l.off[5]),
                       reinterpret_cast<uint64_t*>(w + l.off[6]),
                       reinterpret_cast<int*>(w + l.off[7]),
                       mode == kModeProbs ? probs : reinterpret_cast<uint16_t*>(w + l.off[8])};
  const int nch = (v + kCh - 1) / kCh;
  switch (dtype) {
    case 0: launch_front<float>(x, n, v, nch, temp, scaled, lut, lut_size, step, mode, tokens, logprobs, ws, st); break;
    case 1:
      launch_front<uint16_t>(x, n, v, nch, temp, scaled, lut, lut_size, step, mode, tokens, logprobs, ws, st);
      break;
    default:
      launch_front<double>(x, n, v, nch, temp, scaled, lut, lut_size, step, mode, tokens, logprobs, ws, st);
      break;
  }
  if (mode != kModeGreedy)
    hipLaunchKernelGGL(chunk_select_kernel, dim3(n, nch), dim3(kT), 0, st, v, nch, top_k, mode, seed, probs, tokens,
                       logprobs, ws);
  return hipGetLastError();
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
