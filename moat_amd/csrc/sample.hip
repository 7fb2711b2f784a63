// Batched token sampling over LM-head logits: the table ("LUT") softmax of the
// reference's numpy sampler, then greedy argmax or a draw from the k most
// probable tokens (antigravity-engine/src/batch_generator.py:187-253,
// antigravity-engine/src/attention.py:60-135).
//
// One workgroup of 1024 threads per row (V <= 32768): thread t holds the
// logits t + 1024 j (j < 32) in registers after one coalesced pass; the fp16
// exp table (up to 32768 entries, 64 KB) and the row's fp16 table values, then
// probabilities, sit in LDS (64 KB).  Steps, with the reference's arithmetic:
//   1. x (f32/f16/f64) divided by the temperature in its own dtype (fp16:
//      divide in f32, round to fp16), then rounded to f32; the row maximum
//      (NaN-propagating) and the first index of the raw maximum (NaN first).
//   2. table index size-1-trunc(min(|x - max| / step, size-1)) (f32 division,
//      correctly rounded) -> e, the table's fp16 value.
//   3. sum of e in numpy's float32 order: pairwise sums of 8192-element chunks
//      (the reduction buffer) added in sequence from 0; inside a chunk,
//      halves split at multiples of 8 down to blocks of at most 128, each
//      summed with 8 strided accumulators, then its tail.  The tree is walked
//      in parallel: 8 chains per leaf, one lane per node one level above the
//      leaves (up to 64 per chunk), shuffles for the levels above.
//   4. p = fp16(e / sum) (f32 division).
//   5. greedy: log of p[argmax] (float32 log, then fp16, as numpy's fp16 log);
//      sampling: the k largest p by (p descending, index ascending) from two
//      8-bit histogram passes over the fp16 bits of p and an index-ordered
//      scan of the ties at the threshold, the k values summed in numpy's order
//      (8 accumulators) and normalised in f32, the cumulative sum in f64
//      divided by its last value, the first entry above the row's uniform
//      draw; log of the full-softmax p of that token.
// A row whose maximum is NaN or infinite (where the reference's table index
// is undefined) gets the argmax rule's token and a NaN log-probability, and
// NaN probabilities.
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
constexpr int kSSlots = 128;  // leaves per chunk: at most 64 nodes one level up, two children each
constexpr int kSNodes = kSSlots / 2;  // one wave per chunk holds those nodes
constexpr int kSMaxK = 64;

enum SampleMode { kModeProbs = 0, kModeGreedy = 1, kModeSample = 2 };

struct SampleShared {
  uint16_t lut[kSMaxLut];
  uint16_t e[kSMaxV];  // table value of each element, then its probability (fp16 bits)
  float chain[kSMaxChunks][kSSlots][8];
  float chunk_sum[kSMaxChunks];
  float wave_max[kSWaves];
  double wave_best[kSWaves];
  int wave_idx[kSWaves];
  int wave_flags[kSWaves];
  uint32_t hist[256];
  uint32_t tie_count[kSPer];
  uint32_t wave_cnt[kSWaves];
  int cand[kSMaxK];
  uint32_t n_cand;
  int sorted_idx[kSMaxK];
  uint16_t sorted_key[kSMaxK];
  float sum;
  float row_max;
  int argmax;
  int bad;
  int sel[4];
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
// raw value for the argmax (exact in double for every input dtype)
__device__ __forceinline__ double raw_d(float r) { return (double)r; }
__device__ __forceinline__ double raw_d(double r) { return r; }
__device__ __forceinline__ double raw_d(uint16_t r) { return (double)h2f(r); }

struct Best {
  double v;
  int idx;   // -1: none
  int nan;
};

// a before b under np.argmax: NaN first, then the larger value, then the smaller index
__device__ __forceinline__ bool before(const Best& a, const Best& b) {
  if (a.idx < 0) return false;
  if (b.idx < 0) return true;
  if (a.nan != b.nan) return a.nan;
  if (!a.nan && a.v != b.v) return a.v > b.v;
  return a.idx < b.idx;
}

__device__ __forceinline__ float max_nan(float a, float b) { return (isnan(a) || isnan(b)) ? NAN : fmaxf(a, b); }

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
    if ((i >> l) & 1) {
      a0 += h;
      sz -= h;
    } else {
      sz = h;
    }
  }
}

__device__ __forceinline__ float leaf_value(const SampleShared& S, int c, int slot, int tail_from, int tail) {
  const float* r = S.chain[c][slot];
  float v = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (int k = 0; k < tail; ++k) v = v + h2f(S.e[tail_from + k]);
  return v;
}

// numpy's float32 sum of the row's e values (S.e[0..v)), into S.sum.
__device__ void row_sum(SampleShared& S, int v) {
  const int t = threadIdx.x;
  const int nchunks = (v + kSChunk - 1) / kSChunk;
  // chains: (chunk, leaf slot, accumulator j)
  for (int cid = t; cid < nchunks * kSSlots * 8; cid += kSThreads) {
    const int c = cid / (kSSlots * 8), slot = (cid >> 3) & (kSSlots - 1), j = cid & 7;
    const int base = c * kSChunk, nc = min(kSChunk, v - base), q = nc >> 3, r = nc & 7;
    if (nc < 8) continue;
    const int d = leaf_depth(q, r);
    const int p = d ? 1 << (d - 1) : 1;
    const int i = slot >> 1, ch = slot & 1;
    if (i >= p) continue;
    int a0, sz;
    walk(i, d ? d - 1 : 0, q, a0, sz);
    const bool leaf = d == 0 || 8 * sz + (i == p - 1 ? r : 0) <= 128;
    int b0, b1;
    if (leaf) {
      if (ch) continue;
      b0 = a0;
      b1 = a0 + sz;
    } else {
      const int h = sz >> 1;
      b0 = ch ? a0 + h : a0;
      b1 = ch ? a0 + sz : a0 + h;
    }
    const uint16_t* ep = S.e + base + j;
    float acc = h2f(ep[8 * b0]);
    for (int b = b0 + 1; b < b1; ++b) acc = acc + h2f(ep[8 * b]);
    S.chain[c][slot][j] = acc;
  }
  __syncthreads();
  // nodes one level above the leaves (lane i of wave c for chunk c), then the
  // levels above by shuffles inside the wave
  if (t < nchunks * kSNodes) {
    const int c = t / kSNodes, i = t % kSNodes;
    const int base = c * kSChunk, nc = min(kSChunk, v - base), q = nc >> 3, r = nc & 7;
    float nv = 0.f;
    int p = 1;
    if (nc < 8) {
      if (i == 0)
        for (int k = 0; k < nc; ++k) nv = nv + h2f(S.e[base + k]);
    } else {
      const int d = leaf_depth(q, r);
      p = d ? 1 << (d - 1) : 1;
      if (i < p) {
        int a0, sz;
        walk(i, d ? d - 1 : 0, q, a0, sz);
        const bool last = i == p - 1;
        const int tail = last ? r : 0;
        const int tail_from = base + 8 * q;
        if (d == 0 || 8 * sz + tail <= 128) {
          nv = leaf_value(S, c, 2 * i, tail_from, tail);
        } else {
          nv = leaf_value(S, c, 2 * i, tail_from, 0) + leaf_value(S, c, 2 * i + 1, tail_from, tail);
        }
      }
    }
    for (int m = p; m > 1; m >>= 1) {
      const float a = __shfl(nv, 2 * i, kSNodes);
      const float b = __shfl(nv, 2 * i + 1, kSNodes);
      nv = a + b;
    }
    if (i == 0) S.chunk_sum[c] = nv;
  }
  __syncthreads();
  if (t == 0) {
    float s = 0.f;
    for (int c = 0; c < nchunks; ++c) s = s + S.chunk_sum[c];
    S.sum = s > 0.f ? s : 1.f;
  }
  __syncthreads();
}

// Highest 8-bit bin b with at least `need` keys at or above it (bins above
// hold fewer); `above` = the keys in bins above b.  Wave 0 only.
__device__ void find_bin(const uint32_t* hist, uint32_t need, int& bin, uint32_t& above) {
  const int lane = threadIdx.x & 63;
  const uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
  const uint32_t own = h0 + h1 + h2 + h3;
  // suffix sum over lanes (lane and above)
  uint32_t suf = own;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = __shfl_down(suf, o, 64);
    if (lane + o < 64) suf += u;
  }
  const uint32_t higher = suf - own;  // keys in lanes above this one
  int b = -1;
  uint32_t ab = 0;
  if (higher < need && suf >= need) {
    uint32_t acc = higher;
    const uint32_t hs[4] = {h0, h1, h2, h3};
    for (int k = 3; k >= 0; --k) {
      if (acc + hs[k] >= need) {
        b = 4 * lane + k;
        ab = acc;
        break;
      }
      acc += hs[k];
    }
  }
  // exactly one lane found it
  const unsigned long long m = __ballot(b >= 0);
  const int src = __ffsll((long long)m) - 1;
  bin = __shfl(b, src, 64);
  above = __shfl(ab, src, 64);
}

// Append a selected index (the selection yields exactly min(k, v) of them;
// the bound only keeps a miscount inside the array).
__device__ __forceinline__ void push_cand(SampleShared& S, int i) {
  const uint32_t pos = atomicAdd(&S.n_cand, 1u);
  if (pos < kSMaxK) S.cand[pos] = i;
}

template <typename T>
__global__ void __launch_bounds__(kSThreads) lut_sample_kernel(const T* __restrict__ x, int v, double temp, int scaled,
                                                               const uint16_t* __restrict__ lut, int lut_size,
                                                               float step, int mode, int top_k, uint64_t seed,
                                                               int32_t* __restrict__ tokens,
                                                               float* __restrict__ logprobs,
                                                               uint16_t* __restrict__ probs) {
  __shared__ SampleShared S;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int row = blockIdx.x;
  const T* xr = x + (int64_t)row * v;

  for (int i = t; i < lut_size; i += kSThreads) S.lut[i] = lut[i];

  // 1. scaled values, row maximum, argmax of the raw values
  float xs[kSPer];
  float mx = -INFINITY;
  int has_nan = 0;
  Best best = {0.0, -1, 0};
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const int i = t + j * kSThreads;
    xs[j] = 0.f;
    if (i < v) {
      const T r = xr[i];
      const float s = scaled ? scale_conv(r, temp) : conv(r);
      xs[j] = s;
      if (isnan(s)) has_nan = 1;
      else mx = fmaxf(mx, s);
      const double rd = raw_d(r);
      const Best c = {rd, i, isnan(rd) ? 1 : 0};
      if (before(c, best)) best = c;
    }
  }
  float wmx = has_nan ? NAN : mx;
  for (int o = 32; o > 0; o >>= 1) {
    wmx = max_nan(wmx, __shfl_xor(wmx, o, 64));
    Best other = {__shfl_xor(best.v, o, 64), __shfl_xor(best.idx, o, 64), __shfl_xor(best.nan, o, 64)};
    if (before(other, best)) best = other;
  }
  if (lane == 0) {
    S.wave_max[wv] = wmx;
    S.wave_best[wv] = best.v;
    S.wave_idx[wv] = best.idx;
    S.wave_flags[wv] = best.nan;
  }
  if (t < 256) S.hist[t] = 0;
  if (t < kSPer) S.tie_count[t] = 0;
  if (t < kSMaxK) {
    S.cand[t] = 0;
    S.sorted_idx[t] = 0;
    S.sorted_key[t] = 0;
  }
  if (t == 0) S.n_cand = 0;
  __syncthreads();
  if (t == 0) {
    float m = S.wave_max[0];
    Best b = {S.wave_best[0], S.wave_idx[0], S.wave_flags[0]};
    for (int w = 1; w < kSWaves; ++w) {
      m = max_nan(m, S.wave_max[w]);
      const Best o = {S.wave_best[w], S.wave_idx[w], S.wave_flags[w]};
      if (before(o, b)) b = o;
    }
    S.row_max = m;
    S.argmax = b.idx;
    S.bad = isfinite(m) ? 0 : 1;
  }
  __syncthreads();
  const int bad = S.bad;
  const float m = S.row_max;

  if (bad) {
    if (probs)
      for (int i = t; i < v; i += kSThreads) probs[(int64_t)row * v + i] = 0x7E00;
    if (t == 0 && mode != kModeProbs) {
      tokens[row] = S.argmax;
      logprobs[row] = NAN;
    }
    return;
  }

  // 2. table values
  const float top = (float)(lut_size - 1);
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const int i = t + j * kSThreads;
    if (i < v) {
      const float a = __fdiv_rn(fabsf(xs[j] - m), step);
      const int idx = (int)fminf(a, top);
      S.e[i] = S.lut[lut_size - 1 - idx];
    }
  }
  __syncthreads();

  // 3. numpy-order sum
  row_sum(S, v);
  const float sum = S.sum;

  // 4. probabilities
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const int i = t + j * kSThreads;
    if (i < v) {
      const uint16_t pb = f2h(__fdiv_rn(h2f(S.e[i]), sum));
      S.e[i] = pb;
      if (probs) probs[(int64_t)row * v + i] = pb;
    }
  }
  if (mode == kModeProbs) return;
  __syncthreads();

  if (mode == kModeGreedy) {
    if (t == 0) {
      const int tok = S.argmax;
      const float p = h2f(S.e[tok]);
      tokens[row] = tok;
      logprobs[row] = h2f(f2h((float)log((double)p)));  // f32 log, then fp16 (numpy's fp16 log)
    }
    return;
  }

  // 5. top-k selection: two histogram passes over the fp16 bits of p
  const uint32_t kk = (uint32_t)min(top_k, v);
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const int i = t + j * kSThreads;
    if (i < v) atomicAdd(&S.hist[S.e[i] >> 8], 1u);
  }
  __syncthreads();
  if (wv == 0) {
    int b;
    uint32_t above;
    find_bin(S.hist, kk, b, above);
    if (lane == 0) {
      S.sel[0] = b;
      S.sel[1] = (int)above;
    }
  }
  __syncthreads();
  const int b1 = S.sel[0];
  const uint32_t above1 = (uint32_t)S.sel[1];
  if (t < 256) S.hist[t] = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const int i = t + j * kSThreads;
    if (i < v && (S.e[i] >> 8) == b1) atomicAdd(&S.hist[S.e[i] & 255], 1u);
  }
  __syncthreads();
  if (wv == 0) {
    int b;
    uint32_t above;
    find_bin(S.hist, kk - above1, b, above);
    if (lane == 0) {
      S.sel[2] = (b1 << 8) | b;
      S.sel[3] = (int)(kk - above1 - above);  // ties at the threshold to take, lowest index first
    }
  }
  __syncthreads();
  const uint16_t thr = (uint16_t)S.sel[2];
  const uint32_t need = (uint32_t)S.sel[3];
  // keys above the threshold, and the ties per 1024-element chunk
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const int i = t + j * kSThreads;
    if (i < v) {
      const uint16_t k = S.e[i];
      if (k > thr) push_cand(S, i);
      else if (k == thr) atomicAdd(&S.tie_count[j], 1u);
    }
  }
  __syncthreads();
  // the chunk where the ties run out
  if (wv == 0) {
    const uint32_t cnt = lane < kSPer ? S.tie_count[lane] : 0u;
    uint32_t inc = cnt;
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t u = __shfl_up(inc, o, 64);
      if (lane >= o) inc += u;
    }
    const unsigned long long hit = __ballot(inc >= need && lane < kSPer);
    const int J = hit ? __ffsll((long long)hit) - 1 : 0;
    const uint32_t before_j = __shfl(inc - cnt, J, 64);
    if (lane == 0) {
      S.sel[0] = J;
      S.sel[1] = (int)(need - before_j);
    }
  }
  __syncthreads();
  const int J = S.sel[0];
  const uint32_t need_j = (uint32_t)S.sel[1];
  for (int j = 0; j < J; ++j) {
    const int i = t + j * kSThreads;
    if (i < v && S.e[i] == thr) push_cand(S, i);
  }
  const int iJ = t + J * kSThreads;
  const bool tie = iJ < v && S.e[iJ] == thr;
  const unsigned long long bal = __ballot(tie);
  if (lane == 0) S.wave_cnt[wv] = (uint32_t)__popcll(bal);
  __syncthreads();
  if (tie) {
    uint32_t rank = (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
    for (int w = 0; w < wv; ++w) rank += S.wave_cnt[w];
    if (rank < need_j) push_cand(S, iJ);
  }
  __syncthreads();
  // order: p descending, index ascending
  if (t < (int)kk) {
    const int mi = S.cand[t];
    const uint16_t mk = S.e[mi];
    uint32_t rank = 0;
    for (uint32_t o = 0; o < kk; ++o) {
      const int oi = S.cand[o];
      const uint16_t ok = S.e[oi];
      rank += (ok > mk || (ok == mk && oi < mi)) ? 1u : 0u;
    }
    if (rank < kk) {
      S.sorted_idx[rank] = mi;
      S.sorted_key[rank] = mk;
    }
  }
  __syncthreads();
  if (t == 0) {
    // the k probabilities' sum in numpy's order (at most 64: one block)
    float s;
    if (kk < 8) {
      s = 0.f;
      for (uint32_t o = 0; o < kk; ++o) s = s + h2f(S.sorted_key[o]);
    } else {
      float r8[8];
      for (int j = 0; j < 8; ++j) r8[j] = h2f(S.sorted_key[j]);
      uint32_t o = 8;
      for (; o < kk - (kk % 8); o += 8)
        for (int j = 0; j < 8; ++j) r8[j] = r8[j] + h2f(S.sorted_key[o + j]);
      s = ((r8[0] + r8[1]) + (r8[2] + r8[3])) + ((r8[4] + r8[5]) + (r8[6] + r8[7]));
      for (; o < kk; ++o) s = s + h2f(S.sorted_key[o]);
    }
    // cumulative distribution in f64, divided by its last entry
    double total = 0.0;
    for (uint32_t o = 0; o < kk; ++o)
      total += s > 0.f ? (double)__fdiv_rn(h2f(S.sorted_key[o]), s) : 1.0 / (double)kk;
    const double u = row_uniform(seed, row);
    double c = 0.0;
    uint32_t pick = kk - 1;
    for (uint32_t o = 0; o < kk; ++o) {
      c += s > 0.f ? (double)__fdiv_rn(h2f(S.sorted_key[o]), s) : 1.0 / (double)kk;
      if (__ddiv_rn(c, total) > u) {
        pick = o;
        break;
      }
    }
    const int tok = S.sorted_idx[pick];
    const float pc = h2f(S.sorted_key[pick]);
    tokens[row] = tok;
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

}  // namespace

hipError_t launch_lut_sample(const void* x, int dtype, int n, int v, double temp, int scaled, const uint16_t* lut,
                             int lut_size, float step, int mode, int top_k, uint64_t seed, int32_t* tokens,
                             float* logprobs, uint16_t* probs, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const dim3 grid(n), block(kSThreads);
  switch (dtype) {
    case 0:
      hipLaunchKernelGGL(lut_sample_kernel<float>, grid, block, 0, st, static_cast<const float*>(x), v, temp, scaled,
                         lut, lut_size, step, mode, top_k, seed, tokens, logprobs, probs);
      break;
    case 1:
      hipLaunchKernelGGL(lut_sample_kernel<uint16_t>, grid, block, 0, st, static_cast<const uint16_t*>(x), v, temp,
                         scaled, lut, lut_size, step, mode, top_k, seed, tokens, logprobs, probs);
      break;
    default:
      hipLaunchKernelGGL(lut_sample_kernel<double>, grid, block, 0, st, static_cast<const double*>(x), v, temp,
                         scaled, lut, lut_size, step, mode, top_k, seed, tokens, logprobs, probs);
      break;
  }
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
