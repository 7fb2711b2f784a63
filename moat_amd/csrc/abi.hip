// C ABI of libmoat_int4.so: argument validation (before any HIP call),
// planning of the GEMM launch, and dispatch to the kernels.
#include <stdint.h>

#include <atomic>
#include <mutex>

#include <hip/hip_runtime.h>

#include "../../include/moat_int4.h"
#include "handoff.h"

namespace moat {
hipError_t launch_dequant_stream(const uint8_t* sb, int64_t n_sb, uint16_t* out, hipStream_t st);
hipError_t launch_pack_nibbles(const int8_t* q, int64_t n, uint8_t* packed, hipStream_t st);
hipError_t launch_unpack_nibbles(const uint8_t* packed, int64_t n_bytes, int8_t* q, hipStream_t st);
hipError_t launch_group_dequant(const void* q, int q_dtype, const void* scales, int scale_dtype, int64_t n_groups,
                                int group_size, int table_mode, uint16_t* out, int32_t* err_flag, hipStream_t st);
hipError_t launch_lut_gather(const int64_t* q, int64_t n, int index_mode, const uint16_t* lut, int64_t lut_rows,
                             int lut_len, uint16_t* out, hipStream_t st);
hipError_t launch_any_negative(const int64_t* q, int64_t n, int32_t* flag, hipStream_t st);
hipError_t launch_to_f16(const void* src, int src_dtype, int64_t n, uint16_t* out, hipStream_t st);
hipError_t launch_i8_div_to_f16(const int8_t* q, int64_t n, float divisor, uint16_t* out, hipStream_t st);
hipError_t launch_clear(void* p, int64_t bytes, hipStream_t st);
hipError_t launch_quantize(const void* w, int dtype, int64_t n, int gsize, int scale_mode, int8_t* q,
                           uint16_t* scales, hipStream_t st);
hipError_t launch_pack_superblocks(const int8_t* q, const uint16_t* scales, int64_t n_sb, uint8_t* sb,
                                   hipStream_t st);
hipError_t launch_quantize_pack(const void* w, int dtype, int64_t n, int scale_mode, uint8_t* sb, hipStream_t st);
int gemm_col_tiles(int m);
int gemm_rounds(int k);
bool gemm_records_eligible(int k, int m);
int gemm_records_tiles(int m);
int gemm_records_groups(int m, int group_tiles);
bool gemm_records_shares_tiles(int k, int m, int group_tiles, int wgs);
bool gemm_groups_shared(int64_t groups, int64_t rounds, int wgs);
int gemm_fused_groups(int mode, int mats, int m);
hipError_t launch_gemm_fused(int mode, const uint16_t* x, const uint8_t* const* sbs, float* const* ys, uint16_t* h,
                             int mats, int n, int k, int m, int wgs, int depth, int finish, float* partials,
                             uint32_t* status, hipStream_t stream);
int sample_max_vocab();
int64_t sample_workspace_bytes(int n, int v, bool with_e);
hipError_t launch_lut_sample(const void* x, int dtype, int n, int v, double temp, int scaled, const uint16_t* lut,
                             int lut_size, float step, int mode, int top_k, uint64_t seed, int32_t* tokens,
                             float* logprobs, uint16_t* probs, void* workspace, hipStream_t st);
hipError_t launch_lut_lookup(const float* x, int64_t n, const uint16_t* lut, int lut_size, float step, uint16_t* out,
                             hipStream_t st);
hipError_t launch_gemm(int algo, const uint16_t* x, const uint8_t* sb, float* y, int n, int k, int m, int splits,
                       int batch, int finish, int front, int group, int waves, float* partials,
                       uint32_t* counters, uint32_t* status, int tile_order, hipStream_t stream);
hipError_t launch_records_to_tiles(const uint8_t* sb, int k, int m, uint8_t* tiles, hipStream_t stream);
hipError_t launch_swiglu_f32(const float* gu, int n, int m, int64_t ld, uint16_t* h, hipStream_t stream);
hipError_t launch_stream_read(const void* src, int64_t bytes, uint32_t* sink, int blocks, hipStream_t st);
hipError_t launch_gemm_strips(const uint16_t* x, const uint8_t* w, float* y, int n, int k, int m, int wgs, int depth,
                              int waves, bool dot, float* slots, uint32_t* status, hipStream_t stream);
hipError_t launch_records_to_strips(const uint8_t* sb, int k, int m, uint8_t* strips, hipStream_t stream);
hipError_t launch_strips_to_records(const uint8_t* strips, int k, int m, uint8_t* sb, hipStream_t stream);
int strips_waves(int n, int waves);
int strips_depth(int n, int waves, int depth);
hipError_t launch_gemm_strips_wide(const uint16_t* x, const uint8_t* w, float* y, int n, int k, int m, int wgs,
                                   int su, int depth, float* slots, uint32_t* status, hipStream_t stream);
hipError_t launch_gemm_strip_groups(const uint16_t* x, const uint8_t* w, float* y, int n, int k, int m, int wgs,
                                    int depth, float* slots, uint32_t* status, hipStream_t stream);
hipError_t launch_gemm_strips_swiglu(const uint16_t* x, const uint8_t* w, uint16_t* h, int n, int k, int m, int wgs,
                                     int per, hipStream_t stream);
int strip_groups_slot_bytes(int n);
void dense_plan(int k, int m, int splits_req, int* blocks, int* rounds, int* per, int* splits);
int64_t dense_slot_bytes(int n, int blocks, int splits);
int64_t dense_counter_bytes();
hipError_t launch_dense_gemm(const uint16_t* x, const uint16_t* w, uint16_t* y, int n, int k, int m, int splits_req,
                             float* slots, uint32_t* counters, hipStream_t stream);
}  // namespace moat

namespace {

constexpr int kMaxN = 32;
constexpr int kMaxDot2N = 8;
// A fixed 64 KB block at the start of the workspace holds the sticky status
// word (first 256 bytes) and the general kernel's split-K counters, so that
// no call's partials (which follow the block) can overlap the counter words
// of a call with more column tiles: 16320 tiles = M up to 2,088,960.
constexpr int64_t kCounterBlockBytes = 64 * 1024;
constexpr int kMaxColTiles = (int)((kCounterBlockBytes - moat::kWsStatusBytes) / 4);

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int32_t status_of(hipError_t e) { return e == hipSuccess ? MOAT_OK : MOAT_ERR_HIP; }

struct GemmPlan {
  int algo;
  int splits;
  int batch;
  int finish;  // kernel-side FinishMode: 0 device atomics, 1 fences, 2 second kernel
  int front;   // kernel-side front end: 0 direct, 1 LDS DMA, 2 vector loads + LDS, 3 record stream
  int group;   // record stream: 256-column tiles per workgroup
  int waves;   // record stream: waves per workgroup (4 or 8)
  int64_t counter_bytes;
  int64_t workspace_bytes;
};

bool gemm_shape_ok(int32_t n, int32_t k, int32_t m) {
  if (n < 1 || n > kMaxN || k < 1 || m < 32 || (m % 32) != 0) return false;
  if (((int64_t)k * (int64_t)m) % 256 != 0) return false;
  // byte offsets of one 32-row round are 32-bit in the kernels
  if ((int64_t)m * 33 * 18 > (int64_t)0xFFFFFFFF) return false;
  if (moat::gemm_col_tiles(m) > kMaxColTiles) return false;
  return true;
}

bool options_ok(const moat_int4_gemm_options* o, int32_t n) {
  if (!o) return true;
  if (o->algo < 0 || o->algo > 2 || o->splits < 0) return false;
  if (o->batch < 0 || o->batch > 5) return false;
  if (o->finish < 0 || o->finish > 3) return false;
  if (o->front < 0 || o->front > 4) return false;
  if (o->group != 0 && o->group != 1 && o->group != 2 && o->group != 4) return false;
  if (o->waves != 0 && o->waves != 4 && o->waves != 8) return false;
  if (o->algo == MOAT_GEMM_DOT2 && n > kMaxDot2N) return false;
  return true;
}

// Kernel and K-split choice.  The split count trades parallelism (a column
// tile is 128 columns, so M/128 workgroups alone leave most of the 256 CUs
// idle at these sizes) against partial-sum traffic, which is
// splits * N * M * 8 bytes against 0.5625 * K * M bytes of weights; it is kept
// below a quarter of the weight stream.
// Record-stream launch plan for `groups` tile groups of `group` tiles each
// (`tiles` tiles in all).  Workgroups: a multiple of the group count (so that
// the workgroups of neighbouring groups read the same rows at the same time
// and share 128-byte lines in L2), about 8 rounds per workgroup, at most one
// per CU, and a K split whose fp32 partials stay well below the weight stream.
void plan_records(GemmPlan& p, int32_t n, int32_t k, int64_t groups, int64_t tiles, int group, int waves,
                  const moat_int4_gemm_options& opt, bool fill_cus) {
  const int rounds = moat::gemm_rounds(k);
  // ring depth (LDS: waves x depth x 7 or 8 KB; the launch clamps it to the LDS)
  const int depth = opt.batch ? opt.batch : (waves == 8 ? 2 : (n <= 16 ? 3 : 2));
  int64_t splits;
  if (opt.splits > 0) {
    splits = opt.splits;
  } else {
    // about 8 rounds per workgroup: 2 per wave with 4 waves, 1 with 8
    splits = (tiles * rounds / 8 + groups / 2) / groups;
    if (splits > 8) splits = 8;  // beyond 8 the hand-off costs more than the shorter loop saves
    // no more workgroups than the 256 CUs hold at once (a second wave of
    // workgroups would double the time): one per CU, as the kernel's
    // registers (over 128 per lane) leave room for one wave per SIMD with 4
    // waves per workgroup, two with 8
    const int64_t resident = 256;
    const int64_t cap_wgs = resident / groups > 0 ? resident / groups : 1;
    if (splits > cap_wgs) splits = cap_wgs;
    // above 16 rows the partial sums (N x 256 floats per workgroup) weigh:
    // stop at about one workgroup per CU
    if (n > 16) {
      const int64_t one_per_cu = 256 / groups > 2 ? 256 / groups : 2;
      if (splits > one_per_cu) splits = one_per_cu;
    }
    int64_t by_traffic = k / (16 * n);
    if (by_traffic < 2) by_traffic = 2;
    if (splits > by_traffic) splits = by_traffic;
    // ... but not below about 64 workgroups (up to 8 per group): with few
    // column tiles the loop, not the partials, is the longer part
    int64_t floor_splits = (64 + groups - 1) / groups;
    if (floor_splits > 8) floor_splits = 8;
    if (floor_splits > cap_wgs) floor_splits = cap_wgs;
    if (splits < floor_splits) splits = floor_splits;
    if (splits < 1) splits = 1;
    // prefer a count that divides the rounds: every workgroup then holds
    // one segment of one tile group (a range that crosses a group boundary
    // costs a second segment, measured ~3 us per call)
    for (int64_t s = splits; s * 2 >= splits; --s) {
      if (rounds % s == 0) {
        splits = s;
        break;
      }
    }
  }
  int64_t wgs = groups * splits;
  const int64_t items = groups * rounds;
  // Up to 8 rows, with at least 8 rounds per workgroup, fill every CU even
  // when the split count leaves some idle: stream-K ranges then cross tile
  // boundaries (a second segment in some workgroups), which costs less than
  // the idle CUs when the weight stream is the bound.  Measured at K=8192 x
  // M=28672 (224 -> 256 workgroups, N = 1..8): 5-9 % faster on the tile
  // order, unchanged on the row order; slower above 8 rows.  (Single
  // projections only: the fused launches keep the split count.)
  if (fill_cus && opt.splits <= 0 && n <= 8 && wgs < 256 && items >= 8 * 256) wgs = 256;
  if (wgs > items) wgs = items;
  // the kernel addresses the partials with 32-bit byte offsets
  const int64_t max_wgs = (int64_t)0xFFFFFFFF / ((int64_t)2 * group * n * 256 * (int64_t)sizeof(float));
  if (wgs > max_wgs) wgs = max_wgs;
  p.splits = (int)wgs;
  p.group = group;
  p.waves = waves;
  p.batch = depth;
  // shared tile groups: summed in the kernel by the workgroup that owns the
  // group (MOAT_FINISH_DEVICE_ATOMICS or MOAT_FINISH_FENCES) or by a fix-up
  // kernel (MOAT_FINISH_SECOND_KERNEL).  Automatic: in the kernel while the
  // owner reads at most 64 KB of partials (n x 1 KB per tile and
  // contributor), which saves the second launch; beyond that the owner's
  // one CU is slower than the fix-up kernel spread over many.
  if (opt.finish == MOAT_FINISH_AUTO) {
    const int64_t per_group = (wgs + groups - 1) / groups;  // workgroups sharing a tile group
    p.finish = (int64_t)n * group * (per_group - 1) <= 64 ? 0 : 2;
  } else {
    p.finish = opt.finish == MOAT_FINISH_SECOND_KERNEL ? 2 : 0;
  }
  p.front = 3;
  // the partials follow the fixed counter block, which other calls sharing
  // the workspace rely on staying zero
  const bool shared = moat::gemm_groups_shared(groups, rounds, p.splits);
  p.counter_bytes = shared ? kCounterBlockBytes : 0;
  p.workspace_bytes = shared ? p.counter_bytes + (int64_t)2 * p.splits * group * n * 256 * (int64_t)sizeof(float) : 0;
}

// x_vec: X rows can be read 16 bytes at a time (x 16-byte aligned, k % 8 ==
// 0), which the record-stream kernel needs.
GemmPlan plan_gemm(int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* o, bool x_vec) {
  moat_int4_gemm_options opt = {0, 0, 0, 0, 0, 0, 0};
  if (o) opt = *o;
  GemmPlan p;
  const bool records_ok = moat::gemm_records_eligible(k, m) && x_vec;
  // the record-stream kernel (matrix cores) serves every N when the shape allows it
  const bool records = records_ok && opt.algo != MOAT_GEMM_DOT2 &&
                       (opt.front == MOAT_FRONT_AUTO || opt.front == MOAT_FRONT_RECORDS);
  if (opt.algo != MOAT_GEMM_AUTO) p.algo = opt.algo;
  else p.algo = (records || n > 2) ? MOAT_GEMM_MFMA : MOAT_GEMM_DOT2;
  const int rounds = moat::gemm_rounds(k);
  if (records) {
    // Record-stream kernel.  Tiles per workgroup: 1 (its 4 waves split K four
    // ways), measured fastest at every benchmark shape but the largest, where
    // 2 ties.
    const int group = opt.group ? opt.group : 1;
    // 8 waves per workgroup only up to 16 rows (the accumulators of 32 rows
    // need more registers than 8 waves leave a lane)
    const int waves = (opt.waves && n <= 16) ? opt.waves : 4;
    plan_records(p, n, k, moat::gemm_records_groups(m, group), moat::gemm_records_tiles(m), group, waves, opt, true);
    return p;
  }
  const int tiles = moat::gemm_col_tiles(m);
  int splits = opt.splits;
  if (splits <= 0) {
    const int target_wgs = 640;
    int s = (target_wgs + tiles / 2) / tiles;
    const int by_rounds = rounds / 4 > 0 ? rounds / 4 : 1;
    const double cap_d = 0.25 * 0.5625 * (double)k / (8.0 * (double)n);
    const int by_traffic = cap_d >= 1.0 ? (int)cap_d : 1;
    if (s > by_rounds) s = by_rounds;
    if (s > by_traffic) s = by_traffic;
    if (s < 1) s = 1;
    splits = s;
  }
  if (splits > rounds) splits = rounds;
  p.splits = splits;
  const int per_wave = (rounds + 4 * splits - 1) / (4 * splits);  // rounds per wave
  // rounds whose loads a wave issues at once
  p.batch = opt.batch ? opt.batch : (per_wave >= 4 ? 4 : (per_wave >= 2 ? 2 : 1));
  // automatic hand-off: a second kernel sums the partials (measured cheapest at every N)
  p.finish = opt.finish ? opt.finish - 1 : 2;
  p.front = opt.front == MOAT_FRONT_DIRECT ? 0 : (opt.front == MOAT_FRONT_LDS_DMA ? 1 : 2);
  p.group = 1;
  p.waves = 4;
  if (splits > 1) {
    p.counter_bytes = kCounterBlockBytes;
    p.workspace_bytes = p.counter_bytes + (int64_t)splits * n * m * 4;
  } else {
    p.counter_bytes = 0;
    p.workspace_bytes = 0;
  }
  return p;
}

// Fused launches (the kernel's RecMode values).
constexpr int kFusedMulti = 1;
constexpr int kFusedSwiglu = 2;
constexpr int kMaxFusedMats = 4;

bool fused_shape_ok(int32_t count, int32_t n, int32_t k, int32_t m) {
  return count >= 1 && count <= kMaxFusedMats && gemm_shape_ok(n, k, m) && moat::gemm_records_eligible(k, m);
}

GemmPlan plan_fused(int mode, int32_t count, int32_t n, int32_t k, int32_t m) {
  GemmPlan p = {};
  const moat_int4_gemm_options opt = {0, 0, 0, 0, 0, 0, 0};
  const int64_t tiles = moat::gemm_records_tiles(m);
  const int group = mode == kFusedSwiglu ? 2 : 1;  // SwiGLU: a gate tile and an up tile per group
  plan_records(p, n, k, moat::gemm_fused_groups(mode, count, m), (mode == kFusedSwiglu ? 2 : count) * tiles, group,
               4, opt, false);
  p.algo = MOAT_GEMM_MFMA;
  return p;
}

int32_t run_fused(int mode, const uint16_t* x, const uint8_t* const* sbs, float* const* ys, uint16_t* h, int32_t count,
                  int32_t n, int32_t k, int32_t m, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  const GemmPlan p = plan_fused(mode, count, n, k, m);
  float* partials = nullptr;
  uint32_t* status = nullptr;
  if (p.workspace_bytes > 0) {
    if (!workspace || workspace_bytes < p.workspace_bytes || !aligned(workspace, 16)) return MOAT_ERR_WORKSPACE;
    status = static_cast<uint32_t*>(workspace);
    partials = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + p.counter_bytes);
  }
  return status_of(moat::launch_gemm_fused(mode, x, sbs, ys, h, count, n, k, m, p.splits, p.batch, p.finish,
                                           partials, status, stream));
}

// Row count (rows x 1024 threads, the launches' first grid dimension, stays
// below 2^32) and vocabulary (64 chunks of 8192 logits) of the sampling calls.
bool sample_sizes_ok(int32_t n, int32_t v) {
  return n >= 0 && n <= (1 << 21) && v >= 1 && v <= moat::sample_max_vocab();
}

// Shared checks of the sampling entry points: dtype, 1 <= v <= 524288 (64
// chunks of 8192 logits), table of 2..2^24 fp16 entries (indices exact in
// float32), positive finite step, at most 2^21 rows.
bool sample_args_ok(const void* x, int32_t dtype, int32_t n, int32_t v, const uint16_t* lut, int32_t lut_size,
                    float step) {
  if (dtype != MOAT_DTYPE_F32 && dtype != MOAT_DTYPE_F16 && dtype != MOAT_DTYPE_F64) return false;
  if (!sample_sizes_ok(n, v)) return false;
  if (lut_size < 2 || lut_size > (1 << 24)) return false;
  if (!(step > 0.f) || step == INFINITY) return false;
  if (n == 0) return true;
  const uintptr_t elem = dtype == MOAT_DTYPE_F32 ? 4 : dtype == MOAT_DTYPE_F16 ? 2 : 8;
  return x && lut && aligned(x, elem) && aligned(lut, 2);
}

// The sampling workspace: present, large enough and 256-byte aligned.
bool sample_ws_ok(int32_t n, int32_t v, bool with_e, const void* workspace, int64_t workspace_bytes) {
  return n == 0 || (workspace && aligned(workspace, 256) &&
                    workspace_bytes >= moat::sample_workspace_bytes(n, v, with_e));
}


// Scratch of moat_int4_gemm_noalloc: one static device array, which every
// GPU the library runs on holds (its own copy, at its own address) until the
// process ends.  Its address on a device comes from hipGetSymbolAddress with
// that device current, once per device; host code uses only that address (the
// array's name in host code is a host-side stand-in, not device memory).
// Calls that use it always hand split-K partials to the fix-up kernel, which
// needs nothing to start at zero: whatever an earlier call left there is
// overwritten before it is read.
constexpr int64_t kNoallocScratchBytes = 16 << 20;

}  // namespace

static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The scratch address on the current device (looked up on its first use).
int32_t noalloc_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return MOAT_ERR_HIP;
  if (dev < 0 || dev >= kMaxDevices) return MOAT_ERR_INVALID;
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      size_t bytes = 0;
      if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return MOAT_ERR_HIP;
      if (hipGetSymbolSize(&bytes, HIP_SYMBOL(scratch)) != hipSuccess || bytes < (size_t)kNoallocScratchBytes)
        return MOAT_ERR_HIP;
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return MOAT_OK;
}

// The GEMM over records in row order (tile_order 0) or tile order (1).  With
// `noalloc`, the workspace is the library's own scratch: any split-K plan
// hands its partials to the fix-up kernel (no in-kernel hand-off, so no
// status word and nothing that must start at zero), and a plan needing more
// than the scratch holds is refused.
int32_t gemm_call(const uint16_t* x_f16, const uint8_t* superblocks, float* y_f32, int32_t n, int32_t k, int32_t m,
                  const moat_int4_gemm_options* options, void* workspace, int64_t workspace_bytes, int tile_order,
                  hipStream_t stream, bool noalloc = false) {
  if (!gemm_shape_ok(n, k, m) || !options_ok(options, n)) return MOAT_ERR_INVALID;
  if (!x_f16 || !superblocks || !y_f32) return MOAT_ERR_INVALID;
  if (!aligned(x_f16, 2) || !aligned(superblocks, 16) || !aligned(y_f32, 4)) return MOAT_ERR_INVALID;
  const bool x_vec = aligned(x_f16, 16) && (k % 8) == 0;
  const GemmPlan p = plan_gemm(n, k, m, options, x_vec);
  if (noalloc) {
    if (p.workspace_bytes > kNoallocScratchBytes) return MOAT_ERR_TOO_LARGE;
    if (p.workspace_bytes > 0) {
      const int32_t st = noalloc_scratch(&workspace);
      if (st != MOAT_OK) return st;
      workspace_bytes = kNoallocScratchBytes;
    }
  }
  if (p.algo == MOAT_GEMM_DOT2 && n > kMaxDot2N) return MOAT_ERR_INVALID;
  // tile order: the record-stream kernel only (whole 256-column tiles, whole
  // 32-row rounds, 16-byte X rows)
  if (tile_order && (p.front != 3 || (m % 256) != 0 || (k % 32) != 0 || !aligned(x_f16, 16) || (k % 8) != 0))
    return MOAT_ERR_INVALID;
  float* partials = nullptr;
  uint32_t* counters = nullptr;
  uint32_t* status = nullptr;
  if (p.workspace_bytes > 0) {
    if (!workspace || workspace_bytes < p.workspace_bytes || !aligned(workspace, 16)) return MOAT_ERR_WORKSPACE;
    status = noalloc ? nullptr : static_cast<uint32_t*>(workspace);
    counters = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + moat::kWsStatusBytes);
    partials = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + p.counter_bytes);
  }
  return status_of(moat::launch_gemm(p.algo, x_f16, superblocks, y_f32, n, k, m, p.splits, p.batch, p.finish,
                                     p.front, p.group, p.waves, partials, counters, status, tile_order, stream));
}


// ---- strip order

// Rows of X one strip-kernel launch takes; more rows run as several launches.
constexpr int kStripRowsPerLaunch = 8;
// At most one workgroup per CU (the kernel's LDS allows no second): all of a
// launch's workgroups are resident together, so a strip's owner never waits
// for a workgroup that cannot start.
constexpr int64_t kStripMaxWorkgroups = 256;

// K % 32 == 0 with at least 64 units of 32 rows per strip (K >= 2048: a
// wave's stage then meets at most one strip boundary), M % 32 == 0.
bool strips_shape_ok(int32_t n, int32_t k, int32_t m) {
  if (n < 1 || n > kMaxN || k < 2048 || (k % 32) != 0 || m < 32 || (m % 32) != 0) return false;
  if ((int64_t)(m / 32) * (k / 32) > ((int64_t)1 << 30)) return false;  // unit indices are 32-bit
  if ((int64_t)kMaxN * k * 2 > ((int64_t)1 << 31)) return false;  // X offsets are 32-bit
  return true;
}

struct StripPlan {
  int kind;  // kStripSlices, kStripGroups or kStripWide
  bool dot;  // the strip kernel's v_dot2 variant (options algo = MOAT_GEMM_DOT2, N <= 4)
  int su;    // the wide strip kernel's units a stage (0: its default)
  int wgs;
  int depth;
  int waves;
  int64_t workspace_bytes;
};

// Kernel choice (options `group`): 0 automatic, 1 the strip-group kernel,
// 2 the strip kernel (8 rows a launch), 3 the wide strip kernel.
constexpr int kStripSlices = 0, kStripGroups = 1, kStripWide = 2;

bool strip_options_ok(const moat_int4_gemm_options* o) {
  return !o || (o->splits >= 0 && o->batch >= 0 && (o->waves == 0 || o->waves == 4 || o->waves == 8 || o->waves == 12) &&
                o->group >= 0 && o->group <= 3 &&
                (o->front == 0 || o->front == 1 || o->front == 2 || o->front == 4 || o->front == 8) &&
                (o->algo == MOAT_GEMM_AUTO || o->algo == MOAT_GEMM_MFMA || o->algo == MOAT_GEMM_DOT2));
}

// The strip kernel: workgroups as strip_workgroups (at most 256, one per
// CU: the kernel's LDS leaves room for one).  Shared strips need the status
// word and one slot of 8 x 32 floats per workgroup, after the fixed 64 KB
// block.
// The wide strip kernel: all N rows in one launch, the same workgroup ranges
// and hand-off, slots of N x 32 floats per workgroup.  The strip-group
// kernel, over (group of 8 strips, unit) items when the records span fewer
// than 2^32 bytes (its copy offsets are 32-bit): up to 256 workgroups of at
// least 16 items and slots of 8 waves x 2 or 4 KB per workgroup.
// Workgroups of the strip and wide strip kernels.  Whole strips per
// workgroup (nothing handed between workgroups; ceil(strips / 256) strips
// each) unless that workgroup's work exceeds the even split over 256
// workgroups by more than 64 units, the measured cost of a hand-off: the
// split then spreads the units over all 256 CUs, at least 16 units each.
// (Measured: K=2048 x M=2048, 64 strips, 4.6 against 5.7 us at N = 1 as 64
// whole strips; K=5632 x M=2048 6.5 against 9.3 us at N = 16 split over 256;
// K=2048 x M=11264, 352 strips, 8.1 against 8.6 us as 2 strips each.)
int strip_workgroups(int64_t strips, int64_t units, int splits) {
  const int64_t total = strips * units;
  int64_t wgs;
  if (splits > 0) {
    wgs = splits < kStripMaxWorkgroups ? splits : kStripMaxWorkgroups;
  } else {
    const int64_t per = (strips + kStripMaxWorkgroups - 1) / kStripMaxWorkgroups;  // strips a workgroup
    const int64_t even = (total + kStripMaxWorkgroups - 1) / kStripMaxWorkgroups;
    if (per * units <= even + 64) wgs = (strips + per - 1) / per;
    else wgs = total / 16 < kStripMaxWorkgroups ? (total / 16 > 0 ? total / 16 : 1) : kStripMaxWorkgroups;
  }
  return (int)(wgs > total ? total : wgs);
}

StripPlan plan_strips(int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* o) {
  StripPlan p = {};
  const int64_t strips = m / 32, units = k / 32;
  const int forced = o ? o->group : 0;
  p.dot = o && o->algo == MOAT_GEMM_DOT2;
  if (p.dot) {  // the strip kernel's VALU variant: N <= 4 only
    p.kind = kStripSlices;
    const int64_t total = strips * units;
    p.wgs = strip_workgroups(strips, units, o->splits);
    const int64_t wgs = p.wgs;
    const int waves = o->waves ? o->waves : (total / wgs <= 256 ? 12 : 8);
    p.waves = moat::strips_waves(n, waves);
    p.depth = 2;
    const int64_t base = total / wgs, rem = total % wgs;
    const bool shared = !(rem == 0 && base % units == 0);
    p.workspace_bytes = shared ? kCounterBlockBytes + wgs * kStripRowsPerLaunch * 32 * (int64_t)sizeof(float) : 0;
    return p;
  }
  const bool groups_fit = strips * units * 576 < ((int64_t)1 << 32);
  const int64_t weights = (int64_t)k * m;
  p.kind = kStripSlices;
  if (forced == 3) {
    p.kind = kStripWide;
  } else if (forced == 1) {
    if (groups_fit) p.kind = kStripGroups;
  } else if (forced == 0) {
    // measured: the wide kernel is the fastest for N >= 5 and, on matrices
    // under 2^27 weights, for every N; the strip kernel (1, 2 or 4 rows
    // staged, 64-unit stages) for N <= 4 on larger ones; the strip-group
    // kernel (X staged once for 8 strips) for N > 16 from 2^27 weights
    if (n > 16 && weights >= ((int64_t)1 << 27) && groups_fit) p.kind = kStripGroups;
    else if (n >= 5 || weights < ((int64_t)1 << 27)) p.kind = kStripWide;
  }
  if (p.kind == kStripGroups) {
    const int64_t total = (strips + 7) / 8 * units;
    int64_t wgs;
    if (o && o->splits > 0) wgs = o->splits < kStripMaxWorkgroups ? o->splits : kStripMaxWorkgroups;
    else wgs = total / 16 < 256 ? (total / 16 > 0 ? total / 16 : 1) : 256;
    if (wgs > total) wgs = total;
    p.wgs = (int)wgs;
    // ring depth 2 (3 on request): 2 measured 4-6 % faster (K=8192 x M=28672,
    // N = 17 and 32: 42.6 / 43.5 against 45.4 / 46.0 us)
    p.depth = o && o->batch == 3 ? 3 : 2;
    p.waves = 8;
    const int64_t base = total / wgs, rem = total % wgs;
    const bool shared = !(rem == 0 && base % units == 0);
    p.workspace_bytes = shared ? kCounterBlockBytes + wgs * 8 * (int64_t)moat::strip_groups_slot_bytes(n) : 0;
    return p;
  }
  const int64_t total = strips * units;
  p.wgs = strip_workgroups(strips, units, o ? o->splits : 0);
  const int64_t wgs = p.wgs;
  const int64_t base = total / wgs, rem = total % wgs;
  const bool shared = !(rem == 0 && base % units == 0);
  if (p.kind == kStripWide) {  // 8 waves; slots of n x 32 floats
    p.waves = 8;
    p.depth = o ? o->batch : 0;  // 0: two stages
    p.su = o ? o->front : 0;
    p.workspace_bytes = shared ? kCounterBlockBytes + wgs * n * 32 * (int64_t)sizeof(float) : 0;
    return p;
  }
  const int rows = n < kStripRowsPerLaunch ? n : kStripRowsPerLaunch;
  // 12 waves (4-unit stages) for ranges of at most 256 units, 8 beyond
  const int waves = o && o->waves ? o->waves : (total / wgs <= 256 ? 12 : 8);
  p.waves = moat::strips_waves(rows, waves);
  p.depth = moat::strips_depth(rows, p.waves, o ? o->batch : 0);
  p.workspace_bytes = shared ? kCounterBlockBytes + wgs * kStripRowsPerLaunch * 32 * (int64_t)sizeof(float) : 0;
  return p;
}

int sample_dtype(int32_t dtype) { return dtype == MOAT_DTYPE_F32 ? 0 : dtype == MOAT_DTYPE_F16 ? 1 : 2; }

// Dense fp16 product: rows of X a launch; the workspace holds a fixed area
// of counter words (one per 64-column block), then the split sums.
constexpr int32_t kDenseRowsPerLaunch = 32;
constexpr int32_t kDenseMaxSplits = 1024;

bool dense_shape_ok(int32_t n, int32_t k, int32_t m, int32_t splits) {
  return n >= 1 && k >= 8 && (k % 8) == 0 && m >= 8 && (m % 8) == 0 && splits >= 0 && splits <= kDenseMaxSplits &&
         (int64_t)k * m <= ((int64_t)1 << 40) && (int64_t)n * k <= ((int64_t)1 << 40) &&
         (int64_t)n * m <= ((int64_t)1 << 40);
}

int64_t dense_workspace_bytes(int32_t n, int32_t k, int32_t m, int32_t splits) {
  int blocks = 0, rounds = 0, per = 0, sp = 0;
  moat::dense_plan(k, m, splits, &blocks, &rounds, &per, &sp);
  if (sp <= 1) return 0;
  const int rows = n < kDenseRowsPerLaunch ? n : kDenseRowsPerLaunch;
  return moat::dense_counter_bytes() + moat::dense_slot_bytes(rows, blocks, sp);
}

bool spans_overlap(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + (uintptr_t)b_bytes && y < x + (uintptr_t)a_bytes;
}

}  // namespace

extern "C" {

int32_t moat_int4_version(void) { return MOAT_INT4_VERSION_MAJOR * 100 + MOAT_INT4_VERSION_MINOR; }

const char* moat_int4_status_string(int32_t status) {
  switch (status) {
    case MOAT_OK: return "ok";
    case MOAT_ERR_INVALID: return "invalid argument (shape, size, pointer or alignment)";
    case MOAT_ERR_HIP: return "HIP runtime error";
    case MOAT_ERR_WORKSPACE: return "workspace missing or too small";
    case MOAT_ERR_TOO_LARGE: return "the call needs more split-K scratch than moat_int4_gemm_noalloc holds (16 MB)";
    default: return "unknown status";
  }
}

int32_t moat_int4_dequant(const uint8_t* superblocks, int64_t n_superblocks, uint16_t* out_f16, hipStream_t stream) {
  if (n_superblocks < 0) return MOAT_ERR_INVALID;
  if (n_superblocks == 0) return MOAT_OK;
  if (!superblocks || !out_f16 || !aligned(superblocks, 16) || !aligned(out_f16, 16)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_dequant_stream(superblocks, n_superblocks, out_f16, stream));
}

int64_t moat_int4_gemm_ex_workspace_size(int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* options) {
  if (!gemm_shape_ok(n, k, m) || !options_ok(options, n)) return -1;
  // the plan depends on whether X can be read 16 bytes at a time, which the
  // size query cannot see: enough for either plan
  const int64_t a = plan_gemm(n, k, m, options, true).workspace_bytes;
  const int64_t b = plan_gemm(n, k, m, options, false).workspace_bytes;
  return a > b ? a : b;
}

int64_t moat_int4_gemm_workspace_size(int32_t n, int32_t k, int32_t m) {
  return moat_int4_gemm_ex_workspace_size(n, k, m, nullptr);
}

int32_t moat_int4_gemm_ex(const uint16_t* x_f16, const uint8_t* superblocks, float* y_f32, int32_t n, int32_t k,
                          int32_t m, const moat_int4_gemm_options* options, void* workspace, int64_t workspace_bytes,
                          hipStream_t stream) {
  return gemm_call(x_f16, superblocks, y_f32, n, k, m, options, workspace, workspace_bytes, 0, stream);
}

int32_t moat_int4_gemm_tiles(const uint16_t* x_f16, const uint8_t* tiles, float* y_f32, int32_t n, int32_t k,
                             int32_t m, const moat_int4_gemm_options* options, void* workspace,
                             int64_t workspace_bytes, hipStream_t stream) {
  return gemm_call(x_f16, tiles, y_f32, n, k, m, options, workspace, workspace_bytes, 1, stream);
}

int32_t moat_int4_records_to_strips(const uint8_t* superblocks, int32_t k, int32_t m, uint8_t* strips,
                                    hipStream_t stream) {
  if (k < 8 || (k % 8) != 0 || m < 32 || (m % 32) != 0) return MOAT_ERR_INVALID;
  if ((int64_t)k * (m / 32) > ((int64_t)1 << 40)) return MOAT_ERR_INVALID;
  if (!superblocks || !strips || !aligned(superblocks, 16) || !aligned(strips, 16)) return MOAT_ERR_INVALID;
  const int64_t bytes = (int64_t)k * m / 256 * 144;
  const uintptr_t a = reinterpret_cast<uintptr_t>(superblocks), b = reinterpret_cast<uintptr_t>(strips);
  if (a < b + (uintptr_t)bytes && b < a + (uintptr_t)bytes) return MOAT_ERR_INVALID;  // the copies overlap
  return status_of(moat::launch_records_to_strips(superblocks, k, m, strips, stream));
}

int32_t moat_int4_strips_to_records(const uint8_t* strips, int32_t k, int32_t m, uint8_t* superblocks,
                                    hipStream_t stream) {
  if (k < 8 || (k % 8) != 0 || m < 32 || (m % 32) != 0) return MOAT_ERR_INVALID;
  if ((int64_t)k * (m / 32) > ((int64_t)1 << 40)) return MOAT_ERR_INVALID;
  if (!superblocks || !strips || !aligned(superblocks, 16) || !aligned(strips, 16)) return MOAT_ERR_INVALID;
  const int64_t bytes = (int64_t)k * m / 256 * 144;
  const uintptr_t a = reinterpret_cast<uintptr_t>(superblocks), b = reinterpret_cast<uintptr_t>(strips);
  if (a < b + (uintptr_t)bytes && b < a + (uintptr_t)bytes) return MOAT_ERR_INVALID;  // the copies overlap
  return status_of(moat::launch_strips_to_records(strips, k, m, superblocks, stream));
}

int64_t moat_int4_gemm_strips_workspace_size(int32_t n, int32_t k, int32_t m,
                                             const moat_int4_gemm_options* options) {
  if (!strips_shape_ok(n, k, m) || !strip_options_ok(options) || (options && options->algo == MOAT_GEMM_DOT2 && n > 4))
    return -1;
  return plan_strips(n, k, m, options).workspace_bytes;
}

int32_t moat_int4_gemm_strips(const uint16_t* x_f16, const uint8_t* strips, float* y_f32, int32_t n, int32_t k,
                              int32_t m, const moat_int4_gemm_options* options, void* workspace,
                              int64_t workspace_bytes, hipStream_t stream) {
  if (!strips_shape_ok(n, k, m) || !strip_options_ok(options) || (options && options->algo == MOAT_GEMM_DOT2 && n > 4))
    return MOAT_ERR_INVALID;
  if (!x_f16 || !strips || !y_f32 || !aligned(x_f16, 16) || !aligned(strips, 16) || !aligned(y_f32, 4))
    return MOAT_ERR_INVALID;
  const StripPlan p = plan_strips(n, k, m, options);
  float* slots = nullptr;
  uint32_t* status = nullptr;
  if (p.workspace_bytes > 0) {
    if (!workspace || workspace_bytes < p.workspace_bytes || !aligned(workspace, 16)) return MOAT_ERR_WORKSPACE;
    status = static_cast<uint32_t*>(workspace);
    slots = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kCounterBlockBytes);
  }
  if (p.kind == kStripGroups)
    return status_of(moat::launch_gemm_strip_groups(x_f16, strips, y_f32, n, k, m, p.wgs, p.depth, slots, status,
                                                    stream));
  if (p.kind == kStripWide)
    return status_of(moat::launch_gemm_strips_wide(x_f16, strips, y_f32, n, k, m, p.wgs, p.su, p.depth, slots, status,
                                                   stream));
  // 8 rows of X per launch; the launches share the workspace in stream order
  for (int32_t r0 = 0; r0 < n; r0 += kStripRowsPerLaunch) {
    const int32_t rows = n - r0 < kStripRowsPerLaunch ? n - r0 : kStripRowsPerLaunch;
    const hipError_t e = moat::launch_gemm_strips(x_f16 + (int64_t)r0 * k, strips, y_f32 + (int64_t)r0 * m, rows,
                                                  k, m, p.wgs, p.depth, p.waves, p.dot, slots, status, stream);
    if (e != hipSuccess) return MOAT_ERR_HIP;
  }
  return MOAT_OK;
}

int32_t moat_int4_interleave_strips(const uint8_t* gate_strips, const uint8_t* up_strips, int32_t k, int32_t m,
                                    uint8_t* gate_up_strips, hipStream_t stream) {
  if (k < 8 || (k % 8) != 0 || m < 32 || (m % 32) != 0) return MOAT_ERR_INVALID;
  if ((int64_t)k * (m / 32) > ((int64_t)1 << 40)) return MOAT_ERR_INVALID;
  if (!gate_strips || !up_strips || !gate_up_strips) return MOAT_ERR_INVALID;
  const int64_t strip_bytes = (int64_t)k * 18;  // 32 columns of k rows: k / 8 records
  const int64_t bytes = strip_bytes * (m / 32);
  const uintptr_t o = reinterpret_cast<uintptr_t>(gate_up_strips);
  const uintptr_t g = reinterpret_cast<uintptr_t>(gate_strips), u = reinterpret_cast<uintptr_t>(up_strips);
  if ((g < o + (uintptr_t)(2 * bytes) && o < g + (uintptr_t)bytes) || (u < o + (uintptr_t)(2 * bytes) && o < u + (uintptr_t)bytes))
    return MOAT_ERR_INVALID;  // the output overlaps an input
  // strip c of gate -> strip 2c, strip c of up -> strip 2c + 1: two strided copies
  hipError_t e = hipMemcpy2DAsync(gate_up_strips, (size_t)(2 * strip_bytes), gate_strips, (size_t)strip_bytes,
                                  (size_t)strip_bytes, (size_t)(m / 32), hipMemcpyDeviceToDevice, stream);
  if (e == hipSuccess)
    e = hipMemcpy2DAsync(gate_up_strips + strip_bytes, (size_t)(2 * strip_bytes), up_strips, (size_t)strip_bytes,
                         (size_t)strip_bytes, (size_t)(m / 32), hipMemcpyDeviceToDevice, stream);
  return status_of(e);
}

int32_t moat_int4_gemm_strips_swiglu(const uint16_t* x_f16, const uint8_t* gate_up_strips, uint16_t* h_f16, int32_t n,
                                     int32_t k, int32_t m, const moat_int4_gemm_options* options, hipStream_t stream) {
  if (m < 32 || (m % 32) != 0 || m > (1 << 29) || !strips_shape_ok(n, k, 2 * m) || !strip_options_ok(options))
    return MOAT_ERR_INVALID;
  if (!x_f16 || !gate_up_strips || !h_f16 || !aligned(x_f16, 16) || !aligned(gate_up_strips, 16) ||
      !aligned(h_f16, 8))
    return MOAT_ERR_INVALID;
  // whole gate/up pairs per workgroup (nothing is handed between workgroups)
  const int64_t pairs = m / 32;
  int64_t want = options && options->splits > 0 ? options->splits : kStripMaxWorkgroups;
  if (want > kStripMaxWorkgroups) want = kStripMaxWorkgroups;
  const int64_t per = (pairs + want - 1) / want;
  const int64_t wgs = (pairs + per - 1) / per;
  return status_of(
      moat::launch_gemm_strips_swiglu(x_f16, gate_up_strips, h_f16, n, k, m, (int)wgs, (int)per, stream));
}

int32_t moat_int4_records_to_tiles(const uint8_t* superblocks, int32_t k, int32_t m, uint8_t* tiles,
                                   hipStream_t stream) {
  if (k < 1 || m < 256 || (m % 256) != 0) return MOAT_ERR_INVALID;
  if ((int64_t)k * (m / 256) > ((int64_t)1 << 40)) return MOAT_ERR_INVALID;
  if (!superblocks || !tiles || !aligned(superblocks, 16) || !aligned(tiles, 16)) return MOAT_ERR_INVALID;
  const int64_t bytes = (int64_t)k * (m / 256) * 144;
  const uintptr_t a = reinterpret_cast<uintptr_t>(superblocks), b = reinterpret_cast<uintptr_t>(tiles);
  if (a < b + (uintptr_t)bytes && b < a + (uintptr_t)bytes) return MOAT_ERR_INVALID;  // the copies overlap
  return status_of(moat::launch_records_to_tiles(superblocks, k, m, tiles, stream));
}

int32_t moat_int4_gemm(const uint16_t* x_f16, const uint8_t* superblocks, float* y_f32, int32_t n, int32_t k,
                       int32_t m, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  return moat_int4_gemm_ex(x_f16, superblocks, y_f32, n, k, m, nullptr, workspace, workspace_bytes, stream);
}

int32_t moat_int4_gemm_noalloc(const uint16_t* x_f16, const uint8_t* superblocks, float* y_f32, int32_t n, int32_t k,
                               int32_t m, hipStream_t stream) {
  const moat_int4_gemm_options opt = {0, 0, 0, MOAT_FINISH_SECOND_KERNEL, 0, 0, 0};
  return gemm_call(x_f16, superblocks, y_f32, n, k, m, &opt, nullptr, 0, 0, stream, true);
}

int64_t moat_int4_gemm_multi_workspace_size(int32_t count, int32_t n, int32_t k, int32_t m) {
  if (!fused_shape_ok(count, n, k, m)) return -1;
  return plan_fused(kFusedMulti, count, n, k, m).workspace_bytes;
}

int32_t moat_int4_gemm_multi(const uint16_t* x_f16, const uint8_t* const* superblocks, float* const* y_f32,
                             int32_t count, int32_t n, int32_t k, int32_t m, void* workspace, int64_t workspace_bytes,
                             hipStream_t stream) {
  if (!fused_shape_ok(count, n, k, m) || !x_f16 || !superblocks || !y_f32 || !aligned(x_f16, 16))
    return MOAT_ERR_INVALID;
  for (int i = 0; i < count; ++i) {
    if (!superblocks[i] || !y_f32[i] || !aligned(superblocks[i], 16) || !aligned(y_f32[i], 4)) return MOAT_ERR_INVALID;
  }
  return run_fused(kFusedMulti, x_f16, superblocks, y_f32, nullptr, count, n, k, m, workspace, workspace_bytes,
                   stream);
}

int64_t moat_int4_gemm_swiglu_workspace_size(int32_t n, int32_t k, int32_t m) {
  if (!fused_shape_ok(2, n, k, m)) return -1;
  return plan_fused(kFusedSwiglu, 2, n, k, m).workspace_bytes;
}

int32_t moat_int4_gemm_swiglu(const uint16_t* x_f16, const uint8_t* gate_superblocks, const uint8_t* up_superblocks,
                              uint16_t* h_f16, int32_t n, int32_t k, int32_t m, void* workspace,
                              int64_t workspace_bytes, hipStream_t stream) {
  if (!fused_shape_ok(2, n, k, m) || !x_f16 || !gate_superblocks || !up_superblocks || !h_f16) return MOAT_ERR_INVALID;
  if (!aligned(x_f16, 16) || !aligned(gate_superblocks, 16) || !aligned(up_superblocks, 16) || !aligned(h_f16, 8))
    return MOAT_ERR_INVALID;
  const uint8_t* sbs[2] = {gate_superblocks, up_superblocks};
  return run_fused(kFusedSwiglu, x_f16, sbs, nullptr, h_f16, 2, n, k, m, workspace, workspace_bytes, stream);
}

int32_t moat_int4_stream_read(const void* src, int64_t bytes, int32_t workgroups, uint32_t* sink,
                              hipStream_t stream) {
  if (bytes < 0 || (bytes % 16) != 0 || workgroups < 0) return MOAT_ERR_INVALID;
  if (bytes == 0) return MOAT_OK;
  if (!src || !sink || !aligned(src, 16) || !aligned(sink, 4)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_stream_read(src, bytes, sink, workgroups, stream));
}

int32_t moat_int4_workspace_status(const void* workspace, int64_t workspace_bytes, int32_t* status_out,
                                   hipStream_t stream) {
  if (!status_out || !workspace || workspace_bytes < moat::kWsStatusBytes || !aligned(workspace, 4))
    return MOAT_ERR_INVALID;
  uint32_t word = 0;
  hipError_t e = hipMemcpyAsync(&word, workspace, sizeof(word), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return MOAT_ERR_HIP;
  *status_out = (int32_t)word;
  return MOAT_OK;
}

int32_t moat_int4_workspace_clear(void* workspace, int64_t bytes, hipStream_t stream) {
  if (bytes < 0) return MOAT_ERR_INVALID;
  if (bytes == 0) return MOAT_OK;
  if (!workspace) return MOAT_ERR_INVALID;
  return status_of(moat::launch_clear(workspace, bytes, stream));
}

int32_t moat_int4_quantize(const void* w, int32_t w_dtype, int64_t n, int32_t group_size, int32_t scale_mode,
                           int8_t* q_out, uint16_t* scales_out, hipStream_t stream) {
  if (n < 0 || group_size < 1 || (n % group_size) != 0) return MOAT_ERR_INVALID;
  if (w_dtype != MOAT_DTYPE_F32 && w_dtype != MOAT_DTYPE_F16 && w_dtype != MOAT_DTYPE_F64) return MOAT_ERR_INVALID;
  if (scale_mode != MOAT_SCALE_F32 && scale_mode != MOAT_SCALE_F16) return MOAT_ERR_INVALID;
  if (n == 0) return MOAT_OK;
  if (!w || !q_out || !scales_out) return MOAT_ERR_INVALID;
  const uintptr_t wa = w_dtype == MOAT_DTYPE_F64 ? 8 : (w_dtype == MOAT_DTYPE_F32 ? 4 : 2);
  if (!aligned(w, wa) || !aligned(scales_out, 2)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_quantize(w, w_dtype, n, group_size, scale_mode, q_out, scales_out, stream));
}

int32_t moat_int4_pack_superblocks(const int8_t* q, const uint16_t* scales_f16, int64_t n_superblocks,
                                   uint8_t* superblocks_out, hipStream_t stream) {
  if (n_superblocks < 0) return MOAT_ERR_INVALID;
  if (n_superblocks == 0) return MOAT_OK;
  if (!q || !scales_f16 || !superblocks_out) return MOAT_ERR_INVALID;
  if (!aligned(scales_f16, 2) || !aligned(superblocks_out, 16)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_pack_superblocks(q, scales_f16, n_superblocks, superblocks_out, stream));
}

int32_t moat_int4_quantize_pack(const void* w, int32_t w_dtype, int64_t n, int32_t scale_mode,
                                uint8_t* superblocks_out, hipStream_t stream) {
  if (n < 0 || (n % 256) != 0) return MOAT_ERR_INVALID;
  if (w_dtype != MOAT_DTYPE_F32 && w_dtype != MOAT_DTYPE_F16 && w_dtype != MOAT_DTYPE_F64) return MOAT_ERR_INVALID;
  if (scale_mode != MOAT_SCALE_F32 && scale_mode != MOAT_SCALE_F16) return MOAT_ERR_INVALID;
  if (n == 0) return MOAT_OK;
  if (!w || !superblocks_out || !aligned(superblocks_out, 16)) return MOAT_ERR_INVALID;
  const uintptr_t wa = w_dtype == MOAT_DTYPE_F64 ? 8 : (w_dtype == MOAT_DTYPE_F32 ? 4 : 2);
  if (!aligned(w, wa)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_quantize_pack(w, w_dtype, n, scale_mode, superblocks_out, stream));
}

int32_t moat_int4_pack_nibbles(const int8_t* q, int64_t n, uint8_t* packed_out, hipStream_t stream) {
  if (n < 0 || (n % 2) != 0) return MOAT_ERR_INVALID;
  if (n == 0) return MOAT_OK;
  if (!q || !packed_out) return MOAT_ERR_INVALID;
  return status_of(moat::launch_pack_nibbles(q, n, packed_out, stream));
}

int32_t moat_int4_unpack_nibbles(const uint8_t* packed, int64_t n_bytes, int8_t* q_out, hipStream_t stream) {
  if (n_bytes < 0) return MOAT_ERR_INVALID;
  if (n_bytes == 0) return MOAT_OK;
  if (!packed || !q_out) return MOAT_ERR_INVALID;
  return status_of(moat::launch_unpack_nibbles(packed, n_bytes, q_out, stream));
}

int32_t moat_int4_group_dequant(const void* q, int32_t q_dtype, const void* scales, int32_t scale_dtype,
                                int64_t n_groups, int32_t group_size, int32_t table_mode, uint16_t* out_f16,
                                int32_t* err_flag, hipStream_t stream) {
  if (n_groups < 0 || group_size < 1 || (table_mode != 0 && table_mode != 1)) return MOAT_ERR_INVALID;
  if (q_dtype != MOAT_DTYPE_I8 && q_dtype != MOAT_DTYPE_I64 && q_dtype != MOAT_DTYPE_F32) return MOAT_ERR_INVALID;
  if (table_mode == 1 && q_dtype == MOAT_DTYPE_F32) return MOAT_ERR_INVALID;
  if (scale_dtype != MOAT_DTYPE_F16 && scale_dtype != MOAT_DTYPE_F32 && scale_dtype != MOAT_DTYPE_F64)
    return MOAT_ERR_INVALID;
  if (n_groups == 0) return MOAT_OK;
  if (!q || !scales || !out_f16 || (table_mode == 1 && !err_flag)) return MOAT_ERR_INVALID;
  const uintptr_t qa = q_dtype == MOAT_DTYPE_I64 ? 8 : (q_dtype == MOAT_DTYPE_F32 ? 4 : 1);
  const uintptr_t sa = scale_dtype == MOAT_DTYPE_F64 ? 8 : (scale_dtype == MOAT_DTYPE_F32 ? 4 : 2);
  if (!aligned(q, qa) || !aligned(scales, sa) || !aligned(out_f16, 2)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_group_dequant(q, q_dtype, scales, scale_dtype, n_groups, group_size, table_mode,
                                              out_f16, err_flag, stream));
}

int32_t moat_int4_lut_gather(const int64_t* q, int64_t n, int32_t index_mode, const uint16_t* lut_f16,
                             int64_t lut_rows, int32_t lut_len, uint16_t* out_f16, hipStream_t stream) {
  if (n < 0 || index_mode < 0 || index_mode > 2 || lut_rows < 1 || lut_len < 1) return MOAT_ERR_INVALID;
  if ((n % lut_rows) != 0) return MOAT_ERR_INVALID;
  if (n == 0) return MOAT_OK;
  if (!q || !lut_f16 || !out_f16 || !aligned(q, 8) || !aligned(lut_f16, 2) || !aligned(out_f16, 2))
    return MOAT_ERR_INVALID;
  return status_of(moat::launch_lut_gather(q, n, index_mode, lut_f16, lut_rows, lut_len, out_f16, stream));
}

int32_t moat_int4_any_negative(const int64_t* q, int64_t n, int32_t* flag_out, hipStream_t stream) {
  if (n < 0 || !flag_out || !aligned(flag_out, 4)) return MOAT_ERR_INVALID;
  if (n > 0 && (!q || !aligned(q, 8))) return MOAT_ERR_INVALID;
  return status_of(moat::launch_any_negative(q, n, flag_out, stream));
}

int32_t moat_int4_to_f16(const void* src, int32_t src_dtype, int64_t n, uint16_t* out_f16, hipStream_t stream) {
  if (n < 0 || (src_dtype != MOAT_DTYPE_F32 && src_dtype != MOAT_DTYPE_F64)) return MOAT_ERR_INVALID;
  if (n == 0) return MOAT_OK;
  if (!src || !out_f16) return MOAT_ERR_INVALID;
  if (!aligned(src, src_dtype == MOAT_DTYPE_F64 ? 8 : 4) || !aligned(out_f16, 2)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_to_f16(src, src_dtype, n, out_f16, stream));
}

int32_t moat_int4_swiglu_f32(const float* gu_f32, int32_t n, int32_t m, int64_t ld, uint16_t* h_f16,
                             hipStream_t stream) {
  if (n < 0 || m < 0 || (m % 4) != 0 || ld < 2 * (int64_t)m || (ld % 4) != 0) return MOAT_ERR_INVALID;
  if (n == 0 || m == 0) return MOAT_OK;
  if (!gu_f32 || !h_f16 || !aligned(gu_f32, 16) || !aligned(h_f16, 8)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_swiglu_f32(gu_f32, n, m, ld, h_f16, stream));
}

int32_t moat_int4_i8_div_to_f16(const int8_t* q, int64_t n, float divisor, uint16_t* out_f16, hipStream_t stream) {
  if (n < 0 || !(divisor == divisor) || divisor == 0.0f) return MOAT_ERR_INVALID;
  if (n == 0) return MOAT_OK;
  if (!q || !out_f16 || !aligned(out_f16, 2)) return MOAT_ERR_INVALID;
  return status_of(moat::launch_i8_div_to_f16(q, n, divisor, out_f16, stream));
}

// ---- token sampling ----

int64_t moat_sample_workspace_size(int32_t n, int32_t v) {
  return sample_sizes_ok(n, v) ? moat::sample_workspace_bytes(n, v, true) : -1;
}

int64_t moat_lut_softmax_workspace_size(int32_t n, int32_t v) {
  return sample_sizes_ok(n, v) ? moat::sample_workspace_bytes(n, v, false) : -1;
}

int32_t moat_lut_softmax(const void* x, int32_t dtype, int32_t n, int32_t v, const uint16_t* lut_f16,
                         int32_t lut_size, float step, uint16_t* probs_f16, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream) {
  if (!sample_args_ok(x, dtype, n, v, lut_f16, lut_size, step)) return MOAT_ERR_INVALID;
  if (n > 0 && (!probs_f16 || !aligned(probs_f16, 2))) return MOAT_ERR_INVALID;
  if (!sample_ws_ok(n, v, false, workspace, workspace_bytes)) return MOAT_ERR_WORKSPACE;
  return status_of(moat::launch_lut_sample(x, sample_dtype(dtype), n, v, 1.0, 0, lut_f16, lut_size, step, 0, 1, 0,
                                           nullptr, nullptr, probs_f16, workspace, stream));
}

int32_t moat_sample_tokens(const void* logits, int32_t dtype, int32_t n, int32_t v, double temperature,
                           int32_t top_k, uint64_t seed, const uint16_t* lut_f16, int32_t lut_size, float step,
                           int32_t* tokens, float* logprobs, void* workspace, int64_t workspace_bytes,
                           hipStream_t stream) {
  if (!sample_args_ok(logits, dtype, n, v, lut_f16, lut_size, step)) return MOAT_ERR_INVALID;
  if (!(temperature == temperature) || top_k < 1 || top_k > 64) return MOAT_ERR_INVALID;
  if (n > 0 && (!tokens || !logprobs || !aligned(tokens, 4) || !aligned(logprobs, 4))) return MOAT_ERR_INVALID;
  if (!sample_ws_ok(n, v, true, workspace, workspace_bytes)) return MOAT_ERR_WORKSPACE;
  const bool greedy = temperature <= 0.0;
  // logits / max(T, 1e-5) with T rounded to the logits' dtype first (numpy's
  // array / Python float)
  double t = temperature > 1e-5 ? temperature : 1e-5;
  if (dtype == MOAT_DTYPE_F32) t = (double)(float)t;
  if (dtype == MOAT_DTYPE_F16) t = (double)(_Float16)t;
  return status_of(moat::launch_lut_sample(logits, sample_dtype(dtype), n, v, t, greedy ? 0 : 1, lut_f16, lut_size,
                                           step, greedy ? 1 : 2, top_k, seed, tokens, logprobs, nullptr, workspace,
                                           stream));
}

int32_t moat_lut_lookup(const float* x, int64_t n, const uint16_t* lut_f16, int32_t lut_size, float step,
                        uint16_t* out_f16, hipStream_t stream) {
  if (n < 0 || lut_size < 2 || !(step > 0.f) || step == INFINITY) return MOAT_ERR_INVALID;
  if (n == 0) return MOAT_OK;
  if (!x || !lut_f16 || !out_f16 || !aligned(x, 4) || !aligned(lut_f16, 2) || !aligned(out_f16, 2))
    return MOAT_ERR_INVALID;
  return status_of(moat::launch_lut_lookup(x, n, lut_f16, lut_size, step, out_f16, stream));
}

int64_t moat_dense_gemm_workspace_size(int32_t n, int32_t k, int32_t m, int32_t splits) {
  if (!dense_shape_ok(n, k, m, splits)) return -1;
  return dense_workspace_bytes(n, k, m, splits);
}

int32_t moat_dense_gemm(const uint16_t* x_f16, const uint16_t* w_f16, uint16_t* y_f16, int32_t n, int32_t k,
                             int32_t m, int32_t splits, void* workspace, int64_t workspace_bytes,
                             hipStream_t stream) {
  if (!dense_shape_ok(n, k, m, splits)) return MOAT_ERR_INVALID;
  if (!x_f16 || !w_f16 || !y_f16 || !aligned(x_f16, 16) || !aligned(w_f16, 16) || !aligned(y_f16, 2))
    return MOAT_ERR_INVALID;
  const int64_t y_bytes = (int64_t)n * m * 2;
  if (spans_overlap(y_f16, y_bytes, x_f16, (int64_t)n * k * 2) ||
      spans_overlap(y_f16, y_bytes, w_f16, (int64_t)k * m * 2))
    return MOAT_ERR_INVALID;  // the output overlaps an input
  const int64_t need = dense_workspace_bytes(n, k, m, splits);
  uint32_t* counters = nullptr;
  float* slots = nullptr;
  if (need > 0) {
    if (!workspace || workspace_bytes < need || !aligned(workspace, 16)) return MOAT_ERR_WORKSPACE;
    counters = static_cast<uint32_t*>(workspace);
    slots = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + moat::dense_counter_bytes());
  }
  // 32 rows of X a launch; the launches share the workspace in stream order
  for (int32_t r0 = 0; r0 < n; r0 += kDenseRowsPerLaunch) {
    const int32_t rows = n - r0 < kDenseRowsPerLaunch ? n - r0 : kDenseRowsPerLaunch;
    const hipError_t e = moat::launch_dense_gemm(x_f16 + (int64_t)r0 * k, w_f16, y_f16 + (int64_t)r0 * m, rows, k, m,
                                                 splits, slots, counters, stream);
    if (e != hipSuccess) return MOAT_ERR_HIP;
  }
  return MOAT_OK;
}

}  // extern "C"
