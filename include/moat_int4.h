/*
 * moat_int4.h -- C ABI of libmoat_int4.so, the MI355X (gfx950) implementation
 * of moat's INT4 superblock path.
 *
 * Data format: a weight matrix W[K][M] (row-major, flat index k*M + m) is a
 * stream of 144-byte superblocks, one per 256 consecutive flat elements:
 * bytes [0,16) hold 8 little-endian fp16 scales (group g = elements 32g..32g+31),
 * bytes [16,144) hold nibble pairs, element 2j in the LOW nibble of byte j and
 * element 2j+1 in the HIGH nibble, each stored as q+8 in [0,15]
 * (antigravity-engine/src/shaders/batched_gemm.metal:16-20, 146-154;
 * src/dequant.py:116-147).  A dequantized element is fp16(f32(q) * f32(scale)).
 *
 * Conventions (after antigravity-engine/src/antigravity_c_api.h:15-17, 129, 161):
 *  - extern "C", plain pointers and sizes; every pointer is a DEVICE pointer
 *    owned by the caller (no allocation inside any entry point);
 *  - int32 status: 0 = ok, negative = error (see MOAT_ERR_*); arguments are
 *    validated BEFORE any HIP call, so a bad call has no side effect;
 *  - work is enqueued on `stream` and returns without synchronising;
 *  - no mutable globals: calls on distinct streams with distinct output and
 *    workspace buffers may run concurrently.
 *
 * The reference has no C ABI for this path (its hot path is the numpy module
 * src/dequant.py and the Metal kernels in batched_gemm.metal); each entry
 * point names the reference function or kernel whose result it reproduces.
 */
#ifndef MOAT_INT4_H
#define MOAT_INT4_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOAT_INT4_VERSION_MAJOR 0
#define MOAT_INT4_VERSION_MINOR 1

/* status codes */
#define MOAT_OK 0
#define MOAT_ERR_INVALID (-2)     /* bad shape, size, pointer or alignment */
#define MOAT_ERR_HIP (-3)         /* a HIP runtime call or kernel launch failed */
#define MOAT_ERR_WORKSPACE (-4)   /* workspace missing or too small */
#define MOAT_ERR_TOO_LARGE (-5)   /* moat_int4_gemm_noalloc: the plan needs more scratch than it holds */

/* element types for the typed entry points */
#define MOAT_DTYPE_F32 0
#define MOAT_DTYPE_F16 1
#define MOAT_DTYPE_I8 2
#define MOAT_DTYPE_F64 3
#define MOAT_DTYPE_I64 4

/* quantizer scale rules */
#define MOAT_SCALE_F32 0 /* divide by the float32 scale: src/dequant.py:47-53 */
#define MOAT_SCALE_F16 1 /* divide by the fp16-rounded scale: antigravity-engine/src/dequant.py:56-58 */

/* GEMM kernel choice */
#define MOAT_GEMM_AUTO 0
#define MOAT_GEMM_DOT2 1 /* VALU: v_dot2_f32_f16 with a wavefront reduction */
#define MOAT_GEMM_MFMA 2 /* matrix cores: v_mfma_f32_16x16x32_f16 */

/* MAJOR*100 + MINOR */
int32_t moat_int4_version(void);

/* Static text for a status code. */
const char* moat_int4_status_string(int32_t status);

/*
 * Decode n_superblocks 144-byte records into fp16 (n_superblocks*256 values,
 * flat order).  Bit-exact with src/dequant.py:116-147
 * (unpack_superblock_weights) and antigravity-engine/src/shaders/batched_gemm.metal:41-66
 * (dequantize_superblocks_kernel).  superblocks and out: 16-byte aligned.
 */
int32_t moat_int4_dequant(const uint8_t* superblocks, int64_t n_superblocks,
                          uint16_t* out_f16, hipStream_t stream);

/*
 * Y[n][M] (fp32) = X[n][K] (fp16) @ deq(W)[K][M], the batched decode
 * projection for n = 1..32 parallel traces.  Semantics: the reference CPU
 * path, dequantize (src/dequant.py:116-147) then float32 matmul
 * (antigravity-engine/tests/test_batched_speed.py:39-42); replaces the fused
 * kernel antigravity-engine/src/shaders/batched_gemm.metal:116-169.
 * Preconditions: 1 <= n <= 32, k >= 1, m >= 32, m % 32 == 0, (k*m) % 256 == 0;
 * x 2-byte aligned, superblocks 16-byte aligned, y 4-byte aligned.  The
 * record-stream kernel reads X 16 bytes at a time; when x is not 16-byte
 * aligned (or k % 8 != 0) the call plans the general kernel instead, and the
 * size query covers both plans.
 * workspace: device memory of moat_int4_gemm_workspace_size() bytes (may be
 * NULL when that size is 0): a fixed 64 KB block (a sticky status word, then
 * split-K counters) followed by fp32 partials.  Zero-fill it once before
 * first use (e.g. with moat_int4_workspace_clear); every call leaves all of
 * it at zero again (the record-stream kernel's in-kernel hand-off reads a
 * zero word as "partial not written yet"), so one workspace serves calls of
 * any shape.  Calls that share a workspace must not overlap.  m is limited to
 * 2,088,960.
 *
 * The in-kernel hand-off waits a bounded time (about a second) for another
 * workgroup's partial.  Should that ever run out (it needs the other
 * workgroup to be held back from running, e.g. by other work filling the
 * GPU), the call's affected results are NaN and the status word records it
 * (moat_int4_workspace_status); every later call on that workspace then
 * writes NaN instead of results until the workspace is cleared, because a
 * partial stored after the wait ended may still sit in it.
 */
int64_t moat_int4_gemm_workspace_size(int32_t n, int32_t k, int32_t m);
int32_t moat_int4_gemm(const uint16_t* x_f16, const uint8_t* superblocks, float* y_f32,
                       int32_t n, int32_t k, int32_t m,
                       void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * moat_int4_gemm without a workspace: the same product, plan and kernels,
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Split-K partials go to a 16 MB scratch
 * array inside the library, one per GPU, held until the process ends (its
 * address is looked up on the first call on each device); they are always
 * summed by the fix-up kernel, so nothing in the scratch must start at zero.
 * A call whose plan needs more than 16 MB (the general kernel's plan for
 * very wide outputs) returns MOAT_ERR_TOO_LARGE; use moat_int4_gemm with a
 * workspace instead.  Calls on one GPU share that scratch: calls that overlap
 * in time on one GPU (different streams, concurrent graphs) race and must
 * not be issued; calls in order on one stream are fine.  Allocates nothing.
 */
int32_t moat_int4_gemm_noalloc(const uint16_t* x_f16, const uint8_t* superblocks, float* y_f32,
                               int32_t n, int32_t k, int32_t m, hipStream_t stream);

/* Launch choices for moat_int4_gemm_ex; zero-initialise for "automatic". */
typedef struct moat_int4_gemm_options {
  int32_t algo;   /* MOAT_GEMM_*: 0 automatic, 1 dot2 (n <= 8), 2 MFMA */
  int32_t splits; /* K slices per column tile, >= 1; 0 automatic (record-stream kernel: workgroups
                     per tile group, each taking an equal run of (tile group, round) items) */
  int32_t batch;  /* 32-row rounds a wave has in flight (general kernel: 1, 2 or 4 issued
                     together; record-stream kernel: ring depth 1..5); 0 automatic */
  int32_t finish; /* split-K hand-off, MOAT_FINISH_*; 0 automatic */
  int32_t front;  /* weight loads, MOAT_FRONT_*; 0 automatic */
  int32_t group;  /* record-stream kernel: adjacent 256-column tiles per workgroup, 1, 2 or 4
                     (the workgroup's waves split waves / group ways over K); 0 automatic */
  int32_t waves;  /* record-stream kernel: waves per workgroup, 4 or 8 (8 applies for n <= 16,
                     larger n runs on 4); 0 automatic */
} moat_int4_gemm_options;

#define MOAT_FINISH_AUTO 0
/* General kernel: the last workgroup of a column tile to publish its partial
 * sums the tile (ATOMICS, FENCES: how the partials are published), or a
 * second kernel does.  Record-stream kernel: ATOMICS and FENCES both mean the
 * in-kernel hand-off (the workgroup holding a tile group's last round adds
 * the others' device-coherent partials), SECOND_KERNEL the fix-up kernel;
 * automatic: second kernel for the general kernel; for the record-stream
 * kernel in-kernel while the owner reads at most 64 KB of partials, else the
 * fix-up kernel. */
#define MOAT_FINISH_DEVICE_ATOMICS 1 /* partials via device-scope atomic stores/loads, one launch */
#define MOAT_FINISH_FENCES 2         /* partials via plain stores + agent-scope fences, one launch */
#define MOAT_FINISH_SECOND_KERNEL 3  /* partials via plain stores, summed by a second kernel */

#define MOAT_FRONT_AUTO 0
#define MOAT_FRONT_LDS 1     /* 16-byte vector loads staged through LDS (m % 64 == 0; otherwise direct) */
#define MOAT_FRONT_DIRECT 2  /* 4-byte loads straight into registers */
#define MOAT_FRONT_LDS_DMA 3 /* global_load_lds staging (m % 64 == 0; otherwise direct) */
#define MOAT_FRONT_RECORDS 4 /* record-stream kernel: whole 144-byte records per row, 256-column tiles,
                                matrix cores (m % 128 == 0, k % 32 == 0, x 16-byte aligned; otherwise
                                the general kernel) -- the automatic choice when the shape allows it */

/* Same product with the launch choices made by the caller (NULL = all
 * automatic): for measurement and for testing each kernel at every n.
 * Workspace size from the _ex query with the same options. */
int64_t moat_int4_gemm_ex_workspace_size(int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* options);
int32_t moat_int4_gemm_ex(const uint16_t* x_f16, const uint8_t* superblocks, float* y_f32,
                          int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* options,
                          void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Tile order: the same 144-byte records of W[K][M] (M % 256 == 0), stored so
 * that each 256-column tile's K rows of records are contiguous (row r of tile
 * j at record j*K + r) instead of row by row (record r*(M/256) + j).  In the
 * row order a tile's rows lie 144*M/256 bytes apart, and a load-only kernel
 * reads that pattern at about 4 TB/s on MI355X; in tile order each 32-row
 * round of a tile is one 4608-byte block and reads like a plain stream
 * (about 5.6 TB/s).  No counterpart in the reference, whose stream is the row
 * order (src/dequant.py:116-147): a storage order a loader chooses once.
 *
 * moat_int4_records_to_tiles: copies a row-order stream to tile order
 * (k >= 1, m % 256 == 0; both 16-byte aligned, not overlapping).
 * moat_int4_gemm_tiles: moat_int4_gemm_ex over a tile-order stream, with the
 * same plan, kernel and result bits; it needs the record-stream kernel
 * (m % 256 == 0, k % 32 == 0, x 16-byte aligned; MOAT_ERR_INVALID
 * otherwise).  Workspace from moat_int4_gemm_ex_workspace_size.
 */
int32_t moat_int4_records_to_tiles(const uint8_t* superblocks, int32_t k, int32_t m, uint8_t* tiles,
                                   hipStream_t stream);
int32_t moat_int4_gemm_tiles(const uint16_t* x_f16, const uint8_t* tiles, float* y_f32,
                             int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* options,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Strip order: a storage order for the same quantized weights that a loader
 * chooses once (no counterpart in the reference, whose stream is the row
 * order of src/dequant.py:116-147).  Strip g = columns 32g .. 32g+31 of W;
 * strips follow each other in column order, and inside strip g record b
 * (144 bytes) holds rows 8b .. 8b+7: bytes [0,16) the 8 fp16 scales of those
 * rows' group g (row order), then for each column pair j = 0..15 eight bytes
 * at 16 + 8j: byte j of the payload of rows 8b+0, 8b+2, 8b+1, 8b+3, 8b+4,
 * 8b+6, 8b+5, 8b+7 (in that order; low nibble column 32g+2j, high nibble
 * 32g+2j+1, each stored as q + 8 as in the row order).  The q values and
 * scales are those of the row-order stream, bit for bit; a strip is one
 * contiguous run of K x 18 bytes, and the GEMM's workgroups each stream one
 * contiguous range of them.
 *
 * moat_int4_records_to_strips: row order -> strip order (k % 8 == 0,
 * m % 32 == 0; both 16-byte aligned, not overlapping).
 * moat_int4_gemm_strips: Y = X @ deq(W) over a strip-order stream, the same
 * product and tolerance as moat_int4_gemm.  Preconditions: 1 <= n <= 32,
 * k >= 2048, k % 32 == 0, m % 32 == 0; x 16-byte aligned, strips 16-byte
 * aligned, y 4-byte aligned (MOAT_ERR_INVALID otherwise).  All N rows run in
 * one launch.  Workspace as for moat_int4_gemm (zeroed once, left zero,
 * shares the status word), sized by moat_int4_gemm_strips_workspace_size;
 * options: `splits` = workgroups (0 automatic), `group` = kernel (0
 * automatic; 1 the strip-group kernel for N > 8; 2 the strip kernel, 8 rows
 * a launch; 3 the wide strip kernel), `algo` = MOAT_GEMM_DOT2 for the
 * strip kernel's vector-ALU variant (v_dot2_f32_f16 and a reduction across
 * lanes; N <= 4, MOAT_ERR_INVALID beyond), `batch` = ring depth of the strip
 * kernel or the wide strip kernel (2..4, as far as the LDS holds it) or the
 * strip-group kernel (2 or 3), 0 automatic, `front` = units a stage of the
 * wide strip kernel (1, 2 or 4, and 8 up to 8 rows; 0 automatic), `waves` = waves per workgroup
 * of the strip kernel (4, 8 or 12; 0 automatic), the rest ignored.
 */
int32_t moat_int4_records_to_strips(const uint8_t* superblocks, int32_t k, int32_t m, uint8_t* strips,
                                    hipStream_t stream);
/* Strip order -> row order (the inverse of moat_int4_records_to_strips; same
 * preconditions).  No counterpart in the reference: it restores the stream a
 * row-order consumer (dequantize, moat_int4_gemm) reads. */
int32_t moat_int4_strips_to_records(const uint8_t* strips, int32_t k, int32_t m, uint8_t* superblocks,
                                    hipStream_t stream);
int64_t moat_int4_gemm_strips_workspace_size(int32_t n, int32_t k, int32_t m,
                                             const moat_int4_gemm_options* options);
int32_t moat_int4_gemm_strips(const uint16_t* x_f16, const uint8_t* strips, float* y_f32,
                              int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* options,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * The gate and up projections of a SwiGLU MLP with the activation, over
 * strip order: h[n][m] (fp16) = fp16(silu(g) * u), g = f32(x) @
 * f32(deq(W_gate)), u = f32(x) @ f32(deq(W_up)), silu(g) = g / (1 + exp(-g))
 * in fp32 (moat_int4_gemm_swiglu's arithmetic, fp32 g and u).  Replaces the
 * two dispatchGEMM calls and silu_elementwise_mul_kernel of
 * antigravity-engine/src/transformer_engine.mm:694-713
 * (antigravity-engine/src/shaders/transformer_ops.metal:216-232) in one
 * launch.  `gate_up_strips`: both k x m matrices in strip order with their
 * strips interleaved (strip 2c = strip c of W_gate, 2c + 1 = strip c of
 * W_up), as moat_int4_interleave_strips writes it; each workgroup holds
 * whole gate/up pairs and writes h for their 32 columns, so no workspace.
 * Preconditions: 1 <= n <= 32, k >= 2048, k % 32 == 0, m % 32 == 0 (and 2m
 * columns within moat_int4_gemm_strips' limits); x 16-byte aligned,
 * gate_up_strips 16-byte aligned, h 8-byte aligned (MOAT_ERR_INVALID
 * otherwise); options: `splits` = workgroups (0: up to 256), the rest
 * ignored.
 */
int32_t moat_int4_gemm_strips_swiglu(const uint16_t* x_f16, const uint8_t* gate_up_strips, uint16_t* h_f16,
                                     int32_t n, int32_t k, int32_t m, const moat_int4_gemm_options* options,
                                     hipStream_t stream);
/* Interleave two strip-order streams of k x m matrices (moat_int4_records_to_strips
 * output): strip c of gate_strips -> strip 2c, strip c of up_strips -> strip
 * 2c + 1 of gate_up_strips (2 x k x m x 9 / 16 bytes, not overlapping the
 * inputs).  k % 8 == 0, m % 32 == 0.  No counterpart in the reference: the
 * load-time layout of moat_int4_gemm_strips_swiglu's weights. */
int32_t moat_int4_interleave_strips(const uint8_t* gate_strips, const uint8_t* up_strips, int32_t k, int32_t m,
                                    uint8_t* gate_up_strips, hipStream_t stream);

/* Zero `bytes` bytes of device memory with a kernel (no memset node). */
int32_t moat_int4_workspace_clear(void* workspace, int64_t bytes, hipStream_t stream);

/*
 * The sticky status word of a GEMM workspace (workspace_bytes >= 256):
 * *status_out = 0 when every call since the last clear completed its
 * hand-offs, else MOAT_WS_HANDOFF_TIMEOUT (see moat_int4_gemm); recovery is
 * moat_int4_workspace_clear over the whole workspace.  Copies the word to the
 * host after the work queued on `stream` and waits for it (a synchronising
 * call).  No counterpart in the reference, whose CPU path has no hand-off.
 */
#define MOAT_WS_HANDOFF_TIMEOUT 1
int32_t moat_int4_workspace_status(const void* workspace, int64_t workspace_bytes, int32_t* status_out,
                                   hipStream_t stream);

/*
 * A plain streaming read of `bytes` bytes (16-byte aligned, a multiple of
 * 16) with 16-byte loads over `workgroups` workgroups of 256 threads (0:
 * 2048): the read-bandwidth floor against which the GEMM's weight stream is
 * measured.  Nothing is written (`sink`, one device word, is a guard the
 * compiler cannot prove unused).  No counterpart in the reference; for
 * measurement.
 */
int32_t moat_int4_stream_read(const void* src, int64_t bytes, int32_t workgroups, uint32_t* sink,
                              hipStream_t stream);

/*
 * Several projections of one shape that share their activations, in one
 * launch: y_f32[i] = f32(x) @ f32(deq(W_i)) for i < count (count 1..4), the
 * record-stream kernel over the concatenated column tiles.  Replaces
 * back-to-back dispatchGEMM calls on one input, e.g. the Q, K and V
 * projections of antigravity-engine/src/transformer_engine.mm:589-596 (one
 * call for Q, K, V when they have one width; K and V together when grouped
 * queries make them narrower); each product has moat_int4_gemm's semantics
 * and tolerance.
 * `superblocks` and `y_f32` are host arrays of `count` device pointers.
 * Preconditions: those of moat_int4_gemm, and m % 128 == 0, k % 32 == 0, x
 * 16-byte aligned (the record-stream kernel's shapes); otherwise
 * MOAT_ERR_INVALID (call moat_int4_gemm per matrix).  Workspace as for
 * moat_int4_gemm, sized by moat_int4_gemm_multi_workspace_size.
 */
int64_t moat_int4_gemm_multi_workspace_size(int32_t count, int32_t n, int32_t k, int32_t m);
int32_t moat_int4_gemm_multi(const uint16_t* x_f16, const uint8_t* const* superblocks, float* const* y_f32,
                             int32_t count, int32_t n, int32_t k, int32_t m,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Gate and up projections of a SwiGLU MLP fused with the activation:
 * h = fp16(silu(g) * u), g = f32(x) @ f32(deq(W_gate)), u = f32(x) @
 * f32(deq(W_up)), silu(g) = g / (1 + exp(-g)) in fp32.  Replaces the two
 * dispatchGEMM calls and silu_elementwise_mul_kernel of
 * antigravity-engine/src/transformer_engine.mm:694-713
 * (antigravity-engine/src/shaders/transformer_ops.metal:216-232; the
 * reference rounds g and u to fp16 first, this keeps them in fp32).  h is
 * [n][m] fp16, 8-byte aligned: the down projection's input.  Preconditions
 * and workspace as for moat_int4_gemm_multi.
 */
int64_t moat_int4_gemm_swiglu_workspace_size(int32_t n, int32_t k, int32_t m);
int32_t moat_int4_gemm_swiglu(const uint16_t* x_f16, const uint8_t* gate_superblocks,
                              const uint8_t* up_superblocks, uint16_t* h_f16,
                              int32_t n, int32_t k, int32_t m,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * The SwiGLU step alone, for a GEMM that produced gate and up side by side
 * (gu[r][0..m) = g, gu[r][m..2m) = u, rows ld floats apart): h[r][c] =
 * fp16(silu(g) * u) with moat_int4_gemm_swiglu's arithmetic (fp32 g and u,
 * silu(g) = g / (1 + exp(-g)), one rounding to fp16).  The activation of
 * antigravity-engine/src/transformer_engine.mm:694-713 /
 * antigravity-engine/src/shaders/transformer_ops.metal:216-232 after a
 * strip-order GEMM over [W_gate | W_up].  m % 4 == 0, ld >= 2m, ld % 4 == 0;
 * gu 16-byte aligned, h 8-byte aligned.
 */
int32_t moat_int4_swiglu_f32(const float* gu_f32, int32_t n, int32_t m, int64_t ld, uint16_t* h_f16,
                             hipStream_t stream);

/*
 * Group quantizer: for each group of group_size values (w_dtype F32, F16 or F64;
 * F64 is rounded to float32 first, as astype(np.float32) does),
 * alpha = max|w|, s = (alpha == 0 ? 1 : alpha / 7) in float32; q =
 * clip(rint_half_even(w / d), -8, 7) with d = s (MOAT_SCALE_F32, surface A:
 * src/dequant.py:26-55) or d = fp16(s) (MOAT_SCALE_F16, surface B:
 * antigravity-engine/src/dequant.py:22-60); scales_out = fp16(s).
 * n % group_size == 0.  A NaN quotient gives q = 0.
 */
int32_t moat_int4_quantize(const void* w, int32_t w_dtype, int64_t n, int32_t group_size,
                           int32_t scale_mode, int8_t* q_out, uint16_t* scales_out,
                           hipStream_t stream);

/*
 * Serialize q (int8, values taken mod 16 after +8) and fp16 scales into
 * n_superblocks 144-byte records (the writer for the format above; the
 * inverse of src/dequant.py:116-147; nibble rule of
 * antigravity-engine/src/dequant.py:119-124).  superblocks_out 16-byte aligned.
 */
int32_t moat_int4_pack_superblocks(const int8_t* q, const uint16_t* scales_f16,
                                   int64_t n_superblocks, uint8_t* superblocks_out,
                                   hipStream_t stream);

/* Quantize (group 32, rule scale_mode) and serialize in one pass: n % 256 == 0. */
int32_t moat_int4_quantize_pack(const void* w, int32_t w_dtype, int64_t n, int32_t scale_mode,
                                uint8_t* superblocks_out, hipStream_t stream);

/* Nibble pairs without headers, antigravity-engine/src/dequant.py:119-124
 * (repack_to_superblocks' payload); n even. */
int32_t moat_int4_pack_nibbles(const int8_t* q, int64_t n, uint8_t* packed_out, hipStream_t stream);

/* Inverse, antigravity-engine/src/dequant.py:135-156 (unpack_superblock):
 * 2*n_bytes int8 values in [-8, 7]. */
int32_t moat_int4_unpack_nibbles(const uint8_t* packed, int64_t n_bytes, int8_t* q_out,
                                 hipStream_t stream);

/*
 * Per-group dequant of unpacked values, fp16(f32(q) * f32(scales[g])) for the
 * first n_groups*group_size elements (the caller zero-fills any tail).
 * q_dtype: I8, I64 or F32; scale_dtype: F16, F32 or F64 (one per group; an
 * F64 scale is rounded to float32 first, like numpy's float32 * float).
 * table_mode 0: arithmetic_dequantize (antigravity-engine/src/dequant.py:223-252).
 * table_mode 1: lut_dequantize (:183-220), a 16-entry table indexed by q+8
 * with Python's negative-index wrap (q given as I8 or as I64 already reduced
 * to int16); an index outside [-16, 16) leaves the element 0 and sets
 * *err_flag to 1 (err_flag may be NULL in mode 0).
 */
int32_t moat_int4_group_dequant(const void* q, int32_t q_dtype, const void* scales, int32_t scale_dtype,
                                int64_t n_groups, int32_t group_size, int32_t table_mode,
                                uint16_t* out_f16, int32_t* err_flag, hipStream_t stream);

/*
 * Clipped table gather of src/dequant.py:79-112 (lut_dequantize_fp16):
 * out[i] = lut[row(i)][clip(idx(q[i]), 0, lut_len-1)], row(i) = i / (n / lut_rows).
 * index_mode 0: idx = q + 8; 1: idx = int32(q) + 8 (32-bit wrap); 2: idx = int32(q).
 * q is int64, lut fp16 [lut_rows][lut_len]; n % lut_rows == 0.
 */
int32_t moat_int4_lut_gather(const int64_t* q, int64_t n, int32_t index_mode,
                             const uint16_t* lut_f16, int64_t lut_rows, int32_t lut_len,
                             uint16_t* out_f16, hipStream_t stream);

/* *flag_out = 1 if any q[i] < 0 else 0 (int32 on the device); the branch test
 * of src/dequant.py:90. */
int32_t moat_int4_any_negative(const int64_t* q, int64_t n, int32_t* flag_out, hipStream_t stream);

/* out[i] = fp16(f32(q[i]) / divisor), float32 division then one rounding to
 * fp16: numpy's float16 division of int8 values cast to float16 by a float16
 * scalar -- the int8 fallback of antigravity-engine/src/model_loader.py:247
 * (divisor 7).  divisor finite and non-zero. */
int32_t moat_int4_i8_div_to_f16(const int8_t* q, int64_t n, float divisor, uint16_t* out_f16, hipStream_t stream);

/* Round F32 or F64 values to fp16, nearest-even, one rounding (numpy's astype(float16)). */
int32_t moat_int4_to_f16(const void* src, int32_t src_dtype, int64_t n, uint16_t* out_f16,
                         hipStream_t stream);

/*
 * Token sampling from LM-head logits (the numpy path of
 * BatchedRolloutCoordinator.sample_tokens, antigravity-engine/src/batch_generator.py:187-253,
 * and the table softmax it calls, antigravity-engine/src/attention.py:97-135).
 *
 * `lut_f16` is the exp table of ExponentialLUT (attention.py:32-58): lut_size
 * fp16 values of exp over [-range_max, 0], 2 <= lut_size <= 2^24; `step` is
 * range_max / (lut_size - 1) rounded to float32.  Logits are [n][v] of dtype
 * F32, F16 or F64, 0 <= n <= 2^21, 1 <= v <= 524288 (up to 64 chunks of 8192
 * logits, one workgroup each).
 *
 * Both calls take a device workspace, 256-byte aligned, of at least the
 * bytes the size calls below give (sampling: about 2 v + 600 bytes per row;
 * softmax: about 600 bytes per 8192 logits, its table values going to the
 * output buffer; MOAT_ERR_WORKSPACE when missing or short).  It holds the
 * call's intermediate results and one counter word per row, through which
 * the last of a row's workgroups (one per 8192 logits) takes over the row;
 * each call sets them up itself, so the workspace need not be cleared and
 * serves calls of any shape.  Calls that share a workspace must not
 * overlap; use a different workspace from the GEMM's (whose counter words
 * must stay zero).
 */

/* Workspace bytes of a moat_sample_tokens / moat_lut_softmax call over n rows
 * of v logits (0 when n is 0; -1 for sizes outside the limits above).  No
 * counterpart in the reference, whose numpy sampler allocates as it goes. */
int64_t moat_sample_workspace_size(int32_t n, int32_t v);
int64_t moat_lut_softmax_workspace_size(int32_t n, int32_t v);

/*
 * moat_lut_softmax: probs_f16[n][v] = safe_softmax_lut(x) along each row:
 * row max (f32), table index size-1-trunc(min(|x - max| / step, size-1)),
 * numpy's float32 pairwise sum of the table values, fp16(e / sum).  A row
 * whose maximum is NaN or infinite (the reference's index is undefined
 * there) gives NaN.
 */
int32_t moat_lut_softmax(const void* x, int32_t dtype, int32_t n, int32_t v, const uint16_t* lut_f16,
                         int32_t lut_size, float step, uint16_t* probs_f16, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream);

/*
 * moat_sample_tokens: temperature <= 0: greedy, tokens[r] = np.argmax(row r)
 * (first maximum, NaN first), logprobs[r] = fp16(log(p[token])) (an fp16
 * value in a float), p the table softmax of the raw logits.  temperature > 0:
 * p = table softmax of logits / max(temperature, 1e-5) (divided in the
 * logits' dtype); the top_k (1..64; min(top_k, v)) largest p, ordered by p
 * descending then index ascending (the reference leaves the order to
 * np.argpartition), renormalised in float32 (numpy's summation order), one
 * draw u of row r from a counter-based generator (SplitMix64 of seed +
 * (r + 1) * 0x9E3779B97F4A7C15, 53 bits), the first entry of the float64
 * cumulative distribution above u; logprobs[r] = float32 log of the token's
 * full-softmax p (log(1e-10) when p is 0).  tokens int32, logprobs float32.
 * A row whose maximum is NaN or infinite: the argmax token and a NaN log.
 */
int32_t moat_sample_tokens(const void* logits, int32_t dtype, int32_t n, int32_t v, double temperature,
                           int32_t top_k, uint64_t seed, const uint16_t* lut_f16, int32_t lut_size,
                           float step, int32_t* tokens, float* logprobs, void* workspace,
                           int64_t workspace_bytes, hipStream_t stream);

/*
 * Dense fp16 decode product: y[n][m] (fp16) = fp16(f32(x) @ f32(w)), x
 * [n][k] and w [k][m] row-major fp16, the sums in fp32 and each output
 * rounded to fp16 once.  Replaces the reference's two dense kernels behind
 * dispatchGEMM (antigravity-engine/src/transformer_engine.mm:463-500):
 * batched_gemm_simdgroup (antigravity-engine/src/shaders/
 * batched_gemm.metal:74-109; half sums, n a multiple of 8), as launched by
 * metal_runner.cpp:120-143 and antigravity_c_api.cpp:198-216, and the
 * one-row gemv_kernel (antigravity-engine/src/shaders/
 * transformer_ops.metal:270-286; fp32 sums, half out).  One entry serves every
 * n with the GEMV's fp32 sums (the reference's CPU product,
 * antigravity-engine/tests/test_batched_speed.py:31-42, computes the same);
 * row r of a call does not depend on the other rows (bit for bit, the
 * n = 1 call's row).  Preconditions: n >= 1, k >= 8, k % 8 == 0, m >= 8,
 * m % 8 == 0; x and w 16-byte aligned, y 2-byte aligned and not
 * overlapping x or w; 0 <= splits <= 1024 (workgroups a 64-column block's
 * rows are split over; 0 automatic) -- MOAT_ERR_INVALID otherwise.  When
 * moat_dense_gemm_workspace_size (-1 for an invalid shape) is above 0 the
 * call needs a 16-byte aligned workspace of that many bytes
 * (MOAT_ERR_WORKSPACE otherwise), zero-filled before its first use
 * (moat_int4_workspace_clear) and left with its counter words at zero by
 * every call; its split sums stay behind, so it is not shared with the
 * GEMM entry points above.  Calls that overlap on one workspace race.
 */
int64_t moat_dense_gemm_workspace_size(int32_t n, int32_t k, int32_t m, int32_t splits);
int32_t moat_dense_gemm(const uint16_t* x_f16, const uint16_t* w_f16, uint16_t* y_f16, int32_t n, int32_t k,
                        int32_t m, int32_t splits, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ExponentialLUT.lookup (attention.py:60-85): out_f16[i] =
 * lut[size-1-trunc(min(|x[i]| / step, size-1))] for float32 x (NaN -> NaN). */
int32_t moat_lut_lookup(const float* x, int64_t n, const uint16_t* lut_f16, int32_t lut_size, float step,
                        uint16_t* out_f16, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MOAT_INT4_H */
