/*
 * mcke_amd.h -- the C-ABI boundary of the MI355X (gfx950) MCKE kernel layer.
 *
 * Plain pointers, sizes and integer enums only.  Every entry point below replaces
 * one function of the reference's C++ kernel/runtime API (cited per entry); the
 * C++ mirror of that API (include/mcke/...) is written as inline wrappers over
 * these symbols, and Python/ctypes, cgo or JNI bind them directly.
 *
 * Conventions shared by every entry point:
 *   - Return value: an MCKE_STATUS_* code, numerically equal to the reference's
 *     mcke::StatusCode (reference include/mcke/core/status.hpp:42-50).  On failure
 *     mcke_last_error() returns the message for the calling thread.
 *   - All data pointers are caller-owned device memory.  Launchers never allocate,
 *     free or synchronise (reference kernels.hpp:186-197); work is enqueued on
 *     `stream` (a hipStream_t; NULL means the null stream).
 *   - Enum values are the reference's, and GemmVariant is append-only.
 */
#ifndef MCKE_AMD_H_
#define MCKE_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MCKE_ABI_VERSION 1

/* mcke::StatusCode (status.hpp:42-50).  The reference's kCudaError slot carries
 * HIP runtime errors here. */
enum mcke_status {
  MCKE_STATUS_OK = 0,
  MCKE_STATUS_OUT_OF_MEMORY = 1,
  MCKE_STATUS_INVALID_ARGUMENT = 2,
  MCKE_STATUS_FAILED_PRECONDITION = 3,
  MCKE_STATUS_UNIMPLEMENTED = 4,
  MCKE_STATUS_INTERNAL = 5,
  MCKE_STATUS_DEVICE_ERROR = 6
};

/* kernels.hpp:65 */
enum mcke_activation { MCKE_ACT_NONE = 0, MCKE_ACT_RELU = 1, MCKE_ACT_GELU_ERF = 2, MCKE_ACT_GELU_TANH = 3 };
/* kernels.hpp:153 */
enum mcke_reduce_kind { MCKE_REDUCE_SUM = 0, MCKE_REDUCE_MAX = 1, MCKE_REDUCE_MEAN = 2 };
/* kernels.hpp:180 */
enum mcke_reduce_variant { MCKE_REDUCE_SMEM_TREE = 0, MCKE_REDUCE_WARP_SHUFFLE = 1, MCKE_REDUCE_TWO_PASS = 2 };
/* kernels.hpp:218 */
enum mcke_softmax_variant { MCKE_SOFTMAX_THREE_PASS = 0, MCKE_SOFTMAX_ONLINE_ONE_PASS = 1 };
/* gemm_tile.hpp:209-214, append-only; MCKE_GEMM_MFMA_F32 is this build's addition. */
enum mcke_gemm_variant {
  MCKE_GEMM_NAIVE = 0,
  MCKE_GEMM_TILED_SMEM = 1,
  MCKE_GEMM_TILED_REGBLOCK = 2,
  MCKE_GEMM_WARP_TILE = 3,
  MCKE_GEMM_CUBLAS_REF = 4,      /* vendor-library ceiling row (rocBLAS here) */
  MCKE_GEMM_WARP_TILE_NODBUF = 5,
  MCKE_GEMM_WARP_TILE_VEC4 = 6,
  MCKE_GEMM_NAIVE_UNCOALESCED = 7,
  MCKE_GEMM_MFMA_F32 = 8         /* fp32 MFMA, LDS double-buffered (gfx950) */
};

/* GemmTile, gemm_tile.hpp:47-69: block tile bm x bn staged bk deep, per-thread
 * micro-tile tm x tn; threads per block = (bm/tm)*(bn/tn). */
typedef struct mcke_gemm_tile {
  int32_t bm, bn, bk, tm, tn;
} mcke_gemm_tile;

/* GemmKernelAttrs, kernels.hpp:293-299 (+ agprs, which CDNA adds). */
typedef struct mcke_kernel_attrs {
  int32_t regs_per_thread;       /* architectural VGPRs */
  int32_t agprs_per_thread;      /* accumulation VGPRs (0 when unused) */
  uint64_t static_smem_bytes;    /* LDS bytes per workgroup */
  uint64_t local_bytes;          /* scratch (spill) bytes per lane; > 0 means spilling */
  int32_t threads_per_block;
  int32_t max_blocks_per_sm_api; /* hipOccupancyMaxActiveBlocksPerMultiprocessor */
} mcke_kernel_attrs;

/* DeviceInfo snapshot, reference include/mcke/core/device.hpp:29-110. */
typedef struct mcke_device_info {
  int32_t ordinal;
  char name[256];
  char arch[64];                 /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t cc_major, cc_minor;
  uint64_t total_global_mem;
  int32_t sm_count;              /* compute units */
  int32_t warp_size;             /* 64 on CDNA */
  int32_t max_threads_per_block;
  int32_t max_threads_per_sm;
  int32_t max_blocks_per_sm;
  int32_t regs_per_block;
  int32_t regs_per_sm;
  uint64_t shared_mem_per_block;
  uint64_t shared_mem_per_sm;
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width_bits;
  uint64_t l2_cache_bytes;
  double peak_dram_gb_s;         /* spec figure for the part (see mcke_rt_query_device) */
} mcke_device_info;

/* ---- errors -------------------------------------------------------------- */
/* Message of the last failing call on this thread ("" if none). */
const char* mcke_last_error(void);
int mcke_abi_version(void);

/* ---- kernels ------------------------------------------------------------- */
/* launch_vector_add_f32, kernels.hpp:59-60 / elementwise.cu:46-91. */
int mcke_launch_vector_add_f32(const float* a, const float* b, float* out, size_t n,
                               void* stream);

/* launch_bias_act_f32, kernels.hpp:102-106 / bias_act.cu:269-294.
 * y[r,c] = act(x[r,c] + bias[c]); vector_width in {1,2,4} with cols % vw == 0 and
 * x, y, bias aligned to 4*vw bytes, else INVALID_ARGUMENT (never downgraded);
 * x == y rejected; rows == 0 or cols == 0 is a no-op.  max_row_blocks caps the
 * row dimension of the grid (0 = automatic). */
int mcke_launch_bias_act_f32(const float* x, const float* bias, float* y, int64_t rows,
                             int64_t cols, int act, int vector_width, void* stream,
                             int max_row_blocks);

/* launch_bias_add_f32, kernels.hpp:129-131 / bias_act.cu:296-305: the fused kernel
 * with the identity activation. */
int mcke_launch_bias_add_f32(const float* x, const float* bias, float* y, int64_t rows,
                             int64_t cols, int vector_width, void* stream);

/* launch_activation_f32, kernels.hpp:133-135 / bias_act.cu:307-331: y = act(x),
 * the second half of the unfused baseline. */
int mcke_launch_activation_f32(const float* x, float* y, int64_t n, int act,
                               int vector_width, void* stream);

/* max_vector_width_f32, kernels.hpp:143-148: widest of {4,2,1} legal for p, cols. */
int mcke_max_vector_width_f32(const void* p, int64_t cols);

/* row_reduce_workspace_bytes, kernels.hpp:200-202 / reduce.cu:213-218.  Zero for
 * kSmemTree and kWarpShuffle; kTwoPass needs rows * split * 4 bytes (the
 * partials), where this build's split depends on the shape (rows and cols). */
size_t mcke_row_reduce_workspace_bytes(int64_t rows, int64_t cols, int variant);

/* The frozen 7-argument launch_row_reduce_f32, kernels.hpp:204-207 /
 * reduce.cu:285-295: kTwoPass without a workspace is UNIMPLEMENTED. */
int mcke_launch_row_reduce_f32(const float* x, float* out, int64_t rows, int64_t cols,
                               int kind, int variant, void* stream);

/* The 9-argument launch_row_reduce_f32, kernels.hpp:209-213 / reduce.cu:224-280.
 * out[r] = sum / max / mean of row r (mean = sum / cols).  rows == 1 with
 * kTwoPass is the full-tensor reduction.  When there are too few rows to fill
 * the part, kTwoPass splits each long row into column chunks whose partials go
 * to the workspace, and a second launch folds each row's partials in a fixed
 * order; rows that need no split take one launch.  The launcher keeps no state
 * between calls, and the workspace's contents on entry do not matter. */
int mcke_launch_row_reduce_ws_f32(const float* x, float* out, int64_t rows, int64_t cols,
                                  int kind, int variant, float* workspace,
                                  size_t workspace_bytes, void* stream);

/* No counterpart in the reference: kTwoPass (the 9-argument launch above, same
 * kernels, same bits) for callers that cannot allocate -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  It takes no
 * workspace and allocates nothing: the split partials go to a 4 KiB device array
 * the library holds per GPU (1024 partials; this build's split needs at most
 * 511, and a shape needing more is INVALID_ARGUMENT).  Calls that overlap on one
 * GPU share that array and race; calls in one stream's order do not. */
int mcke_launch_row_reduce_noalloc_f32(const float* x, float* out, int64_t rows, int64_t cols,
                                       int kind, void* stream);

/* launch_row_softmax_f32, kernels.hpp:220-223 / softmax.cu:177-199.  x == y
 * rejected; rows > 2^31-1 rejected. */
int mcke_launch_row_softmax_f32(const float* x, float* y, int64_t rows, int64_t cols,
                                int variant, void* stream);

/* launch_gemm_f32, kernels.hpp:265-269 / gemm.cu:829-882.
 * C = alpha*A[m,k]B[k,n] + beta*C, row-major.  C is not read when beta == 0.
 * m == 0 or n == 0 is a no-op; k == 0 gives C = beta*C.  a == c or b == c,
 * negative or > INT32_MAX extents, and (variant, tile) pairs that are not
 * compiled are INVALID_ARGUMENT (no fallback tile). */
int mcke_launch_gemm_f32(const float* a, const float* b, float* c, int64_t m, int64_t n,
                         int64_t k, float alpha, float beta, int variant,
                         const mcke_gemm_tile* tile, void* stream);

/* No reference counterpart: launch_gemm_f32 (kMfmaF32, beta = 0) with
 * launch_bias_act_f32 fused into the GEMM's epilogue,
 *   y[i,j] = act(alpha * (A B)[i,j] + bias[j]),
 * for callers that chain the two (the graph layer's GemmBiasAct node, the MLP
 * block of the benchmark): C never goes to memory and one launch is saved.  The
 * result has the bits of mcke_launch_gemm_f32(a, b, y, m, n, k, alpha, 0,
 * MCKE_GEMM_MFMA_F32, tile) followed by mcke_launch_bias_act_f32(y, bias, y2, m, n,
 * activation, ...).  Validation as mcke_launch_gemm_f32 for kMfmaF32, plus: bias
 * (n floats, any alignment) must not be null, y must not alias a, b or bias, and
 * activation is an mcke_activation value. */
int mcke_launch_gemm_bias_act_f32(const float* a, const float* b, const float* bias, float* y,
                                  int64_t m, int64_t n, int64_t k, float alpha, int activation,
                                  const mcke_gemm_tile* tile, void* stream);

/* gemm_kernel_attrs, kernels.hpp:301-302 / gemm.cu:884-904. */
int mcke_gemm_kernel_attrs(int variant, const mcke_gemm_tile* tile,
                           mcke_kernel_attrs* out);

/* No reference counterpart: the MFMA tile this build would pick for a shape
 * (the callers that do not hand-pick a tile: the graph layer, the benchmark). */
int mcke_gemm_mfma_default_tile(int64_t m, int64_t n, int64_t k, mcke_gemm_tile* out);

/* ---- 16-bit-input GEMM on the matrix cores -------------------------------
 * No counterpart in the reference: its DType enum reserves kF16 and kBF16 for
 * matrix-unit inputs (include/mcke/core/dtype.hpp:33-41, values below) but the
 * only GEMM launcher is fp32 (kernels.hpp:265-269).  Callers: those with 16-bit
 * weights and activations (the graph layer's next dtype, the benchmark). */
enum mcke_dtype { MCKE_DTYPE_F32 = 0, MCKE_DTYPE_F16 = 1, MCKE_DTYPE_BF16 = 2 };

/* C = alpha * A B + beta * C; A (m x k) and B (k x n) row-major in ab_dtype
 * (MCKE_DTYPE_BF16 or MCKE_DTYPE_F16), products accumulated in fp32
 * (v_mfma_f32_32x32x16_{bf16,f16}), C row-major in c_dtype (MCKE_DTYPE_F32 or
 * ab_dtype, rounded to nearest even).  Validation as mcke_launch_gemm_f32: m or
 * n == 0 is a no-op, k == 0 gives C = beta * C, C is not read when beta == 0,
 * a == c / b == c and negative or > INT32_MAX extents are INVALID_ARGUMENT.
 * Tiles (bm,bn,bk,tm,tn): (256,256,64,16,16), (128,128,64,8,8), (64,64,64,4,4);
 * any other tile is INVALID_ARGUMENT.  Any shape and alignment is accepted;
 * k % 8 == 0, n % 8 == 0 and 16-byte aligned a, b, c take the 16-byte path. */
int mcke_launch_gemm_lp(const void* a, const void* b, void* c, int ab_dtype, int c_dtype,
                        int64_t m, int64_t n, int64_t k, float alpha, float beta,
                        const mcke_gemm_tile* tile, void* stream);

/* mcke_gemm_kernel_attrs for the whole-tile kernel of one (dtype pair, tile). */
int mcke_gemm_lp_kernel_attrs(int ab_dtype, int c_dtype, const mcke_gemm_tile* tile,
                              mcke_kernel_attrs* out);

/* The tile this build picks for a 16-bit GEMM of this shape. */
int mcke_gemm_lp_default_tile(int64_t m, int64_t n, int64_t k, mcke_gemm_tile* out);

/* The vendor-library ceiling row of the 16-bit GEMM (rocBLAS gemm_ex, fp32
 * compute), the counterpart of MCKE_GEMM_CUBLAS_REF for these types: same
 * arguments as mcke_launch_gemm_lp without the tile. */
int mcke_launch_gemm_lp_vendor(const void* a, const void* b, void* c, int ab_dtype,
                               int c_dtype, int64_t m, int64_t n, int64_t k, float alpha,
                               float beta, void* stream);

/* ---- runtime: rt::Stream / rt::Event / raw device memory ------------------
 * reference include/mcke/runtime/stream.hpp:82-306, src/core/device.cpp:56-168,
 * src/memory/allocator.cpp:44-73, src/tensor/tensor.cpp:108-138. */
int mcke_rt_get_device_count(int* count);
int mcke_rt_set_device(int ordinal);
int mcke_rt_get_device(int* ordinal);
int mcke_rt_query_device(int ordinal, mcke_device_info* out);
int mcke_rt_device_synchronize(void);

/* Streams are created non-blocking (stream.hpp:29-35) at default priority. */
int mcke_rt_stream_create(void** out_stream);
int mcke_rt_stream_destroy(void* stream);
int mcke_rt_stream_synchronize(void* stream);
/* *done = 1 when all work on the stream has completed. */
int mcke_rt_stream_query(void* stream, int* done);
int mcke_rt_stream_wait_event(void* stream, void* event);

/* timing != 0 creates a timing event; otherwise timing is disabled (cheaper). */
int mcke_rt_event_create(void** out_event, int timing);
int mcke_rt_event_destroy(void* event);
int mcke_rt_event_record(void* event, void* stream);
int mcke_rt_event_query(void* event, int* done);
int mcke_rt_event_synchronize(void* event);
int mcke_rt_event_elapsed_ms(void* start, void* stop, float* ms);

/* Stream capture into a HIP graph (no reference counterpart: the reference plans
 * it as capture_cuda_graph, include/mcke/graph/executor.hpp:23-27).  Capture runs
 * in thread-local mode on a stream this library created.  end_capture
 * instantiates the captured graph and returns the executable graph; launch
 * replays it on `stream`; destroy releases it.  Nothing captured may be a memset
 * (kernels fill memory here, never hipMemsetAsync). */
int mcke_rt_stream_begin_capture(void* stream);
int mcke_rt_stream_end_capture(void* stream, void** out_exec);
int mcke_rt_graph_launch(void* exec, void* stream);
int mcke_rt_graph_destroy(void* exec);

/* Explicit graph assembly, for plans on several streams (no reference
 * counterpart).  Each node's launches are stream-captured on one stream
 * (end_capture_graph returns the captured, not yet instantiated, hipGraph_t),
 * then added to a parent graph after the parent nodes given in deps; no capture
 * ever spans two streams.  add_child adds a child that is a chain of kernel
 * nodes (what one stream's capture of kernel launches gives) as the same chain
 * of kernel nodes, an empty child as an empty node and any other child as a
 * child-graph node; *out_node is the last node added.  The caller keeps the
 * child until the parent and every executable graph made from it are
 * released.  instantiate turns the parent into an
 * executable graph for mcke_rt_graph_launch / mcke_rt_graph_destroy;
 * graph_release frees a graph that is not instantiated (parent or child). */
int mcke_rt_stream_end_capture_graph(void* stream, void** out_graph);
int mcke_rt_graph_create(void** out_graph);
int mcke_rt_graph_add_child(void* graph, void* child, void* const* deps, size_t n_deps,
                            void** out_node);
int mcke_rt_graph_instantiate(void* graph, void** out_exec);
int mcke_rt_graph_release(void* graph);
/* hipGraphUpload: moves an instantiated graph's launch resources to the device
 * ahead of its first mcke_rt_graph_launch on `stream`. */
int mcke_rt_graph_upload(void* exec, void* stream);

/* raw_device_malloc / raw_device_free (device.cpp:104-130): hipMalloc, which is
 * 256-byte aligned; out-of-memory maps to MCKE_STATUS_OUT_OF_MEMORY. */
int mcke_rt_malloc(void** out_ptr, size_t bytes);
int mcke_rt_free(void* ptr);
int mcke_rt_host_alloc(void** out_ptr, size_t bytes); /* pinned host memory */
int mcke_rt_host_free(void* ptr);
/* kind: 0 host->device, 1 device->host, 2 device->device, 3 default (unified VA). */
int mcke_rt_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream);
/* Refused (INVALID_ARGUMENT) while `stream` is being captured into a graph: a
 * captured memset node is not replayed reliably on this stack; capture
 * mcke_fill_u32_async instead. */
int mcke_rt_memset_async(void* dst, int value, size_t bytes, void* stream);
/* No reference counterpart: fills `count` 32-bit words with `value` using a
 * kernel (usable under graph capture, unlike a memset node).  Used by the graph
 * executor to poison its arena between runs. */
int mcke_fill_u32_async(void* dst, uint32_t value, size_t count, void* stream);

/* ---- measured denominators (reference bench/fma_peak.cu, bench/stream_triad.cu) ----
 * mfma_peak: `blocks` workgroups of 256 lanes; every wave issues `iters` x 4
 * independent v_mfma_f32_32x32x2_f32 and no other memory traffic than reading
 * seed[0..255] and writing out[blocks*256].  mcke_mfma_peak_flops() gives the
 * flops of one launch (blocks * 4 waves * iters * 4 * 4096); 0 for bad arguments.
 * The reference measures the vector FMA pipe; the GEMM here runs on the matrix
 * cores, whose fp32 pipe this measures instead.
 * stream_triad: a[i] = scalar * c[i] + b[i] for i < n (12 bytes per element);
 * 16-byte aligned a, b, c; a must not alias b or c. */
uint64_t mcke_mfma_peak_flops(int64_t blocks, int64_t iters);
int mcke_launch_mfma_peak_f32(const float* seed, float* out, int64_t blocks, int64_t iters,
                              void* stream);
int mcke_launch_stream_triad_f32(const float* b, const float* c, float* a, float scalar, int64_t n,
                                 void* stream);
/* stream_copy: y[i] = x[i] for i < n (8 bytes per element), the read+write
 * ceiling (no reference counterpart; the reference's bench measures the triad
 * only); 16-byte aligned x, y; y must not alias x. */
int mcke_launch_stream_copy_f32(const float* x, float* y, int64_t n, void* stream);
/* The 16-bit MFMA counterpart of mfma_peak (no reference counterpart: the
 * ceiling of mcke_launch_gemm_lp): the same 4 chains per wave of
 * v_mfma_f32_32x32x16_{bf16,f16} (ab_dtype MCKE_DTYPE_BF16 or MCKE_DTYPE_F16),
 * 32768 flops each. */
uint64_t mcke_mfma_peak_lp_flops(int64_t blocks, int64_t iters);
int mcke_launch_mfma_peak_lp(int ab_dtype, const float* seed, float* out, int64_t blocks,
                             int64_t iters, void* stream);
/* Engine-clock probe for the 16-bit MFMA forms (no reference counterpart): chains
 * whose operands change with every instruction, as a GEMM's do, from eight
 * operand registers per lane of random 16-bit values (operand_bits: 256 lanes x
 * 8 x 16 bytes, 16-byte aligned).  shape 0 runs v_mfma_f32_32x32x16_{bf16,f16}
 * (4 chains per wave), shape 1 v_mfma_f32_16x16x32_{bf16,f16} (8 chains): the
 * same flops per iteration.  out receives blocks x 256 sums; ticks (2 x blocks)
 * receives, per workgroup, its s_memtime span (engine clock cycles) and its
 * s_memrealtime span (100 MHz ticks), so clock = cycles / (ticks x 10 ns). */
uint64_t mcke_mfma_clock_lp_flops(int64_t blocks, int64_t iters);
int mcke_launch_mfma_clock_lp(int ab_dtype, int shape, const void* operand_bits, float* out,
                              uint64_t* ticks, int64_t blocks, int64_t iters, void* stream);

/* ---- host data generators (bench / test inputs) ----------------------------
 * The same map as the reference's fill_random (tests/reference.hpp:101-109):
 * std::mt19937_64(seed), u = (e >> 40) / 2^24, x = lo + u*(hi - lo).  The normal
 * variant (no reference counterpart) is Box-Muller on 53-bit uniforms from the
 * same engine.  Host memory. */
void mcke_fill_random_f32(float* host, size_t n, uint64_t seed, float lo, float hi);
void mcke_fill_normal_f32(float* host, size_t n, uint64_t seed, float mu, float sigma);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MCKE_AMD_H_ */
