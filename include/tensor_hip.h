/*
 * libtensor_hip.so — the ROCm (gfx950) provider's C ABI.
 *
 * Two groups of entry points:
 *
 *  1. GGUF quantized-linear kernels, in the reference's native entry shape
 *     TensorKernelV1 (src/tensor/include/tensor/abi.h:135-141).  Each validates
 *     the call the way the reference's CPU image wrapper does
 *     (src/tensor/compiler/cpu.py:49-155: ABI version, struct size, flags,
 *     argument count, kinds, dtypes, device, rank/shape/stride/byte_size,
 *     alignment) before it touches device memory, then enqueues asynchronously
 *     on (hipStream_t)call->stream.handle and returns.  They replace the
 *     AKAS GGUF kernels that the reference builds into .tbin images and
 *     launches through Executable.launch -> Device._launch -> cuLaunchKernel
 *     (benchmarks/kernels/showcase/kernels.py:114-119,
 *      benchmarks/kernels/showcase/benchmark.py:276-290,
 *      src/tensor/providers/cuda/device.py:211-229).
 *
 *  2. Runtime services the Python provider binds through ctypes, replacing the
 *     CUDA driver calls of src/tensor/providers/cuda/driver.py:40-145
 *     (memory, copies, streams, events, graphs, device properties).
 *
 * Every function returns TENSOR_OK or a TENSOR_ERROR_* code and, when error
 * is non-null, fills it with a NUL-terminated message.  No C++ exception
 * crosses this boundary.  Kernel calls borrow every descriptor until return;
 * device buffers must stay alive until the stream has finished the work.
 */
#ifndef TENSOR_HIP_H
#define TENSOR_HIP_H

#include "tensor/abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGML block type ids accepted by the GGUF entry points.  Q4_0, Q8_0, Q4_K and Q6_K are
 * the showcase's encodings (benchmarks/kernels/showcase/benchmark.py:122-126 and
 * research/plans/v1-benchmarks.md:297-301); Q4_1, Q5_0, Q5_1, Q2_K, Q3_K and Q5_K are the
 * plan's other basic and K formats (v1-benchmarks.md:297-300), public GGML layouts. */
#define TENSOR_GGML_Q4_0 2u
#define TENSOR_GGML_Q4_1 3u
#define TENSOR_GGML_Q5_0 6u
#define TENSOR_GGML_Q5_1 7u
#define TENSOR_GGML_Q8_0 8u
#define TENSOR_GGML_Q2_K 10u
#define TENSOR_GGML_Q3_K 11u
#define TENSOR_GGML_Q4_K 12u
#define TENSOR_GGML_Q5_K 13u
#define TENSOR_GGML_Q6_K 14u

/* Largest activation row count of the decode GEMV entry. */
#define TENSOR_GGUF_GEMV_MAX_M 8

/* ----------------------------------------------------------- kernels --- */

/*
 * Decode GEMV, out[m, n] = sum_k x[m, k] * dequant(W)[n, k], fp32 accumulate.
 * Replaces AKAS gemv_packed (benchmarks/kernels/showcase/kernels.py:119, the
 * m == 1 branch; arguments [x, w, out] at benchmark.py:293-295, :460-464;
 * numerics benchmark.py:466-472).  Arguments, in order:
 *   0 x    buffer fp16  [M, K], 1 <= M <= TENSOR_GGUF_GEMV_MAX_M
 *   1 w    buffer uint8 [N, K/QK*BLOCK]   raw GGUF rows
 *   2 out  buffer fp16 or fp32 [M, N]
 *   3 type scalar uint32 GGML type id
 * Buffers: device type TENSOR_DEVICE_ROCM, the stream's ordinal, 16-byte
 * aligned addresses, contiguous byte strides.
 * Q4_K at 4 <= M <= 8 with rows whose x does not fit in LDS (plan kernel 3 of
 * tensor_gguf_gemv_plan_v1, e.g. M = 8, K = 12288) splits K across workgroups: its fp32 partial
 * sums go to the library's static scratch (the array of tensor_gguf_gemm_group_noalloc_v1), so
 * such calls share it with that entry and follow its rules: eager calls on different streams
 * take it in turn, replays of captured graphs that overlap on one GPU race.
 */
int32_t tensor_gguf_gemv_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Prefill fused dequant-GEMM, out[m, n] = sum_k fp16(x[m, k]) *
 * fp16(dequant(W)[n, k]), fp32 accumulate.  Replaces AKAS _packed
 * (benchmarks/kernels/showcase/kernels.py:119, the m > 1 branch; numerics
 * benchmark.py:473-477, triton_kernels.py:199-211).  Same arguments as
 * tensor_gguf_gemv_v1 with any M >= 1.
 */
int32_t tensor_gguf_gemm_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Quantized linear with the reference showcase's dispatch: the decode GEMV
 * for M <= TENSOR_GGUF_GEMV_MAX_M, the fused GEMM otherwise
 * (benchmarks/kernels/showcase/kernels.py:114-119 picks gemv_packed for
 * m == 1 and _packed otherwise).  Same arguments as tensor_gguf_gemv_v1.
 */
int32_t tensor_gguf_linear_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Quantized linear in the AKAS packed call form, which the showcase launches unchanged
 * (buffers [x, w, out] at benchmarks/kernels/showcase/benchmark.py:460-464, launched by
 * TensorCall at :276-290; the kernel is specialised on (m, n, k), kernels.py:114-119, so the
 * shape travels as scalars a manifest fixes).  Dispatch as the showcase's: M == 1 is the
 * decode GEMV with x in its own precision (fp32 x times the fp32-decoded weight,
 * benchmark.py:466-472), M > 1 the prefill GEMM with x rounded to fp16 as it is staged
 * (benchmark.py:473-477).  Arguments, in order:
 *   0 x    buffer fp32 or fp16, M*K elements (any rank, contiguous)
 *   1 w    buffer of any integer dtype, exactly N*(K/QK)*BLOCK bytes of raw GGUF rows
 *   2 out  buffer fp32 or fp16, M*N elements (any rank, contiguous)
 *   3 type scalar uint32 GGML type id
 *   4 m, 5 n, 6 k  scalar uint32; K a multiple of the block's QK
 */
int32_t tensor_gguf_packed_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Grouped decode GEMV: out_i[m, n] = sum_k x[m, k] * dequant(W_i)[n, k] for
 * 1 <= c <= TENSOR_GGUF_GEMV_GROUP_MAX matrices that share the activations x
 * (a decoder's gate and up projections, or q, k and v).  No counterpart in the
 * reference: there every linear is its own gemv_packed launch
 * (benchmarks/kernels/showcase/kernels.py:114-119).  The group is one launch
 * of the Q4_K M = 1 kernel when K is a multiple of 4096; for other encodings
 * and shapes it is c launches of tensor_gguf_gemv_v1's kernels in order on the
 * stream.  Arguments, in order:
 *   0        x     buffer fp16  [M, K], 1 <= M <= TENSOR_GGUF_GEMV_MAX_M
 *   2i+1     w_i   buffer uint8 [N_i, K/QK*BLOCK]
 *   2i+2     out_i buffer [M, N_i], one dtype (fp16 or fp32) for all i
 *   2c+1     type  scalar uint32 GGML type id, shared by the group
 */
#define TENSOR_GGUF_GEMV_GROUP_MAX 3
int32_t tensor_gguf_gemv_group_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Grouped prefill GEMM: out_i[m, n] = sum_k fp16(x[m, k]) * fp16(dequant(W_i)[n, k]), fp32
 * accumulate, for 1 <= c <= TENSOR_GGUF_GEMM_GROUP_MAX matrices that share x and K (a layer's
 * q, k and v, or gate and up) in one launch.  No counterpart in the reference, where each linear
 * is its own _packed launch (benchmarks/kernels/showcase/kernels.py:114-119).  When the shape
 * leaves most CUs idle, K is split across workgroups: each writes fp32 partial sums into the
 * workspace and a second kernel adds them in split order (deterministic) and converts; the
 * split is chosen to fit the workspace given (any size; a short one only limits the split).
 * Q4_K, Q5_K, Q6_K, Q8_0 and Q4_0 use the pipelined kernel (Q8_0 / Q4_0 where K is an even
 * number of 64-element steps), at M <= 64 with every N_i <= 4096 on 64 x 64 tiles with K split
 * across workgroups where that fills at least 128 workgroups; the other encodings and shapes
 * take one launch per matrix as tensor_gguf_gemm_v1 runs it.  Arguments, in order:
 *   0        x         buffer fp16  [M, K]
 *   2i+1     w_i       buffer uint8 [N_i, K/QK*BLOCK]
 *   2i+2     out_i     buffer [M, N_i], one dtype (fp16 or fp32) for all i
 *   2c+1     workspace buffer uint8 [bytes], 256-byte aligned (device scratch, clobbered)
 *   2c+2     type      scalar uint32 GGML type id, shared by the group
 */
#define TENSOR_GGUF_GEMM_GROUP_MAX 3
int32_t tensor_gguf_gemm_group_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * tensor_gguf_gemm_group_v1 without the workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts that forbid
 * hipMalloc): arguments [x, w0, out0, .., w(c-1), out(c-1), type].  No counterpart in the
 * reference.  The K split's fp32 partials go to a static device array of the library,
 * TENSOR_GGUF_NOALLOC_SCRATCH_BYTES per GPU, held from load until the process ends; the call
 * allocates nothing, runs the plan tensor_gguf_gemm_group_v1 runs with the workspace
 * tensor_gguf_gemm_workspace_v1 reports and so gives the same bits, and refuses a shape whose
 * split would need more scratch (by construction none does: a split's partials cover at most
 * 256 tiles of 256 x 128 fp32).  Every partial read is written earlier in the same call, so
 * nothing needs clearing.  Calls share the array: an eager call on a different stream from the
 * previous eager call on the GPU first waits (hipStreamWaitEvent) for that call to finish, so
 * eager calls on several streams or threads take the scratch in turn.  Calls captured into a
 * graph are not ordered that way (a replay chooses its stream later): replays of such graphs,
 * and eager calls beside them, that overlap on one GPU race, and the caller serialises them.
 */
#define TENSOR_GGUF_NOALLOC_SCRATCH_BYTES (32u << 20)
int32_t tensor_gguf_gemm_group_noalloc_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Workspace bytes tensor_gguf_gemm_group_v1 would use for this shape (0: it does not split K):
 * n[0 .. count-1] are the matrices' row counts.
 */
int32_t tensor_gguf_gemm_workspace_v1(uint32_t type, int64_t m, int64_t k, const int64_t *n, uint32_t count,
                                      uint64_t *bytes, TensorErrorV1 *error);

/*
 * The plan tensor_gguf_gemm_group_v1 takes for this shape given workspace_bytes of workspace:
 * the pipelined GEMM's tile index and K split across workgroups, and whether the pipelined
 * kernel runs at all (0: each matrix takes the small-M kernel).  No counterpart in the
 * reference, whose showcase searches schedules per case (benchmarks/kernels/showcase/
 * benchmark.py:214-237): with the two entries below a caller re-times the plans the library
 * could take and checks the one it picks.
 */
int32_t tensor_gguf_gemm_plan_v1(uint32_t type, int64_t m, int64_t k, const int64_t *n, uint32_t count,
                                 uint64_t workspace_bytes, int32_t *tile, int32_t *splits, int32_t *pipelined,
                                 TensorErrorV1 *error);

/* Rows, columns and K wave groups per workgroup of pipelined-GEMM tile `tile` (an index from 0;
 * TENSOR_ERROR_ARGUMENT past the last tile).  No counterpart in the reference. */
int32_t tensor_gguf_gemm_tile_v1(int32_t tile, int32_t *bm, int32_t *bn, int32_t *ks, TensorErrorV1 *error);

/*
 * tensor_gguf_gemm_group_v1 on a plan the caller names, for plan sweeps: arguments
 * [x, w0, out0, .., w(c-1), out(c-1), workspace, type, tile, splits] with tile and splits uint32
 * scalars.  TENSOR_ERROR_ARGUMENT when the pipelined kernel cannot run that tile and split on the
 * shape, or the workspace is shorter than the split needs; the same bits as any other plan up to
 * fp32 summation order.  No counterpart in the reference (its schedule search times candidate
 * builds of one kernel, benchmark.py:214-237, :917-932).
 */
int32_t tensor_gguf_gemm_group_plan_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Decode GEMV on Q8_1-quantized activations with integer dot products, GGML's path for quantized
 * matrix-vector products, which the reference measures as its external GGML baseline
 * (benchmarks/kernels/showcase/external_baselines.py:24-58: "GGML may quantize F32 activations
 * to Q8_1", qualified at relative L2 <= 0.02 against the fp32 oracle).  Arguments [x, w, out,
 * type]: x fp16 or fp32 [M, K] (M <= TENSOR_GGUF_GEMV_MAX_M, M * K <= 98304), w the raw rows of
 * a Q4_0, Q8_0, Q4_K or Q6_K matrix, out fp16 or fp32 [M, N].  x is quantized in blocks of 32
 * (d = max|x| / 127, q = roundf(x / d), d and s = d * sum(q) kept as fp16); each weight block's
 * codes meet the activation codes in int32 dot products, scaled per block in fp32.  An
 * alternative to tensor_gguf_gemv_v1, whose numerics are the reference's fp32 decode.
 */
int32_t tensor_gguf_gemv_q8_1_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * The multi-row plan tensor_gguf_gemv_v1 takes for a Q4_K call with 2 <= m <= 8 rows: the kernel
 * (0 sector-aligned tiles with x staged in LDS, 1 multi-tile with x in LDS, 2 x read per wave,
 * 3 sector-aligned tiles with K split across workgroups, then the ranges added in order) and its
 * two launch fields (kernel 0: 16-row tiles per workgroup 1-3 and 1 to stage x before the weight
 * loads are issued; kernel 1: tiles per workgroup 1-2 and super-blocks per wave 2-3; kernel 2:
 * waves splitting K, 4 or 8, and 0; kernel 3: tiles per workgroup 1-16 and K ranges, 2 or 4).  kernel = -1 where the call takes another path
 * (m = 1, the other encodings).  No counterpart in the reference, whose showcase picks
 * schedules by timing them (benchmarks/kernels/showcase/benchmark.py:214-237).
 */
int32_t tensor_gguf_gemv_plan_v1(uint32_t type, int64_t m, int64_t k, int64_t n, int32_t *kernel, int32_t *a,
                                 int32_t *b, TensorErrorV1 *error);

/*
 * tensor_gguf_gemv_v1 for Q4_K at 2 <= M <= 8 on a plan the caller names, for plan sweeps:
 * arguments [x, w, out, type, kernel, a, b], the last three uint32 scalars as reported by
 * tensor_gguf_gemv_plan_v1.  TENSOR_ERROR_ARGUMENT where that kernel cannot run the shape with
 * those fields; results equal the library plan's up to fp32 summation order.  No counterpart in
 * the reference.
 */
int32_t tensor_gguf_gemv_variant_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Decode GEMV of an MLP's gate and up projections with the SwiGLU epilogue:
 * out[m, n] = silu(g) * u, silu(g) = g / (1 + exp(-g)), where g and u are the
 * fp32 sums x[m, :] . dequant(W_gate)[n, :] and x[m, :] . dequant(W_up)[n, :]
 * (nothing is rounded before the epilogue).  Replaces the reference's
 * two-RHS packed-integer matmul with its SwiGLU output
 * (src/tensor/compiler/webgpu/schedules/packed_integer.py:26-31, epilogue
 * :204-205); the showcase path would take two gemv_packed launches and an
 * elementwise kernel.  One launch: the Q4_K M = 1 kernel with gate and up rows
 * in one workgroup when K is a multiple of 4096 (at most 16384), else the
 * generic decode kernels with a gate / up row pair per wave.  Arguments:
 *   0 x      buffer fp16  [M, K], 1 <= M <= TENSOR_GGUF_GEMV_MAX_M
 *   1 w_gate buffer uint8 [N, K/QK*BLOCK]
 *   2 w_up   buffer uint8 [N, K/QK*BLOCK]
 *   3 out    buffer fp16 or fp32 [M, N]
 *   4 type   scalar uint32 GGML type id of both matrices
 */
int32_t tensor_gguf_gemv_swiglu_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/*
 * Dequantize raw GGUF rows: out[n, k] = dequant(W)[n, k], exact in fp32 and
 * round-to-nearest-even in fp16 (block decoding of
 * benchmarks/kernels/showcase/triton_kernels.py:134-181, the decode_ggml
 * device function).  Arguments, in order:
 *   0 w    buffer uint8 [N, K/QK*BLOCK]
 *   1 out  buffer fp16 or fp32 [N, K]
 *   2 type scalar uint32 GGML type id
 */
int32_t tensor_gguf_dequant_v1(const TensorCallV1 *call, TensorErrorV1 *error);

/* ---------------------------------------------------- runtime services --- */

typedef struct TensorHipDeviceInfoV1 {
  char name[256];
  char arch[64];             /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  uint64_t total_memory;     /* bytes */
  uint64_t l2_cache_bytes;
  int32_t compute_units;
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width;
  int32_t max_threads_per_block;
  int32_t max_shared_memory_per_block;
  int32_t warp_size;
  int32_t max_grid[3];
  int32_t max_block[3];
} TensorHipDeviceInfoV1;

int32_t tensor_hip_device_count(int32_t *count, TensorErrorV1 *error);
int32_t tensor_hip_device_info(int32_t ordinal, TensorHipDeviceInfoV1 *info,
                               TensorErrorV1 *error);
int32_t tensor_hip_set_device(int32_t ordinal, TensorErrorV1 *error);
int32_t tensor_hip_device_synchronize(TensorErrorV1 *error);

int32_t tensor_hip_malloc(uint64_t bytes, uint64_t *address, TensorErrorV1 *error);
int32_t tensor_hip_free(uint64_t address, TensorErrorV1 *error);
/* Which device an address belongs to, for DLPack imports (the reference checks an
 * imported pointer with cuPointerGetAttribute, src/tensor/providers/cuda/device.py:296-309):
 * *ordinal = the owning device, *device_memory = 1 for device (or managed) memory,
 * 0 for host memory.  An address this runtime does not know is TENSOR_ERROR_PROVIDER. */
int32_t tensor_hip_pointer_device(uint64_t address, int32_t *ordinal, int32_t *device_memory,
                                  TensorErrorV1 *error);
/* Host <-> device copies are synchronous with respect to the host. */
int32_t tensor_hip_copy_htod(uint64_t dst, const void *src, uint64_t bytes,
                             uint64_t stream, TensorErrorV1 *error);
int32_t tensor_hip_copy_dtoh(void *dst, uint64_t src, uint64_t bytes,
                             uint64_t stream, TensorErrorV1 *error);
/* Device copies, fills and 2-D copies are ordered on the stream. */
int32_t tensor_hip_copy_dtod(uint64_t dst, uint64_t src, uint64_t bytes,
                             uint64_t stream, TensorErrorV1 *error);
int32_t tensor_hip_copy_2d(uint64_t dst, uint64_t dst_pitch, uint64_t src,
                           uint64_t src_pitch, uint64_t width, uint64_t height,
                           uint64_t stream, TensorErrorV1 *error);
int32_t tensor_hip_fill_u8(uint64_t dst, uint8_t value, uint64_t bytes,
                           uint64_t stream, TensorErrorV1 *error);

int32_t tensor_hip_stream_create(uint64_t *stream, TensorErrorV1 *error);
int32_t tensor_hip_stream_destroy(uint64_t stream, TensorErrorV1 *error);
int32_t tensor_hip_stream_synchronize(uint64_t stream, TensorErrorV1 *error);
int32_t tensor_hip_stream_wait_event(uint64_t stream, uint64_t event,
                                     TensorErrorV1 *error);

int32_t tensor_hip_event_create(uint64_t *event, int32_t timing, TensorErrorV1 *error);
int32_t tensor_hip_event_destroy(uint64_t event, TensorErrorV1 *error);
int32_t tensor_hip_event_record(uint64_t event, uint64_t stream, TensorErrorV1 *error);
int32_t tensor_hip_event_synchronize(uint64_t event, TensorErrorV1 *error);
/* Sets *complete to 1 when the event has completed, else 0. */
int32_t tensor_hip_event_query(uint64_t event, int32_t *complete, TensorErrorV1 *error);
int32_t tensor_hip_event_elapsed(float *milliseconds, uint64_t start, uint64_t stop,
                                 TensorErrorV1 *error);

/* Stream capture into a graph (the reference's CudaGraph,
 * src/tensor/providers/cuda/graph.py:8-98). */
int32_t tensor_hip_capture_begin(uint64_t stream, TensorErrorV1 *error);
/* *graph_exec: an opaque handle of the instantiated graph (and the graph it was made from, kept
 * until tensor_hip_graph_destroy); 0 on failure. */
int32_t tensor_hip_capture_end(uint64_t stream, uint64_t *graph_exec, TensorErrorV1 *error);
int32_t tensor_hip_graph_launch(uint64_t graph_exec, uint64_t stream, TensorErrorV1 *error);
int32_t tensor_hip_graph_destroy(uint64_t graph_exec, TensorErrorV1 *error);

/* Hand-built code objects from `hip` artifacts (the reference's cuModuleLoadData /
 * cuModuleGetFunction / cuModuleUnload / cuLaunchKernel path,
 * src/tensor/providers/cuda/device.py:211-229, :359-389).  `image` is a gfx950
 * ELF code object; `*module` and `*function` are opaque handles. */
int32_t tensor_hip_module_load(const void *image, uint64_t bytes, uint64_t *module,
                               TensorErrorV1 *error);
int32_t tensor_hip_module_function(uint64_t module, const char *name, uint64_t *function,
                                   TensorErrorV1 *error);
int32_t tensor_hip_module_unload(uint64_t module, TensorErrorV1 *error);
/* Launches `function` with the call's grid, block, dynamic shared memory and
 * stream; argument i is passed by value in kernel-parameter order: a buffer as
 * its device address, a scalar as its dtype-sized payload.  Header and argument
 * descriptors are checked (ABI version, flags, ROCm stream and buffers on the
 * stream's device, launch bounds) before any HIP call.  The caller guarantees
 * the argument list matches the kernel's parameters (the Python loader checks
 * it against the code object's metadata). */
int32_t tensor_hip_module_launch_v1(uint64_t function, const TensorCallV1 *call,
                                    TensorErrorV1 *error);

/* Library build identity: "tensor_hip <abi> <arch>". */
const char *tensor_hip_version(void);
/* SHA-256 (hex) of the csrc/ and include/ files the library was built from; the Python
 * loader refuses a library whose hash differs from the sources beside it. */
const char *tensor_hip_source_hash(void);

#ifdef __cplusplus
}
#endif
#endif /* TENSOR_HIP_H */
