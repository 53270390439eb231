// Host-side launch descriptors shared by the GGUF kernel translation units.
// Shapes have been validated by the C-ABI entry points before these run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tensor_gguf {

struct GemvArgs {
  const void* x;   // fp16 [m, k] (fp32 when x_f32)
  const void* w;   // raw GGUF rows [n, row_bytes]
  void* out;       // fp16 or fp32 [m, n]
  int type;        // GGML type id
  int m, n, k;
  bool out_half;
  // fp32 activations (the packed call form): the M = 1 GEMV multiplies them in fp32, the
  // GEMM rounds them to fp16 as it stages its activation tiles
  bool x_f32 = false;
  // device memory for a multi-row GEMV plan that splits K across workgroups (its fp32 partial
  // sums); without it such a shape runs the plan that reads x per wave
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
};

struct DequantArgs {
  const void* w;   // raw GGUF rows [n, row_bytes]
  void* out;       // fp16 or fp32 [n, k]
  int type;
  int n, k;
  bool out_half;
};

// Largest M the decode GEMV entry accepts.
constexpr int kGemvMaxM = 8;

// Largest number of matrices one grouped decode GEMV launch covers.
constexpr int kGemvGroupMax = 3;

hipError_t launch_gemv(const GemvArgs& args, hipStream_t stream);
// Decode GEMV of fp32 activations at M = 1, every encoding (args.x_f32).
hipError_t launch_gemv_f32x(const GemvArgs& args, hipStream_t stream);
// Q4_K fast paths (LDS dot2 kernel for M = 1, MFMA kernel for M >= 2); sets
// *handled to false when the shape is not covered by them.
hipError_t launch_gemv_q4k_fast(const GemvArgs& args, hipStream_t stream, bool* handled);
// Grouped M = 1 Q4_K (or Q5_K) GEMV: `count` (<= kGemvGroupMax) matrices sharing x and K in one launch.
// n: the largest row count of the group (the kernel addresses a matrix with 32-bit offsets).
bool gemv_q4k_group_supported(int m, int k, int n);
// waves: rows (one per wave) per workgroup; 0 takes the default, 4 / 8 / 16 fix it (for sweeps)
hipError_t launch_gemv_q4k_group(const GemvArgs* args, int count, hipStream_t stream, int waves = 0);
// Two Q4_K matrices of one shape sharing x at 2 <= M <= 4 (K a multiple of 1024, at most 8192):
// one launch of the sector-aligned kernel with a tile of each per workgroup; *handled is false
// when x does not fit the kernel's LDS.
bool gemv_q4k_pair_supported(const GemvArgs* args, int count);
hipError_t launch_gemv_q4k_pair(const GemvArgs* args, hipStream_t stream, bool* handled);
// Multi-row Q4_K decode GEMV plans (2 <= M <= 8, fp16 x): the kernel and its launch shape.
//   kGemvSec  (gemv_q4k_sec):  a = 16-row tiles per workgroup (1-3), b = 1 to stage x before
//                              the weight loads are issued, 0 to issue them behind x
//   kGemvMt   (gemv_q4k_mt):   a = tiles per workgroup (1-2), b = super-blocks per wave (2-3)
//   kGemvMfma (gemv_q4k_mfma): a = waves per workgroup splitting K (4 or 8), b = 0
//   kGemvSecSplit (gemv_q4k_sec over K ranges, then gemv_q4k_sec_reduce): a = 16-row tiles per
//                              workgroup (1-16), b = K ranges (2 or 4); M >= 4, a workspace
enum { kGemvSec = 0, kGemvMt = 1, kGemvMfma = 2, kGemvSecSplit = 3 };
struct GemvPlan {
  int kernel, a, b;
};
// The plan the library takes for args; false where another path takes the call (other
// encodings, M = 1, M > 8, fp32 x).
bool gemv_q4k_plan(const GemvArgs& args, GemvPlan* plan);
// Whether plan fits args's shape (the launch limits of its kernel).
bool gemv_q4k_plan_fits(const GemvArgs& args, const GemvPlan& plan);
// Bytes of workspace a plan needs (args.workspace, args.workspace_bytes): 0 for all but kGemvSecSplit.
size_t gemv_q4k_plan_workspace(const GemvArgs& args, const GemvPlan& plan);
// Launch a plan that fits (hipErrorInvalidValue otherwise, also for a plan whose workspace
// args does not provide).
hipError_t launch_gemv_q4k_plan(const GemvArgs& args, const GemvPlan& plan, hipStream_t stream);
// Decode GEMV on Q8_1-quantized activations with integer dot products (GGML's path), Q4_0,
// Q8_0, Q4_K and Q6_K, M <= 8, fp16 or fp32 x (args.x_f32); x is quantized inside each
// workgroup, so M * K is bounded by LDS.
bool gemv_q8_1_supported(const GemvArgs& args);
hipError_t launch_gemv_q8_1(const GemvArgs& args, hipStream_t stream);
// Decode GEMV with the SwiGLU epilogue of an MLP: out = silu(x W_gate^T) * (x W_up^T),
// args.w the gate matrix, w_up the up matrix of the same shape and encoding.
hipError_t launch_gemv_swiglu(const GemvArgs& gate, const void* w_up, hipStream_t stream);
// Its fast paths: Q4_K / Q5_K at M = 1 (gate and up rows of one workgroup; waves: 8 or 16 per
// workgroup, 0 the default) and Q4_K at 2 <= M <= 8 (a gate tile and its up tile per workgroup).
hipError_t launch_gemv_q4k_swiglu_fast(const GemvArgs& gate, const void* w_up, hipStream_t stream, bool* handled,
                                       int waves = 0);
// fp32-activation fast path at M = 1 for Q4_K and Q5_K (K a multiple of 4096, at most 16384);
// *handled is false for the other shapes and encodings.
hipError_t launch_gemv_q4k_f32x(const GemvArgs& args, hipStream_t stream, bool* handled);
// The same for Q6_K (K in {4096, 8192, 12288}).
hipError_t launch_gemv_q6k_f32x(const GemvArgs& args, hipStream_t stream, bool* handled);
// Q5_K fast path (the M = 1 Q4_K kernel with the fifth bits; K a multiple of 4096, at most 16384).
hipError_t launch_gemv_q5k_fast(const GemvArgs& args, hipStream_t stream, bool* handled);
// Q6_K fast path (LDS-staged x, M = 1, K in {4096, 8192, 12288}).
hipError_t launch_gemv_q6k_fast(const GemvArgs& args, hipStream_t stream, bool* handled);
// Q2_K / Q3_K fast path (LDS-staged x, per-sub-block decode, M = 1, K in {4096, 8192, 12288, 16384}).
hipError_t launch_gemv_q23k_fast(const GemvArgs& args, hipStream_t stream, bool* handled);
hipError_t launch_dequant(const DequantArgs& args, hipStream_t stream);
hipError_t launch_gemm(const GemvArgs& args, hipStream_t stream);

// Prefill GEMM of up to kGemmGroupMax matrices that share x and K in one launch (a layer's q, k
// and v, or gate and up), optionally with K split across workgroups.
constexpr int kGemmGroupMax = 3;
struct GemmGroupArgs {
  const void* x;                 // fp16 [m, k] (fp32 when x_f32)
  const void* w[kGemmGroupMax];  // raw GGUF rows [n_i, row_bytes]
  void* out[kGemmGroupMax];      // fp16 or fp32 [m, n_i]
  int n[kGemmGroupMax];
  int count;
  int type, m, k;
  bool out_half, x_f32;
};
// What one launch of gemm_pipe reads (kernel argument): per-matrix pointers, column-tile
// boundaries, and for a split launch the fp32 partial sums [splits][m][n_total].
struct GemmJob {
  const uint8_t* w[kGemmGroupMax];
  void* out[kGemmGroupMax];
  int n[kGemmGroupMax];
  int tile_end[kGemmGroupMax];  // cumulative column tiles of matrices 0..i
  int col0[kGemmGroupMax];      // first column of matrix i in the partial sums
  int count, n_total, splits;
  float* partial;
};
// A workgroup tile (index into the pipelined GEMM's tile table) and a cross-workgroup K split.
struct GemmPlan {
  int tile, splits;
  bool small_m = false;  // M <= 64: this plan replaces one small-M launch per matrix
};
// The plan for a shape given the workspace available (0: no cross-workgroup split).
GemmPlan plan_gemm_group(const GemmGroupArgs& args, size_t workspace_bytes);
// Bytes of fp32 partial sums a plan needs (0 when it does not split K).
size_t gemm_group_workspace(const GemmGroupArgs& args, const GemmPlan& plan);
// Whether the pipelined kernel runs this group under this plan: Q4_K, Q5_K, Q6_K, Q8_0 and
// Q4_0, with K whole 64-element steps that the plan's wave groups and splits share evenly.
bool gemm_group_pipelined(const GemmGroupArgs& args, const GemmPlan& plan);
// The pipelined kernel; hipErrorInvalidValue where gemm_group_pipelined is false or the
// workspace is short.  A split plan also launches the in-order reduction of the partial sums.
hipError_t launch_gemm_group_plan(const GemmGroupArgs& args, const GemmPlan& plan, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream);
// Whether the pipelined kernel covers this single-matrix shape (as launch_gemm_pipe runs it).
bool gemm_pipe_supported(const GemvArgs& args);
// Pipelined dequant-GEMM of one matrix; sets *handled to false for the encodings and shapes it
// does not cover.
hipError_t launch_gemm_pipe(const GemvArgs& args, hipStream_t stream, bool* handled);
// Rows, columns and K wave groups of pipelined-GEMM tile `tile`; false past the last tile.
bool gemm_tile_geometry(int tile, int* bm, int* bn, int* ks);
// One tile configuration of the pipelined GEMM by index (tile sweeps and tests).
hipError_t launch_gemm_pipe_config(const GemvArgs& args, hipStream_t stream, int config);

// Small-M dequant-GEMM, every encoding (M <= kSkinnyMaxM, K a multiple of 32): weights
// dequantized into MFMA operands in registers, K split over the 8 waves of a workgroup of
// 16 nt rows of W (nt 1, 2 or 4) and 16 mt rows of x (mt 1, 2 or 4); 0 chooses by shape.
constexpr int kSkinnyMaxM = 64;
bool gemm_skinny_supported(const GemvArgs& args);
hipError_t launch_gemm_skinny(const GemvArgs& args, hipStream_t stream, int nt = 0, int mt = 0);
// Whether launch_gemm takes the small-M kernel for this shape.
bool gemm_small_m(const GemvArgs& args);

}  // namespace tensor_gguf
