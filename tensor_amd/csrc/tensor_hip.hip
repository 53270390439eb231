// C-ABI entry points of libtensor_hip.so: GGUF kernels in the TensorKernelV1
// shape and the runtime services the Python provider binds with ctypes.
// Declarations and their reference counterparts: include/tensor_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>

#include "gguf_launch.h"
#include "tensor_hip.h"

// Scratch of tensor_gguf_gemm_group_noalloc_v1: the fp32 partial sums of a K split.  A split
// plan keeps splits x (256 x 128 tiles) <= 256 workgroups and its partials cover at most
// those tiles, so splits * M * N_total * 4 <= 256 * 256 * 128 * 4 bytes = 32 MiB for any shape.
// Each GPU the library runs on holds its own copy until the process ends.  Host code never
// uses the array's name as an address: scratch_address() resolves this device's copy.
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kScratchDevices = 64;
std::mutex scratch_mutex;

// Per device: the scratch copy's address (nullptr until resolved) and the last eager use of it,
// the stream it ran on and an event recorded after it.
struct ScratchState {
  void* address;
  hipEvent_t done;
  hipStream_t last;
  bool used;
};
ScratchState scratch_state[kScratchDevices];

// The current device's scratch state, set up once per device with that device current (the
// caller has checked that the stream's ordinal is the current device): the copy's address and
// the event that orders eager calls on different streams.  Call with scratch_mutex held.
hipError_t scratch_setup(int ordinal, ScratchState** state) {
  if (ordinal < 0 || ordinal >= kScratchDevices) return hipErrorInvalidDevice;
  ScratchState& s = scratch_state[ordinal];
  if (!s.address) {
    void* resolved = nullptr;
    hipError_t status = hipGetSymbolAddress(&resolved, HIP_SYMBOL(scratch));
    if (status != hipSuccess) return status;
    if (!resolved) return hipErrorInvalidSymbol;
    status = hipEventCreateWithFlags(&s.done, hipEventDisableTiming);
    if (status != hipSuccess) return status;
    s.address = resolved;
  }
  *state = &s;
  return hipSuccess;
}

int32_t fail(TensorErrorV1* error, int32_t code, const char* format, ...) {
  if (error) {
    error->code = code;
    va_list args;
    va_start(args, format);
    std::vsnprintf(error->message, sizeof(error->message), format, args);
    va_end(args);
  }
  return code;
}

int32_t ok(TensorErrorV1* error) {
  if (error) {
    error->code = TENSOR_OK;
    error->message[0] = 0;
  }
  return TENSOR_OK;
}

int32_t hip_fail(TensorErrorV1* error, hipError_t status, const char* what) {
  return fail(error, TENSOR_ERROR_PROVIDER, "%s: %s (%s, %d)", what, hipGetErrorString(status),
              hipGetErrorName(status), (int)status);
}

#define HIP_TRY(expr, what)                                  \
  do {                                                       \
    hipError_t status_ = (expr);                             \
    if (status_ != hipSuccess) return hip_fail(error, status_, what); \
  } while (0)

struct Format {
  int qk;
  int bytes;
};

bool ggml_format(uint64_t type, Format* format) {
  switch (type) {
    case TENSOR_GGML_Q4_0: *format = {32, 18}; return true;
    case TENSOR_GGML_Q4_1: *format = {32, 20}; return true;
    case TENSOR_GGML_Q5_0: *format = {32, 22}; return true;
    case TENSOR_GGML_Q5_1: *format = {32, 24}; return true;
    case TENSOR_GGML_Q8_0: *format = {32, 34}; return true;
    case TENSOR_GGML_Q2_K: *format = {256, 84}; return true;
    case TENSOR_GGML_Q3_K: *format = {256, 110}; return true;
    case TENSOR_GGML_Q4_K: *format = {256, 144}; return true;
    case TENSOR_GGML_Q5_K: *format = {256, 176}; return true;
    case TENSOR_GGML_Q6_K: *format = {256, 210}; return true;
    default: return false;
  }
}

// Common header checks of every kernel call (src/tensor/compiler/cpu.py:59-66).
// Pure descriptor checks only: nothing here touches the HIP runtime, so every
// argument error is reported before any device state is consulted.
int32_t check_call(const TensorCallV1* call, uint32_t arguments, TensorErrorV1* error) {
  if (!call || call->abi_version != TENSOR_ABI_VERSION || call->struct_size < sizeof(TensorCallV1))
    return fail(error, TENSOR_ERROR_ABI, "unsupported call ABI");
  if (call->flags || call->argument_count != arguments || !call->arguments)
    return fail(error, TENSOR_ERROR_ARGUMENT, "invalid argument count or flags");
  if (call->stream.device_type != TENSOR_DEVICE_ROCM || call->stream.device_ordinal < 0)
    return fail(error, TENSOR_ERROR_PROVIDER, "ROCm calls need a ROCm stream");
  return TENSOR_OK;
}

// The stream's ordinal must be the calling thread's current HIP device.
int32_t check_device(const TensorCallV1* call, TensorErrorV1* error) {
  int device = -1;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return hip_fail(error, status, "hipGetDevice");
  if (call->stream.device_ordinal != device)
    return fail(error, TENSOR_ERROR_PROVIDER, "stream ordinal %d is not the current device %d",
                (int)call->stream.device_ordinal, device);
  return TENSOR_OK;
}

// One call's use of the library's scratch (after check_device).  The scratch is one array per
// device: an eager call on another stream than the previous eager call first waits for that
// call's event, and the lease holds scratch_mutex from acquire to release so that host threads
// cannot interleave between the wait and the record.  Under stream capture nothing is waited for
// or recorded (the graph's replays choose their streams later).
class ScratchLease {
 public:
  int32_t acquire(const TensorCallV1* call, hipStream_t stream, TensorErrorV1* error) {
    lock_.lock();
    hipError_t status = scratch_setup(call->stream.device_ordinal, &state_);
    if (status != hipSuccess) return hip_fail(error, status, "scratch set-up");
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    status = hipStreamIsCapturing(stream, &capture);
    if (status != hipSuccess) return hip_fail(error, status, "hipStreamIsCapturing");
    eager_ = capture == hipStreamCaptureStatusNone;
    if (eager_ && state_->used && state_->last != stream) {
      status = hipStreamWaitEvent(stream, state_->done, 0);
      if (status != hipSuccess) return hip_fail(error, status, "hipStreamWaitEvent(scratch)");
    }
    return TENSOR_OK;
  }
  // After the call's launches: an eager call records its event.
  int32_t release(hipStream_t stream, TensorErrorV1* error) {
    if (eager_) {
      const hipError_t status = hipEventRecord(state_->done, stream);
      if (status != hipSuccess) return hip_fail(error, status, "hipEventRecord(scratch)");
      state_->last = stream;
      state_->used = true;
    }
    return TENSOR_OK;
  }
  void* address() const { return state_->address; }

 private:
  std::unique_lock<std::mutex> lock_{scratch_mutex, std::defer_lock};
  ScratchState* state_ = nullptr;
  bool eager_ = false;
};

// A multi-row Q4_K GEMV whose plan splits K across workgroups takes its partial sums in the
// scratch: the lease is taken when the plan needs one (a Q4_K call with 2 <= M <= 8).
int32_t gemv_workspace(const TensorCallV1* call, tensor_gguf::GemvArgs* args, const tensor_gguf::GemvPlan& plan,
                       hipStream_t stream, ScratchLease* lease, bool* leased, TensorErrorV1* error) {
  *leased = false;
  const size_t need = tensor_gguf::gemv_q4k_plan_workspace(*args, plan);
  if (need == 0 || need > kScratchBytes) return TENSOR_OK;  // beyond the scratch: the plan without it
  if (int32_t s = lease->acquire(call, stream, error)) return s;
  *leased = true;
  args->workspace = lease->address();
  args->workspace_bytes = kScratchBytes;
  return TENSOR_OK;
}

// A rank-2 contiguous device buffer of one of the allowed dtypes.
int32_t check_matrix(const TensorArgumentV1& arg, const char* name, int ordinal, uint32_t dtype_a,
                     uint32_t dtype_b, TensorErrorV1* error) {
  const TensorBufferV1& b = arg.buffer;
  if (arg.kind != TENSOR_ARG_BUFFER || (arg.dtype != dtype_a && arg.dtype != dtype_b) ||
      b.dtype != arg.dtype)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: wrong argument kind or dtype", name);
  if (b.device_type != TENSOR_DEVICE_ROCM || b.device_ordinal != ordinal || !b.address ||
      b.address % 16 || b.rank != 2 || !b.shape || !b.strides)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: invalid buffer descriptor", name);
  const uint64_t item = arg.dtype == TENSOR_UINT8 ? 1 : arg.dtype == TENSOR_FLOAT16 ? 2 : 4;
  uint64_t bytes = item;
  for (int axis = 1; axis >= 0; --axis) {
    if (b.shape[axis] <= 0 || b.shape[axis] >= (int64_t)1 << 31 ||
        b.strides[axis] != (int64_t)bytes)
      return fail(error, TENSOR_ERROR_ARGUMENT, "%s: shape, stride or size mismatch", name);
    bytes *= (uint64_t)b.shape[axis];
  }
  if (b.byte_size < bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: insufficient buffer storage", name);
  return TENSOR_OK;
}

int32_t check_type(const TensorArgumentV1& arg, Format* format, TensorErrorV1* error) {
  if (arg.kind != TENSOR_ARG_SCALAR || arg.dtype != TENSOR_UINT32)
    return fail(error, TENSOR_ERROR_ARGUMENT, "type: wrong argument kind or dtype");
  if (arg.scalar >> 32)
    return fail(error, TENSOR_ERROR_ARGUMENT, "type: noncanonical scalar payload");
  if (!ggml_format(arg.scalar, format))
    return fail(error, TENSOR_ERROR_ARGUMENT, "type: unsupported GGML type %llu",
                (unsigned long long)arg.scalar);
  return TENSOR_OK;
}

enum class Op { kGemv, kGemm, kLinear };

int32_t linear_call(const TensorCallV1* call, TensorErrorV1* error, Op op) {
  ok(error);
  if (int32_t s = check_call(call, 4, error)) return s;
  const int ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  Format format;
  if (int32_t s = check_type(a[3], &format, error)) return s;
  if (int32_t s = check_matrix(a[0], "x", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT16, error)) return s;
  if (int32_t s = check_matrix(a[1], "w", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
  if (int32_t s = check_matrix(a[2], "out", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
  const int64_t m = a[0].buffer.shape[0], k = a[0].buffer.shape[1], n = a[1].buffer.shape[0];
  if (k % format.qk || a[1].buffer.shape[1] != k / format.qk * format.bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "w: shape, stride or size mismatch");
  if (a[2].buffer.shape[0] != m || a[2].buffer.shape[1] != n)
    return fail(error, TENSOR_ERROR_ARGUMENT, "out: shape, stride or size mismatch");
  if (op == Op::kGemv && m > tensor_gguf::kGemvMaxM)
    return fail(error, TENSOR_ERROR_ARGUMENT, "x: decode GEMV takes at most %d rows",
                tensor_gguf::kGemvMaxM);
  if (int32_t s = check_device(call, error)) return s;
  tensor_gguf::GemvArgs args;
  args.x = reinterpret_cast<const void*>(a[0].buffer.address);
  args.w = reinterpret_cast<const void*>(a[1].buffer.address);
  args.out = reinterpret_cast<void*>(a[2].buffer.address);
  args.type = (int)a[3].scalar;
  args.m = (int)m;
  args.n = (int)n;
  args.k = (int)k;
  args.out_half = a[2].dtype == TENSOR_FLOAT16;
  hipStream_t stream = reinterpret_cast<hipStream_t>(call->stream.handle);
  const bool gemv = op == Op::kGemv || (op == Op::kLinear && m <= tensor_gguf::kGemvMaxM);
  ScratchLease lease;
  bool leased = false;
  tensor_gguf::GemvPlan plan;
  if (gemv && tensor_gguf::gemv_q4k_plan(args, &plan))
    if (int32_t s = gemv_workspace(call, &args, plan, stream, &lease, &leased, error)) return s;
  hipError_t status = gemv ? tensor_gguf::launch_gemv(args, stream) : tensor_gguf::launch_gemm(args, stream);
  if (status != hipSuccess) return hip_fail(error, status, gemv ? "GGUF GEMV launch" : "GGUF GEMM launch");
  return leased ? lease.release(stream, error) : TENSOR_OK;
}

// Grouped decode GEMV: x shared by `count` (w, out) pairs, arguments
// [x, w0, out0, .., w(c-1), out(c-1), type].
int32_t group_call(const TensorCallV1* call, TensorErrorV1* error) {
  ok(error);
  if (!call || call->abi_version != TENSOR_ABI_VERSION || call->struct_size < sizeof(TensorCallV1))
    return fail(error, TENSOR_ERROR_ABI, "unsupported call ABI");
  const uint32_t argc = call->argument_count;
  if (argc < 4 || argc > 2 + 2 * tensor_gguf::kGemvGroupMax || argc % 2)
    return fail(error, TENSOR_ERROR_ARGUMENT, "invalid argument count or flags");
  if (int32_t s = check_call(call, argc, error)) return s;
  const int count = (int)(argc - 2) / 2;
  const int ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  Format format;
  if (int32_t s = check_type(a[argc - 1], &format, error)) return s;
  if (int32_t s = check_matrix(a[0], "x", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT16, error)) return s;
  const int64_t m = a[0].buffer.shape[0], k = a[0].buffer.shape[1];
  if (m > tensor_gguf::kGemvMaxM)
    return fail(error, TENSOR_ERROR_ARGUMENT, "x: decode GEMV takes at most %d rows", tensor_gguf::kGemvMaxM);
  if (k % format.qk) return fail(error, TENSOR_ERROR_ARGUMENT, "x: K is not a multiple of the block size");
  tensor_gguf::GemvArgs args[tensor_gguf::kGemvGroupMax];
  for (int i = 0; i < count; ++i) {
    const TensorArgumentV1& w = a[1 + 2 * i];
    const TensorArgumentV1& out = a[2 + 2 * i];
    if (int32_t s = check_matrix(w, "w", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
    if (int32_t s = check_matrix(out, "out", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
    const int64_t n = w.buffer.shape[0];
    if (w.buffer.shape[1] != k / format.qk * format.bytes)
      return fail(error, TENSOR_ERROR_ARGUMENT, "w%d: shape, stride or size mismatch", i);
    if (out.buffer.shape[0] != m || out.buffer.shape[1] != n || out.dtype != a[2].dtype)
      return fail(error, TENSOR_ERROR_ARGUMENT, "out%d: shape, stride, size or dtype mismatch", i);
    args[i].x = reinterpret_cast<const void*>(a[0].buffer.address);
    args[i].w = reinterpret_cast<const void*>(w.buffer.address);
    args[i].out = reinterpret_cast<void*>(out.buffer.address);
    args[i].type = (int)a[argc - 1].scalar;
    args[i].m = (int)m;
    args[i].n = (int)n;
    args[i].k = (int)k;
    args[i].out_half = out.dtype == TENSOR_FLOAT16;
  }
  if (int32_t s = check_device(call, error)) return s;
  hipStream_t stream = reinterpret_cast<hipStream_t>(call->stream.handle);
  hipError_t status = hipSuccess;
  bool paired = false;
  int widest = 0;
  for (int i = 0; i < count; ++i) widest = std::max(widest, args[i].n);
  if ((args[0].type == (int)TENSOR_GGML_Q4_K || args[0].type == (int)TENSOR_GGML_Q5_K) &&
      tensor_gguf::gemv_q4k_group_supported((int)m, (int)k, widest)) {
    status = tensor_gguf::launch_gemv_q4k_group(args, count, stream);
  } else if (tensor_gguf::gemv_q4k_pair_supported(args, count) &&
             (status = tensor_gguf::launch_gemv_q4k_pair(args, stream, &paired), paired)) {
    // two equal Q4_K matrices at M > 1: one launch of the multi-row kernel
  } else {
    // no grouped kernel for this shape or encoding: one launch per matrix, same stream order
    for (int i = 0; i < count && status == hipSuccess; ++i) status = tensor_gguf::launch_gemv(args[i], stream);
  }
  if (status != hipSuccess) return hip_fail(error, status, "GGUF grouped GEMV launch");
  return TENSOR_OK;
}

// Gate / up pair with the SwiGLU epilogue: arguments [x, w_gate, w_up, out, type].
int32_t swiglu_call(const TensorCallV1* call, TensorErrorV1* error) {
  ok(error);
  if (int32_t s = check_call(call, 5, error)) return s;
  const int ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  Format format;
  if (int32_t s = check_type(a[4], &format, error)) return s;
  if (int32_t s = check_matrix(a[0], "x", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT16, error)) return s;
  if (int32_t s = check_matrix(a[1], "w_gate", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
  if (int32_t s = check_matrix(a[2], "w_up", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
  if (int32_t s = check_matrix(a[3], "out", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
  const int64_t m = a[0].buffer.shape[0], k = a[0].buffer.shape[1], n = a[1].buffer.shape[0];
  if (m > tensor_gguf::kGemvMaxM)
    return fail(error, TENSOR_ERROR_ARGUMENT, "x: decode GEMV takes at most %d rows", tensor_gguf::kGemvMaxM);
  if (k % format.qk || a[1].buffer.shape[1] != k / format.qk * format.bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "w_gate: shape, stride or size mismatch");
  if (a[2].buffer.shape[0] != n || a[2].buffer.shape[1] != a[1].buffer.shape[1])
    return fail(error, TENSOR_ERROR_ARGUMENT, "w_up: shape differs from w_gate");
  if (a[3].buffer.shape[0] != m || a[3].buffer.shape[1] != n)
    return fail(error, TENSOR_ERROR_ARGUMENT, "out: shape, stride or size mismatch");
  if (int32_t s = check_device(call, error)) return s;
  tensor_gguf::GemvArgs args;
  args.x = reinterpret_cast<const void*>(a[0].buffer.address);
  args.w = reinterpret_cast<const void*>(a[1].buffer.address);
  args.out = reinterpret_cast<void*>(a[3].buffer.address);
  args.type = (int)a[4].scalar;
  args.m = (int)m;
  args.n = (int)n;
  args.k = (int)k;
  args.out_half = a[3].dtype == TENSOR_FLOAT16;
  hipError_t status = tensor_gguf::launch_gemv_swiglu(args, reinterpret_cast<const void*>(a[2].buffer.address),
                                                      reinterpret_cast<hipStream_t>(call->stream.handle));
  if (status != hipSuccess) return hip_fail(error, status, "GGUF SwiGLU GEMV launch");
  return TENSOR_OK;
}

// A contiguous device buffer of any rank holding `items` elements of one of the allowed
// dtypes (dtype_b == 0: any integer dtype, the raw-byte argument of the packed form).
int32_t check_flat(const TensorArgumentV1& arg, const char* name, int ordinal, uint32_t dtype_a, uint32_t dtype_b,
                   uint64_t bytes_wanted, TensorErrorV1* error) {
  const TensorBufferV1& b = arg.buffer;
  uint64_t item = 0;
  switch (arg.dtype) {
    case TENSOR_INT8: case TENSOR_UINT8: item = 1; break;
    case TENSOR_INT16: case TENSOR_UINT16: case TENSOR_FLOAT16: item = 2; break;
    case TENSOR_INT32: case TENSOR_UINT32: case TENSOR_FLOAT32: item = 4; break;
    case TENSOR_INT64: case TENSOR_UINT64: item = 8; break;
    default: break;
  }
  const bool integer = arg.dtype >= TENSOR_INT8 && arg.dtype <= TENSOR_UINT64;
  const bool allowed = dtype_b == 0 ? integer : (arg.dtype == dtype_a || arg.dtype == dtype_b);
  if (arg.kind != TENSOR_ARG_BUFFER || !allowed || !item || b.dtype != arg.dtype)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: wrong argument kind or dtype", name);
  if (b.device_type != TENSOR_DEVICE_ROCM || b.device_ordinal != ordinal || !b.address || b.address % 16 ||
      b.rank < 1 || b.rank > 8 || !b.shape || !b.strides)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: invalid buffer descriptor", name);
  uint64_t bytes = item;
  for (int axis = (int)b.rank - 1; axis >= 0; --axis) {
    if (b.shape[axis] <= 0 || b.shape[axis] >= (int64_t)1 << 40 || b.strides[axis] != (int64_t)bytes)
      return fail(error, TENSOR_ERROR_ARGUMENT, "%s: shape, stride or size mismatch", name);
    bytes *= (uint64_t)b.shape[axis];
    if (bytes > ((uint64_t)1 << 46))
      return fail(error, TENSOR_ERROR_ARGUMENT, "%s: shape, stride or size mismatch", name);
  }
  if (bytes != bytes_wanted)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: holds %llu bytes, the shape needs %llu", name,
                (unsigned long long)bytes, (unsigned long long)bytes_wanted);
  if (b.byte_size < bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: insufficient buffer storage", name);
  return TENSOR_OK;
}

int32_t check_u32(const TensorArgumentV1& arg, const char* name, uint64_t* value, TensorErrorV1* error) {
  if (arg.kind != TENSOR_ARG_SCALAR || arg.dtype != TENSOR_UINT32)
    return fail(error, TENSOR_ERROR_ARGUMENT, "%s: wrong argument kind or dtype", name);
  if (arg.scalar >> 32) return fail(error, TENSOR_ERROR_ARGUMENT, "%s: noncanonical scalar payload", name);
  *value = arg.scalar;
  return TENSOR_OK;
}

// The Q8_1-activation integer-dot decode GEMV: [x, w, out, type], x fp16 or fp32 [M, K].
int32_t gemv_q8_1_call(const TensorCallV1* call, TensorErrorV1* error) {
  ok(error);
  if (int32_t s = check_call(call, 4, error)) return s;
  const int ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  Format format;
  if (int32_t s = check_type(a[3], &format, error)) return s;
  if (int32_t s = check_matrix(a[0], "x", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
  if (int32_t s = check_matrix(a[1], "w", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
  if (int32_t s = check_matrix(a[2], "out", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
  const int64_t m = a[0].buffer.shape[0], k = a[0].buffer.shape[1], n = a[1].buffer.shape[0];
  if (k % format.qk || a[1].buffer.shape[1] != k / format.qk * format.bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "w: shape, stride or size mismatch");
  if (a[2].buffer.shape[0] != m || a[2].buffer.shape[1] != n)
    return fail(error, TENSOR_ERROR_ARGUMENT, "out: shape, stride or size mismatch");
  tensor_gguf::GemvArgs args;
  args.x = reinterpret_cast<const void*>(a[0].buffer.address);
  args.w = reinterpret_cast<const void*>(a[1].buffer.address);
  args.out = reinterpret_cast<void*>(a[2].buffer.address);
  args.type = (int)a[3].scalar;
  args.m = (int)m;
  args.n = (int)n;
  args.k = (int)k;
  args.out_half = a[2].dtype == TENSOR_FLOAT16;
  args.x_f32 = a[0].dtype == TENSOR_FLOAT32;
  if (!tensor_gguf::gemv_q8_1_supported(args))
    return fail(error, TENSOR_ERROR_ARGUMENT,
                "Q8_1 activation GEMV takes Q4_0, Q8_0, Q4_K or Q6_K, M <= %d and M * K <= 98304",
                tensor_gguf::kGemvMaxM);
  if (int32_t s = check_device(call, error)) return s;
  hipError_t status = tensor_gguf::launch_gemv_q8_1(args, reinterpret_cast<hipStream_t>(call->stream.handle));
  if (status != hipSuccess) return hip_fail(error, status, "GGUF Q8_1 GEMV launch");
  return TENSOR_OK;
}

// The multi-row Q4_K decode GEMV on a plan the caller names: [x, w, out, type, kernel, a, b]
// (the plan fields of tensor_gguf::GemvPlan as uint32 scalars).
int32_t gemv_variant_call(const TensorCallV1* call, TensorErrorV1* error) {
  ok(error);
  if (int32_t s = check_call(call, 7, error)) return s;
  const int ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  Format format;
  if (int32_t s = check_type(a[3], &format, error)) return s;
  uint64_t kernel = 0, pa = 0, pb = 0;
  if (int32_t s = check_u32(a[4], "kernel", &kernel, error)) return s;
  if (int32_t s = check_u32(a[5], "a", &pa, error)) return s;
  if (int32_t s = check_u32(a[6], "b", &pb, error)) return s;
  if (int32_t s = check_matrix(a[0], "x", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT16, error)) return s;
  if (int32_t s = check_matrix(a[1], "w", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
  if (int32_t s = check_matrix(a[2], "out", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
  const int64_t m = a[0].buffer.shape[0], k = a[0].buffer.shape[1], n = a[1].buffer.shape[0];
  if (k % format.qk || a[1].buffer.shape[1] != k / format.qk * format.bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "w: shape, stride or size mismatch");
  if (a[2].buffer.shape[0] != m || a[2].buffer.shape[1] != n)
    return fail(error, TENSOR_ERROR_ARGUMENT, "out: shape, stride or size mismatch");
  tensor_gguf::GemvArgs args;
  args.x = reinterpret_cast<const void*>(a[0].buffer.address);
  args.w = reinterpret_cast<const void*>(a[1].buffer.address);
  args.out = reinterpret_cast<void*>(a[2].buffer.address);
  args.type = (int)a[3].scalar;
  args.m = (int)m;
  args.n = (int)n;
  args.k = (int)k;
  args.out_half = a[2].dtype == TENSOR_FLOAT16;
  tensor_gguf::GemvPlan probe;
  if (!tensor_gguf::gemv_q4k_plan(args, &probe))
    return fail(error, TENSOR_ERROR_ARGUMENT, "multi-row GEMV plans take Q4_K with 2 <= M <= 8");
  const tensor_gguf::GemvPlan plan{(int)kernel, (int)pa, (int)pb};
  if (kernel > 3 || pa > 16 || pb > 16 || !tensor_gguf::gemv_q4k_plan_fits(args, plan))
    return fail(error, TENSOR_ERROR_ARGUMENT, "GEMV plan (%u, %u, %u) does not fit this shape", (unsigned)kernel,
                (unsigned)pa, (unsigned)pb);
  if (tensor_gguf::gemv_q4k_plan_workspace(args, plan) > kScratchBytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "GEMV plan (%u, %u, %u): its partial sums exceed the scratch",
                (unsigned)kernel, (unsigned)pa, (unsigned)pb);
  if (int32_t s = check_device(call, error)) return s;
  hipStream_t stream = reinterpret_cast<hipStream_t>(call->stream.handle);
  ScratchLease lease;
  bool leased = false;
  if (int32_t s = gemv_workspace(call, &args, plan, stream, &lease, &leased, error)) return s;
  hipError_t status = tensor_gguf::launch_gemv_q4k_plan(args, plan, stream);
  if (status != hipSuccess) return hip_fail(error, status, "GGUF GEMV launch");
  return leased ? lease.release(stream, error) : TENSOR_OK;
}

// The packed call form: [x, w, out, type, m, n, k] with flat buffers (see tensor_hip.h).
int32_t packed_call(const TensorCallV1* call, TensorErrorV1* error) {
  ok(error);
  if (int32_t s = check_call(call, 7, error)) return s;
  const int ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  Format format;
  if (int32_t s = check_type(a[3], &format, error)) return s;
  uint64_t m = 0, n = 0, k = 0;
  if (int32_t s = check_u32(a[4], "m", &m, error)) return s;
  if (int32_t s = check_u32(a[5], "n", &n, error)) return s;
  if (int32_t s = check_u32(a[6], "k", &k, error)) return s;
  if (!m || !n || !k || m >= (1u << 31) || n >= (1u << 31) || k >= (1u << 31) || k % format.qk)
    return fail(error, TENSOR_ERROR_ARGUMENT, "m, n, k: must be positive int32 with k a multiple of %d", format.qk);
  const uint64_t x_item = a[0].dtype == TENSOR_FLOAT32 ? 4 : 2, out_item = a[2].dtype == TENSOR_FLOAT32 ? 4 : 2;
  if (int32_t s = check_flat(a[0], "x", ordinal, TENSOR_FLOAT32, TENSOR_FLOAT16, m * k * x_item, error)) return s;
  if (int32_t s = check_flat(a[1], "w", ordinal, TENSOR_UINT8, 0, n * (k / format.qk) * format.bytes, error)) return s;
  if (int32_t s = check_flat(a[2], "out", ordinal, TENSOR_FLOAT32, TENSOR_FLOAT16, m * n * out_item, error)) return s;
  if (int32_t s = check_device(call, error)) return s;
  tensor_gguf::GemvArgs args;
  args.x = reinterpret_cast<const void*>(a[0].buffer.address);
  args.w = reinterpret_cast<const void*>(a[1].buffer.address);
  args.out = reinterpret_cast<void*>(a[2].buffer.address);
  args.type = (int)a[3].scalar;
  args.m = (int)m;
  args.n = (int)n;
  args.k = (int)k;
  args.out_half = a[2].dtype == TENSOR_FLOAT16;
  args.x_f32 = a[0].dtype == TENSOR_FLOAT32;
  hipStream_t stream = reinterpret_cast<hipStream_t>(call->stream.handle);
  // the showcase's dispatch: gemv_packed for m == 1, _packed otherwise (kernels.py:114-119)
  hipError_t status;
  if (m == 1) status = args.x_f32 ? tensor_gguf::launch_gemv_f32x(args, stream) : tensor_gguf::launch_gemv(args, stream);
  else status = tensor_gguf::launch_gemm(args, stream);
  if (status != hipSuccess) return hip_fail(error, status, m == 1 ? "GGUF packed GEMV launch" : "GGUF packed GEMM launch");
  return TENSOR_OK;
}

// Grouped prefill GEMM: [x, w0, out0, .., w(c-1), out(c-1), workspace, type] with a caller's
// workspace (has_workspace), or [x, w0, out0, .., type] on the library's static scratch.
// The scratch form runs the plan the caller's form runs with the workspace that
// tensor_gguf_gemm_workspace_v1 reports, so the two give the same bits.
// forced: the plan comes from two trailing uint32 scalars (tile, splits) after the type.
int32_t gemm_group_call(const TensorCallV1* call, TensorErrorV1* error, bool has_workspace, bool forced = false) {
  ok(error);
  if (!call || call->abi_version != TENSOR_ABI_VERSION || call->struct_size < sizeof(TensorCallV1))
    return fail(error, TENSOR_ERROR_ABI, "unsupported call ABI");
  const uint32_t tail = forced ? 2 : 0;  // scalars after the type
  const uint32_t argc = call->argument_count, fixed = (has_workspace ? 3 : 2) + tail;
  if (argc < fixed + 2 || argc > fixed + 2 * tensor_gguf::kGemmGroupMax || (argc - fixed) % 2)
    return fail(error, TENSOR_ERROR_ARGUMENT, "invalid argument count or flags");
  if (int32_t s = check_call(call, argc, error)) return s;
  const int count = (int)(argc - fixed) / 2, ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  uint64_t forced_tile = 0, forced_splits = 0;
  if (forced) {
    if (int32_t s = check_u32(a[argc - 2], "tile", &forced_tile, error)) return s;
    if (int32_t s = check_u32(a[argc - 1], "splits", &forced_splits, error)) return s;
  }
  Format format;
  if (int32_t s = check_type(a[argc - 1 - tail], &format, error)) return s;
  if (int32_t s = check_matrix(a[0], "x", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT16, error)) return s;
  const int64_t m = a[0].buffer.shape[0], k = a[0].buffer.shape[1];
  if (k % format.qk) return fail(error, TENSOR_ERROR_ARGUMENT, "x: K is not a multiple of the block size");
  tensor_gguf::GemmGroupArgs group{};
  group.x = reinterpret_cast<const void*>(a[0].buffer.address);
  for (int i = 0; i < count; ++i) {
    const TensorArgumentV1& w = a[1 + 2 * i];
    const TensorArgumentV1& out = a[2 + 2 * i];
    if (int32_t s = check_matrix(w, "w", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
    if (int32_t s = check_matrix(out, "out", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
    if (w.buffer.shape[1] != k / format.qk * format.bytes)
      return fail(error, TENSOR_ERROR_ARGUMENT, "w%d: shape, stride or size mismatch", i);
    if (out.buffer.shape[0] != m || out.buffer.shape[1] != w.buffer.shape[0] || out.dtype != a[2].dtype)
      return fail(error, TENSOR_ERROR_ARGUMENT, "out%d: shape, stride, size or dtype mismatch", i);
    group.w[i] = reinterpret_cast<const void*>(w.buffer.address);
    group.out[i] = reinterpret_cast<void*>(out.buffer.address);
    group.n[i] = (int)w.buffer.shape[0];
  }
  group.count = count;
  group.type = (int)a[argc - 1 - tail].scalar;
  group.m = (int)m;
  group.k = (int)k;
  group.out_half = a[2].dtype == TENSOR_FLOAT16;
  void* workspace = nullptr;
  size_t workspace_bytes = SIZE_MAX;
  if (has_workspace) {
    const TensorArgumentV1& ws = a[argc - 2 - tail];
    const TensorBufferV1& b = ws.buffer;
    if (ws.kind != TENSOR_ARG_BUFFER || ws.dtype != TENSOR_UINT8 || b.dtype != TENSOR_UINT8)
      return fail(error, TENSOR_ERROR_ARGUMENT, "workspace: wrong argument kind or dtype");
    if (b.device_type != TENSOR_DEVICE_ROCM || b.device_ordinal != ordinal || !b.address || b.address % 256 ||
        b.rank != 1 || !b.shape || !b.strides || b.shape[0] <= 0 || b.strides[0] != 1 ||
        b.byte_size < (uint64_t)b.shape[0])
      return fail(error, TENSOR_ERROR_ARGUMENT, "workspace: invalid buffer descriptor");
    workspace = reinterpret_cast<void*>(b.address);
    workspace_bytes = (size_t)b.shape[0];
  }
  tensor_gguf::GemmPlan plan = tensor_gguf::plan_gemm_group(group, workspace_bytes);
  if (forced) {
    plan = tensor_gguf::GemmPlan{(int)forced_tile, (int)forced_splits, true};
    if (forced_tile > 64 || forced_splits > 64 || !tensor_gguf::gemm_group_pipelined(group, plan))
      return fail(error, TENSOR_ERROR_ARGUMENT, "tile %u with %u splits does not fit this shape",
                  (unsigned)forced_tile, (unsigned)forced_splits);
  }
  const size_t need = tensor_gguf::gemm_group_workspace(group, plan);
  if (need > workspace_bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "workspace: the plan needs %zu bytes, %zu available", need,
                workspace_bytes);
  if (!has_workspace) {
    if (need > kScratchBytes)
      return fail(error, TENSOR_ERROR_ARGUMENT,
                  "shape too large: the K split needs %zu bytes of scratch, the library holds %zu", need,
                  kScratchBytes);
    workspace_bytes = kScratchBytes;
  }
  if (int32_t s = check_device(call, error)) return s;
  hipStream_t stream = reinterpret_cast<hipStream_t>(call->stream.handle);
  ScratchLease lease;
  if (!has_workspace) {
    if (int32_t s = lease.acquire(call, stream, error)) return s;
    workspace = lease.address();
  }
  hipError_t status = hipSuccess;
  tensor_gguf::GemvArgs one[tensor_gguf::kGemmGroupMax];
  bool small = true;  // every matrix on the small-M kernel, as tensor_gguf_gemm_v1 would run it
  for (int i = 0; i < count; ++i) {
    one[i].x = group.x;
    one[i].w = group.w[i];
    one[i].out = group.out[i];
    one[i].type = group.type;
    one[i].m = group.m;
    one[i].n = group.n[i];
    one[i].k = group.k;
    one[i].out_half = group.out_half;
    small = small && tensor_gguf::gemm_small_m(one[i]);
  }
  if ((!small || plan.small_m) && tensor_gguf::gemm_group_pipelined(group, plan)) {
    status = tensor_gguf::launch_gemm_group_plan(group, plan, workspace, workspace_bytes, stream);
  } else {
    // the other encodings and shapes, and small M where the plan keeps the small-M kernel, one
    // launch per matrix in order (no workspace: such plans never split K)
    for (int i = 0; i < count && status == hipSuccess; ++i) status = tensor_gguf::launch_gemm(one[i], stream);
  }
  if (status != hipSuccess) return hip_fail(error, status, "GGUF grouped GEMM launch");
  return has_workspace ? TENSOR_OK : lease.release(stream, error);
}

}  // namespace

extern "C" {

int32_t tensor_gguf_gemm_group_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return gemm_group_call(call, error, true);
}

int32_t tensor_gguf_gemm_group_noalloc_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return gemm_group_call(call, error, false);
}

int32_t tensor_gguf_gemm_group_plan_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return gemm_group_call(call, error, true, true);
}

int32_t tensor_gguf_gemm_tile_v1(int32_t tile, int32_t* bm, int32_t* bn, int32_t* ks, TensorErrorV1* error) {
  if (!bm || !bn || !ks || !tensor_gguf::gemm_tile_geometry(tile, bm, bn, ks))
    return fail(error, TENSOR_ERROR_ARGUMENT, "no pipelined GEMM tile %d", (int)tile);
  return ok(error);
}

}  // extern "C"

namespace {

// The group a workspace or plan query describes, checked like a call's shapes.
int32_t query_group(uint32_t type, int64_t m, int64_t k, const int64_t* n, uint32_t count,
                    tensor_gguf::GemmGroupArgs* group, TensorErrorV1* error) {
  Format format;
  if (!n || count < 1 || count > (uint32_t)tensor_gguf::kGemmGroupMax)
    return fail(error, TENSOR_ERROR_ARGUMENT, "invalid workspace query");
  if (!ggml_format(type, &format))
    return fail(error, TENSOR_ERROR_ARGUMENT, "type: unsupported GGML type %u", type);
  if (m < 1 || k < 1 || k % format.qk || m >= (int64_t)1 << 31 || k >= (int64_t)1 << 31)
    return fail(error, TENSOR_ERROR_ARGUMENT, "m, k: must be positive int32 with k a multiple of %d", format.qk);
  *group = tensor_gguf::GemmGroupArgs{};
  for (uint32_t i = 0; i < count; ++i) {
    if (n[i] < 1 || n[i] >= (int64_t)1 << 31) return fail(error, TENSOR_ERROR_ARGUMENT, "n%u: must be a positive int32", i);
    group->n[i] = (int)n[i];
  }
  group->count = (int)count;
  group->type = (int)type;
  group->m = (int)m;
  group->k = (int)k;
  group->out_half = true;
  return TENSOR_OK;
}

}  // namespace

extern "C" {

int32_t tensor_gguf_gemm_workspace_v1(uint32_t type, int64_t m, int64_t k, const int64_t* n, uint32_t count,
                                      uint64_t* bytes, TensorErrorV1* error) {
  tensor_gguf::GemmGroupArgs group;
  if (!bytes) return fail(error, TENSOR_ERROR_ARGUMENT, "invalid workspace query");
  if (int32_t s = query_group(type, m, k, n, count, &group, error)) return s;
  *bytes = tensor_gguf::gemm_group_workspace(group, tensor_gguf::plan_gemm_group(group, SIZE_MAX));
  return ok(error);
}

int32_t tensor_gguf_gemm_plan_v1(uint32_t type, int64_t m, int64_t k, const int64_t* n, uint32_t count,
                                 uint64_t workspace_bytes, int32_t* tile, int32_t* splits, int32_t* pipelined,
                                 TensorErrorV1* error) {
  tensor_gguf::GemmGroupArgs group;
  if (!tile || !splits || !pipelined) return fail(error, TENSOR_ERROR_ARGUMENT, "invalid plan query");
  if (int32_t s = query_group(type, m, k, n, count, &group, error)) return s;
  const tensor_gguf::GemmPlan plan = tensor_gguf::plan_gemm_group(group, (size_t)workspace_bytes);
  bool small = true;  // every matrix on the small-M kernel, as the grouped entry decides
  for (int i = 0; i < group.count; ++i) {
    tensor_gguf::GemvArgs one{};
    one.type = group.type;
    one.m = group.m;
    one.n = group.n[i];
    one.k = group.k;
    one.out_half = true;
    small = small && tensor_gguf::gemm_small_m(one);
  }
  *tile = plan.tile;
  *splits = plan.splits;
  *pipelined = (!small || plan.small_m) && tensor_gguf::gemm_group_pipelined(group, plan);
  return ok(error);
}

int32_t tensor_gguf_gemv_plan_v1(uint32_t type, int64_t m, int64_t k, int64_t n, int32_t* kernel, int32_t* a,
                                 int32_t* b, TensorErrorV1* error) {
  Format format;
  if (!kernel || !a || !b) return fail(error, TENSOR_ERROR_ARGUMENT, "invalid plan query");
  if (!ggml_format(type, &format))
    return fail(error, TENSOR_ERROR_ARGUMENT, "type: unsupported GGML type %u", type);
  if (m < 1 || m > tensor_gguf::kGemvMaxM || k < 1 || k % format.qk || k >= (int64_t)1 << 31 || n < 1 ||
      n >= (int64_t)1 << 31)
    return fail(error, TENSOR_ERROR_ARGUMENT, "m, k, n: 1 <= m <= %d, k a positive multiple of %d, n positive",
                tensor_gguf::kGemvMaxM, format.qk);
  tensor_gguf::GemvArgs args{};
  args.type = (int)type;
  args.m = (int)m;
  args.n = (int)n;
  args.k = (int)k;
  args.out_half = true;
  tensor_gguf::GemvPlan plan{-1, 0, 0};  // -1: the call takes another path (M = 1, other encodings)
  if (!tensor_gguf::gemv_q4k_plan(args, &plan)) plan = tensor_gguf::GemvPlan{-1, 0, 0};
  *kernel = plan.kernel;
  *a = plan.a;
  *b = plan.b;
  return ok(error);
}

int32_t tensor_gguf_gemv_q8_1_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return gemv_q8_1_call(call, error);
}

int32_t tensor_gguf_gemv_variant_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return gemv_variant_call(call, error);
}

int32_t tensor_gguf_packed_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return packed_call(call, error);
}

int32_t tensor_gguf_gemv_swiglu_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return swiglu_call(call, error);
}

int32_t tensor_gguf_gemv_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return linear_call(call, error, Op::kGemv);
}

int32_t tensor_gguf_gemm_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return linear_call(call, error, Op::kGemm);
}

int32_t tensor_gguf_linear_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return linear_call(call, error, Op::kLinear);
}

int32_t tensor_gguf_gemv_group_v1(const TensorCallV1* call, TensorErrorV1* error) {
  return group_call(call, error);
}

int32_t tensor_gguf_dequant_v1(const TensorCallV1* call, TensorErrorV1* error) {
  ok(error);
  if (int32_t s = check_call(call, 3, error)) return s;
  const int ordinal = call->stream.device_ordinal;
  const TensorArgumentV1* a = call->arguments;
  Format format;
  if (int32_t s = check_type(a[2], &format, error)) return s;
  if (int32_t s = check_matrix(a[0], "w", ordinal, TENSOR_UINT8, TENSOR_UINT8, error)) return s;
  if (int32_t s = check_matrix(a[1], "out", ordinal, TENSOR_FLOAT16, TENSOR_FLOAT32, error)) return s;
  const int64_t n = a[0].buffer.shape[0], k = a[1].buffer.shape[1];
  if (a[1].buffer.shape[0] != n || k % format.qk ||
      a[0].buffer.shape[1] != k / format.qk * format.bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "out: shape, stride or size mismatch");
  if (int32_t s = check_device(call, error)) return s;
  tensor_gguf::DequantArgs args;
  args.w = reinterpret_cast<const void*>(a[0].buffer.address);
  args.out = reinterpret_cast<void*>(a[1].buffer.address);
  args.type = (int)a[2].scalar;
  args.n = (int)n;
  args.k = (int)k;
  args.out_half = a[1].dtype == TENSOR_FLOAT16;
  hipError_t status = tensor_gguf::launch_dequant(args, reinterpret_cast<hipStream_t>(call->stream.handle));
  if (status != hipSuccess) return hip_fail(error, status, "GGUF dequant launch");
  return TENSOR_OK;
}

// ------------------------------------------------------ runtime services ---

int32_t tensor_hip_device_count(int32_t* count, TensorErrorV1* error) {
  int value = 0;
  hipError_t status = hipGetDeviceCount(&value);
  if (status == hipErrorNoDevice) value = 0;
  else if (status != hipSuccess) return hip_fail(error, status, "hipGetDeviceCount");
  *count = value;
  return ok(error);
}

int32_t tensor_hip_device_info(int32_t ordinal, TensorHipDeviceInfoV1* info, TensorErrorV1* error) {
  hipDeviceProp_t p;
  HIP_TRY(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
  std::memset(info, 0, sizeof(*info));
  std::snprintf(info->name, sizeof(info->name), "%s", p.name);
  std::snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
  info->total_memory = p.totalGlobalMem;
  info->l2_cache_bytes = (uint64_t)p.l2CacheSize;
  info->compute_units = p.multiProcessorCount;
  info->clock_khz = p.clockRate;
  info->memory_clock_khz = p.memoryClockRate;
  info->memory_bus_width = p.memoryBusWidth;
  info->max_threads_per_block = p.maxThreadsPerBlock;
  info->max_shared_memory_per_block = (int32_t)p.sharedMemPerBlock;
  info->warp_size = p.warpSize;
  for (int i = 0; i < 3; ++i) {
    info->max_grid[i] = p.maxGridSize[i];
    info->max_block[i] = p.maxThreadsDim[i];
  }
  return ok(error);
}

int32_t tensor_hip_set_device(int32_t ordinal, TensorErrorV1* error) {
  HIP_TRY(hipSetDevice(ordinal), "hipSetDevice");
  return ok(error);
}

int32_t tensor_hip_device_synchronize(TensorErrorV1* error) {
  HIP_TRY(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return ok(error);
}

int32_t tensor_hip_malloc(uint64_t bytes, uint64_t* address, TensorErrorV1* error) {
  void* p = nullptr;
  HIP_TRY(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
  *address = reinterpret_cast<uint64_t>(p);
  return ok(error);
}

int32_t tensor_hip_free(uint64_t address, TensorErrorV1* error) {
  HIP_TRY(hipFree(reinterpret_cast<void*>(address)), "hipFree");
  return ok(error);
}

int32_t tensor_hip_pointer_device(uint64_t address, int32_t* ordinal, int32_t* device_memory,
                                  TensorErrorV1* error) {
  if (!ordinal || !device_memory) return fail(error, TENSOR_ERROR_ARGUMENT, "null result pointer");
  hipPointerAttribute_t attributes;
  std::memset(&attributes, 0, sizeof(attributes));
  HIP_TRY(hipPointerGetAttributes(&attributes, reinterpret_cast<const void*>(address)), "hipPointerGetAttributes");
  *ordinal = attributes.device;
  *device_memory = attributes.type == hipMemoryTypeDevice || attributes.type == hipMemoryTypeManaged ? 1 : 0;
  return ok(error);
}

int32_t tensor_hip_copy_htod(uint64_t dst, const void* src, uint64_t bytes, uint64_t stream,
                             TensorErrorV1* error) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(HtoD)");
  HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
  return ok(error);
}

int32_t tensor_hip_copy_dtoh(void* dst, uint64_t src, uint64_t bytes, uint64_t stream,
                             TensorErrorV1* error) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  HIP_TRY(hipMemcpyAsync(dst, reinterpret_cast<const void*>(src), bytes, hipMemcpyDeviceToHost, s),
          "hipMemcpyAsync(DtoH)");
  HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
  return ok(error);
}

int32_t tensor_hip_copy_dtod(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream,
                             TensorErrorV1* error) {
  HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), bytes,
                         hipMemcpyDeviceToDevice, reinterpret_cast<hipStream_t>(stream)),
          "hipMemcpyAsync(DtoD)");
  return ok(error);
}

int32_t tensor_hip_copy_2d(uint64_t dst, uint64_t dst_pitch, uint64_t src, uint64_t src_pitch,
                           uint64_t width, uint64_t height, uint64_t stream, TensorErrorV1* error) {
  HIP_TRY(hipMemcpy2DAsync(reinterpret_cast<void*>(dst), dst_pitch, reinterpret_cast<const void*>(src),
                           src_pitch, width, height, hipMemcpyDeviceToDevice,
                           reinterpret_cast<hipStream_t>(stream)),
          "hipMemcpy2DAsync");
  return ok(error);
}

int32_t tensor_hip_fill_u8(uint64_t dst, uint8_t value, uint64_t bytes, uint64_t stream,
                           TensorErrorV1* error) {
  HIP_TRY(hipMemsetAsync(reinterpret_cast<void*>(dst), value, bytes, reinterpret_cast<hipStream_t>(stream)),
          "hipMemsetAsync");
  return ok(error);
}

int32_t tensor_hip_stream_create(uint64_t* stream, TensorErrorV1* error) {
  hipStream_t s = nullptr;
  HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
  *stream = reinterpret_cast<uint64_t>(s);
  return ok(error);
}

int32_t tensor_hip_stream_destroy(uint64_t stream, TensorErrorV1* error) {
  HIP_TRY(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)), "hipStreamDestroy");
  return ok(error);
}

int32_t tensor_hip_stream_synchronize(uint64_t stream, TensorErrorV1* error) {
  HIP_TRY(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)), "hipStreamSynchronize");
  return ok(error);
}

int32_t tensor_hip_stream_wait_event(uint64_t stream, uint64_t event, TensorErrorV1* error) {
  HIP_TRY(hipStreamWaitEvent(reinterpret_cast<hipStream_t>(stream), reinterpret_cast<hipEvent_t>(event), 0),
          "hipStreamWaitEvent");
  return ok(error);
}

int32_t tensor_hip_event_create(uint64_t* event, int32_t timing, TensorErrorV1* error) {
  hipEvent_t e = nullptr;
  HIP_TRY(hipEventCreateWithFlags(&e, timing ? hipEventDefault : hipEventDisableTiming),
          "hipEventCreateWithFlags");
  *event = reinterpret_cast<uint64_t>(e);
  return ok(error);
}

int32_t tensor_hip_event_destroy(uint64_t event, TensorErrorV1* error) {
  HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "hipEventDestroy");
  return ok(error);
}

int32_t tensor_hip_event_record(uint64_t event, uint64_t stream, TensorErrorV1* error) {
  HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(event), reinterpret_cast<hipStream_t>(stream)),
          "hipEventRecord");
  return ok(error);
}

int32_t tensor_hip_event_synchronize(uint64_t event, TensorErrorV1* error) {
  HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)), "hipEventSynchronize");
  return ok(error);
}

int32_t tensor_hip_event_query(uint64_t event, int32_t* complete, TensorErrorV1* error) {
  hipError_t status = hipEventQuery(reinterpret_cast<hipEvent_t>(event));
  if (status == hipErrorNotReady) {
    *complete = 0;
    return ok(error);
  }
  if (status != hipSuccess) return hip_fail(error, status, "hipEventQuery");
  *complete = 1;
  return ok(error);
}

int32_t tensor_hip_event_elapsed(float* milliseconds, uint64_t start, uint64_t stop, TensorErrorV1* error) {
  HIP_TRY(hipEventElapsedTime(milliseconds, reinterpret_cast<hipEvent_t>(start),
                              reinterpret_cast<hipEvent_t>(stop)),
          "hipEventElapsedTime");
  return ok(error);
}

int32_t tensor_hip_capture_begin(uint64_t stream, TensorErrorV1* error) {
  HIP_TRY(hipStreamBeginCapture(reinterpret_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal),
          "hipStreamBeginCapture");
  return ok(error);
}

// A captured graph: the instantiated executable graph and the graph it was made from, which
// lives until the executable graph is destroyed (tools that inspect a launched executable
// graph may look its nodes up in the source graph).
struct CapturedGraph {
  hipGraph_t graph;
  hipGraphExec_t exec;
};

int32_t tensor_hip_capture_end(uint64_t stream, uint64_t* graph_exec, TensorErrorV1* error) {
  if (!graph_exec) return fail(error, TENSOR_ERROR_ARGUMENT, "null graph result pointer");
  *graph_exec = 0;
  hipGraph_t graph = nullptr;
  HIP_TRY(hipStreamEndCapture(reinterpret_cast<hipStream_t>(stream), &graph), "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  hipError_t status = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (status != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return hip_fail(error, status, "hipGraphInstantiate");
  }
  CapturedGraph* captured = new (std::nothrow) CapturedGraph{graph, exec};
  if (!captured) {
    (void)hipGraphExecDestroy(exec);
    (void)hipGraphDestroy(graph);
    return fail(error, TENSOR_ERROR_PROVIDER, "out of host memory for a captured graph");
  }
  *graph_exec = reinterpret_cast<uint64_t>(captured);
  return ok(error);
}

int32_t tensor_hip_graph_launch(uint64_t graph_exec, uint64_t stream, TensorErrorV1* error) {
  const CapturedGraph* captured = reinterpret_cast<const CapturedGraph*>(graph_exec);
  if (!captured) return fail(error, TENSOR_ERROR_ARGUMENT, "null graph handle");
  HIP_TRY(hipGraphLaunch(captured->exec, reinterpret_cast<hipStream_t>(stream)), "hipGraphLaunch");
  return ok(error);
}

int32_t tensor_hip_graph_destroy(uint64_t graph_exec, TensorErrorV1* error) {
  CapturedGraph* captured = reinterpret_cast<CapturedGraph*>(graph_exec);
  if (!captured) return fail(error, TENSOR_ERROR_ARGUMENT, "null graph handle");
  const hipError_t exec_status = hipGraphExecDestroy(captured->exec);
  const hipError_t graph_status = hipGraphDestroy(captured->graph);
  delete captured;
  if (exec_status != hipSuccess) return hip_fail(error, exec_status, "hipGraphExecDestroy");
  if (graph_status != hipSuccess) return hip_fail(error, graph_status, "hipGraphDestroy");
  return ok(error);
}

// ----------------------------------------------------------- code objects ---

int32_t tensor_hip_module_load(const void* image, uint64_t bytes, uint64_t* module, TensorErrorV1* error) {
  if (!image || bytes < 64 || !module || std::memcmp(image, "\x7f" "ELF", 4) != 0)
    return fail(error, TENSOR_ERROR_ARGUMENT, "module image is not an ELF code object");
  hipModule_t handle = nullptr;
  HIP_TRY(hipModuleLoadData(&handle, image), "hipModuleLoadData");
  *module = reinterpret_cast<uint64_t>(handle);
  return ok(error);
}

int32_t tensor_hip_module_function(uint64_t module, const char* name, uint64_t* function, TensorErrorV1* error) {
  if (!module || !name || !function) return fail(error, TENSOR_ERROR_ARGUMENT, "invalid module or function name");
  hipFunction_t handle = nullptr;
  HIP_TRY(hipModuleGetFunction(&handle, reinterpret_cast<hipModule_t>(module), name), "hipModuleGetFunction");
  *function = reinterpret_cast<uint64_t>(handle);
  return ok(error);
}

int32_t tensor_hip_module_unload(uint64_t module, TensorErrorV1* error) {
  if (!module) return fail(error, TENSOR_ERROR_ARGUMENT, "invalid module");
  HIP_TRY(hipModuleUnload(reinterpret_cast<hipModule_t>(module)), "hipModuleUnload");
  return ok(error);
}

int32_t tensor_hip_module_launch_v1(uint64_t function, const TensorCallV1* call, TensorErrorV1* error) {
  constexpr uint32_t kMaxArguments = 256;
  if (!call || call->abi_version != TENSOR_ABI_VERSION || call->struct_size < sizeof(TensorCallV1))
    return fail(error, TENSOR_ERROR_ABI, "unsupported call ABI");
  if (!function) return fail(error, TENSOR_ERROR_ARGUMENT, "invalid kernel function");
  if (call->flags || call->argument_count > kMaxArguments || (call->argument_count && !call->arguments))
    return fail(error, TENSOR_ERROR_ARGUMENT, "invalid argument count or flags");
  if (call->stream.device_type != TENSOR_DEVICE_ROCM || call->stream.device_ordinal < 0)
    return fail(error, TENSOR_ERROR_PROVIDER, "ROCm calls need a ROCm stream");
  uint64_t threads = 1;
  for (int d = 0; d < 3; ++d) {
    if (call->grid[d] < 1 || call->grid[d] > 0x7FFFFFFFu || call->block[d] < 1)
      return fail(error, TENSOR_ERROR_ARGUMENT, "launch dimensions must be positive int32");
    threads *= call->block[d];
  }
  if (threads > 1024) return fail(error, TENSOR_ERROR_ARGUMENT, "launch block exceeds 1024 threads");
  void* parameters[kMaxArguments];
  for (uint32_t i = 0; i < call->argument_count; ++i) {
    const TensorArgumentV1& arg = call->arguments[i];
    if (arg.kind == TENSOR_ARG_BUFFER) {
      const TensorBufferV1& b = arg.buffer;
      if (b.device_type != TENSOR_DEVICE_ROCM || b.device_ordinal != call->stream.device_ordinal || !b.address ||
          b.dtype != arg.dtype)
        return fail(error, TENSOR_ERROR_ARGUMENT, "argument %u: buffer is not on the stream's ROCm device", i);
      parameters[i] = const_cast<uint64_t*>(&b.address);
    } else if (arg.kind == TENSOR_ARG_SCALAR) {
      parameters[i] = const_cast<uint64_t*>(&arg.scalar);  // little-endian: the value is in the low bytes
    } else {
      return fail(error, TENSOR_ERROR_ARGUMENT, "argument %u: unknown kind %u", i, (unsigned)arg.kind);
    }
  }
  if (int32_t status = check_device(call, error)) return status;
  HIP_TRY(hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(function), call->grid[0], call->grid[1],
                                call->grid[2], call->block[0], call->block[1], call->block[2],
                                call->shared_memory_bytes, reinterpret_cast<hipStream_t>(call->stream.handle),
                                call->argument_count ? parameters : nullptr, nullptr),
          "hipModuleLaunchKernel");
  return ok(error);
}

const char* tensor_hip_version(void) { return "tensor_hip 1.4 gfx950"; }

}  // extern "C"
