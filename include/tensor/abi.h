/*
 * Tensor runtime call ABI, version 1 (layout-compatible with minor 3).
 *
 * This header restates the descriptor contract of the reference runtime
 * (src/tensor/include/tensor/abi.h:10-152) so that a ROCm provider consumes the
 * very same bytes a CUDA or CPU provider does.  Every structure below has the
 * size and field offsets fixed by that contract (asserted at the end); the
 * only addition is the ROCm device type, which follows DLPack's kDLROCM = 10
 * as the reference documents device types 1 and 2 following DLPack
 * (docs/reference/runtime-abi.md:71).
 */
#ifndef TENSOR_ABI_H
#define TENSOR_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Versioning and flags. */
#define TENSOR_ABI_VERSION 1u
#define TENSOR_ABI_MINOR 3u
#define TENSOR_EXEC_ASYNC 1u
#define TENSOR_EVENT_KNOWN_COMPLETE 1u

/* Device types (DLPack numbering; 256 is the reference's WebGPU id). */
#define TENSOR_DEVICE_CPU 1u
#define TENSOR_DEVICE_CUDA 2u
#define TENSOR_DEVICE_ROCM 10u
#define TENSOR_DEVICE_WEBGPU 256u

/* Argument kinds. */
#define TENSOR_ARG_BUFFER 1u
#define TENSOR_ARG_SCALAR 2u
#define TENSOR_ARG_OPAQUE_BUFFER 3u

/* Status codes returned by every entry point. */
#define TENSOR_OK 0
#define TENSOR_ERROR_ABI 1
#define TENSOR_ERROR_ARGUMENT 2
#define TENSOR_ERROR_PROVIDER 3

/* Permanent element type ids.  A scalar argument stores its value in the low
 * sizeof(type) bytes of the 64-bit scalar field, little-endian, upper bytes 0. */
enum TensorDTypeV1 {
  TENSOR_BOOL = 1,
  TENSOR_INT8 = 2,
  TENSOR_UINT8 = 3,
  TENSOR_INT16 = 4,
  TENSOR_UINT16 = 5,
  TENSOR_INT32 = 6,
  TENSOR_UINT32 = 7,
  TENSOR_INT64 = 8,
  TENSOR_UINT64 = 9,
  TENSOR_FLOAT16 = 10,
  TENSOR_FLOAT32 = 11,
  TENSOR_FLOAT64 = 12,
  TENSOR_BFLOAT16 = 13
};

/* A contiguous buffer: device address, capacity in bytes, shape and BYTE
 * strides (never element strides). */
typedef struct TensorBufferV1 {
  uint64_t address;
  uint64_t byte_size;
  const int64_t *shape;
  const int64_t *strides;
  uint32_t rank;
  uint32_t dtype;
  uint32_t device_type;
  int32_t device_ordinal;
} TensorBufferV1;

/* One call argument: a buffer (kind 1), a scalar (kind 2) or a session-owned
 * opaque buffer handle (kind 3). */
typedef struct TensorArgumentV1 {
  uint32_t kind;
  uint32_t dtype;
  TensorBufferV1 buffer;
  uint64_t scalar;
} TensorArgumentV1;

/* Stream identity.  For ROCm, handle is a hipStream_t (0 = null stream). */
typedef struct TensorStreamV1 {
  uint32_t device_type;
  int32_t device_ordinal;
  uint64_t handle;
} TensorStreamV1;

/* A complete call: arguments in the executable's declared order, launch
 * geometry and the stream the work is ordered on. */
typedef struct TensorCallV1 {
  uint32_t abi_version;
  uint32_t struct_size;
  const TensorArgumentV1 *arguments;
  uint32_t argument_count;
  uint32_t flags;
  uint32_t grid[3];
  uint32_t block[3];
  uint64_t shared_memory_bytes;
  TensorStreamV1 stream;
} TensorCallV1;

/* Status plus a bounded, always NUL-terminated UTF-8 diagnostic. */
typedef struct TensorErrorV1 {
  int32_t code;
  char message[508];
} TensorErrorV1;

/* External scratch requirements of an executable (ABI 1.1: always zero). */
typedef struct TensorWorkspaceRequirementsV1 {
  uint64_t byte_size;
  uint32_t alignment;
  uint32_t device_type;
  uint32_t flags;
  uint32_t reserved;
} TensorWorkspaceRequirementsV1;

/* Session-qualified identity of a loaded executable. */
typedef struct TensorExecutableV1 {
  uint32_t abi_version;
  uint32_t struct_size;
  uint32_t device_type;
  int32_t device_ordinal;
  uint64_t session;
  uint64_t handle;
  uint32_t argument_count;
  uint32_t flags;
  TensorWorkspaceRequirementsV1 workspace;
} TensorExecutableV1;

/* Session-qualified identity of a completion event. */
typedef struct TensorEventV1 {
  uint32_t abi_version;
  uint32_t struct_size;
  uint32_t device_type;
  int32_t device_ordinal;
  uint64_t session;
  uint64_t handle;
  uint32_t flags;
  uint32_t reserved;
} TensorEventV1;

/* The one native entry shape.  The call and its descriptor arrays are
 * borrowed until return; device storage must stay alive until the stream has
 * completed the work.  Errors are reported through the return value and the
 * error record, never by exceptions. */
typedef int32_t (*TensorKernelV1)(const TensorCallV1 *, TensorErrorV1 *);

#ifdef __cplusplus
} /* extern "C" */
static_assert(sizeof(TensorBufferV1) == 48, "TensorBufferV1 layout");
static_assert(sizeof(TensorArgumentV1) == 64, "TensorArgumentV1 layout");
static_assert(sizeof(TensorStreamV1) == 16, "TensorStreamV1 layout");
static_assert(sizeof(TensorCallV1) == 72, "TensorCallV1 layout");
static_assert(sizeof(TensorErrorV1) == 512, "TensorErrorV1 layout");
static_assert(sizeof(TensorWorkspaceRequirementsV1) == 24, "workspace layout");
static_assert(sizeof(TensorExecutableV1) == 64, "TensorExecutableV1 layout");
static_assert(sizeof(TensorEventV1) == 40, "TensorEventV1 layout");
#else
_Static_assert(sizeof(TensorBufferV1) == 48, "TensorBufferV1 layout");
_Static_assert(sizeof(TensorArgumentV1) == 64, "TensorArgumentV1 layout");
_Static_assert(sizeof(TensorCallV1) == 72, "TensorCallV1 layout");
_Static_assert(sizeof(TensorErrorV1) == 512, "TensorErrorV1 layout");
#endif

#endif /* TENSOR_ABI_H */
