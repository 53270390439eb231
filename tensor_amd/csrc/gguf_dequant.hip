// GGUF rows -> fp32 or fp16 matrix [n, k].
//
// The element values follow benchmarks/kernels/showcase/triton_kernels.py:134-181
// in fp32 with the reference's operation order; every product is exact in fp32
// and Q4_K's final subtraction is the only rounding, so the fp32 output is the
// exact reference value and the fp16 output is its round-to-nearest-even
// (subnormals kept).  The fused GEMM decodes its tiles with the same
// per-element arithmetic (decode8 in gguf_decode.h).
#include "gguf_decode.h"
#include "gguf_launch.h"

namespace tensor_gguf {

template <int TYPE, typename OutT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w,
                                                      OutT* __restrict__ out, int n, int k) {
  constexpr int QK = (TYPE == kQ4_K || TYPE == kQ6_K) ? 256 : 32;
  constexpr int BYTES = TYPE == kQ4_K ? 144 : TYPE == kQ6_K ? 210 : TYPE == kQ8_0 ? 34 : 18;
  const size_t groups = (size_t)n * (k / 8);
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += stride) {
    const size_t row = g / (size_t)(k / 8);
    const int col = (int)(g - row * (size_t)(k / 8)) * 8;
    const uint8_t* block = w + row * (size_t)(k / QK) * BYTES + (size_t)(col / QK) * BYTES;
    float v[8];
    decode8<TYPE>(block, col % QK, v);
    OutT* dst = out + row * (size_t)k + col;
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = (OutT)v[i];
  }
}

template <typename OutT>
static hipError_t launch_typed(const DequantArgs& a, hipStream_t stream) {
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const size_t groups = (size_t)a.n * (a.k / 8);
  const unsigned blocks = (unsigned)((groups + 255) / 256 < 65536 ? (groups + 255) / 256 : 65536);
  switch (a.type) {
    case kQ4_K:
      hipLaunchKernelGGL((dequant_kernel<kQ4_K, OutT>), dim3(blocks), dim3(256), 0, stream, w, out, a.n, a.k);
      break;
    case kQ6_K:
      hipLaunchKernelGGL((dequant_kernel<kQ6_K, OutT>), dim3(blocks), dim3(256), 0, stream, w, out, a.n, a.k);
      break;
    case kQ8_0:
      hipLaunchKernelGGL((dequant_kernel<kQ8_0, OutT>), dim3(blocks), dim3(256), 0, stream, w, out, a.n, a.k);
      break;
    case kQ4_0:
      hipLaunchKernelGGL((dequant_kernel<kQ4_0, OutT>), dim3(blocks), dim3(256), 0, stream, w, out, a.n, a.k);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const DequantArgs& a, hipStream_t stream) {
  return a.out_half ? launch_typed<_Float16>(a, stream) : launch_typed<float>(a, stream);
}

}  // namespace tensor_gguf
