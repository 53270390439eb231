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
  constexpr int QK = Block<TYPE>::QK;
  constexpr int BYTES = Block<TYPE>::BYTES;
  const size_t groups = (size_t)n * (k / 8);
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += stride) {
    const size_t row = g / (size_t)(k / 8);
    const int col = (int)(g - row * (size_t)(k / 8)) * 8;
    const uint8_t* block = w + row * (size_t)(k / QK) * BYTES + (size_t)(col / QK) * BYTES;
    float v[8];
    decode8<TYPE>(block, col % QK, v);
    OutT* dst = out + row * (size_t)k + col;
    if constexpr (sizeof(OutT) == 2) {
      // the cast of each fp32 value (never a fused single rounding of the exact value)
      *reinterpret_cast<uint4*>(dst) = make_uint4(half2_from_fp32(v[0], v[1]), half2_from_fp32(v[2], v[3]),
                                                  half2_from_fp32(v[4], v[5]), half2_from_fp32(v[6], v[7]));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[i] = (OutT)v[i];
    }
  }
}

template <int TYPE, typename OutT>
static hipError_t launch_type(const uint8_t* w, OutT* out, const DequantArgs& a, unsigned blocks,
                              hipStream_t stream) {
  hipLaunchKernelGGL((dequant_kernel<TYPE, OutT>), dim3(blocks), dim3(256), 0, stream, w, out, a.n, a.k);
  return hipGetLastError();
}

template <typename OutT>
static hipError_t launch_typed(const DequantArgs& a, hipStream_t stream) {
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const size_t groups = (size_t)a.n * (a.k / 8);
  const unsigned blocks = (unsigned)((groups + 255) / 256 < 65536 ? (groups + 255) / 256 : 65536);
  switch (a.type) {
    case kQ4_K: return launch_type<kQ4_K>(w, out, a, blocks, stream);
    case kQ6_K: return launch_type<kQ6_K>(w, out, a, blocks, stream);
    case kQ8_0: return launch_type<kQ8_0>(w, out, a, blocks, stream);
    case kQ4_0: return launch_type<kQ4_0>(w, out, a, blocks, stream);
    case kQ4_1: return launch_type<kQ4_1>(w, out, a, blocks, stream);
    case kQ5_0: return launch_type<kQ5_0>(w, out, a, blocks, stream);
    case kQ5_1: return launch_type<kQ5_1>(w, out, a, blocks, stream);
    case kQ2_K: return launch_type<kQ2_K>(w, out, a, blocks, stream);
    case kQ3_K: return launch_type<kQ3_K>(w, out, a, blocks, stream);
    case kQ5_K: return launch_type<kQ5_K>(w, out, a, blocks, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dequant(const DequantArgs& a, hipStream_t stream) {
  return a.out_half ? launch_typed<_Float16>(a, stream) : launch_typed<float>(a, stream);
}

}  // namespace tensor_gguf
