// SwiGLU of a decode step's gate and up projections, shipped as a `hip` executable bundle
// (tensor_amd/kernels/swiglu.tbin, loaded with Device.load(path)):
//   out[i] = silu(gate[i]) * up[i] = gate[i] / (1 + exp(-gate[i])) * up[i]
// over M x N fp16 elements, evaluated in fp32 and rounded once to fp16.  Each thread
// handles eight consecutive elements with 16-byte loads and stores; the last partial
// group of eight falls back to element accesses.
#include <hip/hip_runtime.h>
#include <cstdint>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ _Float16 swiglu(_Float16 g, _Float16 u) {
  const float gf = (float)g;
  return (_Float16)(gf / (1.0f + expf(-gf)) * (float)u);
}

extern "C" __global__ __launch_bounds__(256) void tensor_swiglu_f16(const _Float16* __restrict__ gate,
                                                                    const _Float16* __restrict__ up,
                                                                    _Float16* __restrict__ out, uint32_t M,
                                                                    uint32_t N) {
  const uint64_t count = (uint64_t)M * N;
  const uint64_t first = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (first + 8 <= count) {
    const half8_t g = *reinterpret_cast<const half8_t*>(gate + first);
    const half8_t u = *reinterpret_cast<const half8_t*>(up + first);
    half8_t r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = swiglu(g[i], u[i]);
    *reinterpret_cast<half8_t*>(out + first) = r;
  } else {
    for (uint64_t i = first; i < count; ++i) out[i] = swiglu(gate[i], up[i]);
  }
}
