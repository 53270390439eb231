/*
 * ORACLE — test infrastructure only.  Never linked into, loaded by or called
 * from the product path (tensor_amd/).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load the library built from this file.
 *
 * Scalar C restatement of the reference's GGUF block decoding and of the
 * quantized-linear numerics it is checked against.
 *
 *   Block formats (GGML types 2, 8, 12, 14; types 3, 6, 7, 10, 11 and 13 below
 *   decode_q4_1 follow the public GGML block definitions, with no reference code):
 *     Q4_0  benchmarks/kernels/showcase/triton_kernels.py:135-142
 *     Q4_K  benchmarks/kernels/showcase/triton_kernels.py:143-162
 *     Q6_K  benchmarks/kernels/showcase/triton_kernels.py:163-180
 *     Q8_0  not in the reference's code (named only in
 *           research/plans/v1-benchmarks.md:301); restated from the public
 *           GGML block definition: fp16 d, 32 x int8, y = d * q.
 *   Decode GEMV numerics: fp32 operands, fp32 accumulation
 *     (benchmarks/kernels/showcase/benchmark.py:466-472).
 *   Prefill GEMM numerics: fp16(x) . fp16(dequant(W)), fp32 accumulation
 *     (benchmarks/kernels/showcase/triton_kernels.py:199-211,
 *      benchmark.py:473-477).
 *   CPU entry shape: TensorKernelV1 (src/tensor/include/tensor/abi.h:135-141),
 *     validated like the CPU provider's generated wrapper
 *     (src/tensor/compiler/cpu.py:49-155) and invoked synchronously through
 *     ctypes as src/tensor/providers/cpu.py:191-197 does.
 *
 * The decoders here walk each block the way a block is laid out (sub-block by
 * sub-block); the NumPy oracle (gguf_ref.py) instead evaluates the reference's
 * per-element index formulas.  The two are independent and the tests require
 * them to agree bit for bit.
 *
 * Parity pins (tests/test_oracle.py): pack-then-decode round trips through an
 * independent encoder for every scale/min/code field, exhaustive 6-bit
 * scale/min packing, closed forms for d=1/dmin=0 blocks, the exactness of every
 * fp32 product, fp16 conversion against numpy, and textbook fp64 products.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "tensor/abi.h"

#define GGML_Q4_0 2
#define GGML_Q4_1 3
#define GGML_Q5_0 6
#define GGML_Q5_1 7
#define GGML_Q8_0 8
#define GGML_Q2_K 10
#define GGML_Q3_K 11
#define GGML_Q4_K 12
#define GGML_Q5_K 13
#define GGML_Q6_K 14

/* ---------------------------------------------------------------- fp16 --- */

/* IEEE binary16 -> binary32, exact for every input (including subnormals). */
float oracle_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exponent = (h >> 10) & 31u;
  uint32_t mantissa = h & 1023u;
  uint32_t bits;
  if (exponent == 31u) {
    bits = sign | 0x7F800000u | (mantissa << 13);
  } else if (exponent != 0u) {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  } else if (mantissa == 0u) {
    bits = sign;
  } else {
    /* subnormal: value = mantissa * 2^-24, exact in binary32 */
    float value = (float)mantissa * 5.9604644775390625e-8f;
    memcpy(&bits, &value, 4);
    bits |= sign;
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

/* IEEE binary32 -> binary16, round to nearest even, with overflow to inf,
 * gradual underflow and NaN quieting. */
uint16_t oracle_float_to_half(float f) {
  uint32_t bits;
  memcpy(&bits, &f, 4);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  uint32_t exponent = (bits >> 23) & 255u;
  uint32_t mantissa = bits & 0x7FFFFFu;
  if (exponent == 255u) {
    return sign | 0x7C00u | (mantissa ? (0x200u | (mantissa >> 13)) : 0u);
  }
  int e = (int)exponent - 127;
  if (e > 15) return sign | 0x7C00u;
  if (e >= -14) {
    /* normal half candidate: keep 10 mantissa bits, round the other 13 */
    uint32_t half = ((uint32_t)(e + 15) << 10) | (mantissa >> 13);
    uint32_t rest = mantissa & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (half & 1u))) half += 1u;
    return sign | (uint16_t)half; /* a carry into exponent 31 yields inf */
  }
  if (e < -25) return sign; /* below half of the smallest subnormal */
  /* subnormal half: value / 2^-24 rounded to an integer, ties to even */
  uint32_t full = mantissa | 0x800000u; /* value = full * 2^(e-23) */
  int shift = -e - 1;                   /* 2^(e-23) / 2^-24 = 2^(e+1) */
  uint32_t quotient = full >> shift;
  uint32_t remainder = full & ((1u << shift) - 1u);
  uint32_t halfway = 1u << (shift - 1);
  if (remainder > halfway || (remainder == halfway && (quotient & 1u)))
    quotient += 1u;
  return sign | (uint16_t)quotient;
}

static float load_half(const uint8_t *p) {
  return oracle_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
}

/* ------------------------------------------------------------- formats --- */

int oracle_block_geometry(int type, int *elements, int *bytes) {
  switch (type) {
    case GGML_Q4_0: *elements = 32; *bytes = 18; return 0;
    case GGML_Q4_1: *elements = 32; *bytes = 20; return 0;
    case GGML_Q5_0: *elements = 32; *bytes = 22; return 0;
    case GGML_Q5_1: *elements = 32; *bytes = 24; return 0;
    case GGML_Q8_0: *elements = 32; *bytes = 34; return 0;
    case GGML_Q2_K: *elements = 256; *bytes = 84; return 0;
    case GGML_Q3_K: *elements = 256; *bytes = 110; return 0;
    case GGML_Q4_K: *elements = 256; *bytes = 144; return 0;
    case GGML_Q5_K: *elements = 256; *bytes = 176; return 0;
    case GGML_Q6_K: *elements = 256; *bytes = 210; return 0;
    default: return -1;
  }
}

static void decode_q4_0(const uint8_t *block, float *out) {
  float d = load_half(block);
  const uint8_t *qs = block + 2;
  for (int j = 0; j < 16; ++j) {
    out[j] = (float)((int)(qs[j] & 15u) - 8) * d;
    out[j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
  }
}

static void decode_q8_0(const uint8_t *block, float *out) {
  float d = load_half(block);
  const int8_t *qs = (const int8_t *)(block + 2);
  for (int j = 0; j < 32; ++j) out[j] = d * (float)qs[j];
}

/* The 12 scale bytes hold eight 6-bit (scale, min) pairs. */
static void q4k_scale_min(const uint8_t *s, int sub, int *scale, int *min) {
  if (sub < 4) {
    *scale = s[sub] & 63;
    *min = s[sub + 4] & 63;
  } else {
    *scale = (s[sub + 4] & 15) | ((s[sub - 4] >> 6) << 4);
    *min = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4);
  }
}

static void decode_q4_k(const uint8_t *block, float *out) {
  float d = load_half(block);
  float dmin = load_half(block + 2);
  const uint8_t *scales = block + 4;
  const uint8_t *qs = block + 16;
  /* four 64-element groups; each 32-byte slice holds two sub-blocks */
  for (int group = 0; group < 4; ++group) {
    for (int half = 0; half < 2; ++half) {
      int sub = 2 * group + half, scale, min;
      q4k_scale_min(scales, sub, &scale, &min);
      float ds = d * (float)scale; /* exact: 11 + 6 significant bits */
      float dm = dmin * (float)min;
      for (int l = 0; l < 32; ++l) {
        int q = (qs[32 * group + l] >> (4 * half)) & 15;
        /* ds*q is exact (<= 21 bits); the subtraction rounds once */
        out[64 * group + 32 * half + l] = ds * (float)q - dm;
      }
    }
  }
}

static void decode_q6_k(const uint8_t *block, float *out) {
  const uint8_t *ql = block;
  const uint8_t *qh = block + 128;
  const int8_t *scales = (const int8_t *)(block + 192);
  float d = load_half(block + 208);
  for (int half = 0; half < 2; ++half) {
    for (int l = 0; l < 32; ++l) {
      const uint8_t lo_a = ql[64 * half + l];
      const uint8_t lo_b = ql[64 * half + 32 + l];
      const uint8_t hi = qh[32 * half + l];
      int q[4];
      q[0] = (lo_a & 15) | (((hi >> 0) & 3) << 4);
      q[1] = (lo_b & 15) | (((hi >> 2) & 3) << 4);
      q[2] = (lo_a >> 4) | (((hi >> 4) & 3) << 4);
      q[3] = (lo_b >> 4) | (((hi >> 6) & 3) << 4);
      for (int quarter = 0; quarter < 4; ++quarter) {
        int index = 128 * half + 32 * quarter + l;
        /* (q-32)*sc*d: every factor and partial product is exact in fp32 */
        out[index] = (float)(q[quarter] - 32) * (float)scales[index / 16] * d;
      }
    }
  }
}

/* ---- the other GGML encodings (public GGML block definitions; no reference code) ----
 *   Q4_1  fp16 d | fp16 m | 16 B nibbles                    y = q*d + m
 *   Q5_0  fp16 d | u32 qh | 16 B nibbles                    y = (q - 16)*d, q = nibble | qh bit << 4
 *   Q5_1  fp16 d | fp16 m | u32 qh | 16 B nibbles           y = q*d + m
 *   Q2_K  16 B scales (lo: scale, hi: min) | 64 B 2-bit codes | fp16 d | fp16 dmin
 *                                                           y = d*sc*q - dmin*m
 *   Q3_K  32 B high-bit mask | 64 B 2-bit codes | 12 B 6-bit scales | fp16 d
 *                                                           y = d*(sc - 32)*(q - (hbit ? 0 : 4))
 *   Q5_K  fp16 d | fp16 dmin | 12 B 6-bit scales/mins (as Q4_K) | 32 B high bits | 128 B nibbles
 *                                                           y = d*sc*q - dmin*m
 * Every product is exact in fp32; Q4_1, Q5_1, Q2_K and Q5_K round once, in the final
 * addition or subtraction. */

static uint32_t load_u32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

static void decode_q4_1(const uint8_t *block, float *out) {
  float d = load_half(block), m = load_half(block + 2);
  const uint8_t *qs = block + 4;
  for (int j = 0; j < 16; ++j) {
    out[j] = (float)(qs[j] & 15u) * d + m;
    out[j + 16] = (float)(qs[j] >> 4) * d + m;
  }
}

static void decode_q5(const uint8_t *block, float *out, int with_min) {
  float d = load_half(block);
  float m = with_min ? load_half(block + 2) : 0.0f;
  const uint8_t *tail = block + (with_min ? 4 : 2);
  uint32_t qh = load_u32(tail);
  const uint8_t *qs = tail + 4;
  for (int j = 0; j < 16; ++j) {
    int lo = (int)((qs[j] & 15u) | (((qh >> j) & 1u) << 4));
    int hi = (int)((qs[j] >> 4) | (((qh >> (j + 16)) & 1u) << 4));
    if (with_min) {
      out[j] = (float)lo * d + m;
      out[j + 16] = (float)hi * d + m;
    } else {
      out[j] = (float)(lo - 16) * d;
      out[j + 16] = (float)(hi - 16) * d;
    }
  }
}

static void decode_q2_k(const uint8_t *block, float *out) {
  const uint8_t *scales = block, *qs = block + 16;
  float d = load_half(block + 80), dmin = load_half(block + 82);
  for (int half = 0; half < 2; ++half) {        /* 128 elements per 32 code bytes */
    for (int shift = 0; shift < 4; ++shift) {   /* 2-bit planes, 32 elements each */
      for (int part = 0; part < 2; ++part) {    /* 16 elements per scale byte */
        int index = 128 * half + 32 * shift + 16 * part;
        uint8_t sc = scales[index / 16];
        float dl = d * (float)(sc & 15), ml = dmin * (float)(sc >> 4);
        for (int l = 0; l < 16; ++l) {
          int q = (qs[32 * half + 16 * part + l] >> (2 * shift)) & 3;
          out[index + l] = dl * (float)q - ml;
        }
      }
    }
  }
}

/* Q3_K's 16 six-bit scales: low nibbles in bytes 0-7 (scales 0-7 low, 8-15 high nibble),
 * the top two bits in bytes 8-11 (scale s in byte 8 + s%4, bits 2*(s/4)). */
static int q3k_scale(const uint8_t *s, int index) {
  int low = index < 8 ? (s[index] & 15) : (s[index - 8] >> 4);
  int high = (s[8 + (index & 3)] >> (2 * (index >> 2))) & 3;
  return (low | (high << 4)) - 32;
}

static void decode_q3_k(const uint8_t *block, float *out) {
  const uint8_t *hmask = block, *qs = block + 32, *scales = block + 96;
  float d = load_half(block + 108);
  for (int half = 0; half < 2; ++half) {
    for (int shift = 0; shift < 4; ++shift) {
      int bit = 4 * half + shift;               /* high-bit plane of these 32 elements */
      for (int l = 0; l < 32; ++l) {
        int index = 128 * half + 32 * shift + l;
        int q = ((qs[32 * half + l] >> (2 * shift)) & 3) - (((hmask[l] >> bit) & 1) ? 0 : 4);
        out[index] = d * (float)q3k_scale(scales, index / 16) * (float)q;
      }
    }
  }
}

static void decode_q5_k(const uint8_t *block, float *out) {
  float d = load_half(block), dmin = load_half(block + 2);
  const uint8_t *scales = block + 4, *qh = block + 16, *qs = block + 48;
  for (int group = 0; group < 4; ++group) {
    for (int half = 0; half < 2; ++half) {
      int sub = 2 * group + half, scale, min;
      q4k_scale_min(scales, sub, &scale, &min);
      float ds = d * (float)scale, dm = dmin * (float)min;
      for (int l = 0; l < 32; ++l) {
        int q = ((qs[32 * group + l] >> (4 * half)) & 15) | (((qh[l] >> sub) & 1) << 4);
        out[64 * group + 32 * half + l] = ds * (float)q - dm;
      }
    }
  }
}

int oracle_decode_block(int type, const uint8_t *block, float *out) {
  switch (type) {
    case GGML_Q4_0: decode_q4_0(block, out); return 0;
    case GGML_Q4_1: decode_q4_1(block, out); return 0;
    case GGML_Q5_0: decode_q5(block, out, 0); return 0;
    case GGML_Q5_1: decode_q5(block, out, 1); return 0;
    case GGML_Q8_0: decode_q8_0(block, out); return 0;
    case GGML_Q2_K: decode_q2_k(block, out); return 0;
    case GGML_Q3_K: decode_q3_k(block, out); return 0;
    case GGML_Q4_K: decode_q4_k(block, out); return 0;
    case GGML_Q5_K: decode_q5_k(block, out); return 0;
    case GGML_Q6_K: decode_q6_k(block, out); return 0;
    default: return -1;
  }
}

/* Decode an N x K matrix stored as N rows of K/QK consecutive blocks. */
int oracle_dequantize(int type, const uint8_t *raw, int64_t n, int64_t k,
                      float *out) {
  int qk, bytes;
  if (oracle_block_geometry(type, &qk, &bytes) || k % qk) return -1;
  int64_t blocks = n * (k / qk);
  for (int64_t b = 0; b < blocks; ++b)
    oracle_decode_block(type, raw + b * bytes, out + b * qk);
  return 0;
}

/* --------------------------------------------------------- the products --- */

static int g_threads = 1;

void oracle_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/*
 * out[m,n] = sum_k x[m,k] * W[n,k] with fp32 accumulation in k order.
 * mode 0 (decode):  fp32 x times fp32 dequantized W.
 * mode 1 (prefill): fp16-rounded x times fp16-rounded dequantized W.
 * x_half: x given as fp16 bits (else fp32).  out_half: write fp16 bits (RNE).
 */
int oracle_linear(int type, int mode, const void *x, int x_half,
                  const uint8_t *raw, void *out, int out_half, int64_t m,
                  int64_t n, int64_t k) {
  int qk, bytes;
  if (oracle_block_geometry(type, &qk, &bytes) || k % qk || m < 1 || n < 1)
    return -1;
  float *xf = (float *)malloc(sizeof(float) * (size_t)(m * k));
  if (!xf) return -2;
  for (int64_t i = 0; i < m * k; ++i) {
    float v = x_half ? oracle_half_to_float(((const uint16_t *)x)[i])
                     : ((const float *)x)[i];
    if (mode == 1) v = oracle_half_to_float(oracle_float_to_half(v));
    xf[i] = v;
  }
  const int64_t blocks_per_row = k / qk;
  int status = 0;
#ifdef _OPENMP
#pragma omp parallel num_threads(g_threads)
#endif
  {
    float *row = (float *)malloc(sizeof(float) * (size_t)k);
    if (!row) {
      status = -2;
    } else {
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
      for (int64_t r = 0; r < n; ++r) {
        const uint8_t *src = raw + r * blocks_per_row * bytes;
        for (int64_t b = 0; b < blocks_per_row; ++b)
          oracle_decode_block(type, src + b * bytes, row + b * qk);
        if (mode == 1)
          for (int64_t i = 0; i < k; ++i)
            row[i] = oracle_half_to_float(oracle_float_to_half(row[i]));
        for (int64_t mi = 0; mi < m; ++mi) {
          const float *xr = xf + mi * k;
          float acc = 0.0f;
          for (int64_t i = 0; i < k; ++i) acc += xr[i] * row[i];
          if (out_half)
            ((uint16_t *)out)[mi * n + r] = oracle_float_to_half(acc);
          else
            ((float *)out)[mi * n + r] = acc;
        }
      }
      free(row);
    }
  }
  free(xf);
  return status;
}

/* ---------------------------------------------- TensorKernelV1 CPU entry --- */

static int32_t fail(TensorErrorV1 *error, int32_t code, const char *message) {
  if (error) {
    error->code = code;
    snprintf(error->message, sizeof(error->message), "%s", message);
  }
  return code;
}

static int check_buffer(const TensorArgumentV1 *arg, uint32_t rank,
                        uint64_t itemsize) {
  const TensorBufferV1 *b = &arg->buffer;
  if (arg->kind != TENSOR_ARG_BUFFER || b->dtype != arg->dtype ||
      b->device_type != TENSOR_DEVICE_CPU || b->device_ordinal != 0 ||
      !b->address || b->rank != rank || !b->shape || !b->strides)
    return -1;
  uint64_t expected = itemsize;
  for (int axis = (int)rank - 1; axis >= 0; --axis) {
    if (b->shape[axis] <= 0 || b->strides[axis] != (int64_t)expected) return -1;
    expected *= (uint64_t)b->shape[axis];
  }
  return b->byte_size >= expected ? 0 : -1;
}

/*
 * CPU baselines of the decode path (mode 0: fp32 operands, benchmark.py:466-472)
 * and of the prefill path (mode 1: fp16-rounded operands, benchmark.py:473-477),
 * invoked exactly as the reference CPU provider invokes a native image.
 * Arguments, in order:
 *   x    fp16 [M, K]
 *   w    uint8 [N, K/QK*BLOCK]  (raw GGUF rows)
 *   out  fp16 or fp32 [M, N]
 *   type uint32 scalar GGML type id (2, 8, 12, 14, ...)
 */
static int32_t linear_cpu(const TensorCallV1 *call, TensorErrorV1 *error, int mode) {
  if (error) {
    error->code = 0;
    error->message[0] = 0;
  }
  if (!call || call->abi_version != TENSOR_ABI_VERSION ||
      call->struct_size < sizeof(TensorCallV1))
    return fail(error, TENSOR_ERROR_ABI, "unsupported call ABI");
  if (call->flags || call->argument_count != 4 || !call->arguments)
    return fail(error, TENSOR_ERROR_ARGUMENT, "invalid argument count or flags");
  if (call->stream.device_type != TENSOR_DEVICE_CPU ||
      call->stream.device_ordinal || call->stream.handle)
    return fail(error, TENSOR_ERROR_PROVIDER,
                "CPU calls need the synchronous CPU stream");
  const TensorArgumentV1 *a = call->arguments;
  if (a[3].kind != TENSOR_ARG_SCALAR || a[3].dtype != TENSOR_UINT32 ||
      (a[3].scalar >> 32))
    return fail(error, TENSOR_ERROR_ARGUMENT, "type: wrong argument kind or dtype");
  int type = (int)a[3].scalar, qk, bytes;
  if (oracle_block_geometry(type, &qk, &bytes))
    return fail(error, TENSOR_ERROR_ARGUMENT, "type: unsupported GGML type");
  if (a[0].dtype != TENSOR_FLOAT16 || check_buffer(&a[0], 2, 2))
    return fail(error, TENSOR_ERROR_ARGUMENT, "x: invalid buffer descriptor");
  if (a[1].dtype != TENSOR_UINT8 || check_buffer(&a[1], 2, 1))
    return fail(error, TENSOR_ERROR_ARGUMENT, "w: invalid buffer descriptor");
  int out_half = a[2].dtype == TENSOR_FLOAT16;
  if ((!out_half && a[2].dtype != TENSOR_FLOAT32) ||
      check_buffer(&a[2], 2, out_half ? 2 : 4))
    return fail(error, TENSOR_ERROR_ARGUMENT, "out: invalid buffer descriptor");
  int64_t m = a[0].buffer.shape[0], k = a[0].buffer.shape[1];
  int64_t n = a[1].buffer.shape[0];
  if (k % qk || a[1].buffer.shape[1] != k / qk * bytes)
    return fail(error, TENSOR_ERROR_ARGUMENT, "w: shape, stride or size mismatch");
  if (a[2].buffer.shape[0] != m || a[2].buffer.shape[1] != n)
    return fail(error, TENSOR_ERROR_ARGUMENT, "out: shape, stride or size mismatch");
  if (oracle_linear(type, mode, (const void *)a[0].buffer.address, 1,
                    (const uint8_t *)a[1].buffer.address,
                    (void *)a[2].buffer.address, out_half, m, n, k))
    return fail(error, TENSOR_ERROR_PROVIDER, "CPU kernel failed");
  return TENSOR_OK;
}

int32_t tensor_gguf_gemv_cpu_v1(const TensorCallV1 *call, TensorErrorV1 *error) {
  return linear_cpu(call, error, 0);
}

int32_t tensor_gguf_gemm_cpu_v1(const TensorCallV1 *call, TensorErrorV1 *error) {
  return linear_cpu(call, error, 1);
}
