// A native host of libtensor_hip.so: C++ and the C ABI only (tensor/abi.h, tensor_hip.h),
// no Python, no HIP headers.  It opens the library with dlopen, binds the entry points by
// name and drives them with TensorCallV1 descriptors, the way the reference's native host
// drives a CPU image (src/tensor/native/host.cpp:51-131).
//
//   host check <libtensor_hip.so>   malformed calls only: every one must be refused by the
//                                   descriptor checks, before any HIP call (no GPU needed)
//   host gpu <libtensor_hip.so>     the same checks, then real calls on device 0: the showcase's
//                                   packed form at M = 1 (fp32 GEMV) and M = 4 (fp16 GEMM), and
//                                   the rank-2 linear entry, on blocks whose products are exact,
//                                   with the device memory, stream and copies of the library's
//                                   own runtime services
//
// Prints one JSON line; exit status 0 only when every check passed.
#include <tensor/abi.h>
#include <tensor_hip.h>

#include <dlfcn.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

template <class F>
F bind(void* library, const char* name) {
  void* symbol = dlsym(library, name);
  if (!symbol) throw std::runtime_error(std::string("missing symbol ") + name);
  return reinterpret_cast<F>(symbol);
}

struct Library {
  void* handle;
  TensorKernelV1 packed, linear;
  decltype(&tensor_hip_device_count) device_count;
  decltype(&tensor_hip_set_device) set_device;
  decltype(&tensor_hip_malloc) malloc_;
  decltype(&tensor_hip_free) free_;
  decltype(&tensor_hip_copy_htod) htod;
  decltype(&tensor_hip_copy_dtoh) dtoh;
  decltype(&tensor_hip_stream_create) stream_create;
  decltype(&tensor_hip_stream_synchronize) stream_sync;
  decltype(&tensor_hip_stream_destroy) stream_destroy;

  explicit Library(const char* path) {
    handle = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!handle) throw std::runtime_error(dlerror());
    packed = bind<TensorKernelV1>(handle, "tensor_gguf_packed_v1");
    linear = bind<TensorKernelV1>(handle, "tensor_gguf_linear_v1");
    device_count = bind<decltype(device_count)>(handle, "tensor_hip_device_count");
    set_device = bind<decltype(set_device)>(handle, "tensor_hip_set_device");
    malloc_ = bind<decltype(malloc_)>(handle, "tensor_hip_malloc");
    free_ = bind<decltype(free_)>(handle, "tensor_hip_free");
    htod = bind<decltype(htod)>(handle, "tensor_hip_copy_htod");
    dtoh = bind<decltype(dtoh)>(handle, "tensor_hip_copy_dtoh");
    stream_create = bind<decltype(stream_create)>(handle, "tensor_hip_stream_create");
    stream_sync = bind<decltype(stream_sync)>(handle, "tensor_hip_stream_synchronize");
    stream_destroy = bind<decltype(stream_destroy)>(handle, "tensor_hip_stream_destroy");
  }
};

void check(int32_t status, const TensorErrorV1& error, const char* what) {
  if (status) throw std::runtime_error(std::string(what) + ": " + error.message);
}

// One call's descriptor storage: buffers first, then uint32 scalars.
struct Call {
  std::vector<int64_t> shapes, strides;
  std::vector<TensorArgumentV1> args;
  TensorCallV1 call{};

  Call(std::vector<std::vector<int64_t>> buffer_shapes, std::vector<uint32_t> dtypes, std::vector<uint64_t> addresses,
       std::vector<uint64_t> scalars, uint64_t stream) {
    size_t total = 0;
    for (auto& s : buffer_shapes) total += s.size();
    shapes.reserve(total);
    strides.reserve(total);
    args.resize(buffer_shapes.size() + scalars.size());
    for (size_t i = 0; i < buffer_shapes.size(); ++i) {
      const int64_t item = dtypes[i] == TENSOR_FLOAT32 ? 4 : dtypes[i] == TENSOR_FLOAT16 ? 2 : 1;
      const size_t first = shapes.size();
      for (int64_t extent : buffer_shapes[i]) shapes.push_back(extent), strides.push_back(0);
      int64_t bytes = item;
      for (size_t axis = buffer_shapes[i].size(); axis-- > 0;) {
        strides[first + axis] = bytes;
        bytes *= buffer_shapes[i][axis];
      }
      TensorArgumentV1& a = args[i];
      a.kind = TENSOR_ARG_BUFFER;
      a.dtype = dtypes[i];
      a.buffer = {addresses[i], (uint64_t)bytes, &shapes[first], &strides[first], (uint32_t)buffer_shapes[i].size(),
                  dtypes[i], TENSOR_DEVICE_ROCM, 0};
    }
    for (size_t j = 0; j < scalars.size(); ++j) {
      TensorArgumentV1& a = args[buffer_shapes.size() + j];
      a.kind = TENSOR_ARG_SCALAR;
      a.dtype = TENSOR_UINT32;
      a.scalar = scalars[j];
    }
    call = {TENSOR_ABI_VERSION, sizeof(TensorCallV1), args.data(), (uint32_t)args.size(), 0, {1, 1, 1}, {256, 1, 1}, 0,
            {TENSOR_DEVICE_ROCM, 0, stream}};
  }
};

constexpr int kN = 64, kK = 256, kBlocks = kK / 32, kRowBytes = kBlocks * 18;

// Q4_0 rows with d = 0.5 and code (n + j) % 16 at element j: weight (code - 8) / 2.
std::vector<uint8_t> q4_0_rows() {
  std::vector<uint8_t> raw((size_t)kN * kRowBytes);
  for (int n = 0; n < kN; ++n)
    for (int b = 0; b < kBlocks; ++b) {
      uint8_t* block = &raw[(size_t)n * kRowBytes + b * 18];
      block[0] = 0x00, block[1] = 0x38;  // fp16 0.5
      for (int j = 0; j < 16; ++j) {
        const int lo = (n + 32 * b + j) % 16, hi = (n + 32 * b + j + 16) % 16;
        block[2 + j] = (uint8_t)(lo | (hi << 4));
      }
    }
  return raw;
}

float weight(int n, int k) { return (float)(((n + k) % 16) - 8) * 0.5f; }

// Malformed variants of a well-formed call; each must be refused with its status.
int negative_checks(TensorKernelV1 entry, const Call& good, const char* name) {
  struct Case {
    const char* what;
    int32_t want;
    void (*tamper)(TensorCallV1&, std::vector<TensorArgumentV1>&);
  };
  const Case cases[] = {
      {"abi_version 2", TENSOR_ERROR_ABI, [](TensorCallV1& c, std::vector<TensorArgumentV1>&) { c.abi_version = 2; }},
      {"struct_size 8", TENSOR_ERROR_ABI, [](TensorCallV1& c, std::vector<TensorArgumentV1>&) { c.struct_size = 8; }},
      {"flags 1", TENSOR_ERROR_ARGUMENT, [](TensorCallV1& c, std::vector<TensorArgumentV1>&) { c.flags = 1; }},
      {"x float64", TENSOR_ERROR_ARGUMENT,
       [](TensorCallV1&, std::vector<TensorArgumentV1>& a) { a[0].dtype = a[0].buffer.dtype = TENSOR_FLOAT64; }},
      {"x byte_size 4", TENSOR_ERROR_ARGUMENT,
       [](TensorCallV1&, std::vector<TensorArgumentV1>& a) { a[0].buffer.byte_size = 4; }},
      {"w on the CPU", TENSOR_ERROR_ARGUMENT,
       [](TensorCallV1&, std::vector<TensorArgumentV1>& a) { a[1].buffer.device_type = TENSOR_DEVICE_CPU; }},
      {"CPU stream", TENSOR_ERROR_PROVIDER,
       [](TensorCallV1& c, std::vector<TensorArgumentV1>&) { c.stream.device_type = TENSOR_DEVICE_CPU; }},
  };
  int passed = 0;
  for (const Case& c : cases) {
    std::vector<TensorArgumentV1> args = good.args;
    TensorCallV1 call = good.call;
    call.arguments = args.data();
    c.tamper(call, args);
    TensorErrorV1 error{};
    std::memset(error.message, 'x', sizeof(error.message));
    const int32_t status = entry(&call, &error);
    if (status != c.want || error.code != c.want || std::strlen(error.message) >= sizeof(error.message))
      throw std::runtime_error(std::string(name) + ": " + c.what + " gave status " + std::to_string(status));
    ++passed;
  }
  return passed;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc != 3 || (std::string(argv[1]) != "check" && std::string(argv[1]) != "gpu"))
      throw std::runtime_error("usage: host check|gpu libtensor_hip.so");
    const bool gpu = std::string(argv[1]) == "gpu";
    Library lib(argv[2]);
    // Fake, never dereferenced addresses for the refusal checks (16-byte aligned).
    const uint64_t fx = 0x100000, fw = 0x200000, fo = 0x300000;
    const Call packed_shape({{1 * kK}, {(int64_t)kN * kRowBytes}, {1 * kN}},
                            {TENSOR_FLOAT32, TENSOR_UINT8, TENSOR_FLOAT32}, {fx, fw, fo},
                            {TENSOR_GGML_Q4_0, 1, kN, kK}, 0);
    const Call linear_shape({{1, kK}, {kN, kRowBytes}, {1, kN}}, {TENSOR_FLOAT16, TENSOR_UINT8, TENSOR_FLOAT32},
                            {fx, fw, fo}, {TENSOR_GGML_Q4_0}, 0);
    int negatives = negative_checks(lib.packed, packed_shape, "packed");
    negatives += negative_checks(lib.linear, linear_shape, "linear");
    int exact = 0;
    if (gpu) {
      TensorErrorV1 error{};
      int32_t count = 0;
      check(lib.device_count(&count, &error), error, "device count");
      if (count < 1) throw std::runtime_error("no HIP device");
      check(lib.set_device(0, &error), error, "set device");
      uint64_t stream = 0;
      check(lib.stream_create(&stream, &error), error, "stream");
      const std::vector<uint8_t> raw = q4_0_rows();
      constexpr int kM = 4;
      std::vector<float> x((size_t)kM * kK);
      for (int m = 0; m < kM; ++m)
        for (int k = 0; k < kK; ++k) x[(size_t)m * kK + k] = (float)((m * 7 + k * 3) % 9 - 4) * 0.25f;
      uint64_t dx = 0, dw = 0, dout = 0;
      check(lib.malloc_(x.size() * 4, &dx, &error), error, "malloc x");
      check(lib.malloc_(raw.size(), &dw, &error), error, "malloc w");
      check(lib.malloc_((size_t)kM * kN * 4, &dout, &error), error, "malloc out");
      check(lib.htod(dx, x.data(), x.size() * 4, stream, &error), error, "copy x");
      check(lib.htod(dw, raw.data(), raw.size(), stream, &error), error, "copy w");
      for (int m : {1, kM}) {
        Call call({{(int64_t)m * kK}, {(int64_t)raw.size()}, {(int64_t)m * kN}},
                  {TENSOR_FLOAT32, TENSOR_UINT8, TENSOR_FLOAT32}, {dx, dw, dout}, {TENSOR_GGML_Q4_0, (uint64_t)m, kN, kK},
                  stream);
        std::vector<float> nan((size_t)m * kN, NAN), out((size_t)m * kN);
        check(lib.htod(dout, nan.data(), nan.size() * 4, stream, &error), error, "fill out");
        check(lib.packed(&call.call, &error), error, "packed call");
        check(lib.stream_sync(stream, &error), error, "synchronize");
        check(lib.dtoh(out.data(), dout, out.size() * 4, stream, &error), error, "copy out");
        // every weight, activation and partial sum is a multiple of 1/8 below 2^11: exact in
        // fp16 and fp32, so any summation order gives the exact value
        for (int i = 0; i < m; ++i)
          for (int n = 0; n < kN; ++n) {
            double want = 0;
            for (int k = 0; k < kK; ++k) want += (double)x[(size_t)i * kK + k] * weight(n, k);
            if (out[(size_t)i * kN + n] != (float)want)
              throw std::runtime_error("packed m=" + std::to_string(m) + " out[" + std::to_string(i) + "," +
                                       std::to_string(n) + "] = " + std::to_string(out[(size_t)i * kN + n]) +
                                       ", want " + std::to_string(want));
          }
        ++exact;
      }
      for (auto address : {dx, dw, dout}) check(lib.free_(address, &error), error, "free");
      check(lib.stream_destroy(stream, &error), error, "stream destroy");
    }
    dlclose(lib.handle);
    std::cout << "{\"status\":\"passed\",\"mode\":\"" << argv[1] << "\",\"abi\":" << TENSOR_ABI_VERSION
              << ",\"negative_checks\":" << negatives << ",\"exact_calls\":" << exact << "}\n";
    return 0;
  } catch (const std::exception& error) {
    std::cerr << error.what() << "\n";
    return 1;
  }
}
