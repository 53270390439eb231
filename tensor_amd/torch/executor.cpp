// Native executor of tensor_amd.torch: replays a bound TensorCallV1 with PyTorch tensors'
// pointers written in, on PyTorch's current HIP stream, with the GIL released and no Python
// work per call.
//
// It serves the role of the reference's tensor-torch C++ Plan
// (packages/tensor-torch/src/tensor_torch/native/executor.cpp:74-176), which rebinds pointers
// into CUDA kernel parameters and calls cuLaunchKernel; here a call goes through the
// provider's C ABI (include/tensor/abi.h), whose entry point validates the descriptors and
// picks its own launch geometry as it does for every other caller.
//
// Structure: a Layout is the fixed-size fingerprint a cached call depends on (dtype, device,
// sizes, strides); a CallImage is the plan's private copy of the bound call (descriptor,
// arguments, one flat store for every buffer's shape and stride arrays), so it outlives the
// Python objects that made it; Wires say which operand (inputs, then outputs) feeds which
// buffer argument and the alignment the manifest declares for it.  A prepared plan keeps its
// operands and refuses them once their layout or storage changed; a rebinding plan takes
// inputs of the recorded layouts and allocates its outputs with torch.  Built against torch's
// non-stable C++ ABI: the module name carries torch's major.minor and only a matching build
// is imported.
#include <ATen/ops/empty_strided.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <c10/hip/HIPStream.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/csrc/autograd/python_variable.h>

#include <algorithm>
#include <array>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "tensor/abi.h"

namespace py = pybind11;

namespace {

constexpr uint32_t kRocmDevice = 10;  // TENSOR_DEVICE_ROCM
constexpr uint32_t kBufferKind = 1;   // TENSOR_ARG_BUFFER
constexpr int kMaxRank = 8;

using KernelEntry = int32_t (*)(const TensorCallV1*, TensorErrorV1*);
using ModuleEntry = int32_t (*)(uint64_t, const TensorCallV1*, TensorErrorV1*);

struct Layout {
  at::ScalarType dtype = at::ScalarType::Undefined;
  int device = -1;
  int rank = 0;
  std::array<int64_t, kMaxRank> dims{}, steps{};

  static Layout of(const at::Tensor& t) {
    if (!t.is_cuda()) throw py::value_error("native plans take ROCm tensors");
    if (t.dim() > kMaxRank) throw py::value_error("native plans take tensors of rank 8 or less");
    Layout layout;
    layout.dtype = t.scalar_type();
    layout.device = t.get_device();
    layout.rank = static_cast<int>(t.dim());
    for (int axis = 0; axis < layout.rank; ++axis) {
      layout.dims[axis] = t.size(axis);
      layout.steps[axis] = t.stride(axis);
    }
    return layout;
  }

  bool fits(const at::Tensor& t) const {
    if (!t.is_cuda() || t.scalar_type() != dtype || t.get_device() != device || t.dim() != rank) return false;
    for (int axis = 0; axis < rank; ++axis)
      if (t.size(axis) != dims[axis] || t.stride(axis) != steps[axis]) return false;
    return true;
  }

  at::Tensor allocate() const {
    return at::empty_strided(at::IntArrayRef(dims.data(), rank), at::IntArrayRef(steps.data(), rank),
                             at::TensorOptions().dtype(dtype).device(c10::Device(c10::DeviceType::CUDA, device)));
  }
};

// PyTorch tensors of a Python tuple (or any sequence), in order.
std::vector<at::Tensor> tensors_in(py::handle sequence) {
  py::sequence items = py::reinterpret_borrow<py::sequence>(sequence);
  std::vector<at::Tensor> tensors;
  tensors.reserve(items.size());
  for (size_t i = 0; i < items.size(); ++i) {
    py::handle item = items[i];
    if (!THPVariable_Check(item.ptr())) throw py::type_error("native plans take PyTorch tensors");
    tensors.push_back(THPVariable_Unpack(item.ptr()));
  }
  return tensors;
}

class CallImage {
  TensorCallV1 call_{};
  std::vector<TensorArgumentV1> arguments_;
  std::vector<int64_t> store_;  // every buffer argument's shape, then its strides

 public:
  explicit CallImage(uint64_t address) {
    if (!address) throw py::value_error("a native plan needs a bound call");
    std::memcpy(&call_, reinterpret_cast<const void*>(address), sizeof(call_));
    if (call_.struct_size != sizeof(TensorCallV1) || !call_.arguments || !call_.argument_count)
      throw py::value_error("not a bound TensorCallV1");
    arguments_.assign(call_.arguments, call_.arguments + call_.argument_count);
    size_t extent = 0;
    for (const auto& argument : arguments_)
      if (argument.kind == kBufferKind) extent += 2 * static_cast<size_t>(argument.buffer.rank);
    store_.resize(extent);
    int64_t* cursor = store_.data();
    for (auto& argument : arguments_) {
      if (argument.kind != kBufferKind) continue;
      auto& buffer = argument.buffer;
      std::copy(buffer.shape, buffer.shape + buffer.rank, cursor);
      std::copy(buffer.strides, buffer.strides + buffer.rank, cursor + buffer.rank);
      buffer.shape = cursor;
      buffer.strides = cursor + buffer.rank;
      cursor += 2 * buffer.rank;
    }
    call_.arguments = arguments_.data();
  }

  size_t size() const { return arguments_.size(); }
  bool is_buffer(size_t i) const { return arguments_[i].kind == kBufferKind; }
  void set_address(size_t i, uint64_t address) { arguments_[i].buffer.address = address; }

  const TensorCallV1* on(int ordinal, uint64_t stream) {
    call_.stream.device_type = kRocmDevice;
    call_.stream.device_ordinal = ordinal;
    call_.stream.handle = stream;
    return &call_;
  }
};

struct Wire {
  size_t argument;   // buffer argument of the call
  size_t operand;    // inputs first, then outputs
  uint64_t align;    // the manifest's alignment, bytes
};

class Plan {
  std::string name_;
  uint64_t entry_, function_;  // function_ != 0: a code-object kernel launched by the module entry
  bool prepared_;
  int device_ = -1;
  std::vector<Layout> inputs_, outputs_;
  std::vector<at::Tensor> operands_;       // a prepared plan's tensors
  std::vector<const void*> storage_;       // and their data pointers when prepared
  CallImage image_;
  std::vector<Wire> wires_;
  std::mutex mutex_;

  // Writes the operands into the call and runs it on the device's current HIP stream. False
  // when an operand's pointer is not aligned as its argument requires (nothing has run).
  bool submit(const std::vector<at::Tensor>& operands, int32_t& status, TensorErrorV1& error) {
    c10::DeviceGuard guard(c10::Device(c10::DeviceType::CUDA, device_));
    const auto stream = c10::hip::getCurrentHIPStream(device_);
    for (const Wire& wire : wires_)
      if (reinterpret_cast<uintptr_t>(operands[wire.operand].data_ptr()) % wire.align) return false;
    for (const Wire& wire : wires_) {
      const at::Tensor& t = operands[wire.operand];
      c10::hip::HIPCachingAllocator::recordStream(t.storage().data_ptr(), stream);
      image_.set_address(wire.argument, reinterpret_cast<uint64_t>(t.data_ptr()));
    }
    const TensorCallV1* call = image_.on(device_, reinterpret_cast<uint64_t>(stream.stream()));
    status = function_ ? reinterpret_cast<ModuleEntry>(entry_)(function_, call, &error)
                       : reinterpret_cast<KernelEntry>(entry_)(call, &error);
    return true;
  }

  [[noreturn]] void raise(int32_t status, TensorErrorV1& error) const {
    error.message[sizeof(error.message) - 1] = '\0';
    py::object type = py::module_::import("tensor_amd._native").attr("HipError");
    py::object exception = type(name_, status, std::string(error.message));
    PyErr_SetObject(type.ptr(), exception.ptr());
    throw py::error_already_set();
  }

 public:
  Plan(std::string name, uint64_t entry, uint64_t function, uint64_t call, py::tuple inputs, py::tuple outputs,
       std::vector<std::tuple<size_t, size_t, uint64_t>> bindings, bool prepared)
      : name_(std::move(name)), entry_(entry), function_(function), prepared_(prepared), image_(call) {
    if (!entry_) throw py::value_error("a native plan needs an entry point");
    std::vector<at::Tensor> given = tensors_in(inputs), produced = tensors_in(outputs);
    if (given.empty()) throw py::value_error("a native plan needs tensor inputs");
    for (const auto& t : given) inputs_.push_back(Layout::of(t));
    for (const auto& t : produced) outputs_.push_back(Layout::of(t));
    device_ = inputs_.front().device;
    for (const auto* set : {&inputs_, &outputs_})
      for (const Layout& layout : *set)
        if (layout.device != device_) throw py::value_error("a native plan's tensors must share one device");
    const size_t operands = inputs_.size() + outputs_.size();
    for (const auto& [argument, operand, align] : bindings) {
      if (argument >= image_.size() || !image_.is_buffer(argument) || operand >= operands || !align)
        throw py::value_error("invalid native tensor binding");
      wires_.push_back({argument, operand, align});
    }
    if (prepared_) {
      operands_ = std::move(given);
      operands_.insert(operands_.end(), produced.begin(), produced.end());
      for (const auto& t : operands_) storage_.push_back(t.data_ptr());
    }
  }

  // A prepared plan takes no arguments and returns None. A rebinding plan takes the inputs and
  // returns the outputs, or None when an input's layout differs from the recorded one or its
  // pointer is not aligned as declared (the caller then takes the validated path).
  py::object call(py::args args) {
    std::vector<at::Tensor> operands;
    if (prepared_) {
      if (!args.empty()) throw py::type_error("a prepared native call takes no arguments");
      for (size_t i = 0; i < operands_.size(); ++i) {
        const Layout& layout = i < inputs_.size() ? inputs_[i] : outputs_[i - inputs_.size()];
        if (!layout.fits(operands_[i]) || operands_[i].data_ptr() != storage_[i])
          throw py::value_error("prepared tensor metadata or storage changed");
      }
      operands = operands_;
    } else {
      if (args.size() != inputs_.size()) throw py::value_error("wrong native input count");
      operands = tensors_in(args);
      for (size_t i = 0; i < inputs_.size(); ++i)
        if (!inputs_[i].fits(operands[i])) return py::none();
      for (const Wire& wire : wires_)
        if (wire.operand < inputs_.size() &&
            reinterpret_cast<uintptr_t>(operands[wire.operand].data_ptr()) % wire.align)
          return py::none();
    }
    TensorErrorV1 error{};
    int32_t status = 0;
    bool submitted;
    {
      py::gil_scoped_release release;
      std::lock_guard<std::mutex> lock(mutex_);
      if (!prepared_) {
        c10::DeviceGuard guard(c10::Device(c10::DeviceType::CUDA, device_));
        for (const Layout& layout : outputs_) operands.push_back(layout.allocate());
      }
      submitted = submit(operands, status, error);
    }
    if (!submitted) throw py::value_error("a native output has insufficient pointer alignment");
    if (status) raise(status, error);
    if (prepared_) return py::none();
    auto wrap = [&](size_t i) { return py::reinterpret_steal<py::object>(THPVariable_Wrap(operands[inputs_.size() + i])); };
    if (outputs_.size() == 1) return wrap(0);
    py::tuple result(outputs_.size());
    for (size_t i = 0; i < outputs_.size(); ++i) result[i] = wrap(i);
    return result;
  }
};

}  // namespace

PYBIND11_MODULE(TENSOR_EXECUTOR_MODULE, m) {
  py::class_<Plan>(m, "Plan")
      .def(py::init<std::string, uint64_t, uint64_t, uint64_t, py::tuple, py::tuple,
                    std::vector<std::tuple<size_t, size_t, uint64_t>>, bool>())
      .def("__call__", &Plan::call);
}
