// Native executor of tensor_amd.torch: binds PyTorch tensors into a TensorCallV1 the
// plan owns and calls a HIP provider entry point on PyTorch's current HIP stream, with
// the GIL released and no Python work per call.
//
// Counterpart of the reference's tensor-torch C++ Plan
// (packages/tensor-torch/src/tensor_torch/native/executor.cpp:74-176), which rebinds
// pointers into CUDA kernel parameters and calls cuLaunchKernel.  Here the call goes
// through the provider's C ABI (include/tensor/abi.h), so the entry point validates the
// descriptors and picks its own launch geometry exactly as it does for every other
// caller.  A plan is either fixed (it retains its tensors and checks their storage is
// unchanged) or rebinding (it takes inputs of the recorded metadata and allocates the
// outputs with torch).  Built against torch's non-stable C++ ABI: the module name
// carries torch's major/minor version and only a matching build is imported.
#include <ATen/ops/empty_strided.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <c10/hip/HIPStream.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "tensor/abi.h"

namespace py = pybind11;

namespace {

constexpr uint32_t kDeviceRocm = 10;

using Entry = int32_t (*)(const TensorCallV1*, TensorErrorV1*);
using ModuleEntry = int32_t (*)(uint64_t, const TensorCallV1*, TensorErrorV1*);

struct Spec {
  std::vector<int64_t> sizes, strides;
  at::ScalarType dtype;
  c10::Device device;
  void* pointer;

  explicit Spec(const at::Tensor& t)
      : sizes(t.sizes().vec()), strides(t.strides().vec()), dtype(t.scalar_type()), device(t.device()),
        pointer(t.data_ptr()) {}

  bool matches(const at::Tensor& t, bool fixed) const {
    return t.device() == device && t.scalar_type() == dtype && t.sizes().equals(sizes) &&
           t.strides().equals(strides) && (!fixed || t.data_ptr() == pointer);
  }
};

std::vector<at::Tensor> unpack(py::handle sequence) {
  std::vector<at::Tensor> result;
  for (auto value : py::reinterpret_borrow<py::sequence>(sequence)) {
    if (!THPVariable_Check(value.ptr())) throw py::type_error("the native executor takes PyTorch tensors");
    result.push_back(THPVariable_Unpack(value.ptr()));
  }
  return result;
}

struct Slot {
  size_t argument;   // index into the call's arguments
  size_t tensor;     // inputs first, then outputs
  uint64_t alignment;
};

class Plan {
  std::string name_;
  uint64_t entry_, function_;  // function_ != 0: a code-object kernel launched by the module entry
  bool fixed_;
  c10::Device device_{c10::DeviceType::CUDA, 0};
  std::vector<Spec> inputs_, outputs_;
  std::vector<at::Tensor> retained_;
  std::vector<TensorArgumentV1> arguments_;
  std::vector<std::vector<int64_t>> shapes_, strides_;
  std::vector<Slot> slots_;
  TensorCallV1 call_{};
  std::mutex mutex_;

 public:
  // `call` is the address of a bound TensorCallV1; the plan copies it, its arguments and
  // every buffer's shape and stride arrays, so it outlives the Python objects that made it.
  Plan(std::string name, uint64_t entry, uint64_t function, uint64_t call, py::tuple inputs, py::tuple outputs,
       std::vector<std::tuple<size_t, size_t, uint64_t>> bindings, bool fixed)
      : name_(std::move(name)), entry_(entry), function_(function), fixed_(fixed) {
    if (!entry_ || !call) throw py::value_error("a native plan needs an entry point and a bound call");
    auto in = unpack(inputs), out = unpack(outputs);
    if (in.empty()) throw py::value_error("a native plan needs tensor inputs");
    device_ = in.front().device();
    if (!device_.is_cuda()) throw py::value_error("a native plan needs ROCm tensors");
    for (const auto& t : in) {
      if (t.device() != device_) throw py::value_error("native plan inputs must share a device");
      inputs_.emplace_back(t);
    }
    for (const auto& t : out) {
      if (t.device() != device_) throw py::value_error("native plan outputs must share a device");
      outputs_.emplace_back(t);
    }
    if (fixed_) {
      retained_ = std::move(in);
      retained_.insert(retained_.end(), out.begin(), out.end());
    }
    std::memcpy(&call_, reinterpret_cast<const void*>(call), sizeof(call_));
    if (call_.struct_size != sizeof(TensorCallV1) || !call_.arguments)
      throw py::value_error("not a bound TensorCallV1");
    arguments_.assign(call_.arguments, call_.arguments + call_.argument_count);
    shapes_.resize(arguments_.size());
    strides_.resize(arguments_.size());
    for (size_t i = 0; i < arguments_.size(); ++i) {
      auto& buffer = arguments_[i].buffer;
      if (arguments_[i].kind != 1) continue;
      shapes_[i].assign(buffer.shape, buffer.shape + buffer.rank);
      strides_[i].assign(buffer.strides, buffer.strides + buffer.rank);
      buffer.shape = shapes_[i].data();
      buffer.strides = strides_[i].data();
    }
    call_.arguments = arguments_.data();
    for (const auto& [argument, tensor, alignment] : bindings) {
      if (argument >= arguments_.size() || arguments_[argument].kind != 1 ||
          tensor >= inputs_.size() + outputs_.size() || !alignment)
        throw py::value_error("invalid native tensor binding");
      slots_.push_back({argument, tensor, alignment});
    }
  }

  // Fixed plans take no arguments and return None; rebinding plans take the inputs and
  // return the outputs, or None when an input's metadata differs from the recorded one or
  // its pointer is not aligned as declared (the caller then takes the validated path).
  py::object call(py::args args) {
    if (fixed_ && !args.empty()) throw py::type_error("a prepared native call takes no arguments");
    if (!fixed_ && args.size() != inputs_.size()) throw py::value_error("wrong native input count");
    auto tensors = fixed_ ? retained_ : unpack(args);
    for (size_t i = 0; i < inputs_.size(); ++i) {
      if (inputs_[i].matches(tensors[i], fixed_)) continue;
      if (!fixed_) return py::none();  // other metadata: the caller's validated path decides
      throw py::value_error("prepared tensor metadata or storage changed");
    }
    if (fixed_) {
      for (size_t i = 0; i < outputs_.size(); ++i)
        if (!outputs_[i].matches(tensors[inputs_.size() + i], true))
          throw py::value_error("prepared tensor metadata or storage changed");
    }
    for (const auto& slot : slots_)
      if (slot.tensor < inputs_.size() &&
          reinterpret_cast<uintptr_t>(tensors[slot.tensor].data_ptr()) % slot.alignment)
        return py::none();
    TensorErrorV1 error{};
    int32_t status = 0;
    bool misaligned = false;
    {
      py::gil_scoped_release release;
      std::lock_guard<std::mutex> lock(mutex_);
      c10::DeviceGuard guard(device_);
      auto stream = c10::hip::getCurrentHIPStream(device_.index());
      if (!fixed_)
        for (const auto& spec : outputs_)
          tensors.push_back(at::empty_strided(spec.sizes, spec.strides,
                                              at::TensorOptions().dtype(spec.dtype).device(spec.device)));
      for (const auto& slot : slots_) {
        const auto& tensor = tensors[slot.tensor];
        auto pointer = reinterpret_cast<uint64_t>(tensor.data_ptr());
        if (pointer % slot.alignment) {
          misaligned = true;
          break;
        }
        c10::hip::HIPCachingAllocator::recordStream(tensor.storage().data_ptr(), stream);
        arguments_[slot.argument].buffer.address = pointer;
      }
      if (!misaligned) {
        call_.stream.device_type = kDeviceRocm;
        call_.stream.device_ordinal = device_.index();
        call_.stream.handle = reinterpret_cast<uint64_t>(stream.stream());
        status = function_ ? reinterpret_cast<ModuleEntry>(entry_)(function_, &call_, &error)
                           : reinterpret_cast<Entry>(entry_)(&call_, &error);
      }
    }
    if (misaligned) throw py::value_error("a native output has insufficient pointer alignment");
    if (status) {
      error.message[sizeof(error.message) - 1] = '\0';
      auto type = py::module_::import("tensor_amd._native").attr("HipError");
      auto exception = type(name_, status, std::string(error.message));
      PyErr_SetObject(type.ptr(), exception.ptr());
      throw py::error_already_set();
    }
    if (fixed_) return py::none();
    if (outputs_.size() == 1) return py::reinterpret_steal<py::object>(THPVariable_Wrap(tensors[inputs_.size()]));
    py::tuple result(outputs_.size());
    for (size_t i = 0; i < outputs_.size(); ++i)
      result[i] = py::reinterpret_steal<py::object>(THPVariable_Wrap(tensors[inputs_.size() + i]));
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
