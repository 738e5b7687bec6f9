// light.hpp -- host-side mirror of Light's boundary types for the quantized matmul path.
//
// Light's host code is Go; this C++ layer restates the parts of its API that sit above
// the operator boundary for this path, with the same names, argument meanings and
// error behaviour, and calls libhipq's C ABI (include/hipq.h) below it:
//   DType          dtype/dtype.go:10-102   (codes, block sizes, ByteSize)
//   Device         device/device.go:9-50   (kinds; KindROCm is the new backend)
//   Storage/Tensor storage/, tensor/       (contiguous tensors on one device)
//   Error          Go `error`: an exception carrying the message; kernel-not-found is
//                  distinguishable like errors.Is(err, registry.ErrKernelNotFound)
#pragma once

#include <stdint.h>

#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace light {

// dtype.DType (dtype/dtype.go:13-37).
enum class DType : uint8_t {
  F16, BF16, F32, F64, U8, I8, U16, I16, U32, I32, U64, I64, F8E4M3,
  Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K,
};
const char *DTypeName(DType d);
int BlockElems(DType d);
int BlockBytes(DType d);
int64_t ByteSize(DType d, int64_t n);  // dtype.ByteSize (dtype/dtype.go:95-102)
inline bool IsQuantized(DType d) { return d >= DType::Q4_0; }

// device.Kind (device/device.go:9-15) plus the ROCm backend this library adds.
enum class DeviceKind : uint8_t { CPU = 0, CUDA = 1, WebGPU = 2, ROCm = 3 };
const char *KindName(DeviceKind k);
struct Device {
  DeviceKind kind = DeviceKind::CPU;
  int ordinal = 0;
  bool SameAs(const Device &o) const { return kind == o.kind && ordinal == o.ordinal; }
  std::string str() const;
};
inline Device CPU() { return Device{DeviceKind::CPU, 0}; }
inline Device ROCm(int i = 0) { return Device{DeviceKind::ROCm, i}; }

// A Go error: the message, and whether it wraps registry.ErrKernelNotFound.
class Error : public std::runtime_error {
 public:
  explicit Error(const std::string &m, bool not_found = false) : std::runtime_error(m), not_found_(not_found) {}
  bool IsKernelNotFound() const { return not_found_; }

 private:
  bool not_found_;
};
[[noreturn]] void Fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
// libhipq return code -> Error with hq_last_error().
void Check(int rc);

// Refcounted bytes on one device (storage.Storage).  ROCm bytes come from hq_malloc.
class Storage {
 public:
  Storage(Device dev, size_t bytes);                       // owning
  Storage(Device dev, void *ptr, size_t bytes, bool owned);  // wrap
  ~Storage();
  Storage(const Storage &) = delete;
  Storage &operator=(const Storage &) = delete;
  void *ptr() const { return ptr_; }
  size_t bytes() const { return bytes_; }
  const Device &device() const { return dev_; }

 private:
  Device dev_;
  void *ptr_ = nullptr;
  size_t bytes_ = 0;
  bool owned_ = false;
};

// A contiguous tensor (shape + element offset into a storage).  Quantized dtypes count
// logical elements; their bytes are ByteSize(dtype, n) as in Light.
class Tensor {
 public:
  Tensor() = default;
  static Tensor Empty(DType dt, std::vector<int64_t> shape, Device dev);  // tensor.Empty
  static Tensor Zeros(DType dt, std::vector<int64_t> shape, Device dev);  // tensor.Zeros
  // tensor.FromBytes / tensor.New: copy host bytes to a new tensor on dev.
  static Tensor FromHost(const void *src, size_t bytes, DType dt, std::vector<int64_t> shape, Device dev);
  // Borrow memory owned elsewhere (a device pointer from another framework).
  static Tensor Wrap(void *ptr, DType dt, std::vector<int64_t> shape, Device dev);

  bool defined() const { return st_ != nullptr; }
  DType dtype() const { return dt_; }
  const std::vector<int64_t> &shape() const { return shape_; }
  int Rank() const { return (int)shape_.size(); }
  int64_t Dim(int i) const { return shape_.at(i < 0 ? i + Rank() : i); }
  int64_t NumElements() const;
  int64_t Offset() const { return offset_; }
  Device device() const;
  // Byte address of element Offset() (the CUDAPtr() + offset of storage/cuda.go:373-378).
  void *data() const;
  size_t nbytes() const { return (size_t)ByteSize(dt_, NumElements()); }
  // Same storage, new shape (Reshape of a contiguous tensor).
  Tensor Reshape(std::vector<int64_t> shape) const;
  // Copy to host bytes (tensor.To(CPU) + CPUBytes).
  void ToHost(void *dst, size_t bytes) const;
  std::string ShapeStr() const;

 private:
  std::shared_ptr<Storage> st_;
  DType dt_ = DType::F32;
  std::vector<int64_t> shape_;
  int64_t offset_ = 0;
};

}  // namespace light
