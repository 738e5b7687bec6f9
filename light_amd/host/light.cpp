// light.cpp -- DType tables, Device, Storage and Tensor of the host layer.
#include "light.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/hipq.h"
#include "registry.hpp"

namespace light {

namespace {
// blockInfo (dtype/dtype.go:53-60): {elements per block, bytes per block}.
const int kBlock[][2] = {
    {1, 2}, {1, 2}, {1, 4}, {1, 8}, {1, 1}, {1, 1}, {1, 2}, {1, 2}, {1, 4}, {1, 4}, {1, 8}, {1, 8}, {1, 1},
    {32, 18}, {32, 20}, {32, 22}, {32, 24}, {32, 34}, {32, 36}, {256, 84}, {256, 110}, {256, 144}, {256, 176},
    {256, 210}, {256, 292},
};
const char *kNames[] = {"F16",  "BF16", "F32",  "F64",  "U8",   "I8",   "U16",  "I16",  "U32",
                        "I32",  "U64",  "I64",  "F8E4M3", "Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0",
                        "Q8_1", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_K"};
constexpr int kNumDTypes = sizeof(kNames) / sizeof(kNames[0]);
}  // namespace

const char *DTypeName(DType d) { return (int)d < kNumDTypes ? kNames[(int)d] : "DType(?)"; }
int BlockElems(DType d) { return (int)d < kNumDTypes ? kBlock[(int)d][0] : 0; }
int BlockBytes(DType d) { return (int)d < kNumDTypes ? kBlock[(int)d][1] : 0; }
int64_t ByteSize(DType d, int64_t n) {
  if ((int)d >= kNumDTypes || n < 0) return 0;
  const int64_t be = kBlock[(int)d][0];
  return (n + be - 1) / be * kBlock[(int)d][1];
}

const char *KindName(DeviceKind k) {
  switch (k) {
    case DeviceKind::CPU: return "CPU";
    case DeviceKind::CUDA: return "CUDA";
    case DeviceKind::WebGPU: return "WebGPU";
    case DeviceKind::ROCm: return "ROCm";
  }
  return "?";
}

// Device.String (device/device.go:59, device/cuda.go:20): "CPU", "ROCm(0)".
std::string Device::str() const {
  if (kind == DeviceKind::CPU) return "CPU";
  return std::string(KindName(kind)) + "(" + std::to_string(ordinal) + ")";
}

void Fail(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw Error(buf);
}

void Check(int rc) {
  if (rc != 0) throw Error(hq_last_error());
}

// ---- Storage ----

static void set_device(const Device &d) {
  if (d.kind == DeviceKind::ROCm) Check(hq_set_device(d.ordinal));
}

Storage::Storage(Device dev, size_t bytes) : dev_(dev), bytes_(bytes), owned_(true) {
  if (dev.kind == DeviceKind::CPU) {
    ptr_ = bytes ? ::operator new(bytes) : nullptr;
  } else if (dev.kind == DeviceKind::ROCm) {
    set_device(dev);
    Check(hq_malloc(&ptr_, bytes));
  } else {
    Fail("storage: device %s is not supported by this build", dev.str().c_str());
  }
}

Storage::Storage(Device dev, void *ptr, size_t bytes, bool owned) : dev_(dev), ptr_(ptr), bytes_(bytes), owned_(owned) {}

Storage::~Storage() {
  if (!owned_ || !ptr_) return;
  if (dev_.kind == DeviceKind::CPU)
    ::operator delete(ptr_);
  else if (dev_.kind == DeviceKind::ROCm)
    hq_free(ptr_);
}

// ---- Tensor ----

int64_t Tensor::NumElements() const {
  int64_t n = 1;
  for (int64_t d : shape_) n *= d;
  return n;
}

Device Tensor::device() const { return st_ ? st_->device() : CPU(); }

void *Tensor::data() const {
  if (!st_) return nullptr;
  return static_cast<char *>(st_->ptr()) + ByteSize(dt_, offset_);
}

std::string Tensor::ShapeStr() const {
  std::string s = "[";
  for (size_t i = 0; i < shape_.size(); i++) s += (i ? " " : "") + std::to_string(shape_[i]);
  return s + "]";
}

static void check_shape(const std::vector<int64_t> &shape) {
  for (int64_t d : shape)
    if (d < 0) Fail("tensor: negative dimension in shape");
}

Tensor Tensor::Empty(DType dt, std::vector<int64_t> shape, Device dev) {
  check_shape(shape);
  Tensor t;
  t.dt_ = dt;
  t.shape_ = std::move(shape);
  t.st_ = std::make_shared<Storage>(dev, (size_t)ByteSize(dt, t.NumElements()));
  return t;
}

Tensor Tensor::Zeros(DType dt, std::vector<int64_t> shape, Device dev) {
  Tensor t = Empty(dt, std::move(shape), dev);
  if (!t.nbytes()) return t;
  if (dev.kind == DeviceKind::CPU)
    memset(t.data(), 0, t.nbytes());
  else
    Check(hq_memset(t.data(), 0, t.nbytes(), nullptr));
  return t;
}

Tensor Tensor::FromHost(const void *src, size_t bytes, DType dt, std::vector<int64_t> shape, Device dev) {
  Tensor t = Empty(dt, std::move(shape), dev);
  if (bytes != t.nbytes())
    Fail("tensor.FromBytes: %zu bytes for %s %s (want %zu)", bytes, DTypeName(dt), t.ShapeStr().c_str(), t.nbytes());
  if (!bytes) return t;
  if (dev.kind == DeviceKind::CPU)
    memcpy(t.data(), src, bytes);
  else
    Check(hq_memcpy_h2d(t.data(), src, bytes, nullptr));
  return t;
}

Tensor Tensor::Wrap(void *ptr, DType dt, std::vector<int64_t> shape, Device dev) {
  check_shape(shape);
  Tensor t;
  t.dt_ = dt;
  t.shape_ = std::move(shape);
  t.st_ = std::make_shared<Storage>(dev, ptr, (size_t)ByteSize(dt, t.NumElements()), false);
  return t;
}

Tensor Tensor::Reshape(std::vector<int64_t> shape) const {
  Tensor t = *this;
  t.shape_ = std::move(shape);
  if (t.NumElements() != NumElements())
    Fail("tensor: cannot reshape %s to %s", ShapeStr().c_str(), t.ShapeStr().c_str());
  return t;
}

void Tensor::ToHost(void *dst, size_t bytes) const {
  if (bytes != nbytes()) Fail("tensor: ToHost of %zu bytes from a %zu-byte tensor", bytes, nbytes());
  if (!bytes) return;
  if (device().kind == DeviceKind::CPU)
    memcpy(dst, data(), bytes);
  else
    Check(hq_memcpy_d2h(dst, data(), bytes, nullptr));
}

// ---- registry (internal/registry/registry.go) ----

// Key.String (registry.go:20-22): "op/Kind/DType".

std::string Key::str() const { return op + "/" + KindName(dev) + "/" + DTypeName(dtype); }

bool Key::operator<(const Key &o) const {
  if (op != o.op) return op < o.op;
  if (dev != o.dev) return dev < o.dev;
  return dtype < o.dtype;
}

int64_t Context::attr(const std::string &k) const {
  auto it = attrs.find(k);
  if (it == attrs.end()) Fail("registry: missing attribute %s", k.c_str());
  return it->second.i;
}

namespace {
std::mutex &reg_mu() {
  static std::mutex mu;
  return mu;
}
std::map<Key, Kernel> &kernels() {
  static std::map<Key, Kernel> k;
  return k;
}
}  // namespace

void Register(const Key &k, Kernel fn) {
  std::lock_guard<std::mutex> lk(reg_mu());
  if (kernels().count(k)) throw std::logic_error("registry: duplicate kernel for " + k.str());
  kernels()[k] = std::move(fn);
}

Kernel Lookup(const Key &k) {
  std::lock_guard<std::mutex> lk(reg_mu());
  auto it = kernels().find(k);
  if (it == kernels().end()) throw Error("registry: kernel not found: " + k.str(), true);
  return it->second;
}

std::vector<Key> Registered() {
  std::lock_guard<std::mutex> lk(reg_mu());
  std::vector<Key> out;
  for (auto &kv : kernels()) out.push_back(kv.first);
  return out;
}

}  // namespace light
