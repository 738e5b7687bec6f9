// gguf.hpp -- the GGUF byte path of the quantized-matmul weights: parse a GGUF file's
// header, metadata and tensor table, and move a tensor's raw block bytes to a device.
//
// Restates Light's gguf package for this path (gguf/reader.go, gguf/types.go): the same
// structural checks and error texts at Open, lazily read tensor payloads, TensorBytes /
// Tensor / TensorRowMajor (gguf/reader.go:214-265), and the byte-level gate/up expert
// fusion of the MoE loader (models/llama_gguf.go:174-196).  Tensors keep their GGUF
// block bytes unchanged, which is the layout every libhipq kernel reads, so a loaded
// weight goes to the device with one copy and no repack.
#pragma once

#include <stdint.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "light.hpp"

namespace light {
namespace gguf {

constexpr uint32_t kMagic = 0x46554747;  // "GGUF" (gguf/types.go:10)
constexpr uint32_t kMinVersion = 2, kMaxVersion = 3;

// Metadata value types (gguf/types.go:19-33).
enum ValueType : uint32_t {
  TypeUInt8 = 0, TypeInt8 = 1, TypeUInt16 = 2, TypeInt16 = 3, TypeUInt32 = 4, TypeInt32 = 5,
  TypeFloat32 = 6, TypeBool = 7, TypeString = 8, TypeArray = 9, TypeUInt64 = 10, TypeInt64 = 11,
  TypeFloat64 = 12,
};

// One decoded metadata value: `type` says which member holds it (integers of every width
// in i or u by signedness, both float widths in f).
struct Value {
  uint32_t type = TypeUInt8;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0;
  bool b = false;
  std::string s;
  std::vector<Value> arr;
};

// Random-access input (io.ReaderAt), with its size when it can be learned (-1 otherwise).
class Source {
 public:
  virtual ~Source() = default;
  virtual int64_t Size() const = 0;
  // Copies n bytes at off into dst; throws Error on a short read.
  virtual void ReadAt(void *dst, size_t n, int64_t off) const = 0;
  // A stable pointer to [off, off + n) when the whole input is addressable (memory,
  // mapped file), else nullptr.
  virtual const uint8_t *Direct(int64_t off, size_t n) const { return nullptr; }
};
// In-memory bytes; sized = false hides the size (an input of unknown length).
std::shared_ptr<Source> MemorySource(std::vector<uint8_t> bytes, bool sized = true);
// A file mapped read-only.
std::shared_ptr<Source> FileSource(const std::string &path);

struct TensorInfo {
  std::string name;
  DType dtype = DType::F32;
  std::vector<int64_t> dims;  // file order, innermost first (ne[0] is contiguous)
  uint64_t offset = 0;        // relative to the data section
  int64_t bytes = 0;          // payload length
};

class File {
 public:
  // gguf.Open: parses and validates the header, metadata and tensor table.
  static std::shared_ptr<File> Open(std::shared_ptr<Source> src);

  uint32_t version = 0;
  std::map<std::string, Value> meta;
  std::map<std::string, TensorInfo> tensors;
  std::vector<std::string> order;      // tensor names in declaration order
  std::vector<std::string> key_order;  // metadata keys in declaration order
  int64_t data_base = 0;

  const TensorInfo &Info(const std::string &name) const;  // "gguf: tensor %q not found"
  std::vector<uint8_t> TensorBytes(const std::string &name) const;
  // Dims in file order.
  Tensor LoadTensor(const std::string &name, Device dev) const;
  // Dims reversed into row-major order: a Linear weight [in, out] in the file is (out, in).
  Tensor TensorRowMajor(const std::string &name, Device dev) const;
  // Copies the payload of `name` into dst (bytes = the payload length) on dst's device.
  void CopyTensorTo(const std::string &name, void *dst, Device dev) const;
  // The payload bytes: a pointer into the input when it is addressable (memory, mapped
  // file), else read into *tmp.
  const uint8_t *Payload(const std::string &name, std::vector<uint8_t> *tmp) const;

  bool String(const std::string &key, std::string *out) const;
  bool Int64(const std::string &key, int64_t *out) const;
  bool Float64(const std::string &key, double *out) const;

 private:
  // The tensor's byte range is addressable and its last byte readable (before allocation).
  void ProbeData(const TensorInfo &ti, const std::string &name) const;
  std::shared_ptr<Source> src_;
};

// The MoE expert stacks of one layer (prefix "blk.N."): gate and up fused byte-wise into
// one (E, 2I, H) tensor -- expert e's I gate rows, then its I up rows, the layout
// moe_gemm_q's gated and plain launches read -- and down as (E, H, I) row-major.  F16 /
// BF16 stacks are widened to F32, as Light casts them (models/llama_gguf.go:202-206).
struct ExpertStacks {
  Tensor gate_up, down;
};
ExpertStacks LoadExperts(const File &f, const std::string &prefix, Device dev);

// ggml type code <-> Light dtype (gguf/types.go:61-156).
DType DTypeFromGGML(uint32_t t);

}  // namespace gguf
}  // namespace light
